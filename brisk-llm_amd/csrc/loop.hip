// The persistent token loop: one launch runs n_steps forward steps.
//
// Every workgroup of the grid (one per CU) stays resident for the launch and
// walks the same phases as the one-kernel-per-phase path:
//
//   per layer:  A  Q/K/V rows of attn_norm(h)                 (src/model.cpp:996-1015)
//               B  Q/K norms, RoPE, K/V cache write, attention (:1020-1093)
//               C  O rows of (sub-normed) att, residual add    (:1095-1111)
//               D  gate/up rows of ffn_norm(h), SiLU / relu^2  (:1111-1143)
//               F  down rows of (sub-normed) act, residual add (:1144-1162)
//   full steps: H  output_norm(h) -> output rows -> logits and the greedy pick
//
// There are no grid barriers.  Every vector one phase hands to the next (q, k,
// v, att, h, act, attention partials) is stored as 64-bit words, each holding a
// value and the tag of the (step, layer, phase) that produced it, written with
// one system-scope store (which goes past the per-XCD L2s).  A consumer polls
// the words it needs until their tags match, so a hand-off costs one memory
// round trip.  A buffer is only rewritten after all its readers are done with
// it: every producer of a phase has consumed, directly or through the phases in
// between, the outputs of every reader of the previous contents.  The greedy
// pick is the one all-to-all wait: each workgroup of phase H folds its best
// (logit, index) into the step's key, then counts itself done; the next step
// starts from the key once all have.  Waits are bounded: on expiry a workgroup
// raises the error flag and every waiter leaves, so a launch always drains.
#include "phases.h"
#include "loop.h"

namespace bh {

constexpr unsigned kSpinLimit = 1u << 24;

// A field of a layer descriptor (read-only for the launch), read through the
// constant address space: the compiler reads it with scalar loads, which go
// through the scalar cache and are counted by lgkmcnt, so the read does not
// wait for the vector memory operations in flight (weight loads issued ahead,
// hand-off stores); a vector load of it would, as the vector memory counter
// retires in order.
template <class T>
__device__ __forceinline__ T sld(const T* p) {
    static_assert(sizeof(T) % 4 == 0 && alignof(T) >= 4, "sld: whole dwords");
    typedef const __attribute__((address_space(4))) uint32_t* cptr;
    uint32_t w[sizeof(T) / 4];
#pragma unroll
    for (size_t i = 0; i < sizeof(T) / 4; ++i) w[i] = ((cptr)p)[i];
    T v;
    __builtin_memcpy(&v, w, sizeof(T));
    return v;
}

__device__ __forceinline__ bool loop_failed(const LoopArgs& g) {
    return __hip_atomic_load(g.error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Tagged values into LDS, by the whole workgroup: up to three (src, dst, n)
// segments awaited together; false when the launch is being abandoned.
struct TSeg {
    const unsigned long long* src;
    float* dst;
    int n;
};

// Tagged values into LDS: word i of n at at(i) -> (src, dst), by the whole
// workgroup (kWg, ends with a barrier) or by one wave (no barrier).  Each thread
// requests kGetPer words before checking any, so a round costs one memory round
// trip.  While words are missing, each wave polls a single word (the first
// missing word of its lowest lane still waiting, the same address in every
// lane, one memory request), then fetches its missing words again: polling
// traffic stays at one request a wave, so it does not queue the weight and
// cache loads of the compute units behind it.  False when abandoning.
template <int kGetPer, bool kWg, class At>
__device__ __forceinline__ bool tgather(const LoopArgs& g, unsigned tag, int n, At at) {
    const int nt = kWg ? kThreads : 64, me = kWg ? static_cast<int>(threadIdx.x) : static_cast<int>(threadIdx.x & 63);
    bool fail = false;
    for (int base0 = 0; base0 < n && !fail; base0 += kGetPer * nt) {
        const int base = base0 + me;
        unsigned long long w[kGetPer];
        const unsigned long long* src[kGetPer];
        float* dst[kGetPer];
        bool have[kGetPer];
#pragma unroll
        for (int u = 0; u < kGetPer; ++u) {
            const int i = base + u * nt;
            have[u] = i >= n;
            at(i < n ? i : n - 1, src[u], dst[u]);  // unconditional loads (no branches between them)
            w[u] = tload(src[u]);
        }
        unsigned spins = 0;
        while (true) {
            bool all = true;
            const unsigned long long* first = src[0];
#pragma unroll
            for (int u = kGetPer - 1; u >= 0; --u) {
                if (!have[u]) {
                    if (static_cast<unsigned>(w[u] >> 32) == tag) {
                        *dst[u] = __uint_as_float(static_cast<unsigned>(w[u]));
                        have[u] = true;
                    } else {
                        first = src[u];
                        all = false;
                    }
                }
            }
            const unsigned long long miss = __ballot(!all);
            if (miss == 0) break;
            const int leader = __ffsll(static_cast<long long>(miss)) - 1;
            const uintptr_t fa = reinterpret_cast<uintptr_t>(first);
            const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(fa), leader);
            const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(fa >> 32), leader);
            const unsigned long long* poll = reinterpret_cast<const unsigned long long*>((static_cast<uintptr_t>(hi) << 32) | lo);
            while (static_cast<unsigned>(tload(poll) >> 32) != tag) {
                if (++spins > kSpinLimit) {
                    atomicExch(g.error, 1);
                    fail = true;
                    break;
                }
                if ((spins & 63) == 0 && loop_failed(g)) {
                    fail = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            if (fail) break;
#pragma unroll
            for (int u = 0; u < kGetPer; ++u)
                if (!have[u]) w[u] = tload(src[u]);
        }
    }
    if (kWg) return !__syncthreads_or(fail);
    return !fail;
}

template <int kGetPer = 4>
__device__ __forceinline__ bool tget_segs(const LoopArgs& g, unsigned tag, TSeg s0, TSeg s1 = TSeg{nullptr, nullptr, 0},
                                          TSeg s2 = TSeg{nullptr, nullptr, 0}) {
    const int n01 = s0.n + s1.n, n = n01 + s2.n;
    return tgather<kGetPer, true>(g, tag, n, [&](int i, const unsigned long long*& src, float*& dst) {
        if (i < s0.n) { src = s0.src + i; dst = s0.dst + i; }
        else if (i < n01) { src = s1.src + (i - s0.n); dst = s1.dst + (i - s0.n); }
        else { src = s2.src + (i - n01); dst = s2.dst + (i - n01); }
    });
}

__device__ __forceinline__ bool tget_vec(const LoopArgs& g, const unsigned long long* src, unsigned tag, float* dst, int n) {
    return tget_segs<>(g, tag, TSeg{src, dst, n});
}

// One tagged value (a residual row), by one thread.
__device__ __forceinline__ bool tget_one(const LoopArgs& g, const unsigned long long* src, unsigned tag, float& v) {
    unsigned spins = 0;
    unsigned long long w;
    while (static_cast<unsigned>((w = tload(src)) >> 32) != tag) {
        if (++spins > kSpinLimit) {
            atomicExch(g.error, 1);
            return false;
        }
        if ((spins & 63) == 0 && loop_failed(g)) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    v = __uint_as_float(static_cast<unsigned>(w));
    return true;
}

template <int kGetPer, class At>
__device__ __forceinline__ bool tget_fn(const LoopArgs& g, unsigned tag, int n, At at) {
    return tgather<kGetPer, true>(g, tag, n, at);
}

// ---------------------------------------------------------------- shared memory

constexpr int kGroupRows = kThreads;  // rows of one tile group (one summing lane each)

struct GemvLds {
    ActLds a;
    ActLds a2;  // the pushed phase D's activation block (block 0)
    alignas(16) float terms[kTermCap];
    float sums[kGroupRows];
    float sums2[64];
    double red[4];
    float x[kMaxCols];  // the phase's input vector
};
// The spread exact attention (phase_b_spread): stage 1 scores a chunk of
// positions, stage 2 turns a head's scores into weights and sums one 32-wide
// slice of the values, streaming the cached values in chunks of positions.
constexpr int kSpreadSlice = 32;                 // value dimensions a stage-2 task (one Q8_0 block a head)
constexpr int kSpreadHpk = 4;                    // query heads a key/value head, at most
constexpr int kSpreadChunk = 320;                // positions a stage-1 task, at most
constexpr int kSpreadScores = 16384;             // heads-per-kv x positions (padded to 8), at most
constexpr int kSpreadStage = 256;                // positions a stage-2 chunk
constexpr int kVtStride = kSpreadStage + 8;      // halves a transposed value row (16-byte aligned, banks staggered)
// s_waitcnt vmcnt(N), other counters unconstrained (gfx9 encoding: vmcnt bits 3:0 and 15:14,
// expcnt 6:4, lgkmcnt 11:8)
template <int N>
__device__ __forceinline__ void wait_vm_le() {
    static_assert(N >= 0 && N < 16, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

struct SpreadStage1 {
    alignas(16) float q[kSpreadHpk * 128];       // the query heads, normed and rotated
    alignas(16) float kcur[128];                 // (writer) this token's key
    alignas(16) uint16_t kst[kSpreadChunk * 128];   // the chunk's keys [position][dim]
};
struct SpreadStage2 {
    alignas(16) float kcur[128];                 // this token's key (its cache row)
    alignas(16) float vcur[kSpreadSlice];        // this token's values of the slice
    alignas(16) float sc[kSpreadScores];         // scores, then weights: [head][position, rows padded to 8]
    alignas(16) uint16_t vraw[2][kSpreadStage * kSpreadSlice];  // cached values of two chunks [position][dim]
    alignas(16) uint16_t vt[2][kSpreadSlice * kVtStride];       // the same, transposed [dim][position]
    float mx[kSpreadHpk][4];     // [head][wave]
    double red[kSpreadHpk][4];
};
union SpreadLds {
    SpreadStage1 s1;
    SpreadStage2 s2;
};

// The resident attention (short contexts): workgroup b < heads * (head_dim / 64)
// takes query head b / (head_dim / 64) and a 64-wide slice of its values.  It
// holds the layer's cached keys of that head's kv head and its value slice,
// transposed, in LDS.  They are loaded after the workgroup's attention of the
// layer before (at the start of a step for layer 0), while the other phases
// run, so the attention itself waits only for this token's q, k and v.
constexpr int kResMax = 320;                     // positions (this token's included)
constexpr int kResSlice = 64;                    // value dimensions a task (one wave of chains)
constexpr int kResVt = kResMax + 8;              // halves a transposed value row (16-byte aligned)
constexpr int kResStage = 128;                   // value rows staged at a time for the transpose
struct ResLds {
    alignas(16) uint16_t keys[kResMax * 128];    // [position][dim], 16-byte pieces swizzled by position
    alignas(16) uint16_t vt[kResSlice * kResVt];                // [dim][position]
    alignas(16) uint16_t vstage[kResStage * kResSlice];         // value rows [position][dim]
    alignas(16) float sc[kResVt];                // scores, then weights
    alignas(16) float q[128];
    alignas(16) float kcur[128];
    alignas(16) float vcur[kResSlice];
    float mx[4];
    double red[4];
};

union LoopLds {
    GemvLds g;
    AttnLds att;
    AttnPoolLds pool;
    SpreadLds spread;
    ResLds res;
};

// Trace: workgroup 0's wall clock at point `pt` of phase `ph` of every (step,
// layer), and every workgroup's at one chosen (step, layer) (trace_step, trace_layer).
struct Stamps {
    unsigned long long* w0;
    unsigned long long* all;
};
constexpr int kTraceW0 = 65536, kTraceAll = 1 << 19;
__device__ __forceinline__ Stamps pst_ptr(const LoopArgs& g, int step, int l, int ph) {
    Stamps st{nullptr, nullptr};
    if (g.trace == nullptr) return st;
    if (blockIdx.x == 0) st.w0 = g.trace + kTraceW0 + (static_cast<size_t>(step * g.n_layers + l) * 8 + ph) * 8;
    if (step == g.trace_step && l == g.trace_layer) st.all = g.trace + kTraceAll + static_cast<size_t>(ph) * 8 * 1024;
    return st;
}
__device__ __forceinline__ void pst(const Stamps& st, int pt) {
    if (threadIdx.x == 0 && (st.w0 != nullptr || st.all != nullptr)) {
        const unsigned long long t = wall_clock64();
        if (st.w0 != nullptr) st.w0[pt] = t;
        if (st.all != nullptr) {
            st.all[pt * 1024 + blockIdx.x] = t;
            st.all[65536 + pt * 1024 + blockIdx.x] = clock64();
        }
    }
}

__device__ __forceinline__ unsigned tag_of(const LoopArgs& g, int step, int layer, int phase) {
    return g.tag_base + static_cast<unsigned>((step * g.n_layers + layer) * 8 + phase);
}

// Quantised activation of the input vector in s.x (rms_norm'd by w when given).
// The norm weight chunks are in `ar` already (act_issue_w, before the input wait).
template <uint32_t T>
__device__ __forceinline__ void prologue_lds(const Packed& m, ActRegs& ar, const float* w, float eps, GemvLds& s) {
    const int cols = static_cast<int>(m.cols);
    act_issue_x<PlainIO>(ar, s.x, cols);
    act_finish<PlainIO>(ar, s.x, w, eps, cols, takes_q8_k(T), act_bits(m), s.a, s.red);
}

// The embedding row of `token` (embedding_row, src/model.cpp:27-70) into s.x.
// The loop is built for an embedding of its output's format (find_loop_kernel checks it).
template <uint32_t TE>
__device__ __forceinline__ void embed_to_lds(const LoopArgs& g, int token, GemvLds& s) {
    for (uint32_t e = threadIdx.x; e < g.embd.cols; e += kThreads) s.x[e] = dequant_elem<TE>(g.embd, static_cast<uint32_t>(token), e);
    __syncthreads();
}

constexpr int kLoopUnits = 2;  // units per thread in the loop's tiles (the tile plan keeps to it)
// ... in the output projection's tiles (fewer for the K-quant formats' larger units)
__host__ __device__ constexpr int head_units(uint32_t type) { return (type == kQ4_K || type == kQ5_K || type == kQ6_K) ? 2 : 4; }

// The tiles t = blockIdx.x, + G, ... of a phase, streamed one ahead: a tile's
// weights are requested before the phase's input has arrived and before the
// previous tile is computed, so their latency overlaps the wait and the work.
// `row_of(t, m, R)` maps a tile to (matrix, first row); `done(t, sums)` is the
// epilogue.  `ready()` waits for the input and prepares the activation; it runs
// once, after the first tile's loads are issued.  Returns false when abandoning.
// The tiles go to workgroups first, first + 1, ... (first > 0 keeps the first
// workgroups, busy elsewhere, out of the phase).
template <uint32_t T, int M, class RowOf, class Ready, class Done>
__device__ __forceinline__ bool run_tiles(int total, GemvLds& s, RowOf row_of, Ready ready, Done done,
                                          Stamps st = Stamps{nullptr, nullptr}, int first = 0, int count = 0) {
    const int G = count > 0 ? count : static_cast<int>(gridDim.x) - first;
    int t = static_cast<int>(blockIdx.x) - first;
    if (t < 0 || t >= total || t >= G) return true;
    Tile<T, M> ta, tb;
    Packed ma, mb;  // by value: a pointer to a kernel-argument member would force a private copy
    uint32_t ra, rb = 0;
    int Ra, Rb = 0;
    row_of(t, ma, ra, Ra);
    ta.load(ma, ra, Ra);
    if (!ready()) return false;
    // Tiles go in groups: their terms side by side in LDS, then one row-sum pass
    // for all the group's rows (one lane a row), so a workgroup with several
    // tiles pays the serial block-order sum once, not once a tile.
    const uint32_t units = ma.cols / Unit<T>::kElems, stride = term_stride(units);
    int gfirst = t, grows = 0;
    auto flush = [&]() -> bool {
        pst(st, 3);
        __syncthreads();
        row_sums(s.terms, stride, units, grows, s.sums);
        __syncthreads();
        pst(st, 4);
        int off = 0;
        for (int u = gfirst; off < grows; u += G) {
            Packed mu;
            uint32_t r0;
            int Ru;
            row_of(u, mu, r0, Ru);
            if (!done(u, mu, r0, s.sums + off)) return false;
            off += Ru;
        }
        pst(st, 5);
        grows = 0;
        return true;
    };
    auto fits = [&](int more) { return (grows + more) * static_cast<int>(stride) <= kTermCap && grows + more <= kGroupRows; };
    // the next tile's loads are issued on every path (the last tile re-reads
    // itself), so the wait for the current tile leaves them in flight
    while (true) {
        row_of(t + G < total ? t + G : t, mb, rb, Rb);
        tb.load(mb, rb, Rb);
        ta.terms(ma, s.a, s.terms + grows * stride);
        grows += Ra;
        if (t + G >= total || !fits(Rb)) {
            if (!flush()) return false;
            gfirst = t + G;
        }
        t += G;
        if (t >= total) break;
        row_of(t + G < total ? t + G : t, ma, ra, Ra);
        ta.load(ma, ra, Ra);
        tb.terms(mb, s.a, s.terms + grows * stride);
        grows += Rb;
        if (t + G >= total || !fits(Ra)) {
            if (!flush()) return false;
            gfirst = t + G;
        }
        t += G;
        if (t >= total) break;
    }
    return true;
}

// ---------------------------------------------------------------- phases

// Bytes a block takes in each of a matrix's planes (plane_bytes for one block).
__device__ __forceinline__ void block_plane_bytes(uint32_t type, uint32_t (&b)[3]) {
    b[0] = b[1] = b[2] = 0;
    switch (type) {
        case kQ4_0: b[0] = 16; b[1] = 2; break;
        case kQ4_1: b[0] = 16; b[1] = 2; b[2] = 2; break;
        case kQ5_0: b[0] = 16; b[1] = 2; b[2] = 4; break;
        case kQ8_0: b[0] = 32; b[1] = 2; break;
        case kQ4_K: b[0] = 128; b[1] = 16; b[2] = 16; break;
        case kQ5_K: b[0] = 128; b[1] = 16; b[2] = 48; break;
        case kQ6_K: b[0] = 128; b[1] = 64; b[2] = 20; break;
        case kTQ2_0: b[0] = 64; b[1] = 2; break;
        default: break;
    }
}

// Rows [row0, row0 + R) of m, every plane, one dword a 128-byte line (a line a thread, up to four
// a thread), loaded and waited for in one asm block (no register receives data after it ends).
__device__ __forceinline__ void touch_rows(const Packed& m, uint32_t row0, int R) {
    uint32_t b[3];
    block_plane_bytes(m.type, b);
    const size_t nb = m.cols / block_elems(m.type);
    const uint8_t* planes[3] = {m.p0, m.p1, m.p2};
    const uint8_t* addr[4];
    int n = 0;
    size_t line = threadIdx.x;
    for (int k = 0; k < 3 && n < 4; ++k) {
        if (b[k] == 0) continue;
        const size_t off = static_cast<size_t>(row0) * nb * b[k], len = static_cast<size_t>(R) * nb * b[k];
        const size_t lines = (len + 127) / 128;
        while (line < lines && n < 4) {
            addr[n++] = planes[k] + off + line * 128;
            line += kThreads;
        }
        line -= lines;  // this thread's line index in the next plane
    }
    if (n == 0) return;
    for (int i = n; i < 4; ++i) addr[i] = addr[0];
    uint32_t d0, d1, d2, d3;
    asm volatile(
        "global_load_dword %0, %4, off\n\t"
        "global_load_dword %1, %5, off\n\t"
        "global_load_dword %2, %6, off\n\t"
        "global_load_dword %3, %7, off\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(d0), "=&v"(d1), "=&v"(d2), "=&v"(d3)
        : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3])
        : "memory");
}

// The phase-A tile workgroup b takes in the layer of L (one-format Q/K/V, the plan run_tiles
// follows), touched into L2 by touch_rows.
__device__ __forceinline__ void a_touch(const LoopArgs& g, const LayerDev& L) {
    const int first = g.res_ok ? g.res_n : 0, G = static_cast<int>(gridDim.x) - first;
    const int nq = g.tiles_qkv[0] + g.tiles_qkv[1], total = nq + g.tiles_qkv[2];
    const int t = static_cast<int>(blockIdx.x) - first;  // the first tile: the loads run_tiles issues before its input wait
    if (t < 0 || t >= total || t >= G) return;
    const int i = t < g.tiles_qkv[0] ? 0 : t < nq ? 1 : 2;
    const int tt = i == 0 ? t : i == 1 ? t - g.tiles_qkv[0] : t - nq;
    const Packed m = i == 0 ? sld(&L.q) : i == 1 ? sld(&L.k) : sld(&L.v);
    const int R = g.R_qkv[i];
    const uint32_t row0 = static_cast<uint32_t>(tt) * R;
    touch_rows(m, row0, row0 + R <= m.rows ? R : static_cast<int>(m.rows - row0));
}

// A: Q, K, V rows (one format, or Q/K's and then V's).
template <uint32_t TQ, uint32_t TV, uint32_t TE>
__device__ __forceinline__ bool phase_a(const LoopArgs& g, const LayerDev& L, int step, int l, int token, GemvLds& s) {
    const Packed L_q = sld(&L.q);
    const Packed L_k = sld(&L.k);
    const Packed L_v = sld(&L.v);
    const float* L_attn_norm = sld(&L.attn_norm);
    const int nq = g.tiles_qkv[0] + g.tiles_qkv[1];
    const int total = nq + g.tiles_qkv[2];
    const unsigned tag = tag_of(g, step, l, 1);
    const Stamps st = pst_ptr(g, step, l, 0);
    auto input = [&]() -> bool {
        if (l == 0) {
            embed_to_lds<TE>(g, token, s);
            return true;
        }
        const bool ok = tget_vec(g, g.ht, tag_of(g, step, l - 1, 5), s.x, g.embd_dim);
        pst(st, 1);
        return ok;
    };
    auto row_of = [&](int t, Packed& m, uint32_t& row0, int& R) {
        const int i = t < g.tiles_qkv[0] ? 0 : t < nq ? 1 : 2;
        const int tt = i == 0 ? t : i == 1 ? t - g.tiles_qkv[0] : t - nq;
        m = i == 0 ? L_q : i == 1 ? L_k : L_v;
        R = g.R_qkv[i];
        row0 = static_cast<uint32_t>(tt) * R;
    };
    auto done = [&](int t, const Packed& m, uint32_t row0, const float* sums) -> bool {
        unsigned long long* out = t < g.tiles_qkv[0] ? g.qt : t < nq ? g.kt : g.vt;
        const int R = t < g.tiles_qkv[0] ? g.R_qkv[0] : t < nq ? g.R_qkv[1] : g.R_qkv[2];
        const uint32_t r = threadIdx.x;
        if (r < static_cast<uint32_t>(R) && row0 + r < m.rows) tput(out + row0 + r, sums[r], tag);
        return true;
    };
    if (TQ == TV) {
        auto ready = [&]() -> bool {
            ActRegs ar;
            act_issue_w(ar, L_attn_norm, static_cast<int>(L_q.cols));
            if (!input()) return false;
            prologue_lds<TQ>(L_q, ar, L_attn_norm, g.eps, s);
            pst(st, 2);
            return true;
        };
        // with the resident attention its workgroups (the first res_n) take no tiles
        return run_tiles<TQ, kLoopUnits>(total, s, row_of, ready, done, st, g.res_ok ? g.res_n : 0);
    }
    // Q and K in their format, then V's tiles (same activation family, its own width)
    if (static_cast<int>(blockIdx.x) >= total) return true;
    bool have_input = false;
    if (!run_tiles<TQ, kLoopUnits>(nq, s, row_of, [&]() -> bool {
            ActRegs ar;
            act_issue_w(ar, L_attn_norm, static_cast<int>(L_q.cols));
            if (!input()) return false;
            have_input = true;
            prologue_lds<TQ>(L_q, ar, L_attn_norm, g.eps, s);
            return true;
        }, done))
        return false;
    if (!have_input && !input()) return false;
    // V tiles continue round-robin after Q's and K's
    const int G = static_cast<int>(gridDim.x);
    const int first = nq % G, me = (static_cast<int>(blockIdx.x) - first + G) % G;
    if (me >= g.tiles_qkv[2]) return true;
    {
        ActRegs ar;
        act_issue_w(ar, L_attn_norm, static_cast<int>(L_v.cols));
        prologue_lds<TV>(L_v, ar, L_attn_norm, g.eps, s);
    }
    for (int t = me; t < g.tiles_qkv[2]; t += G) {
        const uint32_t row0 = static_cast<uint32_t>(t) * g.R_qkv[2];
        Tile<TV, kLoopUnits> tile;
        tile.load(L_v, row0, g.R_qkv[2]);
        tile.sums(L_v, s.a, s.terms, s.sums);
        done(nq + t, L_v, row0, s.sums);
    }
    return true;
}

__device__ __forceinline__ AttnArgs attn_args(const LoopArgs& g, const LayerDev& L, int step, int l) {
    const float* L_q_norm = sld(&L.q_norm);
    const float* L_k_norm = sld(&L.k_norm);
    const int L_rope = sld(&L.rope);
    const float* L_q_bias = sld(&L.q_bias);
    const float* L_k_bias = sld(&L.k_bias);
    const float* L_v_bias = sld(&L.v_bias);
    uint16_t* L_kc = sld(&L.kc);
    uint16_t* L_vc = sld(&L.vc);
    AttnArgs a{};
    a.qnorm = L_q_norm; a.knorm = L_k_norm; a.rope = L_rope ? g.rope : nullptr; a.eps = g.eps; a.neox = g.neox;
    a.qbias = L_q_bias; a.kbias = L_k_bias; a.vbias = L_v_bias; a.rope_dim = g.rope_dim;
    a.kcache = L_kc; a.vcache = L_vc; a.ctx = g.ctx; a.head_dim = g.head_dim; a.heads = g.heads;
    a.kv_heads = g.kv_heads; a.scale = g.scale; a.max_splits = g.max_splits;
    a.stamps = g.trace != nullptr ? g.trace + 65536 + (static_cast<size_t>(step * g.n_layers + l) * 8 + 1) * 8 : nullptr;
    return a;
}

// ---------------------------------------------------------------- per-head exact attention

// Tagged values into LDS by one wave (no barrier); false when abandoning.
template <int K>
__device__ __forceinline__ bool wget_segs(const LoopArgs& g, unsigned tag, TSeg s0, TSeg s1, TSeg s2) {
    const int n01 = s0.n + s1.n, n = n01 + s2.n;
    return tgather<K, false>(g, tag, n, [&](int i, const unsigned long long*& src, float*& dst) {
        if (i < s0.n) { src = s0.src + i; dst = s0.dst + i; }
        else if (i < n01) { src = s1.src + (i - s0.n); dst = s1.dst + (i - s0.n); }
        else { src = s2.src + (i - n01); dst = s2.dst + (i - n01); }
    });
}

// chunk_issue by the `nt` threads of rank 0 .. nt - 1 (nt a multiple of 64).
__device__ __forceinline__ void chunk_issue_by(uint16_t* lds, const uint16_t* base, int p0, int n_pos, int hd, bool swz, int rank,
                                               int nt) {
    const int P = kv_pieces(hd), mask = swz ? kv_mask(hd) : 0;
    const int pieces = n_pos * P;
    const uint8_t* src = reinterpret_cast<const uint8_t*>(base + static_cast<size_t>(p0) * hd);
    uint8_t* dst = reinterpret_cast<uint8_t*>(lds);
    const int wave_first = rank & ~63;
    for (int k = 0; k * nt < pieces; ++k) {
        const int i = k * nt + rank;
        if (i < pieces) {
            const int p = i / P, c = (i - p * P) ^ (p & mask);
            __builtin_amdgcn_global_load_lds((global_cvoid_ptr)(src + (static_cast<size_t>(p) * P + c) * 16),
                                             (lds_void_ptr)(dst + (k * nt + wave_first) * 16), 16, 0, 0);
        }
    }
}

// Attention of query head h on workgroup h, in the reference's order (scores
// by dot_f32's 16 lane partials, softmax with a double sum, value sums in
// position order; see attn_exact_pool).  Wave 0 awaits this token's q (head
// h), k and v (kv head h / hpk) while waves 1-3 stage the cached keys (and
// values), so the hand-off polls are not queued behind the cache loads.  Every
// query head of a kv head normalises and rotates the same k; the first one
// also stores the new cache rows (system-scope stores, complete before its
// outputs are published, for the other workgroups that read them in later
// steps).  Needs L <= kSplit * kPoolChunks.
template <int HD, class O>
__device__ __forceinline__ bool attn_head_pool(const LoopArgs& lg, const AttnArgs& g, AttnPoolLds& sp, int h, int pos, unsigned tin,
                                               const O& o) {
    AttnLds& s = sp.a;
    const int hd = HD != 0 ? HD : g.head_dim, hpk = g.heads / g.kv_heads, kv = h / hpk, t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63, L = pos + 1;
    const int n = pool_nchunks(L), last = (L - 1) / kSplit;
    const bool early = pool_values_early(L), writer = h % hpk == 0;
    const uint16_t* kbase = g.kcache + static_cast<size_t>(kv) * g.ctx * hd;
    const uint16_t* vbase = g.vcache + static_cast<size_t>(kv) * g.ctx * hd;
    bool fail = false;
    attn_stamp(g, h, 0);
    if (wave == 0) {
        fail = !wget_segs<8>(lg, tin, TSeg{lg.qt + h * hd, s.q, hd}, TSeg{lg.kt + kv * hd, s.kcur, hd},
                             TSeg{lg.vt + kv * hd, s.vcur, hd});
    } else {
        for (int c = 0; c < n; ++c) {
            const int nn = chunk_cached(c, L);
            if (nn > 0) chunk_issue_by(sp.chunk(c), kbase, c * kSplit, nn, hd, true, t - 64, kThreads - 64);
        }
        if (early)
            for (int c = 0; c < n; ++c) {
                const int nn = chunk_cached(c, L);
                if (nn > 0) chunk_issue_by(sp.chunk(n + c), vbase, c * kSplit, nn, hd, false, t - 64, kThreads - 64);
            }
    }
    if (__syncthreads_or(fail)) {
        __builtin_amdgcn_s_waitcnt(0);
        return false;
    }
    attn_stamp(g, h, 1);
    // q_norm / k_norm and RoPE (src/model.cpp:1026-1041), k and v rounded to fp16 as the cache holds them
    const float* rope = g.rope != nullptr ? g.rope + static_cast<size_t>(pos) * g.rope_dim : nullptr;
    if (wave == 0) head_norm_rope(s.q, g.qbias != nullptr ? g.qbias + h * hd : nullptr, g.qnorm, rope, hd, g.rope_dim, g.neox, g.eps);
    else if (wave == 1) {
        head_norm_rope(s.kcur, g.kbias != nullptr ? g.kbias + kv * hd : nullptr, g.knorm, rope, hd, g.rope_dim, g.neox, g.eps);
        for (int i = lane; i < hd; i += 64) s.kcur[i] = h2f(f2h(s.kcur[i]));
    } else if (wave == 2) {
        for (int i = lane; i < hd; i += 64) s.vcur[i] = h2f(f2h(g.vbias != nullptr ? s.vcur[i] + gmem(g.vbias)[kv * hd + i] : s.vcur[i]));
    }
    __builtin_amdgcn_s_waitcnt(0);  // waves 1-3: the staged keys (and values) have landed
    __syncthreads();
    attn_stamp(g, h, 2);
    pool_put_current(sp.chunk(last), s.kcur, L, hd, true);
    if (early) pool_put_current(sp.chunk(n + last), s.vcur, L, hd, false);
    if (writer && t >= 128) {  // waves 2-3 store the new cache rows (store_f16, src/kernels_f32.cpp:248-250)
        const int i = 2 * (t - 128);
        if (i < hd) {
            uint16_t* kr = g.kcache + (static_cast<size_t>(kv) * g.ctx + pos) * hd;
            uint16_t* vr = g.vcache + (static_cast<size_t>(kv) * g.ctx + pos) * hd;
            const uint32_t kw = f2h(s.kcur[i]) | (static_cast<uint32_t>(f2h(s.kcur[i + 1])) << 16);
            const uint32_t vw = f2h(s.vcur[i]) | (static_cast<uint32_t>(f2h(s.vcur[i + 1])) << 16);
            __hip_atomic_store(gmem(reinterpret_cast<uint32_t*>(kr + i)), kw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(gmem(reinterpret_cast<uint32_t*>(vr + i)), vw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
    __syncthreads();
    // ---- scores, one position a lane
    for (int p = t; p < L; p += kThreads) {
        const int c = p / kSplit, r = p - c * kSplit;
        float v;
        if (HD != 0) v = score_lane<(HD != 0 ? HD : 128) / 16>(s.q, sp.chunk(c), r, HD / 8, HD / 8 - 1);
        else {
            const int per = hd / 16, P = kv_pieces(hd), mask = kv_mask(hd);
            v = per == 8 ? score_lane<8>(s.q, sp.chunk(c), r, P, mask) : per == 6 ? score_lane<6>(s.q, sp.chunk(c), r, P, mask)
              : per == 4 ? score_lane<4>(s.q, sp.chunk(c), r, P, mask) : score_lane<2>(s.q, sp.chunk(c), r, P, mask);
        }
        s.sc[p] = v * g.scale;
    }
    __syncthreads();
    attn_stamp(g, h, 3);
    const int vfirst = early ? n : 0;
    if (!early)  // the keys are consumed: the values take their buffers
        for (int c = 0; c < n; ++c) {
            const int nn = chunk_cached(c, L);
            if (nn > 0) chunk_issue(sp.chunk(c), vbase, c * kSplit, nn, hd, false);
        }
    // ---- softmax over the four waves: max, e = expf(s - max), double sum, w = e * (float)(1 / sum)
    float m = -INFINITY;
    for (int p = t; p < L; p += kThreads) m = fmaxf(m, s.sc[p]);
    m = wave_max(m);
    if (lane == 0) s.mx[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(s.mx[0], s.mx[1]), fmaxf(s.mx[2], s.mx[3]));
    double part = 0.0;
    for (int p = t; p < L; p += kThreads) {
        const float e = ref_expf_s(s.sc[p] - m);
        s.sc[p] = e;
        part += static_cast<double>(e);
    }
    part = wave_sum(part);
    if (lane == 0) s.red[0][wave] = part;
    __syncthreads();
    const float scale = static_cast<float>(1.0 / (((s.red[0][0] + s.red[0][1]) + s.red[0][2]) + s.red[0][3]));
    for (int p = t; p < L; p += kThreads) s.sc[p] *= scale;
    __builtin_amdgcn_s_waitcnt(0);  // values staged (late case); the writer's cache rows are in memory
    if (!early) pool_put_current(sp.chunk(last), s.vcur, L, hd, false);
    __syncthreads();
    attn_stamp(g, h, 4);
    // ---- value sums in position order, one chain a lane
    if (t < hd) {
        const int d = t, full = L & ~7;
        const float* w = s.sc;
        const uint16_t* vcol = sp.chunk(vfirst) + d;
        auto vat = [&](int p) -> const uint16_t* { return vcol + (p >> 6) * (kSplit * 128) + (p & 63) * hd; };
        float a = 0.0f;
        float4 wa0, wa1, wb0, wb1;
        uint16_t va[8], vb[8];
        int p = 0;
        if (full > 0) {
            wa0 = *reinterpret_cast<const float4*>(w);
            wa1 = *reinterpret_cast<const float4*>(w + 4);
#pragma unroll
            for (int u = 0; u < 8; ++u) va[u] = vat(0)[u * hd];
            for (; p + 16 <= full; p += 16) {
                {
                    const float* wn = w + p + 8;
                    wb0 = *reinterpret_cast<const float4*>(wn);
                    wb1 = *reinterpret_cast<const float4*>(wn + 4);
                    const uint16_t* vn = vat(p + 8);
#pragma unroll
                    for (int u = 0; u < 8; ++u) vb[u] = vn[u * hd];
                }
                a += wa0.x * h2f(va[0]); a += wa0.y * h2f(va[1]); a += wa0.z * h2f(va[2]); a += wa0.w * h2f(va[3]);
                a += wa1.x * h2f(va[4]); a += wa1.y * h2f(va[5]); a += wa1.z * h2f(va[6]); a += wa1.w * h2f(va[7]);
                if (p + 16 < full) {
                    const float* wn = w + p + 16;
                    wa0 = *reinterpret_cast<const float4*>(wn);
                    wa1 = *reinterpret_cast<const float4*>(wn + 4);
                    const uint16_t* vn = vat(p + 16);
#pragma unroll
                    for (int u = 0; u < 8; ++u) va[u] = vn[u * hd];
                }
                a += wb0.x * h2f(vb[0]); a += wb0.y * h2f(vb[1]); a += wb0.z * h2f(vb[2]); a += wb0.w * h2f(vb[3]);
                a += wb1.x * h2f(vb[4]); a += wb1.y * h2f(vb[5]); a += wb1.z * h2f(vb[6]); a += wb1.w * h2f(vb[7]);
            }
            if (p < full) {
                a += wa0.x * h2f(va[0]); a += wa0.y * h2f(va[1]); a += wa0.z * h2f(va[2]); a += wa0.w * h2f(va[3]);
                a += wa1.x * h2f(va[4]); a += wa1.y * h2f(va[5]); a += wa1.z * h2f(va[6]); a += wa1.w * h2f(va[7]);
                p += 8;
            }
        }
        for (; p < L; ++p) a += w[p] * h2f(*vat(p));
        o.att(h * hd + d, a);
    }
    attn_stamp(g, h, 5);
    return true;
}

// ---------------------------------------------------------------- spread exact attention

// Attention in the reference's order (src/model.cpp:1050-1093, src/kernels_f32.cpp:256-284),
// spread over the grid so that no workgroup streams a whole head's cache:
//
//  stage 1, task (kv, c) on workgroup n2 + kv * per_kv + c: the query heads of
//    key/value head kv (bias, q_norm, RoPE), then their scores against the
//    positions of chunk c, each dot_f32(q, k) * scale (16 lane sums, then the
//    lanes added in order).  The task holding this token's position also
//    normalises and rotates its key, rounds it to fp16 and stores the cache row.
//    Scores go out as tagged words, [kv][head][position] packed by length L.
//  stage 2, task (kv, slice) on workgroup kv * slices + slice: every score of
//    the group's heads, softmax (max, expf, double sum, multiply by the float of
//    1 / sum), then out[h][d] = sum over positions in order of w[h][p] v[p][d]
//    (each product rounded, then added) for the slice's 32 dimensions, one
//    chain a lane.  It also rounds this token's values of the slice to fp16 and
//    stores them into the cache row.
//
// A stage-1 task reads its chunk's keys and a stage-2 task its slice's values;
// both are requested before the task's inputs are awaited.  Every cache row a
// task stores is in memory before the task publishes (s_waitcnt), so later
// steps, which depend on what it published, see it.
// The rotation pair of lane `lane` in a head of hd values rotated whole
// (apply_rope, src/model.cpp:100-115): (i, i + hd / 2) in the NeoX layout,
// (2 i, 2 i + 1) otherwise; lanes from hd / 2 on hold none.
struct Pair {
    int ia, ib;
    bool live;
};
__device__ __forceinline__ Pair rope_pair(int lane, int hd, int neox) {
    Pair p;
    p.live = lane < hd / 2;
    p.ia = neox ? lane : 2 * lane;
    p.ib = neox ? lane + hd / 2 : 2 * lane + 1;
    if (!p.live) p.ia = p.ib = 0;
    return p;
}

// The per-lane constants of a head's norm and rotation, fetched before the inputs arrive.
struct PairConst {
    float wa, wb, c, sn;
};
__device__ __forceinline__ PairConst pair_const(const Pair& p, const float* w, const float* rope_row) {
    PairConst k{1.0f, 1.0f, 1.0f, 0.0f};
    if (p.live) {
        if (w != nullptr) { k.wa = gmem(w)[p.ia]; k.wb = gmem(w)[p.ib]; }
        if (rope_row != nullptr) {
            const int i = static_cast<int>(threadIdx.x & 63);
            k.c = rope_row[2 * i];
            k.sn = rope_row[2 * i + 1];
        }
    }
    return k;
}

// Bias, RMS norm (float squares summed in double, src/model.cpp:87-97) and
// rotation of one head in LDS (v), by one wave, each lane on its pair in registers.
__device__ __forceinline__ void pair_norm_rope(float* v, const Pair& p, const PairConst& k, const float* bias, bool norm,
                                               bool rope, int hd, float eps) {
    float a = p.live ? v[p.ia] : 0.0f, b = p.live ? v[p.ib] : 0.0f;
    if (bias != nullptr && p.live) {
        a = a + gmem(bias)[p.ia];
        b = b + gmem(bias)[p.ib];
    }
    if (norm) {
        double s2 = static_cast<double>(a * a);
        s2 += static_cast<double>(b * b);
        const float scale = rms_scale(wave_sum(s2), hd, eps);
        a = a * scale * k.wa;
        b = b * scale * k.wb;
    }
    if (rope) {
        const float x0 = a, x1 = b;
        a = x0 * k.c - x1 * k.sn;
        b = x0 * k.sn + x1 * k.c;
    }
    if (p.live) {
        v[p.ia] = a;
        v[p.ib] = b;
    }
}

__device__ __forceinline__ bool spread_stage1(const LoopArgs& g, const AttnArgs& a, SpreadStage1& s, int kv, int p0, int p1,
                                              int pos, unsigned tin, unsigned tsc, const Stamps& st) {
    const int hd = a.head_dim, hpk = g.sp_hpk, t = threadIdx.x, wave = t >> 6, Lc = pos + 1;
    const bool writer = p1 == Lc;
    const int cached = (writer ? pos : p1) - p0;
    const float* rope_row = a.rope != nullptr ? a.rope + static_cast<size_t>(pos) * a.rope_dim : nullptr;
    const Pair pr = rope_pair(t & 63, hd, a.neox);
    // the norm and rotation constants of the head(s) this wave will take (queries: q_norm, the writer's key:
    // k_norm).  Wave 0 only polls: a load issued before its poll would hold the poll's results back
    // until it returned (a wave's loads complete in order).
    PairConst kq{1.0f, 1.0f, 1.0f, 0.0f}, kk{1.0f, 1.0f, 1.0f, 0.0f};
    if (wave != 0) {
        kq = pair_const(pr, a.qnorm, rope_row);
        kk = pair_const(pr, a.knorm, rope_row);
    }
    bool fail = false;
    if (wave == 0) {  // this token's query heads (and, for the writer, key) while the others stage the keys
        pst(st, 4);
        fail = !wget_segs<8>(g, tin, TSeg{g.qt + kv * hpk * hd, s.q, hpk * hd},
                             writer ? TSeg{g.kt + kv * hd, s.kcur, hd} : TSeg{nullptr, nullptr, 0}, TSeg{nullptr, nullptr, 0});
        pst(st, 6);
    } else if (cached > 0) {
        chunk_issue_by(s.kst, a.kcache + static_cast<size_t>(kv) * a.ctx * hd, p0, cached, hd, false, t - 64, kThreads - 64);
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (__syncthreads_or(fail)) return false;
    pst(st, 1);
    // q_norm / k_norm and RoPE (src/model.cpp:1026-1041) by waves 1..3; the key rounded to fp16 as the cache holds it
    for (int h = wave - 1; wave > 0 && h < hpk + (writer ? 1 : 0); h += kThreads / 64 - 1) {
        if (h < hpk)
            pair_norm_rope(s.q + h * hd, pr, kq, a.qbias != nullptr ? a.qbias + (kv * hpk + h) * hd : nullptr, a.qnorm != nullptr,
                           rope_row != nullptr, hd, a.eps);
        else {
            pair_norm_rope(s.kcur, pr, kk, a.kbias != nullptr ? a.kbias + kv * hd : nullptr, a.knorm != nullptr, rope_row != nullptr,
                           hd, a.eps);
            for (int i = t & 63; i < hd; i += 64) s.kst[(pos - p0) * hd + i] = f2h(s.kcur[i]);
        }
    }
    __syncthreads();
    pst(st, 2);
    // scores: 4 threads a (head, position), thread r holding dot_f32's lanes 4 r .. 4 r + 3; the
    // lanes are added in order (0 + lane 0 + ... + lane 15), each thread adding its four to the
    // running sum it takes from the thread before it
    const int n = p1 - p0, items = hpk * n, per = hd / 16, r = t & 3;
    for (int base = 0; base < items; base += kThreads / 4) {
        const int it = base + (t >> 2);
        const bool live = it < items;
        const int h = live ? it / n : 0, p = live ? it - h * n : 0;
        float l0 = 0.0f, l1 = 0.0f, l2 = 0.0f, l3 = 0.0f;
        const float* q = s.q + h * hd + 4 * r;
        const uint16_t* k = s.kst + p * hd + 4 * r;
        for (int m = 0; m < per; ++m) {
            const float4 qv = *reinterpret_cast<const float4*>(q + 16 * m);
            const uint2 kw = *reinterpret_cast<const uint2*>(k + 16 * m);
            l0 += mul_h<false>(qv.x, kw.x);
            l1 += mul_h<true>(qv.y, kw.x);
            l2 += mul_h<false>(qv.z, kw.y);
            l3 += mul_h<true>(qv.w, kw.y);
        }
        float sum = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float prev = __shfl_up(sum, 1, 4);
            if (r == u) sum = ((((u == 0 ? 0.0f : prev) + l0) + l1) + l2) + l3;
        }
        if (live && r == 3)
            tput(g.sct + static_cast<size_t>(kv * hpk + h) * Lc + p0 + p, sum * a.scale, tsc);
    }
    pst(st, 3);
    return true;
}

// A value chain of the exact attention over positions [p, full) (full - p a multiple of 8):
// acc += w[q] * v[q] in position order, w the float weights and v the fp16 values of one
// dimension (transposed rows), both in LDS.  Eight positions a round, each round's three LDS
// reads issued two rounds ahead as inline assembly with counted waits (the compiler would wait
// for every read before the first use); the products are v_fma_mix_f32's rounded float products.
__device__ __forceinline__ float value_chain(const float* w, const uint16_t* vrow, int p, int full, float acc) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    struct Round {
        f4 w0, w1;
        u4 v;
    };
    typedef __attribute__((address_space(3))) const void* lds_cptr;
    const uint32_t wb = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_cptr)w));
    const uint32_t vb = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_cptr)vrow));
    auto rd = [&](int q) {
        const int qc = q < full ? q : full - 8;  // past the end: the last round again (unused)
        Round r;
        asm volatile("ds_read_b128 %0, %1" : "=v"(r.w0) : "v"(wb + 4 * qc));
        asm volatile("ds_read_b128 %0, %1 offset:16" : "=v"(r.w1) : "v"(wb + 4 * qc));
        asm volatile("ds_read_b128 %0, %1" : "=v"(r.v) : "v"(vb + 2 * qc));
        return r;
    };
    // one round: the eight products (v_fma_mix_f32, as mul_h) issued ahead of their adds, in one
    // asm block so each add's product is formed while the add before it completes
    auto sum = [&](const Round& r) {
        float p0, p1, p2, p3, p4, p5, p6, p7;
        asm volatile(
            "v_fma_mix_f32 %1, %9, %17, %19 op_sel_hi:[0,1,0]\n\t"
            "v_fma_mix_f32 %2, %10, %17, %19 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
            "v_fma_mix_f32 %3, %11, %18, %19 op_sel_hi:[0,1,0]\n\t"
            "v_add_f32 %0, %0, %1\n\t"
            "v_fma_mix_f32 %4, %12, %18, %19 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
            "v_add_f32 %0, %0, %2\n\t"
            "v_fma_mix_f32 %5, %13, %20, %19 op_sel_hi:[0,1,0]\n\t"
            "v_add_f32 %0, %0, %3\n\t"
            "v_fma_mix_f32 %6, %14, %20, %19 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
            "v_add_f32 %0, %0, %4\n\t"
            "v_fma_mix_f32 %7, %15, %21, %19 op_sel_hi:[0,1,0]\n\t"
            "v_add_f32 %0, %0, %5\n\t"
            "v_fma_mix_f32 %8, %16, %21, %19 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
            "v_add_f32 %0, %0, %6\n\t"
            "v_add_f32 %0, %0, %7\n\t"
            "v_add_f32 %0, %0, %8"
            : "+v"(acc), "=&v"(p0), "=&v"(p1), "=&v"(p2), "=&v"(p3), "=&v"(p4), "=&v"(p5), "=&v"(p6), "=&v"(p7)
            : "v"(r.w0.x), "v"(r.w0.y), "v"(r.w0.z), "v"(r.w0.w), "v"(r.w1.x), "v"(r.w1.y), "v"(r.w1.z), "v"(r.w1.w),
              "v"(r.v.x), "v"(r.v.y), "v"(-0.0f), "v"(r.v.z), "v"(r.v.w));
    };
    if (full <= p) return acc;
    // rounds at p, p + 8, ...: ra and rb hold the next two; three rounds an iteration, the names
    // rotated rather than copied; each wait leaves the later round's three reads in flight
    Round ra = rd(p), rb = rd(p + 8), rc;
    for (; p + 24 <= full; p += 24) {
        asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(ra.w0), "+v"(ra.w1), "+v"(ra.v));
        rc = rd(p + 16);
        sum(ra);
        asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(rb.w0), "+v"(rb.w1), "+v"(rb.v));
        ra = rd(p + 24);
        sum(rb);
        asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(rc.w0), "+v"(rc.w1), "+v"(rc.v));
        rb = rd(p + 32);
        sum(rc);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(ra.w0), "+v"(ra.w1), "+v"(ra.v), "+v"(rb.w0), "+v"(rb.w1), "+v"(rb.v));
    if (p < full) { sum(ra); p += 8; }
    if (p < full) sum(rb);
    return acc;
}

// The whole workgroup's softmax of H heads' long rows, all heads in each pass: one barrier a
// pass for all of them, and the heads' exp chains interleaved.  Each head's max, exps, partial
// sums (thread t: positions t, t + 256, ..; then the wave sum; then the four waves in order)
// and scale are what it gets on its own.
template <int H>
__device__ __forceinline__ void spread_softmax_long(SpreadStage2& s, int Ls, int Lc) {
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    float m[H];
#pragma unroll
    for (int h = 0; h < H; ++h) m[h] = -INFINITY;
    for (int p = t; p < Lc; p += kThreads)
#pragma unroll
        for (int h = 0; h < H; ++h) m[h] = fmaxf(m[h], s.sc[h * Ls + p]);
#pragma unroll
    for (int h = 0; h < H; ++h) {
        m[h] = wave_max(m[h]);
        if (lane == 0) s.mx[h][wave] = m[h];
    }
    __syncthreads();
    double part[H];
#pragma unroll
    for (int h = 0; h < H; ++h) {
        m[h] = fmaxf(fmaxf(s.mx[h][0], s.mx[h][1]), fmaxf(s.mx[h][2], s.mx[h][3]));
        part[h] = 0.0;
    }
    for (int p = t; p < Lc; p += kThreads)
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const float e = ref_expf_s(s.sc[h * Ls + p] - m[h]);
            s.sc[h * Ls + p] = e;
            part[h] += static_cast<double>(e);
        }
#pragma unroll
    for (int h = 0; h < H; ++h) {
        part[h] = wave_sum(part[h]);
        if (lane == 0) s.red[h][wave] = part[h];
    }
    __syncthreads();
    float scale[H];
#pragma unroll
    for (int h = 0; h < H; ++h) scale[h] = static_cast<float>(1.0 / (((s.red[h][0] + s.red[h][1]) + s.red[h][2]) + s.red[h][3]));
    for (int p = t; p < Lc; p += kThreads)
#pragma unroll
        for (int h = 0; h < H; ++h) s.sc[h * Ls + p] *= scale[h];
}

template <class O>
__device__ __forceinline__ bool spread_stage2(const LoopArgs& g, const AttnArgs& a, SpreadStage2& s, int kv, int d0, int pos,
                                              unsigned tin, unsigned tsc, const O& o, const Stamps& st) {
    const int hd = a.head_dim, hpk = a.heads / a.kv_heads, t = threadIdx.x, wave = t >> 6, lane = t & 63, Lc = pos + 1;
    const int Ls = (Lc + 7) & ~7, chunks = (Lc + kSpreadStage - 1) / kSpreadStage, chains = hpk * kSpreadSlice;
    // chain waves hold one (head, dimension) chain a lane; the others stage the cached values
    const int cw = (chains + 63) / 64, r = t - 64 * cw, nt = kThreads - 64 * cw, wave_first = r & ~63;
    const float* rope_row = a.rope != nullptr ? a.rope + static_cast<size_t>(pos) * a.rope_dim : nullptr;
    const uint8_t* vsrc = reinterpret_cast<const uint8_t*>(a.vcache + static_cast<size_t>(kv) * a.ctx * hd + d0);
    // chunk c's cached rows of the slice (4 pieces of 16 bytes a position) into vraw[c & 1], by the staging waves
    auto issue = [&](int c) {
        const int p0 = c * kSpreadStage, np = (pos < p0 + kSpreadStage ? pos : p0 + kSpreadStage) - p0, pieces = np * 4;
        uint8_t* dst = reinterpret_cast<uint8_t*>(s.vraw[c & 1]);
        for (int k = 0; k * nt < pieces; ++k) {
            const int i = k * nt + r;
            if (i < pieces)
                __builtin_amdgcn_global_load_lds((global_cvoid_ptr)(vsrc + static_cast<size_t>(p0 + (i >> 2)) * hd * 2 + (i & 3) * 16),
                                                 (lds_void_ptr)(dst + (k * nt + wave_first) * 16), 16, 0, 0);
        }
    };
    // ... transposed to [dim][position] in vt[c & 1] (each staging wave its own pieces: whole 8 x 8
    // blocks of 8 positions by 8 dimensions in registers, the rest a half at a time); the last chunk
    // also takes this token's values of the slice, rounded to fp16 with the bias, at position pos
    auto transpose = [&](int c) {
        const int p0 = c * kSpreadStage, np = (pos < p0 + kSpreadStage ? pos : p0 + kSpreadStage) - p0;
        const uint16_t* raw = s.vraw[c & 1];
        uint16_t* vt = s.vt[c & 1];
        const int blocks = (np >> 3) * (kSpreadSlice / 8);
        for (int bi = r; bi < blocks; bi += nt) {
            const int pb = (bi >> 2) * 8, c8 = (bi & 3) * 8;
            uint32_t in[8][4];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint4 w = *reinterpret_cast<const uint4*>(raw + (pb + q) * kSpreadSlice + c8);
                in[q][0] = w.x; in[q][1] = w.y; in[q][2] = w.z; in[q][3] = w.w;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // byte selectors: the low (even j) or high (odd j) half of each of two words
                const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
                uint4 o4;
                o4.x = __builtin_amdgcn_perm(in[1][j >> 1], in[0][j >> 1], sel);
                o4.y = __builtin_amdgcn_perm(in[3][j >> 1], in[2][j >> 1], sel);
                o4.z = __builtin_amdgcn_perm(in[5][j >> 1], in[4][j >> 1], sel);
                o4.w = __builtin_amdgcn_perm(in[7][j >> 1], in[6][j >> 1], sel);
                *reinterpret_cast<uint4*>(vt + (c8 + j) * kVtStride + pb) = o4;
            }
        }
        const int tail0 = np & ~7, tail = (np - tail0) * kSpreadSlice;
        for (int i = r; i < tail; i += nt) {
            const int p = tail0 + i / kSpreadSlice, dd = i % kSpreadSlice;
            vt[dd * kVtStride + p] = raw[p * kSpreadSlice + dd];
        }
        if (c == chunks - 1 && r < kSpreadSlice) {
            const float v = a.vbias != nullptr ? s.vcur[r] + gmem(a.vbias)[kv * hd + d0 + r] : s.vcur[r];
            vt[r * kVtStride + pos - p0] = f2h(v);
        }
    };
    bool fail = false;
    if (wave == 0) {
        // this token's key (all of it: its norm spans the head) and values of the slice; the key
        // normalised and rotated, then the slice of both rows rounded to fp16 into the cache rows
        // (store_f16, src/kernels_f32.cpp:248-250)
        const Pair pr = rope_pair(lane, hd, a.neox);
        fail = !wget_segs<4>(g, tin, TSeg{g.kt + kv * hd, s.kcur, hd}, TSeg{g.vt + kv * hd + d0, s.vcur, kSpreadSlice},
                             TSeg{nullptr, nullptr, 0});
        // (the norm and rotation constants requested after the poll: loads issued before it would hold
        // its results back)
        const PairConst kk = pair_const(pr, a.knorm, rope_row);
        if (!fail) {
            pair_norm_rope(s.kcur, pr, kk, a.kbias != nullptr ? a.kbias + kv * hd : nullptr, a.knorm != nullptr, rope_row != nullptr,
                           hd, a.eps);
            if (lane < kSpreadSlice / 2) {
                const int d = 2 * lane;
                uint16_t* kr = a.kcache + (static_cast<size_t>(kv) * a.ctx + pos) * hd + d0;
                uint16_t* vr = a.vcache + (static_cast<size_t>(kv) * a.ctx + pos) * hd + d0;
                const uint16_t k0 = f2h(s.kcur[d0 + d]), k1 = f2h(s.kcur[d0 + d + 1]);
                const float b0 = a.vbias != nullptr ? gmem(a.vbias)[kv * hd + d0 + d] : 0.0f;
                const float b1 = a.vbias != nullptr ? gmem(a.vbias)[kv * hd + d0 + d + 1] : 0.0f;
                const uint16_t v0 = f2h(a.vbias != nullptr ? s.vcur[d] + b0 : s.vcur[d]);
                const uint16_t v1 = f2h(a.vbias != nullptr ? s.vcur[d + 1] + b1 : s.vcur[d + 1]);
                __hip_atomic_store(gmem(reinterpret_cast<uint32_t*>(kr + d)), k0 | (static_cast<uint32_t>(k1) << 16), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
                __hip_atomic_store(gmem(reinterpret_cast<uint32_t*>(vr + d)), v0 | (static_cast<uint32_t>(v1) << 16), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
    } else if (wave >= cw) {
        issue(0);
        if (chunks > 1) issue(1);
    }
    if (__syncthreads_or(fail)) {
        __builtin_amdgcn_s_waitcnt(0);
        return false;
    }
    if (wave >= cw) {  // the first chunk transposed, the third requested
        __builtin_amdgcn_s_waitcnt(0);
        transpose(0);
        if (chunks > 2) issue(2);
    }
    // every score of the group, a head a padded row
    bool ok = true;
    for (int h0 = 0; h0 < hpk && ok; h0 += 3) {
        auto seg = [&](int h) {
            return h < hpk ? TSeg{g.sct + static_cast<size_t>(kv * hpk + h) * Lc, s.sc + h * Ls, Lc} : TSeg{nullptr, nullptr, 0};
        };
        ok = tget_segs<8>(g, tsc, seg(h0), seg(h0 + 1), seg(h0 + 2));
    }
    if (!ok) {
        __builtin_amdgcn_s_waitcnt(0);
        return false;
    }
    pst(st, 4);
    // softmax of each head's row (softmax_f32, src/kernels_f32.cpp:275-285): a wave a head on short
    // rows (no barriers), the whole workgroup on a head on long ones
    if (Lc <= 1024) {
        for (int h = wave; h < hpk; h += kThreads / 64) {
            float* sc = s.sc + h * Ls;
            float m = -INFINITY;
            for (int p = lane; p < Lc; p += 64) m = fmaxf(m, sc[p]);
            m = wave_max(m);
            double part = 0.0;
            for (int p = lane; p < Lc; p += 64) {
                const float e = ref_expf_s(sc[p] - m);
                sc[p] = e;
                part += static_cast<double>(e);
            }
            const float scale = static_cast<float>(1.0 / wave_sum(part));
            for (int p = lane; p < Lc; p += 64) sc[p] *= scale;
        }
    } else {
        switch (hpk) {
            case 1: spread_softmax_long<1>(s, Ls, Lc); break;
            case 2: spread_softmax_long<2>(s, Ls, Lc); break;
            case 3: spread_softmax_long<3>(s, Ls, Lc); break;
            default: spread_softmax_long<4>(s, Ls, Lc); break;
        }
    }
    __syncthreads();
    pst(st, 5);
    // value sums, one (head, dimension) chain a lane, positions in order (weighted_sum_f32, :265-273),
    // chunk by chunk; while the chain waves sum chunk c, the staging waves transpose chunk c + 1 and
    // request chunk c + 3 (into the raw buffer chunk c + 1 leaves)
    const bool chain = t < chains;
    const int h = chain ? t / kSpreadSlice : 0, d = t - h * kSpreadSlice;
    const float* w = s.sc + h * Ls;
    float acc = 0.0f;
    for (int c = 0; c < chunks; ++c) {
        if (chain) {
            const int p0 = c * kSpreadStage, pe = Lc < p0 + kSpreadStage ? Lc : p0 + kSpreadStage;
            const uint16_t* vrow = s.vt[c & 1] + d * kVtStride - p0;
            const int full = p0 + ((pe - p0) & ~7);
            int p = p0;
            acc = value_chain(w, vrow, p0, full, acc);
            p = full;
            for (; p < pe; ++p) acc += mul_h<false>(w[p], vrow[p]);
        } else if (wave >= cw && c + 1 < chunks) {
            __builtin_amdgcn_s_waitcnt(0);
            transpose(c + 1);
            if (c + 3 < chunks) issue(c + 3);
        }
        __syncthreads();
    }
    if (chain) {
        if (t < kSpreadSlice / 2) __builtin_amdgcn_s_waitcnt(0);  // the cache rows are in memory before any output
        o.att((kv * hpk + h) * hd + d0 + d, acc);
    }
    pst(st, 6);
    return true;
}

// ---------------------------------------------------------------- resident attention

// The resident attention's task of workgroup b: query head h, kv head kv, value slice at d0.
struct ResTask {
    int h, kv, d0;
};
__device__ __forceinline__ ResTask res_task(const LoopArgs& g, int b) {
    const int ns = g.head_dim / kResSlice, h = b / ns;
    return ResTask{h, h / g.sp_hpk, (b - h * ns) * kResSlice};
}

// Rows [0, n) of kv head kv's key cache (whole heads) and of the value slice at
// d0, the values transposed to [dim][position], into LDS; by the whole
// workgroup, ends with a barrier.  Keys go straight in by global_load_lds;
// values through a staging buffer.
__device__ __forceinline__ void res_preload(const AttnArgs& a, ResLds& s, const ResTask& k, int n) {
    const int hd = a.head_dim, t = threadIdx.x, P = hd / 8;
    const uint8_t* ksrc = reinterpret_cast<const uint8_t*>(a.kcache + static_cast<size_t>(k.kv) * a.ctx * hd);
    uint8_t* kdst = reinterpret_cast<uint8_t*>(s.keys);
    // LDS slot c of key row p holds the row's 16-byte piece c ^ (p & (P - 1)), so the score
    // loop's reads (consecutive positions at one piece) spread over the banks
    for (int base = 0; base < n * P; base += kThreads) {
        const int i = base + t, p = i / P, c = (i % P) ^ (p & (P - 1));
        if (i < n * P)
            __builtin_amdgcn_global_load_lds((global_cvoid_ptr)(ksrc + (static_cast<size_t>(p) * P + c) * 16),
                                             (lds_void_ptr)(kdst + (base + (t & ~63)) * 16), 16, 0, 0);
    }
    constexpr int VP = kResSlice / 8;  // 16-byte pieces a value row of the slice
    const uint8_t* vsrc = reinterpret_cast<const uint8_t*>(a.vcache + static_cast<size_t>(k.kv) * a.ctx * hd + k.d0);
    uint8_t* vdst = reinterpret_cast<uint8_t*>(s.vstage);
    for (int c0 = 0; c0 < n; c0 += kResStage) {
        const int np = n - c0 < kResStage ? n - c0 : kResStage, pieces = np * VP;
        for (int base = 0; base < pieces; base += kThreads) {
            const int i = base + t;
            if (i < pieces)
                __builtin_amdgcn_global_load_lds((global_cvoid_ptr)(vsrc + static_cast<size_t>(c0 + i / VP) * hd * 2 + (i % VP) * 16),
                                                 (lds_void_ptr)(vdst + (base + (t & ~63)) * 16), 16, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        // 8 x 8 blocks (8 positions by 8 dimensions) transposed in registers, the rest a half at a time
        const int blocks = (np >> 3) * VP;
        for (int bi = t; bi < blocks; bi += kThreads) {
            const int pb = (bi / VP) * 8, c8 = (bi % VP) * 8;
            uint32_t in[8][4];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint4 w = *reinterpret_cast<const uint4*>(s.vstage + (pb + q) * kResSlice + c8);
                in[q][0] = w.x; in[q][1] = w.y; in[q][2] = w.z; in[q][3] = w.w;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
                uint4 o4;
                o4.x = __builtin_amdgcn_perm(in[1][j >> 1], in[0][j >> 1], sel);
                o4.y = __builtin_amdgcn_perm(in[3][j >> 1], in[2][j >> 1], sel);
                o4.z = __builtin_amdgcn_perm(in[5][j >> 1], in[4][j >> 1], sel);
                o4.w = __builtin_amdgcn_perm(in[7][j >> 1], in[6][j >> 1], sel);
                *reinterpret_cast<uint4*>(s.vt + (c8 + j) * kResVt + c0 + pb) = o4;
            }
        }
        const int tail0 = np & ~7, tail = (np - tail0) * kResSlice;
        for (int i = t; i < tail; i += kThreads) {
            const int p = tail0 + i / kResSlice, dd = i % kResSlice;
            s.vt[dd * kResVt + c0 + p] = s.vstage[p * kResSlice + dd];
        }
        __syncthreads();
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

// Scores of the resident attention (dot_f32, src/kernels_f32.cpp:256-262, times
// the scale) for every position: 4 threads a position, thread r holding
// dot_f32's lanes 4 r .. 4 r + 3 over the PER 16-value steps of the head, its
// query values in registers; quad g walks positions g, g + 64, ...; the lanes
// are added in order along the quad (each thread adding its four to the
// running sum broadcast from the thread before).
template <int PER>
__device__ __forceinline__ void res_scores(ResLds& s, int Lc, float scale) {
    float mx = -INFINITY;  // the scores' max, for the softmax: each wave's into s.mx
    constexpr int hd = PER * 16, P = hd / 8;
    const int t = threadIdx.x, r = t & 3, g = t >> 2;
    float4 qr[PER];
#pragma unroll
    for (int m = 0; m < PER; ++m) qr[m] = *reinterpret_cast<const float4*>(s.q + 16 * m + 4 * r);
    for (int p = g; p < Lc; p += kThreads / 4) {
        const uint16_t* k = s.keys + p * hd + 4 * (r & 1);
        uint2 kw[PER];
#pragma unroll
        for (int m = 0; m < PER; ++m) kw[m] = *reinterpret_cast<const uint2*>(k + (((2 * m + (r >> 1)) ^ (p & (P - 1))) << 3));
        float l0 = 0.0f, l1 = 0.0f, l2 = 0.0f, l3 = 0.0f;
#pragma unroll
        for (int m = 0; m < PER; ++m) {
            l0 += mul_h<false>(qr[m].x, kw[m].x);
            l1 += mul_h<true>(qr[m].y, kw[m].x);
            l2 += mul_h<false>(qr[m].z, kw[m].y);
            l3 += mul_h<true>(qr[m].w, kw[m].y);
        }
        float sum = (((0.0f + l0) + l1) + l2) + l3;  // thread 0's part; the others add theirs in turn
        float prev = dpp<0x00>(sum);
        if (r == 1) sum = (((prev + l0) + l1) + l2) + l3;
        prev = dpp<0x55>(sum);
        if (r == 2) sum = (((prev + l0) + l1) + l2) + l3;
        prev = dpp<0xAA>(sum);
        if (r == 3) {
            const float v = ((((prev + l0) + l1) + l2) + l3) * scale;
            s.sc[p] = v;
            mx = fmaxf(mx, v);
        }
    }
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) s.mx[threadIdx.x >> 6] = mx;
}

// The attention of query head k.h for value slice k.d0 at position pos
// (src/model.cpp:1020-1093), in the reference's order: wave 0 awaits this
// token's q head, k and v slice; waves 1 and 2 normalise and rotate the query
// head and the key (pair_norm_rope); the first query head of a kv head stores
// this token's cache rows of the slice; scores by dot_f32's 16 lanes in order
// (4 threads a score); softmax over the four waves (max, glibc expf, double sum,
// multiply by the float reciprocal); value sums one dimension chain a lane in
// position order; the outputs quantised for the O projection.
template <class O>
__device__ __forceinline__ bool res_attend(const LoopArgs& g, const AttnArgs& a, ResLds& s, const ResTask& k, int pos, unsigned tin,
                                           const O& o, const Stamps& st) {
    const int hd = a.head_dim, t = threadIdx.x, wave = t >> 6, lane = t & 63, Lc = pos + 1;
    const int d0 = k.d0, kv = k.kv;
    const float* rope_row = a.rope != nullptr ? a.rope + static_cast<size_t>(pos) * a.rope_dim : nullptr;
    const Pair pr = rope_pair(lane, hd, a.neox);
    PairConst kc{1.0f, 1.0f, 1.0f, 0.0f};
    if (wave == 1) kc = pair_const(pr, a.qnorm, rope_row);  // (wave 0 polls: a load issued before its poll would
    if (wave == 2) kc = pair_const(pr, a.knorm, rope_row);  //  hold the poll's results back)
    bool fail = false;
    if (wave == 0) {
        pst(st, 1);
        fail = !wget_segs<4>(g, tin, TSeg{g.qt + k.h * hd, s.q, hd}, TSeg{g.kt + kv * hd, s.kcur, hd},
                             TSeg{g.vt + kv * hd + d0, s.vcur, kResSlice});
    }
    if (__syncthreads_or(fail)) {
        __builtin_amdgcn_s_waitcnt(0);
        return false;
    }
    pst(st, 2);
    if (wave == 1)
        pair_norm_rope(s.q, pr, kc, a.qbias != nullptr ? a.qbias + k.h * hd : nullptr, a.qnorm != nullptr, rope_row != nullptr, hd, a.eps);
    if (wave == 2)
        pair_norm_rope(s.kcur, pr, kc, a.kbias != nullptr ? a.kbias + kv * hd : nullptr, a.knorm != nullptr, rope_row != nullptr, hd,
                       a.eps);
    __syncthreads();
    // this token's key (fp16, as the cache holds it) and value slice join the LDS copies; the
    // first query head of the kv head stores the slice of both cache rows (store_f16,
    // src/kernels_f32.cpp:248-250)
    const int P = hd / 8;  // 16-byte pieces a key row, swizzled as res_preload stores them
    for (int i = t; i < hd; i += kThreads) s.keys[pos * hd + (((i >> 3) ^ (pos & (P - 1))) << 3) + (i & 7)] = f2h(s.kcur[i]);
    if (t >= 64 && t < 64 + kResSlice) {
        const int d = t - 64;
        const float v = a.vbias != nullptr ? s.vcur[d] + gmem(a.vbias)[kv * hd + d0 + d] : s.vcur[d];
        s.vt[d * kResVt + pos] = f2h(v);
    }
    if (t < kResSlice / 2 && k.h % g.sp_hpk == 0) {  // wave 0, whose output lanes wait for these stores
        const int d = 2 * t;
        uint16_t* kr = a.kcache + (static_cast<size_t>(kv) * a.ctx + pos) * hd + d0;
        uint16_t* vr = a.vcache + (static_cast<size_t>(kv) * a.ctx + pos) * hd + d0;
        const uint16_t k0 = f2h(s.kcur[d0 + d]), k1 = f2h(s.kcur[d0 + d + 1]);
        const float b0 = a.vbias != nullptr ? gmem(a.vbias)[kv * hd + d0 + d] : 0.0f;
        const float b1 = a.vbias != nullptr ? gmem(a.vbias)[kv * hd + d0 + d + 1] : 0.0f;
        const uint16_t v0 = f2h(a.vbias != nullptr ? s.vcur[d] + b0 : s.vcur[d]);
        const uint16_t v1 = f2h(a.vbias != nullptr ? s.vcur[d + 1] + b1 : s.vcur[d + 1]);
        __hip_atomic_store(gmem(reinterpret_cast<uint32_t*>(kr + d)), k0 | (static_cast<uint32_t>(k1) << 16), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(gmem(reinterpret_cast<uint32_t*>(vr + d)), v0 | (static_cast<uint32_t>(v1) << 16), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    }
    __syncthreads();
    pst(st, 3);
    if (hd == 128) res_scores<8>(s, Lc, a.scale);
    else res_scores<4>(s, Lc, a.scale);
    __syncthreads();
    pst(st, 4);
    // softmax (softmax_f32, src/kernels_f32.cpp:275-285) over the four waves: the max, the
    // exponentials with their double sum (a double sum of floats is exact in any grouping over the
    // range here), then every weight times the float reciprocal of the sum
    {
        const float m = fmaxf(fmaxf(s.mx[0], s.mx[1]), fmaxf(s.mx[2], s.mx[3]));  // (res_scores' wave maxima)
        double part = 0.0;
        for (int p = t; p < Lc; p += kThreads) {
            const float e = ref_expf_s(s.sc[p] - m);
            s.sc[p] = e;
            part += static_cast<double>(e);
        }
        part = wave_sum(part);
        if (lane == 0) s.red[wave] = part;
        __syncthreads();
        const float scale = static_cast<float>(1.0 / (((s.red[0] + s.red[1]) + s.red[2]) + s.red[3]));
        for (int p = t; p < Lc; p += kThreads) s.sc[p] *= scale;
    }
    __syncthreads();
    pst(st, 5);
    // value sums (weighted_sum_f32, :265-273): one dimension chain a lane of wave 0, positions in
    // order, eight a round, each round's weights and values read two rounds ahead
    if (wave == 0) {
        const float* w = s.sc;
        const uint16_t* vrow = s.vt + lane * kResVt;
        const int full = Lc & ~7;
        float acc = value_chain(w, vrow, 0, full, 0.0f);
        int p = full;
        for (; p < Lc; ++p) acc += mul_h<false>(w[p], vrow[p]);
        __builtin_amdgcn_s_waitcnt(0);  // the cache rows are in memory before any output
        pst(st, 6);
        o.att(k.h * hd + d0 + lane, acc);
    }
    return true;
}

// This workgroup's part of the spread attention at one context length: a
// stage-2 task (kv2, slice at d0; kv = -1), or stage-1 positions [p0, p1) of
// key/value head kv (empty when the length leaves the chunk out).
struct SpreadGeo {
    int kv, p0, p1, kv2, d0;
};
__device__ __forceinline__ SpreadGeo spread_geo(const LoopArgs& g, int pos) {
    SpreadGeo geo{-1, 0, 0, 0, 0};
    if (!g.spread) return geo;
    const int Lc = pos + 1, b = static_cast<int>(blockIdx.x), per_kv = g.sp_per_kv;
    if (b < g.sp_n2) {
        geo.kv2 = b / g.sp_slices;
        geo.d0 = (b - geo.kv2 * g.sp_slices) * kSpreadSlice;
        return geo;
    }
    int P1 = (Lc + per_kv - 1) / per_kv;
    P1 = P1 < 4 ? 4 : P1;
    const int task = b - g.sp_n2, kv = task / per_kv, c = task - kv * per_kv;
    geo.kv = kv < g.kv_heads ? kv : g.kv_heads;  // past the last head: no task
    geo.p0 = kv < g.kv_heads ? c * P1 : 0;
    geo.p1 = kv < g.kv_heads ? (geo.p0 + P1 < Lc ? geo.p0 + P1 : Lc) : 0;
    if (geo.p0 >= Lc) geo.p1 = geo.p0;
    return geo;
}

// B, spread: the tasks of both stages; a workgroup with neither goes on to phase C.
__device__ __forceinline__ bool phase_b_spread(const LoopArgs& g, const AttnArgs& a, int step, int l, int pos, SpreadLds& s,
                                               const SpreadGeo& geo) {
    const unsigned tin = tag_of(g, step, l, 1), tsc = tag_of(g, step, l, 6), tout = tag_of(g, step, l, 2);
    if (geo.kv < 0) {  // stage 2: (key/value head, slice)
        const TaggedOut o{g.attt, g.pacct, g.pmlt, tout, g.error, g.att_q8, g.heads * g.head_dim};
        return spread_stage2(g, a, s.s2, geo.kv2, geo.d0, pos, tin, tsc, o, pst_ptr(g, step, l, 1));
    }
    if (geo.p0 >= geo.p1) return true;  // no chunk at this length
    return spread_stage1(g, a, s.s1, geo.kv, geo.p0, geo.p1, pos, tin, tsc, pst_ptr(g, step, l, 1));
}

// Whether the spread attention takes a context of L positions (on a grid of G workgroups).
__device__ __forceinline__ bool spread_takes(const LoopArgs& g, int L) {
    const int hpk = g.heads / g.kv_heads, n2 = g.kv_heads * (g.head_dim / kSpreadSlice);
    const int per_kv = (static_cast<int>(gridDim.x) - n2) / g.kv_heads;
    return hpk * ((L + 7) & ~7) <= kSpreadScores && (L + per_kv - 1) / per_kv <= kSpreadChunk;
}

// B: attention, exact (one workgroup per key/value head) or split over (kv, split) slots.
__device__ __forceinline__ bool phase_b(const LoopArgs& g, const LayerDev& L, int step, int l, int pos, LoopLds& lds, const SpreadGeo& geo) {
    const int kvh = g.kv_heads, hpk = g.sp_hpk, hd = g.head_dim, Lc = pos + 1;
    const unsigned tin = tag_of(g, step, l, 1), tout = tag_of(g, step, l, 2);
    const AttnArgs a = attn_args(g, L, step, l);
    const TaggedOut o{g.attt, g.pacct, g.pmlt, tout, g.error, g.att_q8, g.heads * g.head_dim};
    if (g.res_ok && Lc <= kResMax) {
        if (static_cast<int>(blockIdx.x) >= g.res_n) return true;
        return res_attend(g, a, lds.res, res_task(g, blockIdx.x), pos, tin, o, pst_ptr(g, step, l, 1));
    }
    if (g.spread && (g.sp_all || spread_takes(g, Lc))) return phase_b_spread(g, a, step, l, pos, lds.spread, geo);
    if (attn_is_exact(Lc, hpk) && Lc <= kSplit * kPoolChunks && g.head_attn) {
        if (static_cast<int>(blockIdx.x) >= g.heads) return true;
        const int h = blockIdx.x;
        AttnPoolLds& sp = lds.pool;
        if (hd == 128) return attn_head_pool<128>(g, a, sp, h, pos, tin, o);
        if (hd == 64) return attn_head_pool<64>(g, a, sp, h, pos, tin, o);
        return attn_head_pool<0>(g, a, sp, h, pos, tin, o);
    }
    if (attn_is_exact(Lc, hpk) && Lc <= kSplit * kPoolChunks) {
        if (static_cast<int>(blockIdx.x) >= kvh) return true;
        const int kv = blockIdx.x;
        AttnPoolLds& sp = lds.pool;
        attn_stamp(a, kv, 0);
        attn_pool_issue(a, sp, kv, Lc);  // the cached keys (and values) stream in while q/k/v are awaited
        if (!tget_segs<>(g, tin, TSeg{g.qt + kv * hpk * hd, sp.a.q, hpk * hd}, TSeg{g.kt + kv * hd, sp.a.kcur, hd},
                       TSeg{g.vt + kv * hd, sp.a.vcur, hd})) {
            __builtin_amdgcn_s_waitcnt(0);
            return false;
        }
        pst(pst_ptr(g, step, l, 1), 1);
        attn_finish_prologue<true>(a, sp.a, kv, pos, true, false);
        pst(pst_ptr(g, step, l, 1), 2);
        if (hd == 128) attn_exact_pool<128>(a, sp, kv, Lc, o);
        else if (hd == 64) attn_exact_pool<64>(a, sp, kv, Lc, o);
        else attn_exact_pool<0>(a, sp, kv, Lc, o);
        return true;
    }
    // no other case reaches the loop: the session takes the one-kernel-per-phase path for a
    // context that neither the spread nor the pooled exact attention takes whole
    atomicExch(g.error, 1);
    return false;
}

// C: O rows of att, h += O att.  With own_h the residual rows come from the
// workgroup's own copy (it produced them in the previous layer's phase F, or
// from the embedding at layer 0).
template <uint32_t TO>
__device__ __forceinline__ bool phase_c(const LoopArgs& g, const LayerDev& L, int step, int l, int token, GemvLds& s,
                                        float* hown) {
    const Packed L_o = sld(&L.o);
    const float* L_attn_sub = sld(&L.attn_sub);
    const unsigned tag = tag_of(g, step, l, 3), tprev = tag_of(g, step, l - 1, 5);
    const int G = g.n_c;
    const Stamps st = pst_ptr(g, step, l, 2);
    auto row_of = [&](int t, Packed& m, uint32_t& row0, int& R) {
        m = L_o;
        R = g.R_o;
        row0 = static_cast<uint32_t>(t) * R;
    };
    auto ready = [&]() -> bool {
        const int n = g.heads * g.head_dim;
        if (g.att_q8) {  // already quantised by the attention: straight into the activation LDS
            const bool ok = tget_segs<>(g, tag_of(g, step, l, 2), TSeg{g.attt, reinterpret_cast<float*>(s.a.xs), n / 4},
                               TSeg{g.attt + n / 4, s.a.xd, n / 32},
                               TSeg{g.attt + n / 4 + n / 32, reinterpret_cast<float*>(s.a.xsum), n / 32});
            pst(st, 1);
            return ok;
        }
        ActRegs ar;
        act_issue_w(ar, L_attn_sub, n);
        if (!tget_vec(g, g.attt, tag_of(g, step, l, 2), s.x, n)) return false;
        prologue_lds<TO>(L_o, ar, L_attn_sub, g.eps, s);
        return true;
    };
    auto done = [&](int t, const Packed& m, uint32_t row0, const float* sums) -> bool {
        const uint32_t r = threadIdx.x, row = row0 + r;
        bool ok = true;
        if (r < static_cast<uint32_t>(g.R_o) && row < m.rows) {
            float prev = 0.0f;
            const int slot = (t - (static_cast<int>(blockIdx.x) - g.c_first)) / G * g.R_o + static_cast<int>(r);
            if (g.own_h) prev = hown[slot];
            else if (l == 0) prev = dequant_elem(g.embd, static_cast<uint32_t>(token), row);
            else ok = tget_one(g, g.ht + row, tprev, prev);
            const float h = prev + sums[r];  // h += proj (src/model.cpp:1111)
            if (ok) tput(g.ht + row, h, tag);
            if (g.own_h) hown[slot] = h;
        }
        return g.own_h || !__syncthreads_or(!ok);
    };
    return run_tiles<TO, kLoopUnits>(g.tiles_o, s, row_of, ready, done, st, g.c_first, g.n_c);
}

// D: gate/up rows of ffn_norm(h), the gated activation.  A tile is R gate rows
// and the same R up rows; tiles are grouped as in run_tiles (gate terms, then
// up terms, a tile after the other).
template <uint32_t TG>
__device__ __forceinline__ bool phase_d(const LoopArgs& g, const LayerDev& L, int step, int l, GemvLds& s) {
    const Packed L_gate = sld(&L.gate);
    const Packed L_up = sld(&L.up);
    const float* L_ffn_norm = sld(&L.ffn_norm);
    if (static_cast<int>(blockIdx.x) >= g.tiles_gu) return true;
    const unsigned tag = tag_of(g, step, l, 4);
    const int G = static_cast<int>(gridDim.x), R = g.R_gu;
    const uint32_t units = L_gate.cols / Unit<TG>::kElems, stride = term_stride(units);
    Tile<TG, kLoopUnits> tg, tu;
    int t = blockIdx.x;
    uint32_t row0 = static_cast<uint32_t>(t) * R;
    tg.load(L_gate, row0, R);
    tu.load(L_up, row0, R);
    const Stamps st = pst_ptr(g, step, l, 3);
    ActRegs ar;
    act_issue_w(ar, L_ffn_norm, g.embd_dim);
    if (!tget_vec(g, g.ht, tag_of(g, step, l, 3), s.x, g.embd_dim)) return false;
    pst(st, 1);
    prologue_lds<TG>(L_gate, ar, L_ffn_norm, g.eps, s);
    pst(st, 2);
    int gfirst = t, grows = 0;
    while (true) {
        tg.terms(L_gate, s.a, s.terms + grows * stride);
        tu.terms(L_up, s.a, s.terms + (grows + R) * stride);
        grows += 2 * R;
        const int tn = t + G;
        const bool last = tn >= g.tiles_gu;
        if (!last) {  // the next tile's weights stream in while this group finishes
            row0 = static_cast<uint32_t>(tn) * R;
            tg.load(L_gate, row0, R);
            tu.load(L_up, row0, R);
        }
        if (last || (grows + 2 * R) * static_cast<int>(stride) > kTermCap || grows + 2 * R > kGroupRows) {
            pst(st, 3);
            __syncthreads();
            row_sums(s.terms, stride, units, grows, s.sums);
            __syncthreads();
            pst(st, 4);
            for (int u = gfirst, off = 0; off < grows; u += G, off += 2 * R) {
                const uint32_t r = threadIdx.x, r0 = static_cast<uint32_t>(u) * R;
                if (r < static_cast<uint32_t>(R) && r0 + r < L_gate.rows) {
                    const float gv = s.sums[off + r], uv = s.sums[off + R + r];
                    float out;
                    if (g.relu2) {
                        const float q = gv > 0.0f ? gv : 0.0f;
                        out = q * q * uv;  // src/model.cpp:1134-1138
                    } else {
                        out = gv / (1.0f + ref_expf_s(-gv)) * uv;  // src/kernels_f32.cpp:287-289
                    }
                    tput(g.actt + r0 + r, out, tag);
                }
            }
            pst(st, 5);
            grows = 0;
            gfirst = tn;
        }
        if (last) break;
        t = tn;
    }
    return true;
}

// F: down rows of act, h += down act (residual rows from the own copy with own_h).
template <uint32_t TD>
__device__ __forceinline__ bool phase_f(const LoopArgs& g, const LayerDev& L, int step, int l, GemvLds& s, float* hown) {
    const Packed L_down = sld(&L.down);
    const float* L_ffn_sub = sld(&L.ffn_sub);
    const unsigned tag = tag_of(g, step, l, 5), tprev = tag_of(g, step, l, 3);
    const int G = g.n_c;
    auto row_of = [&](int t, Packed& m, uint32_t& row0, int& R) {
        m = L_down;
        R = g.R_d;
        row0 = static_cast<uint32_t>(t) * R;
    };
    const Stamps st = pst_ptr(g, step, l, 4);
    auto ready = [&]() -> bool {
        ActRegs ar;
        act_issue_w(ar, L_ffn_sub, g.ff);
        // the whole input in one round of loads (3072 words: 12 a thread)
        if (!tget_segs<12>(g, tag_of(g, step, l, 4), TSeg{g.actt, s.x, g.ff})) return false;
        pst(st, 1);
        prologue_lds<TD>(L_down, ar, L_ffn_sub, g.eps, s);
        pst(st, 2);
        return true;
    };
    auto done = [&](int t, const Packed& m, uint32_t row0, const float* sums) -> bool {
        const uint32_t r = threadIdx.x, row = row0 + r;
        bool ok = true;
        if (r < static_cast<uint32_t>(g.R_d) && row < m.rows) {
            float prev = 0.0f;
            const int slot = (t - (static_cast<int>(blockIdx.x) - g.c_first)) / G * g.R_d + static_cast<int>(r);
            if (g.own_h) prev = hown[slot];
            else ok = tget_one(g, g.ht + row, tprev, prev);
            const float h = prev + sums[r];  // h += proj (src/model.cpp:1162)
            if (ok) tput(g.ht + row, h, tag);
            if (g.own_h) hown[slot] = h;
        }
        return g.own_h || !__syncthreads_or(!ok);
    };
    return run_tiles<TD, kLoopUnits>(g.tiles_d, s, row_of, ready, done, st, g.c_first, g.n_c);
}

// ---------------------------------------------------------------- the pushed feed-forward block

// Gate/up rows a tile of the pushed phase D: the largest power of two up to 32
// whose units fit 4 a thread.
__device__ __forceinline__ int push_tile_rows(uint32_t units) {
    int r = 32;
    while (r > 1 && static_cast<uint32_t>(r) * units > static_cast<uint32_t>(4 * kThreads)) r >>= 1;
    return r;
}

// quantize_q8_0 (src/quant.cpp:115-142) of one 32-value block held one value a
// lane by lanes 0..31 of a wave (lanes 32..63 run along on their own values,
// results unused) into block 0 of `a`.
__device__ __forceinline__ void quant_block_lanes(float v, ActLds& a) {
    const int lane = threadIdx.x & 63;
    float amax = group_reduce<16>(fabsf(v), [](float x, float y) { return nnmax(x, y); });
    amax = nnmax(amax, __shfl_xor(amax, 16, 64));
    const float d = div127(amax);
    const float inv = d != 0.0f ? rcp_rn(d) : 0.0f;
    const int q = static_cast<int>(rintf(v * inv));
    int sum = group_reduce<16>(q, [](int x, int y) { return x + y; });
    sum += __shfl_xor(sum, 16, 64);
    const int q1 = __shfl_down(q, 1, 64), q2 = __shfl_down(q, 2, 64), q3 = __shfl_down(q, 3, 64);
    if (lane < 32 && (lane & 3) == 0)
        a.xs[lane / 4] = (q & 0xFF) | ((q1 & 0xFF) << 8) | ((q2 & 0xFF) << 16) | (static_cast<uint32_t>(q3) << 24);
    if (lane == 0) {
        a.xd[0] = h2f(f2h(d));
        a.xsum[0] = sum;
    }
}

#ifdef BRISK_NO_PUSH
constexpr bool kPushBuilt = false;
#else
constexpr bool kPushBuilt = true;
#endif
constexpr int kPushDown = 4;    // down rows a thread a chunk
constexpr int kPushChunks = 4;  // chunks at most (rows of h up to 4096)

// D, pushed (src/model.cpp:1111-1162 with the down projection split by its
// input blocks): task j computes gate/up rows 32 j .. 32 j + 31 of
// ffn_norm(h) (each row sum in block order), the gated activation of those 32
// rows (silu(gate) * up, src/kernels_f32.cpp:287-289), its Q8_0 block (the
// block the reference's quantize_q8_0 of the whole activation makes), and the
// down matrix's term of block j for every row: term = (float)acc * d_w * d_x,
// as dot_*_q8_0 forms it.  The terms go out as tagged words dtt[j][row].
// Loads are issued before any store of the task (on gfx9 a wait for a load
// also waits for every store issued before it).
template <uint32_t TG, uint32_t TD>
__device__ __forceinline__ bool phase_d_push(const LoopArgs& g, const LayerDev& L, int step, int l, GemvLds& s) {
    const Packed L_gate = sld(&L.gate);
    const Packed L_up = sld(&L.up);
    const Packed L_down_t = sld(&L.down_t);
    const float* L_ffn_norm = sld(&L.ffn_norm);
    const int G = static_cast<int>(gridDim.x), nb = g.ff / 32, rows = g.embd_dim;
    const int first = (static_cast<int>(blockIdx.x) - g.d_first + G) % G;
    if (first >= nb) return true;
    const unsigned tag = tag_of(g, step, l, 4);
    const Stamps st = pst_ptr(g, step, l, 3);
    const uint32_t units = L_gate.cols / Unit<TG>::kElems, stride = term_stride(units);
    const int R = push_tile_rows(units), per = 32 / R, tiles = 2 * per;  // gate tiles, then up tiles
    auto tile_load = [&](Tile<TG, 4>& t, int j, int k) {
        t.load(k < per ? L_gate : L_up, static_cast<uint32_t>(32 * j + (k % per) * R), R);
    };
    auto tile_terms = [&](const Tile<TG, 4>& t, int k) { t.terms(k < per ? L_gate : L_up, s.a, s.terms + k * R * stride); };
    // the down units of chunk c (every thread issues every load; rows past the matrix re-read its last row)
    auto down_load = [&](Unit<TD> (&u)[kPushDown], int j, int c) {
#pragma unroll
        for (int k = 0; k < kPushDown; ++k) {
            int r = (c * kPushDown + k) * kThreads + static_cast<int>(threadIdx.x);
            r = r < rows ? r : rows - 1;
            u[k].load(L_down_t, static_cast<size_t>(j) * rows + r);
        }
    };
    const int dchunks = (rows + kPushDown * kThreads - 1) / (kPushDown * kThreads);
    bool have_input = false;
    for (int j = first; j < nb; j += G) {
        Unit<TD> du[kPushDown];
        down_load(du, j, 0);
        Tile<TG, 4> t0, t1;
        tile_load(t0, j, 0);
        tile_load(t1, j, 1);
        if (!have_input) {
            ActRegs ar;
            act_issue_w(ar, L_ffn_norm, g.embd_dim);
            if (!tget_vec(g, g.ht, tag_of(g, step, l, 3), s.x, g.embd_dim)) return false;
            pst(st, 1);
            prologue_lds<TG>(L_gate, ar, L_ffn_norm, g.eps, s);
            pst(st, 2);
            have_input = true;
        }
        // two tiles in flight: tile k + 2 is requested once tile k's terms are out
        tile_terms(t0, 0);
        if (tiles > 2) tile_load(t0, j, 2);
        tile_terms(t1, 1);
        for (int k = 2; k < tiles; k += 2) {
            if (k + 1 < tiles) tile_load(t1, j, k + 1);
            tile_terms(t0, k);
            if (k + 2 < tiles) tile_load(t0, j, k + 2);
            if (k + 1 < tiles) tile_terms(t1, k + 1);
        }
        pst(st, 6);
        __syncthreads();
        row_sums(s.terms, stride, units, 64, s.sums);
        __syncthreads();
        pst(st, 3);
        // the gated activation of the block, quantised by wave 0 into block 0 of s.a2
        if (threadIdx.x < 64) {
            const int r = threadIdx.x & 31;
            const float gv = s.sums[r], uv = s.sums[32 + r];
            float out;
            if (g.relu2) {
                const float q = gv > 0.0f ? gv : 0.0f;
                out = q * q * uv;  // src/model.cpp:1134-1138
            } else {
                out = gv / (1.0f + ref_expf_s(-gv)) * uv;  // src/kernels_f32.cpp:287-289
            }
            quant_block_lanes(out, s.a2);
        }
        __syncthreads();
        pst(st, 4);
        // every down term of the task in registers, then the stores
        float dt[kPushChunks][kPushDown];
#pragma unroll
        for (int c = 0; c < kPushChunks; ++c) {
            if (c < dchunks) {
                if (c > 0) down_load(du, j, c);
#pragma unroll
                for (int k = 0; k < kPushDown; ++k) dt[c][k] = du[k].term(0, s.a2);
            }
        }
#pragma unroll
        for (int c = 0; c < kPushChunks; ++c) {
            if (c < dchunks) {
#pragma unroll
                for (int k = 0; k < kPushDown; ++k) {
                    const int r = (c * kPushDown + k) * kThreads + static_cast<int>(threadIdx.x);
                    if (r < rows) tput(g.dtt + static_cast<size_t>(j) * rows + r, dt[c][k], tag);
                }
            }
        }
        pst(st, 5);
        __syncthreads();  // s.a2 and s.terms are rewritten by the next task
    }
    return true;
}

// F, pushed: the rows of h this workgroup owns (phase C's tiles), each h += the
// sum of its terms dtt[0..nb)[row] in block order (as the reference's
// sequential `sum +=`), residual from the own copy.
template <uint32_t TD>
__device__ __forceinline__ bool phase_f_push(const LoopArgs& g, int step, int l, GemvLds& s, float* hown) {
    const int Gc = g.n_c, me = static_cast<int>(blockIdx.x) - g.c_first;
    if (me < 0 || me >= g.tiles_o || me >= Gc) return true;
    const int nb = g.ff / 32, rows = g.embd_dim, R = g.R_o;
    const uint32_t stride = term_stride(static_cast<uint32_t>(nb));
    const unsigned tag = tag_of(g, step, l, 5);
    const Stamps st = pst_ptr(g, step, l, 4);
    // owned rows: slot k * R + r is row (me + k Gc) R + r
    const int ntiles = (g.tiles_o - me + Gc - 1) / Gc, nrows = ntiles * R;
    const int n = nrows * nb;
    const bool ok = tget_fn<4>(g, tag_of(g, step, l, 4), n, [&](int i, const unsigned long long*& src, float*& dst) {
        const int slot = i % nrows, j = i / nrows;
        int row = (me + (slot / R) * Gc) * R + slot % R;
        row = row < rows ? row : rows - 1;
        src = g.dtt + static_cast<size_t>(j) * rows + row;
        dst = s.terms + slot * stride + j;
    });
    if (!ok) return false;
    pst(st, 1);
    row_sums(s.terms, stride, static_cast<uint32_t>(nb), nrows, s.sums);
    __syncthreads();
    pst(st, 4);
    for (int slot = threadIdx.x; slot < nrows; slot += kThreads) {
        const int row = (me + (slot / R) * Gc) * R + slot % R;
        if (row < rows) {
            const float h = hown[slot] + s.sums[slot];  // h += proj (src/model.cpp:1162)
            tput(g.ht + row, h, tag);
            hown[slot] = h;
        }
    }
    pst(st, 5);
    return true;
}

// H: output rows of output_norm(h) -> logits; the workgroup's best key folded
// into keys[step & 1], then the workgroup counted done.
template <uint32_t TH>
__device__ __forceinline__ bool phase_h(const LoopArgs& g, int step, GemvLds& s) {
    if (static_cast<int>(blockIdx.x) >= g.tiles_h) return true;
    unsigned long long best = 0;
    auto row_of = [&](int t, Packed& m, uint32_t& row0, int& R) {
        m = g.out;
        R = g.R_h;
        row0 = static_cast<uint32_t>(t) * R;
    };
    auto ready = [&]() -> bool {
        ActRegs ar;
        act_issue_w(ar, g.out_norm, g.embd_dim);
        if (!tget_vec(g, g.ht, tag_of(g, step, g.n_layers - 1, 5), s.x, g.embd_dim)) return false;
        prologue_lds<TH>(g.out, ar, g.out_norm, g.eps, s);
        return true;
    };
    auto done = [&](int, const Packed& m, uint32_t row0, const float* sums) -> bool {
        const uint32_t r = threadIdx.x, row = row0 + r;
        if (r < static_cast<uint32_t>(g.R_h) && row < m.rows) {
            const float v = sums[r];
            g.logits[row] = v;
            const unsigned long long k = pick_key(v, row);
            best = k > best ? k : best;
        }
        return true;
    };
    if (!run_tiles<TH, head_units(TH)>(g.tiles_h, s, row_of, ready, done)) return false;
    if (threadIdx.x < 64) {
        best = wave_max_u64(best);
        if (threadIdx.x == 0) {
            unsigned long long* key = g.keys + (step & 1);
            const unsigned long long cur = __hip_atomic_load(key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            unsigned long long old = 0;
            if (best > cur) old = atomicMax(key, best);
            // counted done only once the atomicMax has been performed (the address depends on its result)
            atomicAdd(g.done + (step & 1) + (old == ~0ull ? 2 : 0), 1u);
        }
    }
    return true;
}

// The pick of step `step` (all of its phase H done), by one thread.
__device__ __forceinline__ bool wait_pick(const LoopArgs& g, int step, int& token) {
    const int hw = g.tiles_h < static_cast<int>(gridDim.x) ? g.tiles_h : static_cast<int>(gridDim.x);
    // full steps of this parity so far: first_full .. step, every other one
    const unsigned want = static_cast<unsigned>(((step - g.first_full) >> 1) + 1) * static_cast<unsigned>(hw);
    unsigned spins = 0;
    while (__hip_atomic_load(g.done + (step & 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < want) {
        if (++spins > kSpinLimit) {
            atomicExch(g.error, 1);
            return false;
        }
        if ((spins & 63) == 0 && loop_failed(g)) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    const unsigned long long k = __hip_atomic_load(g.keys + (step & 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    token = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(k & 0xFFFFFFFFu));
    return true;
}

// The launch's arguments (the kernel's only argument, at the start of the kernel
// argument segment), re-addressed through an opaque copy of the segment pointer
// at each use: the compiler then reads the fields it needs with scalar loads
// where they are used, instead of holding every value derived from them in
// registers across the whole step loop (which spills).
__device__ __forceinline__ const LoopArgs& lg() {
    const __attribute__((address_space(4))) LoopArgs* p = (const __attribute__((address_space(4))) LoopArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return *(const LoopArgs*)p;
}

template <uint32_t TQ, uint32_t TV, uint32_t TO, uint32_t TG, uint32_t TD, uint32_t TH>
__global__ __launch_bounds__(kThreads) void k_loop(LoopArgs g_arg) {
    (void)g_arg;  // read through lg(), re-addressed at each use
    __shared__ LoopLds lds;
    __shared__ float hown[kOwnRows];
    __shared__ int s_token, s_ok;
    __shared__ SpreadGeo s_geo;
    exp_tab_fill();  // ordered before its first use by the barrier after the first token
    for (int step = 0; step < lg().n_steps; ++step) {
        const int pos = lg().pos0 + step;
        const bool full = step >= lg().first_full;
        // the token of this step: the caller's, or the previous step's pick
        if (threadIdx.x == 0) {
            int token = lg().seq[pos];
            bool ok = true;
            if (step > 0 && pos >= lg().fixed) ok = wait_pick(lg(), step - 1, token);
            if (ok && blockIdx.x == 0) {
                if (step > 0 && pos >= lg().fixed) lg().seq[pos] = token;
                // re-arm the key this step's phase H uses: its last readers (the
                // previous step's starts) are all done, since this step's pick
                // waits on the previous step's phase H, which needed their outputs
                if (step >= 2) __hip_atomic_store(lg().keys + (step & 1), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __builtin_amdgcn_s_waitcnt(0);
            }
            s_token = token;
            s_ok = ok;
        }
        if (threadIdx.x == 0) s_geo = spread_geo(lg(), pos);
        __syncthreads();
        if (!s_ok) return;
        const int token = s_token;
        if (lg().own_h) {  // this workgroup's rows of h: the embedding row (embedding_row, src/model.cpp:27-70)
            const int me = static_cast<int>(blockIdx.x) - lg().c_first;
            for (int t = me, k = 0; me >= 0 && me < lg().n_c && t < lg().tiles_o; t += lg().n_c, ++k)
                for (int r = threadIdx.x; r < lg().R_o; r += kThreads) {
                    const uint32_t row = static_cast<uint32_t>(t * lg().R_o + r);
                    if (row < lg().embd.cols) hown[k * lg().R_o + r] = dequant_elem(lg().embd, static_cast<uint32_t>(token), row);
                }
        }
        // the resident attention's workgroups load layer 0's keys and values
        const bool res = lg().res_ok && pos + 1 <= kResMax && static_cast<int>(blockIdx.x) < lg().res_n;
        if (res) res_preload(attn_args(lg(), lg().layers[0], step, 0), lds.res, res_task(lg(), blockIdx.x), pos);
        for (int l = 0; l < lg().n_layers; ++l) {
            const LayerDev& L = lg().layers[l];
            if (lg().trace != nullptr && blockIdx.x == 0 && threadIdx.x == 0) lg().trace[1 + (step * lg().n_layers + l) * 5] = wall_clock64();
            pst(pst_ptr(lg(), step, l, 0), 0);
            if (!phase_a<TQ, TV, TH>(lg(), L, step, l, token, lds.g)) return;
            if (lg().trace != nullptr) {
                __builtin_amdgcn_s_waitcnt(0);
                pst(pst_ptr(lg(), step, l, 0), 6);
            }
            pst(pst_ptr(lg(), step, l, 0), 7);
            __syncthreads();
            if (lg().trace != nullptr && blockIdx.x == 0 && threadIdx.x == 0) lg().trace[2 + (step * lg().n_layers + l) * 5] = wall_clock64();
            pst(pst_ptr(lg(), step, l, 1), 0);
            if (!phase_b(lg(), L, step, l, pos, lds, s_geo)) return;
            pst(pst_ptr(lg(), step, l, 1), 7);
            __syncthreads();
            // ... and, their attention of this layer done, the next layer's
            if (res && l + 1 < lg().n_layers) res_preload(attn_args(lg(), lg().layers[l + 1], step, l + 1), lds.res, res_task(lg(), blockIdx.x), pos);
            if (lg().trace != nullptr && blockIdx.x == 0 && threadIdx.x == 0) lg().trace[3 + (step * lg().n_layers + l) * 5] = wall_clock64();
            pst(pst_ptr(lg(), step, l, 2), 0);
            if (!phase_c<TO>(lg(), L, step, l, token, lds.g, hown)) return;
            pst(pst_ptr(lg(), step, l, 2), 7);
            __syncthreads();
            if (lg().trace != nullptr && blockIdx.x == 0 && threadIdx.x == 0) lg().trace[4 + (step * lg().n_layers + l) * 5] = wall_clock64();
            pst(pst_ptr(lg(), step, l, 3), 0);
            if constexpr (block_elems(TD) == 32 && kPushBuilt) {
                if (lg().push_ffn) {
                    if (!phase_d_push<TG, TD>(lg(), L, step, l, lds.g)) return;
                } else if (!phase_d<TG>(lg(), L, step, l, lds.g)) {
                    return;
                }
            } else if (!phase_d<TG>(lg(), L, step, l, lds.g)) {
                return;
            }
            pst(pst_ptr(lg(), step, l, 3), 7);
            __syncthreads();
            if (lg().trace != nullptr && blockIdx.x == 0 && threadIdx.x == 0) lg().trace[5 + (step * lg().n_layers + l) * 5] = wall_clock64();
            pst(pst_ptr(lg(), step, l, 4), 0);
            if constexpr (TQ == TV) {
                const int me = static_cast<int>(blockIdx.x) - lg().c_first;
                if (lg().a_touch && l + 1 < lg().n_layers && lg().own_h && me >= 0 && me < lg().n_c) a_touch(lg(), lg().layers[l + 1]);
            }
            if constexpr (block_elems(TD) == 32 && kPushBuilt) {
                if (lg().push_ffn) {
                    if (!phase_f_push<TD>(lg(), step, l, lds.g, hown)) return;
                } else if (!phase_f<TD>(lg(), L, step, l, lds.g, hown)) {
                    return;
                }
            } else if (!phase_f<TD>(lg(), L, step, l, lds.g, hown)) {
                return;
            }
            pst(pst_ptr(lg(), step, l, 4), 7);
            __syncthreads();
        }
        if (full && !phase_h<TH>(lg(), step, lds.g)) return;
        __syncthreads();
    }
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
    // the last step's pick becomes seq[end]; the device position follows
    const int end = lg().pos0 + lg().n_steps;
    if (lg().n_steps > lg().first_full && end < lg().seq_len && end >= lg().fixed) {
        int token = 0;
        if (!wait_pick(lg(), lg().n_steps - 1, token)) return;
        lg().seq[end] = token;
    }
    *lg().pos_out = end;
    if (lg().trace != nullptr) lg().trace[0] = wall_clock64();
}

// ---------------------------------------------------------------- host side

template <uint32_t TQ, uint32_t TV, uint32_t TO, uint32_t TG, uint32_t TD, uint32_t TH>
static const void* loop_kernel() {
    return reinterpret_cast<const void*>(&k_loop<TQ, TV, TO, TG, TD, TH>);
}

// The format mixes the loop is built for: (q/k, v, o, gate/up, down, output).
const void* find_loop_kernel(uint32_t tq, uint32_t tv, uint32_t to, uint32_t tg, uint32_t td, uint32_t th) {
    auto is = [&](uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t e, uint32_t f) {
        return tq == a && tv == b && to == c && tg == d && td == e && th == f;
    };
    if (is(kQ4_0, kQ4_0, kQ4_0, kQ4_0, kQ4_0, kQ8_0)) return loop_kernel<kQ4_0, kQ4_0, kQ4_0, kQ4_0, kQ4_0, kQ8_0>();
    if (is(kQ8_0, kQ8_0, kQ8_0, kQ8_0, kQ8_0, kQ8_0)) return loop_kernel<kQ8_0, kQ8_0, kQ8_0, kQ8_0, kQ8_0, kQ8_0>();
    if (is(kQ4_K, kQ6_K, kQ4_K, kQ4_K, kQ6_K, kQ6_K)) return loop_kernel<kQ4_K, kQ6_K, kQ4_K, kQ4_K, kQ6_K, kQ6_K>();
    if (is(kTQ2_0, kTQ2_0, kTQ2_0, kTQ2_0, kTQ2_0, kQ4_0)) return loop_kernel<kTQ2_0, kTQ2_0, kTQ2_0, kTQ2_0, kTQ2_0, kQ4_0>();
    // Q5_K_M (Q5_K with Q6_K for V, down and the output) and Q5_0 with Q4_1 on the O and down rows
    if (is(kQ5_K, kQ6_K, kQ5_K, kQ5_K, kQ6_K, kQ6_K)) return loop_kernel<kQ5_K, kQ6_K, kQ5_K, kQ5_K, kQ6_K, kQ6_K>();
    if (is(kQ5_0, kQ5_0, kQ4_1, kQ5_0, kQ4_1, kQ8_0)) return loop_kernel<kQ5_0, kQ5_0, kQ4_1, kQ5_0, kQ4_1, kQ8_0>();
    return nullptr;
}

int loop_units_per_thread(uint32_t type, bool head) { return head ? head_units(type) : kLoopUnits; }

bool loop_spread_fits(int heads, int kv_heads, int head_dim, int rope_dim, int grid) {
    if (kv_heads <= 0 || heads % kv_heads != 0 || heads / kv_heads > kSpreadHpk) return false;
    if (head_dim % kSpreadSlice != 0 || head_dim > 128) return false;
    if (rope_dim != head_dim) return false;  // the rotation pairs span the head (no partial rotary)
    return grid - kv_heads * (head_dim / kSpreadSlice) >= kv_heads;  // a stage-1 task a key/value head at least
}

int loop_resident_max() { return kResMax; }

bool loop_pool_covers(int hpk, int positions) { return attn_is_exact(positions, hpk) && positions <= kSplit * kPoolChunks; }

bool loop_spread_covers(int heads, int kv_heads, int head_dim, int grid, int positions) {
    const int per_kv = (grid - kv_heads * (head_dim / kSpreadSlice)) / kv_heads;
    return (heads / kv_heads) * ((positions + 7) & ~7) <= kSpreadScores && (positions + per_kv - 1) / per_kv <= kSpreadChunk;
}

// cooperative: the runtime either places the whole grid at once or fails the
// launch (hipErrorCooperativeLaunchTooLarge).  A plain launch of a grid that
// fits (one workgroup a compute unit, checked against the occupancy at set-up)
// on an otherwise idle device is placed whole as well, and runs about 2%
// faster; if other work holds compute units, the loop's bounded waits expire
// and the launch reports an error instead of hanging.
hipError_t launch_loop(const void* kernel, const LoopArgs& g, int grid, hipStream_t s, bool cooperative) {
    void* args[] = {const_cast<LoopArgs*>(&g)};
    if (cooperative) return hipLaunchCooperativeKernel(kernel, dim3(grid), dim3(kThreads), args, 0, s);
    return hipLaunchKernel(kernel, dim3(grid), dim3(kThreads), args, 0, s);
}

}  // namespace bh
