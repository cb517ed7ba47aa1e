// The persistent token loop: one launch runs n_steps forward steps.
//
// Every workgroup of the grid (one per CU) stays resident for the whole launch
// and walks the same phase sequence as the one-kernel-per-phase path:
//
//   per step:   E  embed: workgroup 0 turns the previous pick (or the caller's
//                  token) into seq[pos] and dequantises its embedding row into h
//   per layer:  A  Q/K/V rows of attn_norm(h)                 (src/model.cpp:996-1015)
//               B  Q/K norms, RoPE, K/V cache write, attention (:1020-1093)
//               C  O rows of (sub-normed) att, residual add    (:1095-1111)
//               D  gate/up rows of ffn_norm(h), SiLU / relu^2  (:1111-1143)
//               F  down rows of (sub-normed) act, residual add (:1144-1162)
//   full steps: H  output_norm(h) -> output rows -> logits, pick key
//
// with a grid barrier after each phase.  The barrier is two-level (groups of
// 32 workgroups, then the groups) on relaxed device-scope atomics with no cache
// maintenance: the vectors handed between phases are written and read with
// system-scope accesses (CoherentIO), which bypass the per-XCD L2s.  Each
// waiting workgroup spins a bounded number of times; on expiry it raises the
// error flag, and every workgroup leaves at its next barrier, so a launch
// always drains.
#include "phases.h"
#include "loop.h"

namespace bh {

constexpr int kGroup = 32;          // workgroups per first-level barrier counter
constexpr int kRootSlot = 64 * 64;  // counters sit 256 bytes apart
constexpr int kReleaseSlot = kRootSlot + 64;
constexpr unsigned kSpinLimit = 1u << 22;

// Grid barrier: returns false when the launch is being abandoned.
__device__ bool grid_barrier(unsigned* bar, unsigned& gen, int* error, unsigned long long* trace = nullptr) {
    __shared__ int abandon;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores and atomics are performed
    __syncthreads();
    if (threadIdx.x == 0) {
        gen += 1;
        const unsigned G = gridDim.x, g = blockIdx.x / kGroup, ngroups = (G + kGroup - 1) / kGroup;
        const unsigned members = G - g * kGroup < kGroup ? G - g * kGroup : kGroup;
        const unsigned old = atomicAdd(bar + g * 64, 1u);
        if (old + 1 == gen * members) {
            // the root add depends on the group add's result, so it is issued after it completed
            const unsigned o2 = atomicAdd(bar + kRootSlot + (old == ~0u ? 1 : 0), 1u);
            if (o2 + 1 == gen * ngroups)
                __hip_atomic_store(bar + kReleaseSlot + (o2 == ~0u ? 1 : 0), gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        unsigned spins = 0;
        int bad = 0;
        while (__hip_atomic_load(bar + kReleaseSlot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < gen) {
            __builtin_amdgcn_s_sleep(1);
            if ((++spins & 255) == 0 && __hip_atomic_load(error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                bad = 1;
                break;
            }
            if (spins > kSpinLimit) {
                atomicExch(error, 1);
                bad = 1;
                break;
            }
        }
        abandon = bad;
        if (trace != nullptr && blockIdx.x == 0) trace[gen] = wall_clock64();
    }
    __syncthreads();
    return abandon == 0;
}

// Shared memory of the loop: the GEMV phases' and the attention phase's layouts overlap.
struct GemvLds {
    ActLds a;
    float terms[kTermCap];
    float sums[64];
    float sums2[64];
    double red[4];
};
union LoopLds {
    GemvLds g;
    AttnLds att;
};

// Rows [row0, row0 + R) of m into out (add: out += ...), activation already in LDS.
template <uint32_t T>
__device__ __forceinline__ void tile_out(const Packed& m, uint32_t row0, int R, GemvLds& s, float* out, bool add) {
    Tile<T> tile;
    tile.load(m, row0, R);
    tile.sums(m, s.a, s.terms, s.sums);
    const uint32_t r = threadIdx.x, row = row0 + r;
    if (r < static_cast<uint32_t>(R) && row < m.rows) {
        const float v = add ? CoherentIO::ld(out + row) + s.sums[r] : s.sums[r];
        CoherentIO::st(out + row, v);
    }
}

template <uint32_t T>
__device__ __forceinline__ void prologue(const Packed& m, const float* x, const float* w, float eps, GemvLds& s) {
    ActRegs ar;
    const int cols = static_cast<int>(m.cols);
    act_issue<CoherentIO>(ar, x, w, cols);
    act_finish<CoherentIO>(ar, x, w, eps, cols, takes_q8_k(T), act_bits(m), s.a, s.red);
}

// One matrix (or up to three, same activation) as a phase: tiles t = blockIdx.x, + G, ...
template <uint32_t T>
__device__ void gemv_phase(const Packed* ms, float* const* outs, const int* R, const int* tiles, int n, const float* x,
                           const float* w, float eps, bool add, GemvLds& s) {
    int total = 0;
    for (int i = 0; i < n; ++i) total += tiles[i];
    if (static_cast<int>(blockIdx.x) >= total) return;
    prologue<T>(ms[0], x, w, eps, s);
    for (int t = blockIdx.x; t < total; t += gridDim.x) {
        int i = 0, tt = t;
        while (i < n - 1 && tt >= tiles[i]) tt -= tiles[i++];
        tile_out<T>(ms[i], static_cast<uint32_t>(tt) * R[i], R[i], s, outs[i], add);
    }
}

template <uint32_t TG>
__device__ void gateup_phase(const LayerDev& L, const LoopArgs& g, GemvLds& s) {
    if (static_cast<int>(blockIdx.x) >= g.tiles_gu) return;
    prologue<TG>(L.gate, g.h, L.ffn_norm, g.eps, s);
    for (int t = blockIdx.x; t < g.tiles_gu; t += gridDim.x) {
        const uint32_t row0 = static_cast<uint32_t>(t) * g.R_gu;
        Tile<TG, (Unit<TG>::kMaxPerThread + 1) / 2> tg, tu;
        tg.load(L.gate, row0, g.R_gu);
        tu.load(L.up, row0, g.R_gu);
        tg.sums(L.gate, s.a, s.terms, s.sums);
        tu.sums(L.up, s.a, s.terms, s.sums2);
        const uint32_t r = threadIdx.x;
        if (r < static_cast<uint32_t>(g.R_gu) && row0 + r < L.gate.rows) {
            const float gv = s.sums[r], uv = s.sums2[r];
            float out;
            if (g.relu2) {
                const float q = gv > 0.0f ? gv : 0.0f;
                out = q * q * uv;  // src/model.cpp:1134-1138
            } else {
                out = gv / (1.0f + ref_expf(-gv)) * uv;  // src/kernels_f32.cpp:287-289
            }
            CoherentIO::st(g.act + row0 + r, out);
        }
    }
}

template <uint32_t TH>
__device__ void head_phase(const LoopArgs& g, unsigned long long* key, GemvLds& s) {
    if (static_cast<int>(blockIdx.x) >= g.tiles_h) return;
    prologue<TH>(g.out, g.h, g.out_norm, g.eps, s);
    unsigned long long best = 0;
    for (int t = blockIdx.x; t < g.tiles_h; t += gridDim.x) {
        const uint32_t row0 = static_cast<uint32_t>(t) * g.R_h;
        Tile<TH> tile;
        tile.load(g.out, row0, g.R_h);
        tile.sums(g.out, s.a, s.terms, s.sums);
        const uint32_t r = threadIdx.x, row = row0 + r;
        if (r < static_cast<uint32_t>(g.R_h) && row < g.out.rows) {
            const float v = s.sums[r];
            g.logits[row] = v;
            const unsigned long long k = pick_key(v, row);
            best = k > best ? k : best;
        }
    }
    if (threadIdx.x < 64) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long other = __shfl_xor(best, o, 64);
            best = other > best ? other : best;
        }
        if (threadIdx.x == 0) {
            const unsigned long long cur = __hip_atomic_load(key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (best > cur) atomicMax(key, best);
        }
    }
}

// Attention with the cache rows written through (system scope), since a row
// written by one workgroup may be read by another in a later step.
__device__ void attn_phase(const LayerDev& L, const LoopArgs& g, int pos, AttnLds& s, unsigned& gen, bool& ok) {
    AttnArgs a{};
    a.q = g.q; a.k = g.k; a.v = g.v; a.qnorm = L.q_norm; a.knorm = L.k_norm; a.rope = g.rope;
    a.eps = g.eps; a.neox = g.neox; a.kcache = L.kc; a.vcache = L.vc; a.pos = nullptr;
    a.ctx = g.ctx; a.head_dim = g.head_dim; a.heads = g.heads; a.kv_heads = g.kv_heads; a.scale = g.scale;
    a.part_acc = g.part_acc; a.part_ml = g.part_ml; a.max_splits = g.max_splits; a.tickets = nullptr; a.out = g.att;
    a.stamps = g.trace != nullptr ? g.trace + 60000 + 8 * (pos % 8) : nullptr;
    const int L_ = pos + 1, hpk = g.heads / g.kv_heads;
    const int kv = static_cast<int>(blockIdx.x) % g.kv_heads, split = static_cast<int>(blockIdx.x) / g.kv_heads;
    if (attn_is_exact(L_, hpk)) {
        if (split == 0) {
            attn_stamp(a, kv, 0);
            attn_prologue<CoherentIO, true>(a, s, kv, pos, true);
            attn_exact<CoherentIO>(a, s, kv, L_);
        }
        return;
    }
    const int ns = (L_ + kSplit - 1) / kSplit;
    // every (kv, split) slot of the grid, round-robin over the workgroups
    for (int slot = blockIdx.x; slot < g.kv_heads * ns; slot += gridDim.x) {
        const int kvs = slot % g.kv_heads, sp = slot / g.kv_heads;
        attn_prologue<CoherentIO, true>(a, s, kvs, pos, sp == pos / kSplit);
        attn_split_partial<CoherentIO>(a, s, kvs, sp, L_);
        __syncthreads();
    }
    ok = grid_barrier(g.bar, gen, g.error, g.trace);
    if (!ok) return;
    if (static_cast<int>(blockIdx.x) < g.kv_heads) attn_split_combine<CoherentIO>(a, static_cast<int>(blockIdx.x), L_);
}

// embedding_row (src/model.cpp:27-70) of `token` into h, by one workgroup.
__device__ void embed_row(const Packed& m, uint32_t r, float* h) {
    const uint32_t cols = m.cols;
    for (uint32_t e = threadIdx.x; e < cols; e += kThreads) CoherentIO::st(h + e, dequant_elem(m, r, e));
}

template <uint32_t TQ, uint32_t TV, uint32_t TO, uint32_t TG, uint32_t TD, uint32_t TH>
__global__ __launch_bounds__(kThreads) void k_loop(LoopArgs g) {
    __shared__ LoopLds lds;
    __shared__ int s_token;
    unsigned gen = 0;
    bool ok = true;
    if (g.trace != nullptr && blockIdx.x == 0 && threadIdx.x == 0) g.trace[0] = wall_clock64();
    for (int step = 0; step < g.n_steps && ok; ++step) {
        const int pos = g.pos0 + step;
        const bool full = step >= g.first_full;
        unsigned long long* key = g.keys + (step & 1);
        // ---- E
        if (blockIdx.x == 0) {
            if (threadIdx.x == 0) {
                int token = g.seq[pos];
                if (step > 0 && pos >= g.fixed) {  // the previous step's pick
                    const unsigned long long k =
                        __hip_atomic_load(g.keys + ((step - 1) & 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    token = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(k & 0xFFFFFFFFu));
                    g.seq[pos] = token;
                }
                __hip_atomic_store(key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_token = token;
            }
            __syncthreads();
            embed_row(g.embd, static_cast<uint32_t>(s_token), g.h);
        }
        if (!(ok = grid_barrier(g.bar, gen, g.error, g.trace))) break;
        for (int l = 0; l < g.n_layers && ok; ++l) {
            const LayerDev& L = g.layers[l];
            // ---- A: Q, K, V (same activation; Q and K share a format, V may differ)
            {
                if (TQ == TV) {
                    const Packed ms[3] = {L.q, L.k, L.v};
                    float* const outs[3] = {g.q, g.k, g.v};
                    gemv_phase<TQ>(ms, outs, g.R_qkv, g.tiles_qkv, 3, g.h, L.attn_norm, g.eps, false, lds.g);
                } else {
                    const Packed ms[2] = {L.q, L.k};
                    float* const outs[2] = {g.q, g.k};
                    gemv_phase<TQ>(ms, outs, g.R_qkv, g.tiles_qkv, 2, g.h, L.attn_norm, g.eps, false, lds.g);
                    __syncthreads();
                    // V's tiles after Q's and K's, on the next workgroups round-robin
                    const int first = (g.tiles_qkv[0] + g.tiles_qkv[1]) % static_cast<int>(gridDim.x);
                    const int me = (static_cast<int>(blockIdx.x) - first + static_cast<int>(gridDim.x)) % static_cast<int>(gridDim.x);
                    if (me < g.tiles_qkv[2]) {
                        prologue<TV>(L.v, g.h, L.attn_norm, g.eps, lds.g);
                        for (int t = me; t < g.tiles_qkv[2]; t += gridDim.x)
                            tile_out<TV>(L.v, static_cast<uint32_t>(t) * g.R_qkv[2], g.R_qkv[2], lds.g, g.v, false);
                    }
                }
            }
            if (!(ok = grid_barrier(g.bar, gen, g.error, g.trace))) break;
            // ---- B
            attn_phase(L, g, pos, lds.att, gen, ok);
            if (!ok) break;
            if (!(ok = grid_barrier(g.bar, gen, g.error, g.trace))) break;
            // ---- C
            {
                const Packed ms[1] = {L.o};
                float* const outs[1] = {g.h};
                gemv_phase<TO>(ms, outs, &g.R_o, &g.tiles_o, 1, g.att, L.attn_sub, g.eps, true, lds.g);
            }
            if (!(ok = grid_barrier(g.bar, gen, g.error, g.trace))) break;
            // ---- D
            gateup_phase<TG>(L, g, lds.g);
            if (!(ok = grid_barrier(g.bar, gen, g.error, g.trace))) break;
            // ---- F
            {
                const Packed ms[1] = {L.down};
                float* const outs[1] = {g.h};
                gemv_phase<TD>(ms, outs, &g.R_d, &g.tiles_d, 1, g.act, L.ffn_sub, g.eps, true, lds.g);
            }
            if (!(ok = grid_barrier(g.bar, gen, g.error, g.trace))) break;
        }
        if (!ok) break;
        if (full) {
            // ---- H
            head_phase<TH>(g, key, lds.g);
            if (!(ok = grid_barrier(g.bar, gen, g.error, g.trace))) break;
        }
    }
    if (!ok || blockIdx.x != 0 || threadIdx.x != 0) return;
    // the last step's pick becomes seq[end]; the device position follows
    const int end = g.pos0 + g.n_steps;
    if (g.n_steps > g.first_full && end < g.seq_len && end >= g.fixed) {
        const unsigned long long k =
            __hip_atomic_load(g.keys + ((g.n_steps - 1) & 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        g.seq[end] = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(k & 0xFFFFFFFFu));
    }
    *g.pos_out = end;
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
    return nullptr;
}

hipError_t launch_loop(const void* kernel, const LoopArgs& g, int grid, hipStream_t s) {
    void* args[] = {const_cast<LoopArgs*>(&g)};
    return hipLaunchKernel(kernel, dim3(grid), dim3(kThreads), args, 0, s);
}

}  // namespace bh
