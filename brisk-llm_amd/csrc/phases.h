// Phase bodies shared by the one-kernel-per-phase path (kernels.hip) and the
// persistent token loop (loop.hip): attention and the greedy-pick key.
#pragma once

#include "launch.h"

namespace bh {

// Element e of row r of a packed matrix, dequantised as embedding_row does
// (src/model.cpp:27-70, src/quant.cpp:196-239).
// T: the format, known at compile time (kF32: read m.type at run time).
template <uint32_t T = kF32>
__device__ inline float dequant_elem(const Packed& m, uint32_t r, uint32_t e) {
    const uint32_t cols = m.cols;
    switch (T != kF32 ? T : m.type) {
        case kQ8_0: {
            const size_t blk = static_cast<size_t>(r) * (cols / 32) + e / 32;
            const float d = h2f(gld<uint16_t>(m.p1, blk));
            return static_cast<float>(static_cast<int8_t>(gmem(m.p0)[blk * 32 + e % 32])) * d;
        }
        case kQ4_0: {
            const size_t blk = static_cast<size_t>(r) * (cols / 32) + e / 32;
            const float d = h2f(gld<uint16_t>(m.p1, blk));
            const uint32_t i = e % 32;
            const uint8_t q = gmem(m.p0)[blk * 16 + (i & 15)];
            return static_cast<float>((i < 16 ? (q & 0x0F) : (q >> 4)) - 8) * d;
        }
        case kQ4_1: {  // q d + m (src/quant.cpp:207-217)
            const size_t blk = static_cast<size_t>(r) * (cols / 32) + e / 32;
            const float d = h2f(gld<uint16_t>(m.p1, blk));
            const float mn = h2f(gld<uint16_t>(m.p2, blk));
            const uint32_t i = e % 32;
            const uint8_t q = gmem(m.p0)[blk * 16 + (i & 15)];
            return static_cast<float>(i < 16 ? (q & 0x0F) : (q >> 4)) * d + mn;
        }
        case kQ5_0: {  // ((nibble | bit e of qh << 4) - 16) d (src/quant.cpp:219-232)
            const size_t blk = static_cast<size_t>(r) * (cols / 32) + e / 32;
            const float d = h2f(gld<uint16_t>(m.p1, blk));
            const uint32_t qh = gld<uint32_t>(m.p2, blk);
            const uint32_t i = e % 32;
            const uint8_t q = gmem(m.p0)[blk * 16 + (i & 15)];
            const int v = (i < 16 ? (q & 0x0F) : (q >> 4)) | static_cast<int>(((qh >> i) & 1u) << 4);
            return static_cast<float>(v - 16) * d;
        }
        case kQ5_K: {  // Q4_K's with bit s of qh[j] on value j of sub-block s (src/quant.cpp:263-283)
            const size_t blk = static_cast<size_t>(r) * (cols / 256) + e / 256;
            const auto meta = gmem(m.p1 + blk * 16);
            const float d = h2f(static_cast<uint16_t>(meta[0] | (meta[1] << 8)));
            const float dmin = h2f(static_cast<uint16_t>(meta[2] | (meta[3] << 8)));
            const int i = e % 256, chunk = i / 64, hi = (i % 64) >= 32, j = i % 32, sb = 2 * chunk + hi;
            const auto dec = gmem(m.p2 + blk * 48);
            const float d1 = d * static_cast<float>(dec[sb]), m1 = dmin * static_cast<float>(dec[8 + sb]);
            const uint8_t q = gmem(m.p0)[blk * 128 + chunk * 32 + j];
            const int v = (hi ? (q >> 4) : (q & 0xF)) | (((dec[16 + j] >> sb) & 1) << 4);
            return d1 * static_cast<float>(v) - m1;
        }
        case kQ4_K: {
            const size_t blk = static_cast<size_t>(r) * (cols / 256) + e / 256;
            const auto meta = gmem(m.p1 + blk * 16);
            const float d = h2f(static_cast<uint16_t>(meta[0] | (meta[1] << 8)));
            const float dmin = h2f(static_cast<uint16_t>(meta[2] | (meta[3] << 8)));
            const int i = e % 256, chunk = i / 64, hi = (i % 64) >= 32, j = i % 32;
            int sc, mn;
            q4k_scale_min(meta + 4, 2 * chunk + hi, sc, mn);
            const float d1 = d * static_cast<float>(sc), m1 = dmin * static_cast<float>(mn);
            const uint8_t q = gmem(m.p0)[blk * 128 + chunk * 32 + j];
            return d1 * static_cast<float>(hi ? (q >> 4) : (q & 0xF)) - m1;
        }
        case kQ6_K: {
            const size_t blk = static_cast<size_t>(r) * (cols / 256) + e / 256;
            const int i = e % 256, half = i / 128, w = i % 128, quarter = w / 32, l = w % 32;
            const auto ql = gmem(m.p0 + blk * 128 + half * 64);
            const auto qh = gmem(m.p1 + blk * 64 + half * 32);
            const auto meta = gmem(m.p2 + blk * 20);
            const int lo = (quarter & 1) ? ql[l + 32] : ql[l];
            const int nib = quarter >= 2 ? (lo >> 4) : (lo & 0xF);
            const int q = (nib | (((qh[l] >> (2 * quarter)) & 3) << 4)) - 32;
            const float d = h2f(static_cast<uint16_t>(meta[16] | (meta[17] << 8)));
            return d * static_cast<float>(static_cast<int8_t>(meta[i / 16])) * static_cast<float>(q);
        }
        default: {  // TQ2_0
            const size_t blk = static_cast<size_t>(r) * (cols / 256) + e / 256;
            const int i = e % 256;
            const int c = (gmem(m.p0)[blk * 64 + (i / 128) * 32 + i % 32] >> (2 * ((i % 128) / 32))) & 3;
            return static_cast<float>(c - 1) * h2f(gld<uint16_t>(m.p1, blk));
        }
    }
}

// Ordered 64-bit key of (logit, index): larger logit first, then smaller index,
// so one atomicMax finds the reference's pick (std::max_element: the first index
// of the maximum, src/sampler.cpp:11-13).  -0 is keyed as +0 (they compare equal).
__device__ __forceinline__ unsigned long long pick_key(float v, uint32_t idx) {
    if (v == 0.0f) v = 0.0f;
    const uint32_t u = __float_as_uint(v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<unsigned long long>(ord) << 32) | (0xFFFFFFFFu - idx);
}



struct AttnLds {
    alignas(16) float q[16 * 128];   // the group's query heads (raw, then normed and rotated)
    float kcur[128], vcur[128];      // this token's key and value (raw, then fp16-rounded)
    alignas(16) float sc[kExactScores + 64];  // scores, then weights: [head][position] (rows may be padded)
    double red[16][4];
    float mx[16];
    float ml[16][2];
    alignas(16) uint16_t kv[2][kSplit * 128];  // two staged chunks of keys or values (kept last: see AttnPoolLds)
};

// The persistent loop's attention space: AttnLds with its chunk buffers
// extended to kPoolChunks, so that a whole context's keys (and, when they fit,
// its values) are staged at once.
constexpr int kPoolChunks = 8;
struct AttnPoolLds {
    AttnLds a;
    alignas(16) uint16_t more[kPoolChunks - 2][kSplit * 128];
    __device__ __forceinline__ uint16_t* chunk(int i) { return &a.kv[0][0] + static_cast<size_t>(i) * kSplit * 128; }
};

// ---------------------------------------------------------------- tagged words

// A 64-bit word holding a float and the tag of the step that produced it,
// written and read with system-scope accesses (past the per-XCD L2s).
__device__ __forceinline__ void tput(unsigned long long* p, float v, unsigned tag) {
    __hip_atomic_store(gmem(p), (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ unsigned long long tload(const unsigned long long* p) {
    return __hip_atomic_load(gmem(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Where attention puts its results: plain floats (one kernel per phase) ...
struct PlainOut {
    float* out;
    float* part_acc;
    float* part_ml;
    __device__ __forceinline__ void att(int i, float v) const { out[i] = v; }
    __device__ __forceinline__ void pacc(size_t i, float v) const { part_acc[i] = v; }
    __device__ __forceinline__ void pml(size_t i, float v) const { part_ml[i] = v; }
    // read after a device-scope fence by the merging workgroup
    __device__ __forceinline__ bool get_pacc(size_t i, float& v) const { v = CoherentIO::ld(part_acc + i); return true; }
    __device__ __forceinline__ bool get_pml(size_t i, float& v) const { v = CoherentIO::ld(part_ml + i); return true; }
};

// ... or tagged words (the persistent loop); reads wait for the tag.
struct TaggedOut {
    unsigned long long* out;
    unsigned long long* part_acc;
    unsigned long long* part_ml;
    unsigned tag;
    int* error;
    int q8;      // publish the attention output quantised (Q8_0), see att_q8_0
    int total;   // values of the whole attention output (heads x head size)
    __device__ __forceinline__ void att(int i, float v) const {
        if (q8) att_q8_0(i, v);
        else tput(out + i, v, tag);
    }
    // The consumer (the O projection, no sub-norm) takes the attention output
    // as quantize_q8_0 makes it (src/quant.cpp:115-142), so the producer
    // quantises it here and publishes the blocks: words [0, total / 4) hold the
    // int8 values four a word, then total / 32 fp16-rounded scales (as floats),
    // then total / 32 block sums.  One value a lane: lanes 32 k .. 32 k + 31 hold
    // a block, and all of them call together.
    __device__ __forceinline__ void att_q8_0(int i, float v) const {
        // the two 16-lane rows of a block combined through scalar reads of their first lanes (no
        // LDS round trip); the quad's bytes gathered by DPP quad broadcasts
        const bool upper = (threadIdx.x & 63) >= 32;
        float amax = group_reduce<16>(fabsf(v), [](float a, float b) { return nnmax(a, b); });
        amax = upper ? nnmax(readlane(amax, 32), readlane(amax, 48)) : nnmax(readlane(amax, 0), readlane(amax, 16));
        const float d = div127(amax);
        const float inv = d != 0.0f ? rcp_rn(d) : 0.0f;
        const int q = static_cast<int>(rintf(v * inv));
        int sum = group_reduce<16>(q, [](int a, int b) { return a + b; });
        sum = upper ? readlane(sum, 32) + readlane(sum, 48) : readlane(sum, 0) + readlane(sum, 16);
        const int q1 = dpp<0x55>(q), q2 = dpp<0xAA>(q), q3 = dpp<0xFF>(q);
        if ((i & 3) == 0) {
            const uint32_t w = (q & 0xFF) | ((q1 & 0xFF) << 8) | ((q2 & 0xFF) << 16) | (static_cast<uint32_t>(q3) << 24);
            tput(out + i / 4, __uint_as_float(w), tag);
        }
        if ((i & 31) == 0) {
            tput(out + total / 4 + i / 32, h2f(f2h(d)), tag);
            tput(out + total / 4 + total / 32 + i / 32, __int_as_float(sum), tag);
        }
    }
    __device__ __forceinline__ void pacc(size_t i, float v) const { tput(part_acc + i, v, tag); }
    __device__ __forceinline__ void pml(size_t i, float v) const { tput(part_ml + i, v, tag); }
    __device__ bool wait(const unsigned long long* p, float& v) const {
        unsigned long long w;
        unsigned spins = 0;
        while (static_cast<unsigned>((w = tload(p)) >> 32) != tag) {
            if (++spins > (1u << 24)) {
                atomicExch(error, 1);
                return false;
            }
            if ((spins & 63) == 0 && __hip_atomic_load(error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) return false;
            __builtin_amdgcn_s_sleep(1);
        }
        v = __uint_as_float(static_cast<unsigned>(w));
        return true;
    }
    __device__ __forceinline__ bool get_pacc(size_t i, float& v) const { return wait(part_acc + i, v); }
    __device__ __forceinline__ bool get_pml(size_t i, float& v) const { return wait(part_ml + i, v); }
};

// The projection bias (add_bias, src/model.cpp:117-119 and :1026-1030), an
// RMS norm over one head (optional weight w) and RoPE (none when rope is
// null), by one wave: the per-head steps of src/model.cpp:1021-1041, with
// rms_norm's float squares summed in double (src/model.cpp:87-97).
__device__ __forceinline__ void head_norm_rope(float* v, const float* bias, const float* w, const float* rope, int hd, int rd,
                                               int neox, float eps) {
    const int lane = threadIdx.x & 63;
    if (bias != nullptr)
        for (int i = lane; i < hd; i += 64) v[i] = v[i] + gmem(bias)[i];
    if (w != nullptr) {
        double s = 0.0;
        for (int i = lane; i < hd; i += 64) s += static_cast<double>(v[i] * v[i]);
        s = wave_sum(s);
        const float scale = rms_scale(s, hd, eps);
        for (int i = lane; i < hd; i += 64) v[i] = v[i] * scale * gmem(w)[i];
    }
    if (rope == nullptr) return;
    const int half = rd / 2;  // only the first rd dimensions rotate (apply_rope, src/model.cpp:100-115)
    for (int i = lane; i < half; i += 64) {
        const float c = rope[2 * i], sn = rope[2 * i + 1];
        const int ia = neox ? i : 2 * i, ib = neox ? i + half : 2 * i + 1;
        const float x0 = v[ia], x1 = v[ib];
        v[ia] = x0 * c - x1 * sn;
        v[ib] = x0 * sn + x1 * c;
    }
}

// This token's raw query heads of the group, and (writer) its raw key and value, into LDS.
template <class IO>
__device__ __forceinline__ void attn_load_raw(const AttnArgs& g, AttnLds& s, int kv, bool writer) {
    const int hd = g.head_dim, hpk = g.heads / g.kv_heads, t = threadIdx.x;
    for (int i = t; i < hpk * hd; i += kThreads) s.q[i] = IO::ld(g.q + kv * hpk * hd + i);
    if (writer)
        for (int i = t; i < hd; i += kThreads) {
            s.kcur[i] = IO::ld(g.k + kv * hd + i);
            s.vcur[i] = IO::ld(g.v + kv * hd + i);
        }
    __syncthreads();
}

// The writer's K and V rows at position pos (store_f16, src/kernels_f32.cpp:248-250),
// from the fp16-rounded values in LDS.  kWriteThrough: system-scope stores, for
// rows another workgroup reads later in the same launch; the caller orders them
// before its later writes (an s_waitcnt before those).
template <bool kWriteThrough>
__device__ __forceinline__ void attn_store_rows(const AttnArgs& g, const AttnLds& s, int kv, int pos) {
    const int hd = g.head_dim, t = threadIdx.x;
    uint16_t* kr = g.kcache + (static_cast<size_t>(kv) * g.ctx + pos) * hd;
    uint16_t* vr = g.vcache + (static_cast<size_t>(kv) * g.ctx + pos) * hd;
    for (int i = 2 * t; i < hd; i += 2 * kThreads) {
        const uint32_t kw = f2h(s.kcur[i]) | (static_cast<uint32_t>(f2h(s.kcur[i + 1])) << 16);
        const uint32_t vw = f2h(s.vcur[i]) | (static_cast<uint32_t>(f2h(s.vcur[i + 1])) << 16);
        if (kWriteThrough) {
            __hip_atomic_store(gmem(reinterpret_cast<uint32_t*>(kr + i)), kw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(gmem(reinterpret_cast<uint32_t*>(vr + i)), vw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        } else {
            *reinterpret_cast<uint32_t*>(kr + i) = kw;
            *reinterpret_cast<uint32_t*>(vr + i) = vw;
        }
    }
}

// Norms and RoPE of the raw q (and k), and the fp16 rounding of the writer's
// k and v in LDS; with `store`, the writer also stores the rows (waiting for
// them when kWriteThrough).  Ends with a barrier.
template <bool kWriteThrough>
__device__ __forceinline__ void attn_finish_prologue(const AttnArgs& g, AttnLds& s, int kv, int pos, bool writer,
                                                     bool store = true) {
    const int hd = g.head_dim, hpk = g.heads / g.kv_heads, t = threadIdx.x;
    const float* rope = g.rope != nullptr ? g.rope + static_cast<size_t>(pos) * g.rope_dim : nullptr;
    const int wave = t >> 6;
    for (int h = wave; h < hpk + (writer ? 1 : 0); h += kThreads / 64) {
        if (h < hpk) head_norm_rope(s.q + h * hd, g.qbias != nullptr ? g.qbias + (kv * hpk + h) * hd : nullptr, g.qnorm, rope, hd, g.rope_dim, g.neox, g.eps);
        else head_norm_rope(s.kcur, g.kbias != nullptr ? g.kbias + kv * hd : nullptr, g.knorm, rope, hd, g.rope_dim, g.neox, g.eps);
    }
    __syncthreads();
    if (writer) {
        for (int i = t; i < hd; i += kThreads) {
            s.kcur[i] = h2f(f2h(s.kcur[i]));
            s.vcur[i] = h2f(f2h(g.vbias != nullptr ? s.vcur[i] + gmem(g.vbias)[kv * hd + i] : s.vcur[i]));
        }
        __syncthreads();
        if (store) {
            attn_store_rows<kWriteThrough>(g, s, kv, pos);
            // the rows are in memory before anything this workgroup writes later is
            if (kWriteThrough) __builtin_amdgcn_s_waitcnt(0);
        }
    }
}

template <class IO, bool kWriteThrough = false>
__device__ __forceinline__ void attn_prologue(const AttnArgs& g, AttnLds& s, int kv, int pos, bool writer) {
    attn_load_raw<IO>(g, s, kv, writer);
    attn_finish_prologue<kWriteThrough>(g, s, kv, pos, writer);
}

// Chunk staging: positions [p0, p0 + n_pos) of one head's cache rows
// ([ctx][hd] fp16, contiguous) straight from global memory into LDS with
// gfx950's global_load_lds_dwordx4 (16 bytes a lane, lane i of a wave at the
// wave's LDS base + 16 i).  Completion: s_waitcnt vmcnt(0) + barrier.
typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef __attribute__((address_space(1))) const void* global_cvoid_ptr;

// Swizzled key layout: 16-byte piece c of chunk row p sits at piece slot
// p * P + (c ^ (p & mask)) (P = hd / 8 pieces a row, mask = P - 1 when P is a
// power of two, else 0), so lanes reading the same piece of different rows hit
// different LDS banks.
__device__ __forceinline__ int kv_pieces(int hd) { return hd / 8; }
__device__ __forceinline__ int kv_mask(int hd) {
    const int P = hd / 8;
    return (P & (P - 1)) == 0 ? P - 1 : 0;
}

__device__ __forceinline__ void chunk_issue(uint16_t* lds, const uint16_t* base, int p0, int n_pos, int hd, bool swz = false) {
    const int P = kv_pieces(hd), mask = swz ? kv_mask(hd) : 0;
    const int pieces = n_pos * P;  // 16-byte pieces
    const uint8_t* src = reinterpret_cast<const uint8_t*>(base + static_cast<size_t>(p0) * hd);
    uint8_t* dst = reinterpret_cast<uint8_t*>(lds);
    const int wave_first = static_cast<int>(threadIdx.x) & ~63;
    for (int k = 0; k * kThreads < pieces; ++k) {
        const int i = k * kThreads + static_cast<int>(threadIdx.x);  // the LDS slot this lane fills
        if (i < pieces) {
            const int p = i / P, c = (i - p * P) ^ (p & mask);
            __builtin_amdgcn_global_load_lds((global_cvoid_ptr)(src + (static_cast<size_t>(p) * P + c) * 16),
                                             (lds_void_ptr)(dst + (k * kThreads + wave_first) * 16), 16, 0, 0);
        }
    }
}

__device__ __forceinline__ void attn_stamp(const AttnArgs& g, int kv, int i) {
    if (g.stamps != nullptr && kv == 0 && threadIdx.x == 0) g.stamps[i] = wall_clock64();
}

// Positions of chunk c (of kSplit) that come from the cache; the current
// position (pos) comes from LDS.
__device__ __forceinline__ int chunk_cached(int c, int L) {
    const int pos = L - 1, p0 = c * kSplit;
    const int n = L - p0 < kSplit ? L - p0 : kSplit;
    return pos - p0 < n ? pos - p0 : n;
}

// Waits for chunk c (staged earlier into buffer c & 1), completes it with the
// current position's row from `cur` (LDS floats, fp16-rounded already) and
// starts staging chunk c + 1 into the other buffer, which overlaps chunk c's
// compute.
__device__ __forceinline__ uint16_t* chunk_advance(AttnLds& s, const uint16_t* base, const float* cur, int c, int nchunks, int L,
                                                   int hd, bool swz = false) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of chunk c have landed
    __syncthreads();                // ... everyone's, and buffer (c + 1) & 1 (chunk c - 1) is consumed
    if (c + 1 < nchunks) {
        const int nn = chunk_cached(c + 1, L);
        if (nn > 0) chunk_issue(s.kv[(c + 1) & 1], base, (c + 1) * kSplit, nn, hd, swz);
    }
    uint16_t* buf = s.kv[c & 1];
    const int p0 = c * kSplit, n = L - p0 < kSplit ? L - p0 : kSplit, ncache = chunk_cached(c, L);
    if (ncache < n) {
        const int P = kv_pieces(hd), mask = swz ? kv_mask(hd) : 0;
        for (int i = threadIdx.x; i < hd; i += kThreads)
            buf[(ncache * P + ((i >> 3) ^ (ncache & mask))) * 8 + (i & 7)] = f2h(cur[i]);
    }
    __syncthreads();
    return buf;
}

// Starts staging the first key chunk of kv head `kv` (positions before the
// current one only: they are in the cache already), e.g. before the current
// token's q/k/v have arrived.
__device__ __forceinline__ void attn_issue_k0(const AttnArgs& g, AttnLds& s, int kv, int L) {
    const int n0 = chunk_cached(0, L);
    if (n0 > 0) chunk_issue(s.kv[0], g.kcache + static_cast<size_t>(kv) * g.ctx * g.head_dim, 0, n0, g.head_dim, true);
}

// One score, dot_f32(q, k_p) (src/kernels_f32.cpp:229-246), by one lane: 16
// lane partials l_j = 0 + q_j k_j + q_(j+16) k_(j+16) + ... (PER terms each),
// then 0 + l_0 + ... + l_15.  k_p is row p of a swizzled chunk (P pieces a
// row); q is in LDS (lanes of one head read the same address: a broadcast).
template <int PER>
__device__ __forceinline__ float score_lane(const float* q, const uint16_t* chunk, int p, int P, int mask) {
    float lane[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) lane[j] = 0.0f;
    const uint4* rows = reinterpret_cast<const uint4*>(chunk);
#pragma unroll
    for (int m = 0; m < PER; ++m) {
        const uint4 k0 = rows[p * P + ((2 * m) ^ (p & mask))];
        const uint4 k1 = rows[p * P + ((2 * m + 1) ^ (p & mask))];
        const float4* q4 = reinterpret_cast<const float4*>(q + 16 * m);
        const float4 qa = q4[0], qb = q4[1], qc = q4[2], qd = q4[3];
        const uint32_t kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
        const float qv[16] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w, qc.x, qc.y, qc.z, qc.w, qd.x, qd.y, qd.z, qd.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint16_t h = static_cast<uint16_t>((j & 1) ? (kw[j >> 1] >> 16) : (kw[j >> 1] & 0xFFFF));
            lane[j] += qv[j] * h2f(h);
        }
    }
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) sum += lane[j];
    return sum;
}

// The reference's attention for one token (src/model.cpp:1050-1093 with the
// portable kernels of src/kernels_f32.cpp:229-284), operation for operation:
//   score_p = dot_f32(q, k_p) * scale, dot_f32 being 16 lane partials over
//             i = j (mod 16) in order, then 0 + lane 0 + ... + lane 15;
//   softmax: max, e_p = expf(s_p - max), sum of e_p in double, w_p = e_p * (float)(1 / sum);
//   out    = 0 + w_0 v_0 + w_1 v_1 + ... in position order (weighted_sum_f32's axpy).
// The one grouping that differs is the double sum, whose rounding can reach the
// float scale only when terms below 2^-20 of the sum lose bits.
// A score is computed by one lane.  store_rows: the writer's K/V rows are stored here, once the first
// key chunk has landed (so that wait does not also wait for the stores).
template <class O>
__device__ __forceinline__ void attn_exact(const AttnArgs& g, AttnLds& s, int kv, int L, const O& o, bool k0_issued = false,
                                           bool store_rows = false) {
    const int hd = g.head_dim, hpk = g.heads / g.kv_heads, t = threadIdx.x, per = hd / 16;
    // the scores in LDS when they fit it, else in the global buffer (same order of every operation)
    float* const scores = L * hpk <= kExactScores ? s.sc : g.gsc + static_cast<size_t>(kv) * hpk * g.ctx;
    const int nchunks = (L + kSplit - 1) / kSplit;
    const uint16_t* kbase = g.kcache + static_cast<size_t>(kv) * g.ctx * hd;
    const uint16_t* vbase = g.vcache + static_cast<size_t>(kv) * g.ctx * hd;
    attn_stamp(g, kv, 1);
    // ---- scores, chunk by chunk
    if (!k0_issued) attn_issue_k0(g, s, kv, L);
    const int P = kv_pieces(hd), mask = kv_mask(hd);
    for (int c = 0; c < nchunks; ++c) {
        const uint16_t* kvb = chunk_advance(s, kbase, s.kcur, c, nchunks, L, hd, true);
        if (c == 0 && store_rows) attn_store_rows<true>(g, s, kv, L - 1);
        const int p0 = c * kSplit, n = L - p0 < kSplit ? L - p0 : kSplit, pairs = hpk * n;
        for (int i = t; i < pairs; i += kThreads) {  // one (head, position) score a lane
            const int gq = i / n, p = i - gq * n;
            const float* q = s.q + gq * hd;
            const float v = per == 8 ? score_lane<8>(q, kvb, p, P, mask) : per == 6 ? score_lane<6>(q, kvb, p, P, mask)
                          : per == 4 ? score_lane<4>(q, kvb, p, P, mask) : score_lane<2>(q, kvb, p, P, mask);
            scores[gq * L + p0 + p] = v * g.scale;
        }
    }
    // the first value chunk streams in while the softmax runs
    __syncthreads();
    attn_stamp(g, kv, 7);
    {
        const int n0 = chunk_cached(0, L);
        if (n0 > 0) chunk_issue(s.kv[0], vbase, 0, n0, hd);
    }
    attn_stamp(g, kv, 2);
    // ---- softmax, a wave per head
    const int wave = t >> 6, wl = t & 63;
    for (int gq = wave; gq < hpk; gq += kThreads / 64) {
        float* sc = scores + gq * L;
        float m = -INFINITY;
        for (int p = wl; p < L; p += 64) m = fmaxf(m, sc[p]);
        m = wave_max(m);
        double part = 0.0;
        for (int p = wl; p < L; p += 64) {
            const float e = ref_expf(sc[p] - m);
            sc[p] = e;
            part += static_cast<double>(e);
        }
        const float scale = static_cast<float>(1.0 / wave_sum(part));
        for (int p = wl; p < L; p += 64) sc[p] *= scale;
    }
    attn_stamp(g, kv, 3);
    // ---- value sums in position order, chunk by chunk
    float acc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = 0.0f;
    const int chains = hpk * hd;
    for (int c = 0; c < nchunks; ++c) {
        const uint16_t* kvb = chunk_advance(s, vbase, s.vcur, c, nchunks, L, hd);
        const int p0 = c * kSplit, n = L - p0 < kSplit ? L - p0 : kSplit;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int ch = t + k * kThreads;
            if (ch < chains) {
                const int gq = ch / hd, d = ch % hd;
                const float* w = scores + gq * L + p0;
                const uint16_t* vv = kvb + d;
                float a = acc[k];
                int p = 0;
                for (; p + 8 <= n; p += 8) {  // loads first, then the adds in position order
                    float wv[8], vf[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        wv[u] = w[p + u];
                        vf[u] = h2f(vv[(p + u) * hd]);
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u) a += wv[u] * vf[u];
                }
                for (; p < n; ++p) a += w[p] * h2f(vv[p * hd]);
                acc[k] = a;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int ch = t + k * kThreads;
        if (ch < chains) o.att(kv * hpk * hd + ch, acc[k]);
    }
    attn_stamp(g, kv, 4);
}

// ---------------------------------------------------------------- pooled exact attention (the loop)

// Where the pooled attention stages chunk c of the keys / values for a context of L.
__device__ __forceinline__ int pool_nchunks(int L) { return (L + kSplit - 1) / kSplit; }
__device__ __forceinline__ bool pool_values_early(int L) { return 2 * pool_nchunks(L) <= kPoolChunks; }

// Issues the cached rows of every key chunk (and of every value chunk when
// both fit the pool) of kv head `kv`; the first LDS access after this waits for
// them, so one memory latency covers the whole context.  Needs L <= kSplit * kPoolChunks.
__device__ __forceinline__ void attn_pool_issue(const AttnArgs& g, AttnPoolLds& s, int kv, int L) {
    const int n = pool_nchunks(L), hd = g.head_dim;
    const uint16_t* kbase = g.kcache + static_cast<size_t>(kv) * g.ctx * hd;
    const uint16_t* vbase = g.vcache + static_cast<size_t>(kv) * g.ctx * hd;
    for (int c = 0; c < n; ++c) {
        const int nn = chunk_cached(c, L);
        if (nn > 0) chunk_issue(s.chunk(c), kbase, c * kSplit, nn, hd, true);
    }
    if (pool_values_early(L))
        for (int c = 0; c < n; ++c) {
            const int nn = chunk_cached(c, L);
            if (nn > 0) chunk_issue(s.chunk(n + c), vbase, c * kSplit, nn, hd, false);
        }
}

// The current position's row (cur, fp16-rounded floats) into its chunk buffer.
__device__ __forceinline__ void pool_put_current(uint16_t* buf, const float* cur, int L, int hd, bool swz) {
    const int pos = L - 1, r = pos % kSplit, P = kv_pieces(hd), mask = swz ? kv_mask(hd) : 0;
    for (int i = threadIdx.x; i < hd; i += kThreads) buf[(r * P + ((i >> 3) ^ (r & mask))) * 8 + (i & 7)] = f2h(cur[i]);
}

// attn_exact's arithmetic (the reference's order, see there) over the pool:
// keys (and values) were issued by attn_pool_issue; the writer's cache rows
// are stored here once the keys have landed.
// HD: the head size when it is a compile-time constant (64, 128), else 0.
template <int HD, class O>
__device__ __forceinline__ void attn_exact_pool(const AttnArgs& g, AttnPoolLds& sp, int kv, int L, const O& o) {
    AttnLds& s = sp.a;
    const int hd = HD != 0 ? HD : g.head_dim, hpk = g.heads / g.kv_heads, t = threadIdx.x, per = hd / 16;
    const int n = pool_nchunks(L), last = (L - 1) / kSplit;
    const int Ls = (L + 3) & ~3;  // score row stride: rows start 16-byte aligned
    const bool early = pool_values_early(L);
    attn_stamp(g, kv, 1);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's key (and value) loads have landed
    pool_put_current(sp.chunk(last), s.kcur, L, hd, true);
    if (early) pool_put_current(sp.chunk(n + last), s.vcur, L, hd, false);
    __syncthreads();
    attn_store_rows<true>(g, s, kv, L - 1);
    attn_stamp(g, kv, 5);
    // ---- scores
    const int P = kv_pieces(hd), mask = kv_mask(hd), pairs = hpk * L;
    for (int i = t; i < pairs; i += kThreads) {  // one (head, position) score a lane
        const int gq = i / L, pos = i - gq * L, c = pos / kSplit, p = pos - c * kSplit;
        const float* q = s.q + gq * hd;
        const uint16_t* buf = sp.chunk(c);
        float v;
        if (HD != 0) v = score_lane<(HD != 0 ? HD : 128) / 16>(q, buf, p, HD / 8, HD / 8 - 1);
        else v = per == 8 ? score_lane<8>(q, buf, p, P, mask) : per == 6 ? score_lane<6>(q, buf, p, P, mask)
               : per == 4 ? score_lane<4>(q, buf, p, P, mask) : score_lane<2>(q, buf, p, P, mask);
        s.sc[gq * Ls + pos] = v * g.scale;
    }
    __syncthreads();
    attn_stamp(g, kv, 2);
    const int vfirst = early ? n : 0;
    if (!early) {  // the keys are consumed: the values take their buffers
        const uint16_t* vbase = g.vcache + static_cast<size_t>(kv) * g.ctx * hd;
        for (int c = 0; c < n; ++c) {
            const int nn = chunk_cached(c, L);
            if (nn > 0) chunk_issue(sp.chunk(c), vbase, c * kSplit, nn, hd, false);
        }
    }
    // ---- softmax, a wave per head
    const int wave = t >> 6, wl = t & 63;
    for (int gq = wave; gq < hpk; gq += kThreads / 64) {
        float* sc = s.sc + gq * Ls;
        float m = -INFINITY;
        for (int p = wl; p < L; p += 64) m = fmaxf(m, sc[p]);
        m = wave_max(m);
        double part = 0.0;
        for (int p = wl; p < L; p += 64) {
            const float e = ref_expf(sc[p] - m);
            sc[p] = e;
            part += static_cast<double>(e);
        }
        const float scale = static_cast<float>(1.0 / wave_sum(part));
        for (int p = wl; p < L; p += 64) sc[p] *= scale;
    }
    if (!early) {
        __builtin_amdgcn_s_waitcnt(0);
        pool_put_current(sp.chunk(last), s.vcur, L, hd, false);
    }
    __syncthreads();
    attn_stamp(g, kv, 3);
    // ---- value sums in position order, one chain a lane (every SIMD busy).  Positions
    // go in batches of 8 (never across a chunk); the next batch's weights and values
    // are read before the current batch's adds, so LDS latency overlaps them.
    const int chains = hpk * hd, full = L & ~7;
    const uint16_t* vpool = sp.chunk(vfirst);
    for (int ch = t; ch < chains; ch += kThreads) {
        const int gq = ch / hd, d = ch % hd;
        const float* w = s.sc + gq * Ls;
        const uint16_t* vcol = vpool + d;
        auto vat = [&](int pos) -> const uint16_t* { return vcol + (pos >> 6) * (kSplit * 128) + (pos & 63) * hd; };
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
            if (p < full) {  // one batch left, in va / wa
                a += wa0.x * h2f(va[0]); a += wa0.y * h2f(va[1]); a += wa0.z * h2f(va[2]); a += wa0.w * h2f(va[3]);
                a += wa1.x * h2f(va[4]); a += wa1.y * h2f(va[5]); a += wa1.z * h2f(va[6]); a += wa1.w * h2f(va[7]);
                p += 8;
            }
        }
        for (; p < L; ++p) a += w[p] * h2f(*vat(p));
        o.att(kv * hpk * hd + ch, a);
    }
    attn_stamp(g, kv, 4);
}

// Split-K (flash-decoding) partials for longer contexts: each workgroup scores
// kSplit positions for all the key/value head's query heads and keeps (max, sum
// of exp, exp-weighted value sum); attn_split_combine then merges the splits
// with the log-sum-exp rescale.  Same mathematics as the reference, different
// rounding order (tolerance, not bit-exact).
template <class O>
__device__ __forceinline__ void attn_split_partial(const AttnArgs& g, AttnLds& s, int kv, int split, int L, const O& o) {
    const int hd = g.head_dim, hpk = g.heads / g.kv_heads, t = threadIdx.x;
    const int p0 = split * kSplit;
    const int n = L - p0 < kSplit ? L - p0 : kSplit;
    const int ncache = chunk_cached(split, L);
    const uint16_t* kbase = g.kcache + static_cast<size_t>(kv) * g.ctx * hd;
    const uint16_t* vbase = g.vcache + static_cast<size_t>(kv) * g.ctx * hd;
    __syncthreads();
    if (ncache > 0) {
        chunk_issue(s.kv[0], kbase, p0, ncache, hd);
        chunk_issue(s.kv[1], vbase, p0, ncache, hd);  // values in flight while scoring
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (ncache < n)
        for (int i = t; i < hd; i += kThreads) {
            s.kv[0][ncache * hd + i] = f2h(s.kcur[i]);
            s.kv[1][ncache * hd + i] = f2h(s.vcur[i]);
        }
    __syncthreads();
    float* sc = s.sc;  // [head][kSplit]
    for (int i = t; i < hpk * kSplit; i += kThreads) {
        const int gq = i / kSplit, p = i % kSplit;
        float acc = -INFINITY;
        if (p < n) {
            acc = 0.0f;
            const uint16_t* kr = s.kv[0] + p * hd;
            const float* q = s.q + gq * hd;
            for (int d = 0; d < hd; ++d) acc += q[d] * h2f(kr[d]);
            acc *= g.scale;
        }
        sc[gq * kSplit + p] = acc;
    }
    __syncthreads();
    const int wave = t >> 6, lane = t & 63;
    for (int gq = wave; gq < hpk; gq += 4) {
        const float sv = sc[gq * kSplit + lane];
        const float mx = wave_max(sv);
        const float e = lane < n ? ref_expf(sv - mx) : 0.0f;
        const float l = wave_sum(e);
        sc[gq * kSplit + lane] = e;
        if (lane == 0) { s.ml[gq][0] = mx; s.ml[gq][1] = l; }
    }
    __syncthreads();
    for (int i = t; i < hpk * hd; i += kThreads) {
        const int gq = i / hd, d = i % hd;
        float acc = 0.0f;
        for (int p = 0; p < n; ++p) acc += sc[gq * kSplit + p] * h2f(s.kv[1][p * hd + d]);
        const size_t slot = static_cast<size_t>(kv * hpk + gq) * g.max_splits + split;
        o.pacc(slot * hd + d, acc);
        if (d == 0) {
            o.pml(slot * 2, s.ml[gq][0]);
            o.pml(slot * 2 + 1, s.ml[gq][1]);
        }
    }
}

// Merges the splits of key/value head kv's query heads into the output.
template <class O>
__device__ __forceinline__ bool attn_split_combine(const AttnArgs& g, int kv, int L, const O& o) {
    const int hd = g.head_dim, hpk = g.heads / g.kv_heads, t = threadIdx.x;
    const int ns = (L + kSplit - 1) / kSplit;
    for (int i = t; i < hpk * hd; i += kThreads) {
        const int gq = i / hd, d = i % hd;
        const size_t base = static_cast<size_t>(kv * hpk + gq) * g.max_splits;
        float M = -INFINITY, v = 0.0f;
        for (int s2 = 0; s2 < ns; ++s2) {
            if (!o.get_pml((base + s2) * 2, v)) return false;
            M = fmaxf(M, v);
        }
        float num = 0.0f, den = 0.0f;
        for (int s2 = 0; s2 < ns; ++s2) {
            float m = 0.0f, l = 0.0f, a = 0.0f;
            if (!o.get_pml((base + s2) * 2, m) || !o.get_pml((base + s2) * 2 + 1, l) || !o.get_pacc((base + s2) * hd + d, a))
                return false;
            const float f = ref_expf(m - M);
            den += l * f;
            num += a * f;
        }
        o.att((kv * hpk + gq) * hd + d, num / den);
    }
    return true;
}


}  // namespace bh
