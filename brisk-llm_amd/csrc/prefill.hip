// Batched prefill: a prompt's tokens go through each layer together, with the
// weight contractions on int8 MFMA.
//
// Exactness.  The reference multiplies block by block: per block (32 values,
// or a K-quant sub-block) an exact int32 dot, then a float term added to the
// row sum in block order (src/quant.cpp:445-596, matmul_generic
// src/kernels.cpp:13-30 runs the same dot per token).  v_mfma_i32_16x16x32_i8
// computes, for 16 rows x 16 tokens, exactly those int32 block dots (K = 32 is
// one block), so the float epilogue here repeats the reference's term and sum
// order per output and every output is bit-identical to the matvec path.
//
// Operand layouts of v_mfma_i32_16x16x32_i8 (wave of 64, lane l):
//   A (16 x 32, rows x k):   lane l holds A[l % 16][8 (l / 16) .. + 7]
//   B (32 x 16, k x tokens): lane l holds B[8 (l / 16) .. + 7][l % 16]
//   D (16 x 16 int32):       lane l holds D[4 (l / 16) + i][l % 16], i = 0..3
//
// Activations for the GEMMs are quantised per token into a planar layout
// (ActPlanar): int8 values [T][cols], scales [T][cols / 32] (Q8_0: one per
// 32; Q8_K: one per 256), int32 sums [T][cols / 16] (Q8_K bsums).
#include "phases.h"
#include "prefill.h"

#include <cstdlib>
#include <string>


namespace bh {

typedef int v4i __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- activations

// One token's row x (rms_norm'd by w when given) quantised into the planar layout.
__global__ __launch_bounds__(kThreads) void k_pre_quant(const float* __restrict__ x, int xstride, const float* __restrict__ w,
                                                         float eps, int cols, int q8k, int bits, ActPlanar out) {
    __shared__ ActLds a;
    __shared__ double red[4];
    const int t = blockIdx.x;
    const float* row = x + static_cast<size_t>(t) * xstride;
    ActRegs ar;
    act_issue(ar, row, w, cols);
    act_finish(ar, row, w, eps, cols, q8k != 0, bits, a, red);
    int32_t* qs = reinterpret_cast<int32_t*>(out.qs + static_cast<size_t>(t) * out.stride);
    for (int i = threadIdx.x; i < cols / 4; i += kThreads) qs[i] = a.xs[i];
    float* d = out.d + static_cast<size_t>(t) * (out.stride / 32);
    for (int i = threadIdx.x; i < cols / 32; i += kThreads) d[i] = a.xd[i];
    int32_t* bs = out.bs + static_cast<size_t>(t) * (out.stride / 16);
    for (int i = threadIdx.x; i < cols / 16; i += kThreads) bs[i] = a.xsum[i];
}

// quantize_q8_k / quantize_q8_0 (src/quant.cpp:115-194) of 256-value block b of token t's row,
// by one wave: lane l holds values 4 l .. 4 l + 3 of the block (the mapping, and so every
// operation, of quant_piece_q8_k / quant_piece_q8_0), straight into the planar layout.
template <bool Q8K>
__device__ __forceinline__ void pre_quant_block(const float (&v)[4], int t, int b, int bits, const ActPlanar& out) {
    const int lane = threadIdx.x & 63, base = b * 256 + 4 * lane;
    int q[4];
    if constexpr (Q8K) {
        float amax;
        const float sel = block_first_absmax(v, amax);
        float d;
        if (amax == 0.0f) {
            d = 0.0f;
            q[0] = q[1] = q[2] = q[3] = 0;
        } else {
            const float extreme = bits == 7 ? 63.0f : 127.0f;
            const float inv = -extreme / sel;
            d = rcp_rn(inv);
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = static_cast<int>(fminf(127.0f, rintf(inv * v[i])));
        }
        int sm = q[0] + q[1] + q[2] + q[3];
        sm = group_reduce<4>(sm, [](int a, int c) { return a + c; });
        if ((lane & 3) == 0) out.bs[static_cast<size_t>(t) * (out.stride / 16) + base / 16] = static_cast<int16_t>(sm);  // bsums are int16
        if (lane == 0) out.d[static_cast<size_t>(t) * (out.stride / 32) + b] = d;
    } else {
        float amax = nnmax(nnmax(fabsf(v[0]), fabsf(v[1])), nnmax(fabsf(v[2]), fabsf(v[3])));
        amax = group_reduce<8>(amax, [](float a, float c) { return nnmax(a, c); });
        const float d = div127(amax);
        const float inv = d != 0.0f ? rcp_rn(d) : 0.0f;
        int sm = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q[i] = static_cast<int>(rintf(v[i] * inv));
            sm += q[i];
        }
        sm = group_reduce<8>(sm, [](int a, int c) { return a + c; });
        if ((lane & 7) == 0) {
            out.d[static_cast<size_t>(t) * (out.stride / 32) + base / 32] = h2f(f2h(d));
            out.bs[static_cast<size_t>(t) * (out.stride / 16) + base / 32] = sm;
        }
    }
    *reinterpret_cast<int32_t*>(out.qs + static_cast<size_t>(t) * out.stride + base) =
        (q[0] & 0xFF) | ((q[1] & 0xFF) << 8) | ((q[2] & 0xFF) << 16) | (q[3] << 24);
}

// Rows with no norm: a wave per (token, 256-value block), four a workgroup.
template <bool Q8K>
__global__ __launch_bounds__(kThreads) void k_pre_quant_blocks(const float* __restrict__ x, int xstride, int cols, int bits, ActPlanar out,
                                                                int ntok) {
    const int nb = cols / 256, g = blockIdx.x * 4 + (threadIdx.x >> 6), t = g / nb, b = g - t * nb;
    if (t >= ntok) return;
    const float4 xv = gld4(x + static_cast<size_t>(t) * xstride + b * 256 + 4 * (threadIdx.x & 63));
    const float v[4] = {xv.x, xv.y, xv.z, xv.w};
    pre_quant_block<Q8K>(v, t, b, bits, out);
}

// rms_norm'd rows (src/model.cpp:87-97): a workgroup per token, wave k taking blocks k, k + 4, ...
// The double sum of squares is grouped as the token path's act_finish groups it (thread 64 k + l
// sums its four values of each of those blocks in order; each wave's sums reduced over the wave,
// then the four added in order), so the scale, and every output, is that path's.  The outputs go
// straight to the planar layout; no width limit (a multiple of 256).
template <bool Q8K>
__global__ __launch_bounds__(kThreads) void k_pre_quant_norm(const float* __restrict__ x, int xstride, const float* __restrict__ w,
                                                              float eps, int cols, int bits, ActPlanar out) {
    __shared__ double red[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, t = blockIdx.x, nb = cols / 256;
    const float* row = x + static_cast<size_t>(t) * xstride;
    constexpr int kHeld = 4;  // blocks a wave keeps in registers between the two passes (rows up to 4096 values)
    float4 held[kHeld];
    double sq = 0.0;
#pragma unroll
    for (int k = 0; k < kHeld; ++k) {
        const int b = wave + 4 * k;
        if (b < nb) {
            held[k] = gld4(row + b * 256 + 4 * lane);
            sq += static_cast<double>(held[k].x * held[k].x); sq += static_cast<double>(held[k].y * held[k].y);
            sq += static_cast<double>(held[k].z * held[k].z); sq += static_cast<double>(held[k].w * held[k].w);
        }
    }
    for (int b = wave + 4 * kHeld; b < nb; b += 4) {
        const float4 v = gld4(row + b * 256 + 4 * lane);
        sq += static_cast<double>(v.x * v.x); sq += static_cast<double>(v.y * v.y);
        sq += static_cast<double>(v.z * v.z); sq += static_cast<double>(v.w * v.w);
    }
    sq = wave_sum(sq);
    if (lane == 0) red[wave] = sq;
    __syncthreads();
    const float scale = rms_scale(((red[0] + red[1]) + red[2]) + red[3], cols, eps);
    for (int k = 0, b = wave; b < nb; ++k, b += 4) {
        const float4 xv = k < kHeld ? held[k < kHeld ? k : 0] : gld4(row + b * 256 + 4 * lane);
        const float4 wv = gld4(w + b * 256 + 4 * lane);
        const float v[4] = {xv.x * scale * wv.x, xv.y * scale * wv.y, xv.z * scale * wv.z, xv.w * scale * wv.w};
        pre_quant_block<Q8K>(v, t, b, bits, out);
    }
}

// GGUF BlockQ8_0 / BlockQ8_K rows (the kernel-level ABI's activation format) into the planar layout.
__global__ void k_pre_planar(const uint8_t* __restrict__ xq, int cols, int q8k, ActPlanar out) {
    const int t = blockIdx.x;
    if (!q8k) {
        const int nb = cols / 32;
        const uint8_t* row = xq + static_cast<size_t>(t) * nb * 34;
        for (int b = threadIdx.x; b < nb; b += blockDim.x) {
            const uint8_t* blk = row + b * 34;
            out.d[static_cast<size_t>(t) * (out.stride / 32) + b] = h2f(static_cast<uint16_t>(blk[0] | (blk[1] << 8)));
            int s = 0;
            for (int i = 0; i < 32; ++i) {
                const int8_t v = static_cast<int8_t>(blk[2 + i]);
                out.qs[static_cast<size_t>(t) * out.stride + b * 32 + i] = v;
                s += v;
            }
            out.bs[static_cast<size_t>(t) * (out.stride / 16) + b] = s;
        }
    } else {
        const int nb = cols / 256;
        const uint8_t* row = xq + static_cast<size_t>(t) * nb * 292;
        for (int b = threadIdx.x; b < nb; b += blockDim.x) {
            const uint8_t* blk = row + b * 292;
            float d;
            __builtin_memcpy(&d, blk, 4);
            out.d[static_cast<size_t>(t) * (out.stride / 32) + b] = d;
            for (int i = 0; i < 256; ++i) out.qs[static_cast<size_t>(t) * out.stride + b * 256 + i] = static_cast<int8_t>(blk[4 + i]);
            for (int g = 0; g < 16; ++g) {
                int16_t v;
                __builtin_memcpy(&v, blk + 260 + 2 * g, 2);
                out.bs[static_cast<size_t>(t) * (out.stride / 16) + b * 16 + g] = v;
            }
        }
    }
}

// ---------------------------------------------------------------- weight fragments

// Eight consecutive weight values (k = kq .. kq + 7 of 32-value sub-block j) of
// one row as signed int8, the A operand of one lane.  Q4_0: nibble - 8;
// Q4_1: nibble 0..15 (the offset m enters through the block sum); Q5_0: 5-bit
// value - 16; Q8_0: as stored; Q4_K: nibble 0..15, Q5_K: 5-bit value 0..31
// (the mins enter through the offsets);
// Q6_K: 6-bit value - 32; TQ2_0: code - 1.  Sign extension is done per byte
// (SWAR): for a field t of n bits, t | ((t & sign) * k) with k filling the
// high bits.
constexpr uint64_t kB01 = 0x0101010101010101ull;

__device__ __forceinline__ uint64_t ld8(const uint8_t* p) { return *reinterpret_cast<const uint64_t*>(p); }

template <uint32_t T>
__device__ __forceinline__ uint64_t frag_a(const Packed& m, uint32_t row, uint32_t j, int kq) {
    if (T == kQ8_0) {
        const uint32_t nsub = m.cols / 32;
        return ld8(m.p0 + (static_cast<size_t>(row) * nsub + j) * 32 + kq);
    } else if (T == kQ4_0) {
        const uint32_t nsub = m.cols / 32;
        const uint64_t w = ld8(m.p0 + (static_cast<size_t>(row) * nsub + j) * 16 + (kq & 15));
        const uint64_t nib = kq < 16 ? (w & (0x0F * kB01)) : ((w >> 4) & (0x0F * kB01));
        const uint64_t t = nib ^ (0x08 * kB01);             // 4-bit two's complement of nib - 8
        return t | ((t & (0x08 * kB01)) * 0x1E);             // sign-extend bit 3
    } else if (T == kQ4_1) {
        const uint32_t nsub = m.cols / 32;
        const uint64_t w = ld8(m.p0 + (static_cast<size_t>(row) * nsub + j) * 16 + (kq & 15));
        return kq < 16 ? (w & (0x0F * kB01)) : ((w >> 4) & (0x0F * kB01));
    } else if (T == kQ5_0) {
        const uint32_t nsub = m.cols / 32;
        const size_t blk = static_cast<size_t>(row) * nsub + j;
        const uint64_t w = ld8(m.p0 + blk * 16 + (kq & 15));
        const uint32_t qh = reinterpret_cast<const uint32_t*>(m.p2)[blk] >> kq;  // bits of values kq .. kq + 7
        const uint64_t hb = static_cast<uint64_t>(spread4_hi(qh, 0)) | (static_cast<uint64_t>(spread4_hi(qh, 4)) << 32);
        const uint64_t u = (kq < 16 ? (w & (0x0F * kB01)) : ((w >> 4) & (0x0F * kB01))) | hb;  // 0..31
        const uint64_t t = u ^ (0x10 * kB01);                                                // 5-bit two's complement of u - 16
        return t | ((t & (0x10 * kB01)) * 0x0E);
    } else if (T == kQ4_K) {
        const uint32_t nsb = m.cols / 256, jj = j & 7;
        const size_t blk = static_cast<size_t>(row) * nsb + j / 8;
        const uint64_t w = ld8(m.p0 + blk * 128 + (jj >> 1) * 32 + kq);
        return (jj & 1) ? ((w >> 4) & (0x0F * kB01)) : (w & (0x0F * kB01));
    } else if (T == kQ5_K) {
        const uint32_t nsb = m.cols / 256, jj = j & 7;
        const size_t blk = static_cast<size_t>(row) * nsb + j / 8;
        const uint64_t w = ld8(m.p0 + blk * 128 + (jj >> 1) * 32 + kq);
        const uint64_t h = ld8(m.p2 + blk * 48 + 16 + kq);
        const uint64_t nib = (jj & 1) ? ((w >> 4) & (0x0F * kB01)) : (w & (0x0F * kB01));
        return nib | (((h >> jj) & kB01) << 4);
    } else if (T == kQ6_K) {
        const uint32_t nsb = m.cols / 256, jj = j & 7, half = jj >> 2, quarter = jj & 3;
        const size_t blk = static_cast<size_t>(row) * nsb + j / 8;
        const uint64_t l = ld8(m.p0 + blk * 128 + half * 64 + (quarter & 1) * 32 + kq);
        const uint64_t h = ld8(m.p1 + blk * 64 + half * 32 + kq);
        const uint64_t nib = quarter >= 2 ? ((l >> 4) & (0x0F * kB01)) : (l & (0x0F * kB01));
        const uint64_t u = nib | (((h >> (2 * quarter)) & (0x03 * kB01)) << 4);  // 0..63
        const uint64_t t = u ^ (0x20 * kB01);                                   // 6-bit two's complement of u - 32
        return t | ((t & (0x20 * kB01)) * 0x06);
    } else {  // TQ2_0
        const uint32_t nsb = m.cols / 256, jj = j & 7;
        const size_t blk = static_cast<size_t>(row) * nsb + j / 8;
        const uint64_t w = ld8(m.p0 + blk * 64 + (jj >> 2) * 32 + kq);
        const uint64_t c = (w >> (2 * (jj & 3))) & (0x03 * kB01);                // 0..2
        const uint64_t t = (c + 0x03 * kB01) & (0x03 * kB01);                   // 2-bit two's complement of c - 1
        return t | ((t & (0x02 * kB01)) * 0x7F);
    }
}

__device__ __forceinline__ v4i mfma(uint64_t a, uint64_t b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(static_cast<long>(a), static_cast<long>(b), c, 0, 0, 0);
}

// ---------------------------------------------------------------- the GEMM

// A workgroup computes 64 rows (4 waves x 16) x 64 tokens (4 groups of 16).
// The K dimension goes in chunks of 256 values (8 sub-blocks; one super-block
// for the K-quants).  Per chunk the workgroup stages the 64 tokens'
// activations (and their scales) in LDS, and each lane holds its weight
// fragments and row scales in registers; both are loaded one chunk ahead, so
// memory latency overlaps the MFMAs and the float epilogue.
constexpr int kRowsPerWg = 64;
constexpr int kChunkCols = kMmChunkCols;
constexpr int kBRow = kChunkCols + 16;  // LDS bytes per token row, padded off the bank period
// Token groups of 16 a workgroup: 4 (64 tokens), or 2 for the K-quants, whose
// integer epilogue holds more state per output.
template <uint32_t T>
__host__ __device__ constexpr int mm_groups() { return (T == kQ4_K || T == kQ5_K || T == kQ6_K) ? 2 : 4; }

template <int G>
struct MmLds {
    alignas(16) int8_t b[16 * G][kBRow];
    float xd[16 * G][8];     // Q8_0: the chunk's 8 block scales; Q8_K: [0] the super-block's
    int32_t bs[16 * G][16];  // Q8_K: the super-block's bsums; Q8_0 (for Q4_1): [0..7] the 8 block sums
};

// One thread's share of a chunk's activations, in flight to LDS.
template <int G>
struct ActStage {
    uint4 q[G];
    float d[2];
    int32_t bs[4];  // Q8_0 with sums: [0..1] as d
};

template <int G>
__device__ __forceinline__ void act_stage_load(ActStage<G>& st, const ActPlanar& x, int ntok, int t0, int c, bool q8k,
                                               bool sums = false) {
    constexpr int kTok = 16 * G;
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < G; ++k) {
        const int idx = k * kThreads + tid, tok = idx >> 4, piece = idx & 15;
        const int t = t0 + tok < ntok ? t0 + tok : ntok - 1;
        st.q[k] = *reinterpret_cast<const uint4*>(x.qs + static_cast<size_t>(t) * x.stride + c * kChunkCols + piece * 16);
    }
    const size_t ds = x.stride / 32, bss = x.stride / 16;
    if (!q8k) {  // kTok tokens x 8 scales
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int idx = k * kThreads + tid, tok = idx >> 3, blk = idx & 7;
            if (tok < kTok) {
                const int t = t0 + tok < ntok ? t0 + tok : ntok - 1;
                st.d[k] = x.d[t * ds + c * 8 + blk];
                if (sums) st.bs[k] = x.bs[t * bss + c * 8 + blk];
            }
        }
    } else {  // kTok tokens x 16 bsums, and kTok scales
        const int tok = tid >> 2;
        if (tok < kTok) {
            const int t = t0 + tok < ntok ? t0 + tok : ntok - 1;
#pragma unroll
            for (int k = 0; k < 4; ++k) st.bs[k] = x.bs[t * bss + c * 16 + (tid & 3) * 4 + k];
        }
        if (tid < kTok) {
            const int t2 = t0 + tid < ntok ? t0 + tid : ntok - 1;
            st.d[0] = x.d[t2 * ds + c];
        }
    }
}

template <int G>
__device__ __forceinline__ void act_stage_store(const ActStage<G>& st, MmLds<G>& L, bool q8k, bool sums = false) {
    constexpr int kTok = 16 * G;
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < G; ++k) {
        const int idx = k * kThreads + tid, tok = idx >> 4, piece = idx & 15;
        *reinterpret_cast<uint4*>(&L.b[tok][piece * 16]) = st.q[k];
    }
    if (!q8k) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int idx = k * kThreads + tid;
            if ((idx >> 3) < kTok) {
                L.xd[idx >> 3][idx & 7] = st.d[k];
                if (sums) L.bs[idx >> 3][idx & 7] = st.bs[k];
            }
        }
    } else {
        if ((tid >> 2) < kTok) {
#pragma unroll
            for (int k = 0; k < 4; ++k) L.bs[tid >> 2][(tid & 3) * 4 + k] = st.bs[k];
        }
        if (tid < kTok) L.xd[tid][0] = st.d[0];
    }
}

// One lane's weights for a chunk: the A fragments of its row (8 sub-blocks) and
// the scales of its 4 output rows.
template <uint32_t T>
struct WChunk {
    uint64_t a[8];
    uint4 sc[4];     // Q4_0/Q4_1/Q5_0/Q8_0: 8 fp16 block scales a row; Q4_K/Q5_K: the decoded scales and mins; TQ2_0: .x = d
    uint32_t s6[4];  // Q6_K: the fp16 d of each row (its int8 scales go in sc); Q4_K/Q5_K: {d, dmin}
    uint4 mn[4];     // Q4_1: 8 fp16 block offsets m a row
};

// The 8 fp16 values of a row's plane at element e0 (a chunk's block scales), or its first nb of
// them (the rest 0) when the row ends inside the chunk: nothing past the row is read.
__device__ __forceinline__ uint4 chunk_halves(const uint8_t* plane, size_t e0, int nb) {
    if (nb >= 8) return *reinterpret_cast<const uint4*>(plane + e0 * 2);
    const uint16_t* h = reinterpret_cast<const uint16_t*>(plane) + e0;
    uint32_t wd[4] = {0u, 0u, 0u, 0u};
    for (int k = 0; k < nb; ++k) wd[k >> 1] |= static_cast<uint32_t>(h[k]) << (16 * (k & 1));
    return make_uint4(wd[0], wd[1], wd[2], wd[3]);
}

// Chunk c's weights; nb of its 8 sub-blocks lie in the row (fewer than 8 only in the last chunk
// of a row of 32-value blocks that is not whole 256-value chunks): the others are not read.
template <uint32_t T>
__device__ __forceinline__ void wchunk_load(WChunk<T>& w, const Packed& m, uint32_t arow, bool arow_ok, const uint32_t orow[4],
                                            int c, int kq, int nb = 8) {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) w.a[jj] = arow_ok && jj < nb ? frag_a<T>(m, arow, c * 8 + jj, kq) : 0ull;
    if (T == kQ4_0 || T == kQ4_1 || T == kQ5_0 || T == kQ8_0) {
        const uint32_t nsub = m.cols / 32;
#pragma unroll
        for (int i = 0; i < 4; ++i) w.sc[i] = chunk_halves(m.p1, static_cast<size_t>(orow[i]) * nsub + c * 8, nb);
        if (T == kQ4_1) {
#pragma unroll
            for (int i = 0; i < 4; ++i) w.mn[i] = chunk_halves(m.p2, static_cast<size_t>(orow[i]) * nsub + c * 8, nb);
        }
    } else if (T == kQ4_K || T == kQ5_K) {
        const uint32_t nsb = m.cols / 256;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const size_t blk = static_cast<size_t>(orow[i]) * nsb + c;
            w.sc[i] = *reinterpret_cast<const uint4*>(m.p2 + blk * (T == kQ5_K ? 48 : 16));
            w.s6[i] = *reinterpret_cast<const uint32_t*>(m.p1 + blk * 16);
        }
    } else if (T == kQ6_K) {
        const uint32_t nsb = m.cols / 256;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t* mp = reinterpret_cast<const uint32_t*>(m.p2 + (static_cast<size_t>(orow[i]) * nsb + c) * 20);
            w.sc[i] = make_uint4(mp[0], mp[1], mp[2], mp[3]);
            w.s6[i] = mp[4];
        }
    } else {
        const uint32_t nsb = m.cols / 256;
        const uint16_t* dw = reinterpret_cast<const uint16_t*>(m.p1);
#pragma unroll
        for (int i = 0; i < 4; ++i) w.sc[i].x = dw[static_cast<size_t>(orow[i]) * nsb + c];
    }
}

__device__ __forceinline__ uint32_t u4_word(const uint4& v, int k) { return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w; }

// Per-lane accumulators: [token group][row i].
template <int G>
struct MmAcc {
    float s[G][4];
};

// The chunk's contribution to the lane's outputs (tokens 16 g + l % 16, rows 4 (l / 16) + i),
// in the reference's term and sum order.
template <uint32_t T, int G>
__device__ __forceinline__ void wchunk_compute(const WChunk<T>& w, const MmLds<G>& L, MmAcc<G>& acc, bool lut16, int nb = 8) {
    constexpr int kGroups = G;
    const int lane = threadIdx.x & 63, kq = (lane >> 4) * 8, tl = lane & 15;
    const v4i zero = {0, 0, 0, 0};
    if (T == kQ4_0 || T == kQ5_0 || T == kQ8_0 || T == kQ4_1) {
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            if (jj >= nb) break;  // past the row (a partial last chunk): no term
            v4i d[kGroups];
#pragma unroll
            for (int g = 0; g < kGroups; ++g)
                d[g] = mfma(w.a[jj], *reinterpret_cast<const uint64_t*>(&L.b[16 * g + tl][jj * 32 + kq]), zero);
            float wd[4], wm[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t word = u4_word(w.sc[i], jj >> 1);
                wd[i] = h2f(static_cast<uint16_t>((jj & 1) ? (word >> 16) : (word & 0xFFFF)));
                if (T == kQ4_1) {
                    const uint32_t mword = u4_word(w.mn[i], jj >> 1);
                    wm[i] = h2f(static_cast<uint16_t>((jj & 1) ? (mword >> 16) : (mword & 0xFFFF)));
                }
            }
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
                const float xd = L.xd[16 * g + tl][jj];
                if (T == kQ4_1) {  // src/quant.cpp:445-456 with the offset term
                    const float xs = xd * static_cast<float>(L.bs[16 * g + tl][jj]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc.s[g][i] += static_cast<float>(d[g][i]) * wd[i] * xd + wm[i] * xs;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc.s[g][i] += static_cast<float>(d[g][i]) * wd[i] * xd;  // src/quant.cpp:445-482
                }
            }
        }
    } else if (T == kQ4_K || T == kQ5_K) {
        int wsum[kGroups][4], osum[kGroups][4];
#pragma unroll
        for (int g = 0; g < kGroups; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) wsum[g][i] = osum[g][i] = 0;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            int sc[4], mn[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sc[i] = static_cast<int>((u4_word(w.sc[i], jj >> 2) >> (8 * (jj & 3))) & 0xFF);
                mn[i] = static_cast<int>((u4_word(w.sc[i], 2 + (jj >> 2)) >> (8 * (jj & 3))) & 0xFF);
            }
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
                const int t = 16 * g + tl;
                const v4i d = mfma(w.a[jj], *reinterpret_cast<const uint64_t*>(&L.b[t][jj * 32 + kq]), zero);
                const int pair = L.bs[t][2 * jj] + L.bs[t][2 * jj + 1];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    wsum[g][i] += sc[i] * d[i];
                    osum[g][i] += mn[i] * pair;
                }
            }
        }
#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            const float xd = L.xd[16 * g + tl][0];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float d = h2f(static_cast<uint16_t>(w.s6[i] & 0xFFFF)), dmin = h2f(static_cast<uint16_t>(w.s6[i] >> 16));
                acc.s[g][i] += xd * (d * static_cast<float>(wsum[g][i]) - dmin * static_cast<float>(osum[g][i]));  // :500-521
            }
        }
    } else if (T == kQ6_K) {
        const bool lo_half = lane < 32;  // lanes 0..31 hold k 0..15 of a sub-block, 32..63 hold k 16..31
        int wsum[kGroups][4];
#pragma unroll
        for (int g = 0; g < kGroups; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) wsum[g][i] = 0;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const uint64_t a0 = lo_half ? w.a[jj] : 0ull, a1 = lo_half ? 0ull : w.a[jj];  // groups 2 jj and 2 jj + 1 of 16
            int s0[4], s1[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t word = u4_word(w.sc[i], jj >> 1);
                const int sh = (jj & 1) * 16;
                s0[i] = static_cast<int8_t>((word >> sh) & 0xFF);
                s1[i] = static_cast<int8_t>((word >> (sh + 8)) & 0xFF);
            }
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
                const uint64_t b = *reinterpret_cast<const uint64_t*>(&L.b[16 * g + tl][jj * 32 + kq]);
                const v4i d0 = mfma(a0, b, zero), d1 = mfma(a1, b, zero);
#pragma unroll
                for (int i = 0; i < 4; ++i) wsum[g][i] += s0[i] * d0[i] + s1[i] * d1[i];
            }
        }
#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            const float xd = L.xd[16 * g + tl][0];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float d = h2f(static_cast<uint16_t>(w.s6[i] & 0xFFFF));
                acc.s[g][i] += xd * d * static_cast<float>(wsum[g][i]);  // src/quant.cpp:549-563
            }
        }
    } else {  // TQ2_0
        v4i d[kGroups];
#pragma unroll
        for (int g = 0; g < kGroups; ++g) d[g] = zero;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)  // the block's int32 sum over its 8 sub-blocks, exact
#pragma unroll
            for (int g = 0; g < kGroups; ++g)
                d[g] = mfma(w.a[jj], *reinterpret_cast<const uint64_t*>(&L.b[16 * g + tl][jj * 32 + kq]), d[g]);
#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            const float xd = L.xd[16 * g + tl][0];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float wv = h2f(static_cast<uint16_t>(w.sc[i].x & 0xFFFF));
                const float a = static_cast<float>(d[g][i]);
                acc.s[g][i] += lut16 ? a * wv * xd : xd * wv * a;  // src/quant.cpp:789-802 / :580-596
            }
        }
    }
}

// out[t * ostride + r] (=, += or gate(out) * up) for a 64-row x 64-token tile.
template <uint32_t T, int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_mm(MmArgs g) {
    constexpr int kGroups = mm_groups<T>(), kTokPerWg = 16 * kGroups;
    __shared__ MmLds<kGroups> L;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, kq = (lane >> 4) * 8;
    const uint32_t r0 = blockIdx.x * kRowsPerWg + wave * 16;
    const int t0 = blockIdx.y * kTokPerWg;
    const bool q8k = takes_q8_k(T);
    const bool lut16 = (g.m.flags & kFlagLut16) != 0;
    // rows of this lane: the A fragment's, and the 4 outputs' (clamped for the scale loads; never stored)
    const uint32_t rmax = g.m.rows - 1;
    const bool wave_ok = r0 <= rmax;
    const uint32_t arow_raw = r0 + (lane & 15);
    const bool arow_ok = arow_raw <= rmax;
    const uint32_t arow = arow_ok ? arow_raw : rmax;
    uint32_t orow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t r = r0 + (lane >> 4) * 4 + i;
        orow[i] = r <= rmax ? r : rmax;
    }
    MmAcc<kGroups> a;
#pragma unroll
    for (int gi = 0; gi < kGroups; ++gi)
#pragma unroll
        for (int i = 0; i < 4; ++i) a.s[gi][i] = 0.0f;
    // chunks of 256 values; a row of 32-value blocks may end inside its last chunk (nb_of < 8
    // blocks there; its activation reads stay inside the planar rows, whose stride is whole chunks)
    const int nc = static_cast<int>((g.m.cols + kChunkCols - 1) / kChunkCols), nsub = static_cast<int>(g.m.cols / 32);
    auto nb_of = [&](int c) { return nsub - 8 * c < 8 ? nsub - 8 * c : 8; };
    ActStage<kGroups> st;
    WChunk<T> w0, w1;  // two chunks in flight
    constexpr bool kSums = T == kQ4_1;
    act_stage_load(st, g.x, g.ntok, t0, 0, q8k, kSums);
    if (wave_ok) {
        wchunk_load<T>(w0, g.m, arow, arow_ok, orow, 0, kq, nb_of(0));
    }
    for (int c = 0; c < nc; c += 2) {
        // chunk c (weights in w0/v0)
        __syncthreads();
        act_stage_store(st, L, q8k, kSums);
        __syncthreads();
        if (c + 1 < nc) {
            act_stage_load(st, g.x, g.ntok, t0, c + 1, q8k, kSums);
            if (wave_ok) {
                wchunk_load<T>(w1, g.m, arow, arow_ok, orow, c + 1, kq, nb_of(c + 1));
            }
        }
        if (wave_ok) {
            wchunk_compute<T>(w0, L, a, lut16, nb_of(c));
        }
        if (c + 1 >= nc) break;
        // chunk c + 1 (weights in w1/v1)
        __syncthreads();
        act_stage_store(st, L, q8k, kSums);
        __syncthreads();
        if (c + 2 < nc) {
            act_stage_load(st, g.x, g.ntok, t0, c + 2, q8k, kSums);
            if (wave_ok) {
                wchunk_load<T>(w0, g.m, arow, arow_ok, orow, c + 2, kq, nb_of(c + 2));
            }
        }
        if (wave_ok) {
            wchunk_compute<T>(w1, L, a, lut16, nb_of(c + 1));
        }
    }
    if (!wave_ok) return;
#pragma unroll
    for (int gi = 0; gi < kGroups; ++gi) {
        const int t = t0 + 16 * gi + (lane & 15);
        if (t >= g.ntok) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = r0 + (lane >> 4) * 4 + i;
            if (r > rmax) continue;
            float* o = g.out + static_cast<size_t>(t) * g.ostride + r;
            const float v = a.s[gi][i];
            if (MODE == kMmStore) {
                *o = v;
            } else if (MODE == kMmAdd) {
                *o = *o + v;  // h += proj (src/model.cpp:1111, :1162)
            } else {  // kMmGated: out holds the gate row, this is up
                const float gv = *o;
                if (g.relu2) {
                    const float q = gv > 0.0f ? gv : 0.0f;
                    *o = q * q * v;  // src/model.cpp:1134-1138
                } else if (g.gelu) {
                    *o = gelu_mul(gv, v);  // src/kernels_f32.cpp:291-296
                } else {
                    *o = gv / (1.0f + ref_expf(-gv)) * v;  // src/kernels_f32.cpp:287-289
                }
            }
        }
    }
}

// ---------------------------------------------------------------- the K-quant GEMM, staged through LDS

// Q4_K / Q6_K (one 256-value super-block a row per chunk).  A workgroup of 4
// waves computes 64 rows x 32 tokens; wave w owns rows 16 w .. + 15 for the
// 32 tokens (2 groups of 16).  Per chunk every operand -- the 64 rows' weight
// planes and the 32 tokens' int8 values, bsums and scales -- is copied global
// -> LDS by global_load_lds (16 bytes a lane, no registers held), and the
// waves read their MFMA fragments from there.  The stage is small (22 KB) and
// the registers few, so several workgroups share a CU and one's copies overlap
// the others' MFMAs.  The arithmetic is wchunk_compute's: exact int32 block
// dots, the reference's float term and sum order.
constexpr int kKqTokMax = 64;
constexpr int kKqCus = 256;  // MI355X compute units (the tile choice aims at a workgroup each)
// tokens a workgroup: 16 G (G token groups share each weight fragment's decode); the
// launcher takes the largest G that still gives a workgroup to every CU

template <uint32_t T>
struct KqStage {
    alignas(16) uint8_t w0[64 * 128];                  // Q4_K nibbles / Q6_K ql: row r piece p at slot r * 8 + (p ^ (r & 7))
    alignas(16) uint8_t wk[T == kQ4_K ? 2048 : 4096];  // Q4_K: p1 [64][16] then p2 [64][16]; Q6_K: qh, row r piece p at r * 4 + (p ^ (r & 3))
    alignas(16) uint32_t wm[T == kQ6_K ? 384 : 1];     // Q6_K: the 20-byte meta of row r at dwords 5 r .. 5 r + 4
    alignas(16) int8_t x[kKqTokMax * 256];             // token t piece p at slot t * 16 + (p ^ (t & 15))
    alignas(16) float xd[64];                          // Q8_K scale of token t (lanes 32..63: a copy)
};

__device__ __forceinline__ void dma16(const void* src, void* lds_wave_base) {
    __builtin_amdgcn_global_load_lds((global_cvoid_ptr)src, (lds_void_ptr)lds_wave_base, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* src, void* lds_wave_base) {
    __builtin_amdgcn_global_load_lds((global_cvoid_ptr)src, (lds_void_ptr)lds_wave_base, 4, 0, 0);
}

// Copies chunk c of rows r0 .. r0 + 63 and tokens t0 .. t0 + 31 into the stage
// (rows and tokens past the ends re-read the last one; their outputs are not stored).
template <uint32_t T, int G>
__device__ __forceinline__ void kq_copy(KqStage<T>& st, const Packed& m, const ActPlanar& x, int ntok, uint32_t r0, int t0, int c) {
    const int tid = threadIdx.x, wave = tid >> 6, wave_first = tid & ~63;
    const uint32_t nsb = m.cols / 256, rmax = m.rows - 1;
    auto rowc = [&](int r) -> size_t {
        const uint32_t rr = r0 + r <= rmax ? r0 + r : rmax;
        return static_cast<size_t>(rr) * nsb + c;
    };
    auto tokc = [&](int t) -> size_t { return static_cast<size_t>(t0 + t < ntok ? t0 + t : ntok - 1); };
#pragma unroll
    for (int k = 0; k < 2; ++k) {  // 64 rows x 8 pieces
        const int slot = k * kThreads + tid, r = slot >> 3, p = (slot & 7) ^ (r & 7);
        dma16(m.p0 + rowc(r) * 128 + p * 16, st.w0 + (k * kThreads + wave_first) * 16);
    }
    if (T == kQ4_K) {  // wave 0: the p1 rows, wave 1: the p2 rows
        if (wave < 2) {
            const int r = tid & 63;
            dma16((wave ? m.p2 : m.p1) + rowc(r) * 16, st.wk + wave_first * 16);
        }
    } else {  // qh: 64 rows x 4 pieces; meta: 320 dwords
        const int r = tid >> 2, p = (tid & 3) ^ (r & 3);
        dma16(m.p1 + rowc(r) * 64 + p * 16, st.wk + wave_first * 16);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int slot = k * kThreads + tid;
            if (slot < 384) {  // waves of slots 320..383 copy row 63's meta again into the spare
                const int sl = slot < 320 ? slot : 319, r2 = sl / 5, j = sl - r2 * 5;
                dma4(m.p2 + rowc(r2) * 20 + j * 4, st.wm + k * kThreads + wave_first);
            }
        }
    }
    const size_t ds = x.stride / 32;
#pragma unroll
    for (int k = 0; k < G; ++k) {  // 16 G tokens x 16 pieces, G a thread
        const int slot = k * kThreads + tid, t = slot >> 4, p = (slot & 15) ^ (t & 15);
        dma16(x.qs + tokc(t) * x.stride + c * 256 + p * 16, st.x + (k * kThreads + wave_first) * 16);
    }
    if (wave == 0) dma4(x.d + tokc(tid & (16 * G - 1)) * ds + c, st.xd);
}

// LDS reads issued as inline assembly.  The compiler waits for every
// outstanding global_load_lds before any LDS read it can see (it cannot tell
// which LDS bytes the copies write), which would drain the next chunk's copies
// before the current chunk is computed.  These reads it does not see; their
// completion is waited for explicitly (lds_wait, which ties the destination
// registers so no use moves above it).
typedef __attribute__((address_space(3))) const void* lds_cvoid_ptr;
__device__ __forceinline__ uint32_t lds_off(const void* p) { return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_cvoid_ptr)p)); }
__device__ __forceinline__ uint64_t ds64(uint32_t a) {
    uint64_t r;
    asm volatile("ds_read_b64 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
__device__ __forceinline__ uint32_t ds32(uint32_t a) {
    uint32_t r;
    asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
typedef unsigned v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4u ds128v(uint32_t a) {
    v4u r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
__device__ __forceinline__ uint4 ds128(uint32_t a) {
    const v4u r = ds128v(a);
    return make_uint4(r.x, r.y, r.z, r.w);
}

// Q4_K with the scales folded into the MFMAs.  For sub-block j of a row,
// weighted = sum_j sc_j dot_j and offsets = sum_j mn_j pair_j (dot_q4_k_q8_k,
// src/quant.cpp:500-521) are exact integers; with sc_j = lo_j + 8 hi_j (3-bit
// digits) and q in 0..15, q lo_j and q hi_j fit int8, so
//   weighted = A_lo + 8 A_hi,  A_lo = sum_k (q_k lo_j(k)) x_k,  A_hi likewise,
//   offsets  = sum_k mn_j(k) x_k   (pair_j is the sum of sub-block j's x),
// three int32 MFMA chains over the super-block, with no per-sub-block integer
// epilogue.  The float term per super-block is the reference's.
// The MFMA is v_mfma_i32_16x16x64_i8 (measured at 2.5 POP/s on register operands,
// against 4.2 for v_mfma_i32_32x32x32_i8: brisk_hip_mfma_rate): lane l
// holds 16 consecutive k of A row l % 16 and of B column l % 16, k = 16 (l / 16)
// .. + 15 of the 64, so lanes 0..31 are sub-block 2 s and lanes 32..63
// sub-block 2 s + 1 of step s, and each lane's digit is its own sub-block's.
__device__ __forceinline__ v4i mfma64(const v4u& a, const v4u& b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, a), __builtin_bit_cast(v4i, b), c, 0, 0, 0);
}

// LDS addresses of a Q4_K stage's parts: the nibble rows, the {d, dmin, scales} and decoded
// scale/min rows (wk, then wk + 1024), the activations and their scales.
struct KqBases {
    uint32_t w0, wk, x, xd;
};
__device__ __forceinline__ KqBases kq_bases(uint32_t base) {
    return KqBases{base + static_cast<uint32_t>(offsetof(KqStage<kQ4_K>, w0)), base + static_cast<uint32_t>(offsetof(KqStage<kQ4_K>, wk)),
                   base + static_cast<uint32_t>(offsetof(KqStage<kQ4_K>, x)), base + static_cast<uint32_t>(offsetof(KqStage<kQ4_K>, xd))};
}

// Fragments read by kq_f64_issue; kq_f64_wait ties each as one 128-bit operand,
// so no copy of a fragment register can be placed before the wait.
struct KqF64 {
    v4u a, b0, b1, b2, b3;  // b0 .. b(G-1) used
};
template <int G>
__device__ __forceinline__ KqF64 kq_f64_issue(const KqBases& b, int s, int ar, int tl, int l16) {
    KqF64 f;
    const int pa = 2 * s + (l16 & 1);  // Q4_K: 32 bytes of nibbles a sub-block pair, low then high
    f.a = ds128v(b.w0 + (ar * 8 + (pa ^ (ar & 7))) * 16);
    const int pb = 4 * s + l16;
    auto bfrag = [&](int g) -> v4u {
        const int t = 16 * g + tl;
        return ds128v(b.x + (t * 16 + (pb ^ (t & 15))) * 16);
    };
    const v4u z = {0u, 0u, 0u, 0u};
    f.b0 = bfrag(0);
    f.b1 = G > 1 ? bfrag(1) : z;
    f.b2 = G > 2 ? bfrag(2) : z;
    f.b3 = G > 3 ? bfrag(3) : z;
    return f;
}
__device__ __forceinline__ void kq_f64_wait(KqF64& f) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f.a), "+v"(f.b0), "+v"(f.b1), "+v"(f.b2), "+v"(f.b3));
}

// Each byte of q (0..15) times d (0..7), as two 16-bit lanes a dword (v_pk_mul_lo_u16, full rate,
// where a 32-bit v_mul_lo_u32 is quarter rate): a byte's product is at most 105, so none carries.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t mul_bytes1(uint32_t q, u16x2 dd) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, q) * dd);
}
__device__ __forceinline__ v4u mul_bytes(const v4u& q, uint32_t d) {
    const u16x2 dd = {static_cast<unsigned short>(d), static_cast<unsigned short>(d)};
    return v4u{mul_bytes1(q.x, dd), mul_bytes1(q.y, dd), mul_bytes1(q.z, dd), mul_bytes1(q.w, dd)};
}

template <int G>
__device__ __forceinline__ void kq_compute_fold(const KqBases& base, MmAcc<G>& acc) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, tl = lane & 15, l16 = lane >> 4;
    const int ar = wave * 16 + tl, orow0 = wave * 16 + l16 * 4;
    const v4i zero = {0, 0, 0, 0};
    // the A row's decoded scales and mins (for the digits), the output rows' d / dmin, the groups' x scales
    v4u scm = ds128v(base.wk + 1024 + ar * 16);
    uint32_t dd[4], xd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        dd[i] = ds32(base.wk + (orow0 + i) * 16);
        xd[i] = i < G ? ds32(base.xd + (16 * i + tl) * 4) : 0u;
    }
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(scm), "+v"(dd[0]), "+v"(dd[1]), "+v"(dd[2]), "+v"(dd[3]), "+v"(xd[0]), "+v"(xd[1]), "+v"(xd[2]),
                   "+v"(xd[3]));
    KqF64 cur = kq_f64_issue<G>(base, 0, ar, tl, l16);
    kq_f64_wait(cur);
    v4i alo[4], ahi[4], amn[4];
#pragma unroll
    for (int g = 0; g < G; ++g) alo[g] = ahi[g] = amn[g] = zero;
    // lanes 32..63 take the odd sub-block of the pair (high nibbles): a shift by 4, not a select
    const uint32_t nib_shift = l16 >= 2 ? 4u : 0u;
    const uint32_t lane_byte = static_cast<uint32_t>(l16 >> 1) * 0x01010101u;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        KqF64 nxt;
        if (st < 3) nxt = kq_f64_issue<G>(base, st + 1, ar, tl, l16);
        const int j = 2 * st + (l16 >> 1);  // this lane's sub-block (j < 4 exactly when st < 2)
        const uint32_t sc = ((st < 2 ? scm.x : scm.y) >> (8 * (j & 3))) & 0xFF;
        // the min byte of sub-block j in all four bytes (v_perm_b32: byte j & 3 of the word, four times)
        const uint32_t m4 = __builtin_amdgcn_perm(0u, st < 2 ? scm.z : scm.w, lane_byte + static_cast<uint32_t>((2 * st) & 3) * 0x01010101u);
        const uint32_t dlo = sc & 7, dhi = sc >> 3;
        const v4u qn = (cur.a >> nib_shift) & 0x0F0F0F0Fu;
        const v4u qlo = mul_bytes(qn, dlo);  // bytes 0..15 times 0..7: no carries between bytes
        const v4u qhi = mul_bytes(qn, dhi);
        const v4u qmn = {m4, m4, m4, m4};
        const v4u bq[4] = {cur.b0, cur.b1, cur.b2, cur.b3};
#pragma unroll
        for (int g = 0; g < G; ++g) {
            alo[g] = mfma64(qlo, bq[g], alo[g]);
            ahi[g] = mfma64(qhi, bq[g], ahi[g]);
            amn[g] = mfma64(qmn, bq[g], amn[g]);
        }
        if (st < 3) {
            kq_f64_wait(nxt);
            cur = nxt;
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float xg = __uint_as_float(xd[g]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int weighted = alo[g][i] + 8 * ahi[g][i], offsets = amn[g][i];
            const float d = h2f(static_cast<uint16_t>(dd[i] & 0xFFFF)), dmin = h2f(static_cast<uint16_t>(dd[i] >> 16));
            acc.s[g][i] += xg * (d * static_cast<float>(weighted) - dmin * static_cast<float>(offsets));  // src/quant.cpp:500-521
        }
    }
}

// Q6_K with its signed 8-bit scales folded into the MFMAs.  Per 16-value
// group g of a super-block, weighted = sum_g sc_g dot_g with dot_g = sum (q - 32) x
// (dot_q6_k_q8_k, src/quant.cpp:549-563).  With sc_g + 128 = sum_i 4^i d_i,g
// (base-4 digits, 0..3), sc_g = d_0 + 4 d_1 + 16 d_2 + 64 (d_3 - 2), and with
// s = q - 32 in -32..31 every s d_i and s (d_3 - 2) fits int8, so
//   weighted = A_0 + 4 A_1 + 16 A_2 + 64 A_3,  A_i = sum_k (s_k m_i,g(k)) x_k,
// four exact int32 MFMA chains over the super-block.  Lane l of step st
// (64 values) holds group 4 st + l / 16, so its multipliers are its own group's.
// Bytes are signed: 2 s per byte is a masked shift, 3 s a carry-free byte add,
// -s and -2 s carry-free byte subtractions from zero.
__device__ __forceinline__ void kq_s23(unsigned w, unsigned& s2, unsigned& s3) {
    s2 = (w << 1) & 0xFEFEFEFEu;
    s3 = ((s2 & 0x7F7F7F7Fu) + (w & 0x7F7F7F7Fu)) ^ ((s2 ^ w) & 0x80808080u);
}
__device__ __forceinline__ unsigned kq_neg(unsigned x) { return (0x80808080u - (x & 0x7F7F7F7Fu)) ^ (~x & 0x80808080u); }

struct Kq6F {
    v4u l, h, b0, b1, b2, b3;  // b0 .. b(G-1) used
};
template <int G>
__device__ __forceinline__ Kq6F kq6_issue(uint32_t base, int st, int ar, int tl, int l16) {
    Kq6F f;
    const int half = st >> 1;
    const int lp = half * 4 + l16, hp = half * 2 + (l16 & 1);
    f.l = ds128v(base + offsetof(KqStage<kQ6_K>, w0) + (ar * 8 + (lp ^ (ar & 7))) * 16);
    f.h = ds128v(base + offsetof(KqStage<kQ6_K>, wk) + (ar * 4 + (hp ^ (ar & 3))) * 16);
    const int pb = 4 * st + l16;
    auto bfrag = [&](int g) -> v4u {
        const int t = 16 * g + tl;
        return ds128v(base + offsetof(KqStage<kQ6_K>, x) + (t * 16 + (pb ^ (t & 15))) * 16);
    };
    const v4u z = {0u, 0u, 0u, 0u};
    f.b0 = bfrag(0);
    f.b1 = G > 1 ? bfrag(1) : z;
    f.b2 = G > 2 ? bfrag(2) : z;
    f.b3 = G > 3 ? bfrag(3) : z;
    return f;
}
__device__ __forceinline__ void kq6_wait(Kq6F& f) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f.l), "+v"(f.h), "+v"(f.b0), "+v"(f.b1), "+v"(f.b2), "+v"(f.b3));
}

template <int G>
__device__ __forceinline__ void kq_compute_fold6(uint32_t base, MmAcc<G>& acc) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, tl = lane & 15, l16 = lane >> 4;
    const int ar = wave * 16 + tl, orow0 = wave * 16 + l16 * 4;
    const v4i zero = {0, 0, 0, 0};
    // the A row's 16 int8 scales (four dwords of its meta), the output rows' d, the groups' x scales
    const uint32_t arow = base + offsetof(KqStage<kQ6_K>, wm) + ar * 20;
    uint32_t s0 = ds32(arow), s1 = ds32(arow + 4), s2 = ds32(arow + 8), s3 = ds32(arow + 12);
    uint32_t dd[4], xd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        dd[i] = ds32(base + offsetof(KqStage<kQ6_K>, wm) + (orow0 + i) * 20 + 16);
        xd[i] = i < G ? ds32(base + offsetof(KqStage<kQ6_K>, xd) + (16 * i + tl) * 4) : 0u;
    }
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(s0), "+v"(s1), "+v"(s2), "+v"(s3), "+v"(dd[0]), "+v"(dd[1]), "+v"(dd[2]), "+v"(dd[3]), "+v"(xd[0]),
                   "+v"(xd[1]), "+v"(xd[2]), "+v"(xd[3]));
    const uint32_t scw[4] = {s0, s1, s2, s3};
    Kq6F cur = kq6_issue<G>(base, 0, ar, tl, l16);
    kq6_wait(cur);
    v4i a0[4], a1[4], a2[4], a3[4];
#pragma unroll
    for (int g = 0; g < G; ++g) a0[g] = a1[g] = a2[g] = a3[g] = zero;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        Kq6F nxt;
        if (st < 3) nxt = kq6_issue<G>(base, st + 1, ar, tl, l16);
        // the lane's 16 values: nibbles of ql (high for odd steps), 2 bits of qh, minus 32
        const int quarter = 2 * (st & 1) + (l16 >> 1);
        const v4u nib = (st & 1) ? ((cur.l >> 4) & 0x0F0F0F0Fu) : (cur.l & 0x0F0F0F0Fu);
        const v4u u = nib | (((cur.h >> (2 * quarter)) & 0x03030303u) << 4);  // 0..63
        const v4u tq = u ^ 0x20202020u;                                         // 6-bit two's complement of u - 32
        const v4u sv = tq | ((tq & 0x20202020u) * 0x06u);
        const int gi = 4 * st + l16;                                            // this lane's group
        const uint32_t scu = ((scw[gi >> 2] >> (8 * (gi & 3))) & 0xFF) ^ 0x80u;  // sc + 128 for int8 sc
        v4u w2, w3;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            unsigned p2, p3;
            kq_s23(sv[k], p2, p3);
            w2[k] = p2;
            w3[k] = p3;
        }
        v4u dg[4];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const uint32_t d = (scu >> (2 * i)) & 3;
            dg[i] = (d & 2) ? ((d & 1) ? w3 : w2) : ((d & 1) ? sv : v4u{0u, 0u, 0u, 0u});
        }
        {  // the top digit less 2: -2, -1, 0 or 1 times s
            const uint32_t d = scu >> 6;
            v4u neg;
#pragma unroll
            for (int k = 0; k < 4; ++k) neg[k] = kq_neg((d & 1) ? sv[k] : w2[k]);
            dg[3] = (d & 2) ? ((d & 1) ? sv : v4u{0u, 0u, 0u, 0u}) : neg;
        }
        const v4u bq[4] = {cur.b0, cur.b1, cur.b2, cur.b3};
#pragma unroll
        for (int g = 0; g < G; ++g) {
            a0[g] = mfma64(dg[0], bq[g], a0[g]);
            a1[g] = mfma64(dg[1], bq[g], a1[g]);
            a2[g] = mfma64(dg[2], bq[g], a2[g]);
            a3[g] = mfma64(dg[3], bq[g], a3[g]);
        }
        if (st < 3) {
            kq6_wait(nxt);
            cur = nxt;
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float xg = __uint_as_float(xd[g]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int weighted = a0[g][i] + 4 * a1[g][i] + 16 * a2[g][i] + 64 * a3[g][i];
            const float d = h2f(static_cast<uint16_t>(dd[i] & 0xFFFF));
            acc.s[g][i] += xg * d * static_cast<float>(weighted);  // src/quant.cpp:549-563
        }
    }
}

// ---------------------------------------------------------------- Q6_K, expanded

// Q6_K matrices the batched prefill multiplies are also held expanded (once, at
// the first prefill): per 16-value group g of a super-block the exact integer
// weight w = sc_g (q - 32) (|w| <= 4096) is split as w = lo + 128 hi with lo in
// -64..63 and hi in -32..32, both int8.  Then dot_q6_k_q8_k's weighted sum
// (src/quant.cpp:549-563) is A_lo + 128 A_hi, A = sum_k w_k x_k, two int32 MFMA
// chains over the super-block with no decoding in the GEMM.
//
// The planes are in the fragment order of v_mfma_i32_32x32x32_i8: for 32-row
// group rg, super-block c, 32-value step s and plane p (lo, hi), 64 lanes x 16
// bytes, lane l holding row 32 rg + l % 32, values 32 s + 16 (l / 32) .. + 15
// of the super-block.  A wave's operand for one step is one coalesced 1 KB load.
// The scales follow as floats: d[(rg * nsb + c) * 32 + r % 32] = h2f(d of row r).
// Rows are padded to a multiple of kMxRows with zero weights.
__global__ void k_q6x_expand(Packed m, int8_t* __restrict__ q, float* __restrict__ dq, uint32_t row_groups) {
    const size_t gid = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint32_t nsb = m.cols / 256;
    const int lane = static_cast<int>(gid & 63), s = static_cast<int>((gid >> 6) & 7);
    const size_t rest = gid >> 9;
    const uint32_t c = static_cast<uint32_t>(rest % nsb), rg = static_cast<uint32_t>(rest / nsb);
    if (rg >= row_groups) return;
    const uint32_t row = rg * 32 + (lane & 31);
    const int kin = s * 32 + (lane >> 5) * 16;  // first value of the lane's group within the super-block
    uint32_t lo[4] = {0, 0, 0, 0}, hi[4] = {0, 0, 0, 0};
    float d = 0.0f;
    if (row < m.rows) {
        const size_t blk = static_cast<size_t>(row) * nsb + c;
        const uint8_t* ql = m.p0 + blk * 128;
        const uint8_t* qh = m.p1 + blk * 64;
        const uint8_t* meta = m.p2 + blk * 20;
        const int sc = static_cast<int8_t>(meta[kin / 16]);
        d = h2f(static_cast<uint16_t>(meta[16] | (meta[17] << 8)));
        for (int b = 0; b < 16; ++b) {  // block_q6_K element order (dequantize_row_q6_K)
            const int k = kin + b, n = k >> 7, j = k & 127, which = j >> 5, l = j & 31;
            const int qlb = ql[n * 64 + l + (which & 1) * 32];
            const int nib = which >= 2 ? qlb >> 4 : qlb & 15;
            const int u = nib | (((qh[n * 32 + l] >> (2 * which)) & 3) << 4);
            const int w = sc * (u - 32);
            const int wl = ((w + 64) & 127) - 64, wh = (w - wl) >> 7;
            lo[b >> 2] |= static_cast<uint32_t>(wl & 0xFF) << (8 * (b & 3));
            hi[b >> 2] |= static_cast<uint32_t>(wh & 0xFF) << (8 * (b & 3));
        }
    }
    uint8_t* o = reinterpret_cast<uint8_t*>(q) + ((((static_cast<size_t>(rg) * nsb + c) * 8 + s) * 2) * 64 + lane) * 16;
    *reinterpret_cast<uint4*>(o) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    *reinterpret_cast<uint4*>(o + 1024) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    if (s == 0 && lane < 32) dq[(static_cast<size_t>(rg) * nsb + c) * 32 + lane] = d;
}

// Q4_K and Q5_K expanded the same way: per 32-value sub-block j the exact integer weight
// w = sc_j q (q in 0..15 or 0..31, sc_j 6-bit: w <= 1953) is split as w = lo + 128 hi (lo 0..127,
// hi 0..15), and dot_q4_k_q8_k / dot_q5_k_q8_k's (src/quant.cpp:500-547)
//   weighted = A_lo + 128 A_hi,  offsets = sum_j mn_j pair_j = sum_k mn_j(k) x_k,
// the offsets a third chain against the sub-block's min byte repeated over the step (a step is
// one sub-block).  Per (rg, c) the scales are 64 floats (the 32 rows' d, then their dmin) and the
// mins 32 rows x 8 bytes.
__global__ void k_kmx_expand(Packed m, int8_t* __restrict__ q, float* __restrict__ dq, uint8_t* __restrict__ mq,
                             uint32_t row_groups) {
    const size_t gid = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint32_t nsb = m.cols / 256;
    const int lane = static_cast<int>(gid & 63), s = static_cast<int>((gid >> 6) & 7);
    const size_t rest = gid >> 9;
    const uint32_t c = static_cast<uint32_t>(rest % nsb), rg = static_cast<uint32_t>(rest / nsb);
    if (rg >= row_groups) return;
    const uint32_t row = rg * 32 + (lane & 31);
    const int h = lane >> 5;  // values 16 h .. 16 h + 15 of sub-block s
    const bool q5 = m.type == kQ5_K;
    uint32_t lo[4] = {0, 0, 0, 0}, hi[4] = {0, 0, 0, 0};
    float d = 0.0f, dmin = 0.0f;
    int mn = 0;
    if (row < m.rows) {
        const size_t blk = static_cast<size_t>(row) * nsb + c;
        const uint8_t* qs = m.p0 + blk * 128 + (s >> 1) * 32;
        const uint8_t* meta = m.p1 + blk * 16;
        const uint8_t* dec = m.p2 + blk * (q5 ? 48 : 16);  // decoded scales, mins (then Q5_K's qh)
        const int sc = dec[s];
        mn = dec[8 + s];
        d = h2f(static_cast<uint16_t>(meta[0] | (meta[1] << 8)));
        dmin = h2f(static_cast<uint16_t>(meta[2] | (meta[3] << 8)));
        for (int b = 0; b < 16; ++b) {
            const int i = 16 * h + b;
            int v = (s & 1) ? qs[i] >> 4 : qs[i] & 15;
            if (q5 && (dec[16 + i] >> s) & 1) v |= 16;
            const int w = sc * v, wl = w & 127, wh = w >> 7;
            lo[b >> 2] |= static_cast<uint32_t>(wl) << (8 * (b & 3));
            hi[b >> 2] |= static_cast<uint32_t>(wh) << (8 * (b & 3));
        }
    }
    const size_t rc = static_cast<size_t>(rg) * nsb + c;
    uint8_t* o = reinterpret_cast<uint8_t*>(q) + (((rc * 8 + s) * 2) * 64 + lane) * 16;
    *reinterpret_cast<uint4*>(o) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    *reinterpret_cast<uint4*>(o + 1024) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    if (lane < 32) {
        mq[(rc * 32 + lane) * 8 + s] = static_cast<uint8_t>(mn);
        if (s == 0) {
            dq[rc * 64 + lane] = d;
            dq[rc * 64 + 32 + lane] = dmin;
        }
    }
}

typedef int v16i __attribute__((ext_vector_type(16)));
__device__ __forceinline__ v16i mfma32(const v4u& a, const v4u& b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i, a), __builtin_bit_cast(v4i, b), c, 0, 0, 0);
}

// 32 G tokens' activations of one super-block (token t piece p at slot t * 16 + (p ^ (t & 15))) and their scales.
template <int G>
struct MxStage {
    alignas(16) int8_t x[32 * G * 256];
    alignas(16) float xd[64];  // G = 1: lanes 32..63 hold a copy
};

template <int G, int W>
__device__ __forceinline__ void mx_copy(MxStage<G>& st, const ActPlanar& x, int ntok, int t0, int c) {
    const int tid = threadIdx.x, wave = tid >> 6, wave_first = tid & ~63;
    auto tokc = [&](int t) -> size_t { return static_cast<size_t>(t0 + t < ntok ? t0 + t : ntok - 1); };
#pragma unroll
    for (int k = 0; k < 8 * G / W; ++k) {  // 32 G tokens x 16 pieces, over W waves
        const int slot = k * 64 * W + tid, t = slot >> 4, p = (slot & 15) ^ (t & 15);
        dma16(x.qs + tokc(t) * x.stride + c * 256 + p * 16, st.x + (k * 64 * W + wave_first) * 16);
    }
    if (wave == 0) dma4(x.d + tokc(tid & (32 * G - 1)) * (x.stride / 32) + c, st.xd);
}

// A wave's operands for one super-block: 8 steps x (lo, hi) fragments, the 16 output rows'
// scales and, for Q4_K / Q5_K (KM), their dmins and the A row's 8 sub-block mins.
template <bool KM>
struct MxA {
    v4u f[16];
    float4 d[4];
    float4 dm[KM ? 4 : 1];
    uint32_t mn[KM ? 2 : 1];
};
template <bool KM>
__device__ __forceinline__ void mx_load(MxA<KM>& a, const int8_t* qw, const float* dw, const uint8_t* mw, int lane) {
    const auto* p = gmem(reinterpret_cast<const v4u*>(qw) + lane);
#pragma unroll
    for (int i = 0; i < 16; ++i) a.f[i] = p[i * 64];
    const float* pd = dw + (lane >> 5) * 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) a.d[q] = gld4(pd + q * 8);
    if constexpr (KM) {
#pragma unroll
        for (int q = 0; q < 4; ++q) a.dm[q] = gld4(pd + 32 + q * 8);
        const uint32_t* pm = reinterpret_cast<const uint32_t*>(mw + (lane & 31) * 8);
        a.mn[0] = gld<uint32_t>(pm, 0);
        a.mn[1] = gld<uint32_t>(pm, 1);
    }
}
__device__ __forceinline__ float f4_at(const float4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// acc[gb] (lane: token 32 gb + l % 32, rows 8 (i / 4) + 4 (l / 32) + i % 4) += this super-block's
// terms, in the reference's term order: Q6_K d_x d_w weighted (dot_q6_k_q8_k, src/quant.cpp:549-563);
// Q4_K / Q5_K d_x (d weighted - dmin offsets) (dot_q4_k_q8_k / dot_q5_k_q8_k, :500-547).
template <int G, bool KM>
__device__ __forceinline__ void mx_compute(uint32_t base, const MxA<KM>& a, float (&acc)[G][16]) {
    const int lane = threadIdx.x & 63, h = lane >> 5;
#pragma unroll
    for (int gb = 0; gb < G; ++gb) {
        const int t = 32 * gb + (lane & 31);
        v4u b[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int p = 2 * s + h;
            b[s] = ds128v(base + offsetof(MxStage<G>, x) + (t * 16 + (p ^ (t & 15))) * 16);
        }
        uint32_t xd = ds32(base + offsetof(MxStage<G>, xd) + (G == 1 ? lane : t) * 4);
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]), "+v"(b[4]), "+v"(b[5]), "+v"(b[6]), "+v"(b[7]), "+v"(xd));
        v16i lo = {}, hi = {}, mo = {};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            lo = mfma32(a.f[2 * s], b[s], lo);
            hi = mfma32(a.f[2 * s + 1], b[s], hi);
            if constexpr (KM) {
                const uint32_t m4 = __builtin_amdgcn_perm(0u, a.mn[s >> 2], static_cast<uint32_t>(s & 3) * 0x01010101u);  // byte s & 3, four times
                mo = mfma32(v4u{m4, m4, m4, m4}, b[s], mo);
            }
        }
        const float xg = __uint_as_float(xd);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int weighted = lo[i] + 128 * hi[i];
            const float d = f4_at(a.d[i >> 2], i & 3);
            if constexpr (KM) {
                const float dmin = f4_at(a.dm[i >> 2], i & 3);
                acc[gb][i] += xg * (d * static_cast<float>(weighted) - dmin * static_cast<float>(mo[i]));
            } else {
                acc[gb][i] += xg * d * static_cast<float>(weighted);
            }
        }
    }
}

// The expanded-Q6_K GEMM: a workgroup of W waves computes 32 W rows (32 a wave) x 32 G tokens.  The
// activations are staged in LDS (two stages, global_load_lds); each wave's weight
// fragments are its own and come straight from global memory a super-block ahead.
// Workgroup b runs on XCD b % 8; when the row tiles divide by 8, each XCD takes whole
// row tiles (every token tile of them), so a row tile's weights are read through one L2.
// s_waitcnt vmcnt(n), the other counters not waited: every vector memory load but the last n has landed.
constexpr int mx_wait_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kMxLoads = 20;    // global loads of one mx_load (16 fragments, 4 scale rows)
constexpr int kMxLoadsKm = 26;  // ... with 4 dmin rows and 2 min words
#ifndef BRISK_MX_BUFS
#define BRISK_MX_BUFS 3
#endif
constexpr int kMxBufs = BRISK_MX_BUFS;  // fragment buffers in flight (unified VGPR/AGPR file: one wave a SIMD)

template <int MODE, int G, int W, bool KM>
__global__ __launch_bounds__(64 * W) void k_mmx(MmArgs g) {
    __shared__ MxStage<G> st[2];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nsb = static_cast<int>(g.m.cols / 256);
    const int rtiles = static_cast<int>((g.m.rows + 32 * W - 1) / (32 * W)), ttiles = (g.ntok + 32 * G - 1) / (32 * G);
    const int b = blockIdx.x;
    int rt, tt;
    if (rtiles % 8 == 0) {
        const int j = b >> 3;
        rt = (b & 7) + 8 * (j / ttiles);
        tt = j % ttiles;
    } else {
        rt = b % rtiles;
        tt = b / rtiles;
    }
    const int t0 = tt * 32 * G;
    const size_t rg = static_cast<size_t>(rt) * W + wave;
    constexpr int DW = KM ? 64 : 32;  // scale floats per (row group, super-block)
    const int8_t* qw = g.qx + rg * nsb * 16384;
    const float* dw = g.qxd + rg * nsb * DW;
    const uint8_t* mw = KM ? g.qxm + rg * nsb * 256 : nullptr;
    float acc[G][16];
#pragma unroll
    for (int gb = 0; gb < G; ++gb)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[gb][i] = 0.0f;
    if (MODE == kMmGated) exp_tab_fill();  // ordered before the epilogue by the loop's barriers
    // kMxBufs fragment buffers: a super-block's fragments are loaded kMxBufs - 1 super-blocks
    // ahead, its activations one ahead.  Each step issues stage (c + 1)'s copies, then the loads
    // of super-block c + kMxBufs - 1, computes c, and waits for everything but the loads still
    // ahead of c + 1 (so c + 1 has landed).  A bare barrier: __syncthreads' fence would wait for
    // all of them.
    MxA<KM> a[kMxBufs];
    auto load = [&](MxA<KM>& dst, int n) { mx_load<KM>(dst, qw + static_cast<size_t>(n) * 16384, dw + n * DW, KM ? mw + n * 256 : nullptr, lane); };
    mx_copy<G, W>(st[0], g.x, g.ntok, t0, 0);
#pragma unroll
    for (int k = 0; k < kMxBufs - 1; ++k) load(a[k], min(k, nsb - 1));  // past the end: the last super-block again,
                                                                          // so the load count stays exact
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int c0 = 0; c0 < nsb; c0 += kMxBufs) {
#pragma unroll
        for (int k = 0; k < kMxBufs; ++k) {
            const int c = c0 + k;
            if (c >= nsb) break;
            if (c + 1 < nsb) mx_copy<G, W>(st[(c + 1) & 1], g.x, g.ntok, t0, c + 1);
            load(a[(k + kMxBufs - 1) % kMxBufs], min(c + kMxBufs - 1, nsb - 1));
            mx_compute<G, KM>(lds_off(&st[c & 1]), a[k], acc);
            __builtin_amdgcn_s_waitcnt(mx_wait_imm((KM ? kMxLoadsKm : kMxLoads) * (kMxBufs - 2)));
            __builtin_amdgcn_s_barrier();
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    const uint32_t rmax = g.m.rows - 1;
#pragma unroll
    for (int gb = 0; gb < G; ++gb) {
        const int t = t0 + 32 * gb + (lane & 31);
        if (t >= g.ntok) continue;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t r = static_cast<uint32_t>(rt) * (32 * W) + wave * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
            if (r > rmax) continue;
            float* o = g.out + static_cast<size_t>(t) * g.ostride + r;
            const float v = acc[gb][i];
            if (MODE == kMmStore) {
                *o = v;
            } else if (MODE == kMmAdd) {
                *o = *o + v;  // h += proj (src/model.cpp:1111, :1162)
            } else {  // kMmGated: out holds the gate row, this is up
                const float gv = *o;
                if (g.relu2) {
                    const float q = gv > 0.0f ? gv : 0.0f;
                    *o = q * q * v;  // src/model.cpp:1134-1138
                } else if (g.gelu) {
                    *o = gelu_mul(gv, v);  // src/kernels_f32.cpp:291-296
                } else {
                    *o = gv / (1.0f + ref_expf_s(-gv)) * v;  // src/kernels_f32.cpp:287-289
                }
            }
        }
    }
}

// TWO: one launch for two store GEMMs of one activation (the same format and width; Q and K):
// row tiles 0 .. of ga's rows, then gb's, each workgroup writing its own matrix's output.
template <uint32_t T, int MODE, int G, bool TWO = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 8))) void k_mmk(MmArgs ga, MmArgs gb) {
    __shared__ KqStage<T> st[2];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t rta = (ga.m.rows + 63) / 64;
    const bool second = TWO && blockIdx.x >= rta;
    MmArgs g = ga;
    if (second) {
        g.m = gb.m;
        g.out = gb.out;
        g.ostride = gb.ostride;
    }
    const uint32_t rt0 = (second ? blockIdx.x - rta : blockIdx.x) * 64;
    const int t0 = blockIdx.y * (16 * G);
    const int nc = static_cast<int>(g.m.cols / 256);
    MmAcc<G> a;
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
#pragma unroll
        for (int i = 0; i < 4; ++i) a.s[gi][i] = 0.0f;
    if (MODE == kMmGated) exp_tab_fill();  // ordered before the epilogue by the loop's barriers
    // two stages: chunk c + 1 is copied while chunk c is computed
    kq_copy<T, G>(st[0], g.m, g.x, g.ntok, rt0, t0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int c = 0; c < nc; ++c) {
        if (c + 1 < nc) kq_copy<T, G>(st[(c + 1) & 1], g.m, g.x, g.ntok, rt0, t0, c + 1);
        if constexpr (T == kQ4_K) kq_compute_fold<G>(kq_bases(lds_off(&st[c & 1])), a);
        else kq_compute_fold6<G>(lds_off(&st[c & 1]), a);
        __builtin_amdgcn_s_waitcnt(0);  // chunk c + 1 has landed (this wave's copies) ...
        __syncthreads();                // ... everyone's, and stage c & 1 is consumed
    }
    const uint32_t rmax = g.m.rows - 1;
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        const int t = t0 + 16 * gi + (lane & 15);
        if (t >= g.ntok) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = rt0 + wave * 16 + (lane >> 4) * 4 + i;
            if (r > rmax) continue;
            float* o = g.out + static_cast<size_t>(t) * g.ostride + r;
            const float v = a.s[gi][i];
            if (MODE == kMmStore) {
                *o = v;
            } else if (MODE == kMmAdd) {
                *o = *o + v;  // h += proj (src/model.cpp:1111, :1162)
            } else {  // kMmGated: out holds the gate row, this is up
                const float gv = *o;
                if (g.relu2) {
                    const float q = gv > 0.0f ? gv : 0.0f;
                    *o = q * q * v;  // src/model.cpp:1134-1138
                } else if (g.gelu) {
                    *o = gelu_mul(gv, v);  // src/kernels_f32.cpp:291-296
                } else {
                    *o = gv / (1.0f + ref_expf_s(-gv)) * v;  // src/kernels_f32.cpp:287-289
                }
            }
        }
    }
}

// ---------------------------------------------------------------- Q4_K gate and up, fused

// The gate and up projections of one row tile in one workgroup: both matrices' chunks are
// staged beside one copy of the activations, and the epilogue applies the gate to the up
// sums in registers (the pair's two launches stored the gate rows and read them back).
// Each sum is the one k_mmk computes, in its term order, so the outputs are the same bits.
struct KqPairStage {
    alignas(16) uint8_t w0[64 * 128];  // gate: as KqStage<kQ4_K>
    alignas(16) uint8_t wk[2048];
    alignas(16) uint8_t u0[64 * 128];  // up
    alignas(16) uint8_t uk[2048];
    alignas(16) int8_t x[kKqTokMax * 256];
    alignas(16) float xd[64];
};

__device__ __forceinline__ void kq_copy_w4k(uint8_t* w0, uint8_t* wk, const Packed& m, uint32_t r0, int c) {
    const int tid = threadIdx.x, wave = tid >> 6, wave_first = tid & ~63;
    const uint32_t nsb = m.cols / 256, rmax = m.rows - 1;
    auto rowc = [&](int r) -> size_t {
        const uint32_t rr = r0 + r <= rmax ? r0 + r : rmax;
        return static_cast<size_t>(rr) * nsb + c;
    };
#pragma unroll
    for (int k = 0; k < 2; ++k) {  // 64 rows x 8 pieces
        const int slot = k * kThreads + tid, r = slot >> 3, p = (slot & 7) ^ (r & 7);
        dma16(m.p0 + rowc(r) * 128 + p * 16, w0 + (k * kThreads + wave_first) * 16);
    }
    if (wave < 2) {  // wave 0: the p1 rows, wave 1: the p2 rows
        const int r = tid & 63;
        dma16((wave ? m.p2 : m.p1) + rowc(r) * 16, wk + wave_first * 16);
    }
}

template <int G>
__device__ __forceinline__ void kq_copy_x(int8_t* xs, float* xd, const ActPlanar& x, int ntok, int t0, int c) {
    const int tid = threadIdx.x, wave = tid >> 6, wave_first = tid & ~63;
    auto tokc = [&](int t) -> size_t { return static_cast<size_t>(t0 + t < ntok ? t0 + t : ntok - 1); };
    const size_t ds = x.stride / 32;
#pragma unroll
    for (int k = 0; k < G; ++k) {  // 16 G tokens x 16 pieces, G a thread
        const int slot = k * kThreads + tid, t = slot >> 4, p = (slot & 15) ^ (t & 15);
        dma16(x.qs + tokc(t) * x.stride + c * 256 + p * 16, xs + (k * kThreads + wave_first) * 16);
    }
    if (wave == 0) dma4(x.d + tokc(tid & (16 * G - 1)) * ds + c, xd);
}

template <int G>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 8))) void k_mmk_pair(MmArgs g) {
    __shared__ KqPairStage st[2];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t rt0 = blockIdx.x * 64;
    const int t0 = blockIdx.y * (16 * G);
    const int nc = static_cast<int>(g.m.cols / 256);
    MmAcc<G> ag, au;
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
#pragma unroll
        for (int i = 0; i < 4; ++i) ag.s[gi][i] = au.s[gi][i] = 0.0f;
    exp_tab_fill();  // ordered before the epilogue by the loop's barriers
    auto copy = [&](KqPairStage& d, int c) {
        kq_copy_w4k(d.w0, d.wk, g.m, rt0, c);
        kq_copy_w4k(d.u0, d.uk, g.m2, rt0, c);
        kq_copy_x<G>(d.x, d.xd, g.x, g.ntok, t0, c);
    };
    copy(st[0], 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int c = 0; c < nc; ++c) {
        if (c + 1 < nc) copy(st[(c + 1) & 1], c + 1);
        KqPairStage& cur = st[c & 1];
        kq_compute_fold<G>(KqBases{lds_off(cur.w0), lds_off(cur.wk), lds_off(cur.x), lds_off(cur.xd)}, ag);
        kq_compute_fold<G>(KqBases{lds_off(cur.u0), lds_off(cur.uk), lds_off(cur.x), lds_off(cur.xd)}, au);
        __builtin_amdgcn_s_waitcnt(0);  // chunk c + 1 has landed (this wave's copies) ...
        __syncthreads();                // ... everyone's, and stage c & 1 is consumed
    }
    const uint32_t rmax = g.m.rows - 1;
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        const int t = t0 + 16 * gi + (lane & 15);
        if (t >= g.ntok) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = rt0 + wave * 16 + (lane >> 4) * 4 + i;
            if (r > rmax) continue;
            float* o = g.out + static_cast<size_t>(t) * g.ostride + r;
            const float gv = ag.s[gi][i], v = au.s[gi][i];
            if (g.relu2) {
                const float q = gv > 0.0f ? gv : 0.0f;
                *o = q * q * v;  // src/model.cpp:1134-1138
            } else if (g.gelu) {
                *o = gelu_mul(gv, v);  // src/kernels_f32.cpp:291-296
            } else {
                *o = gv / (1.0f + ref_expf_s(-gv)) * v;  // src/kernels_f32.cpp:287-289
            }
        }
    }
}

// ---------------------------------------------------------------- per-token work

// Embedding rows of seq[pos0 + t] (embedding_row, src/model.cpp:27-70).
// Gemma's rows are then multiplied by sqrt(embd) (src/model.cpp:899-901; scale 1 elsewhere).
__global__ void k_pre_embed(Packed m, const int* __restrict__ seq, int pos0, float* __restrict__ h, float scale) {
    const int t = blockIdx.x;
    const uint32_t tok = static_cast<uint32_t>(seq[pos0 + t]);
    float* row = h + static_cast<size_t>(t) * m.cols;
    for (uint32_t e = threadIdx.x; e < m.cols; e += blockDim.x) {
        const float v = dequant_elem(m, tok, e);
        row[e] = scale != 1.0f ? v * scale : v;
    }
}

// h[t] += rms_norm(p[t], w) for every row t (src/model.cpp:1113-1121, :1153-1160): a workgroup a row.
__global__ __launch_bounds__(kThreads) void k_pre_post_add(float* __restrict__ h, const float* __restrict__ p,
                                                           const float* __restrict__ w, float eps, int n, float out_scale) {
    __shared__ double red[4];
    const size_t off = static_cast<size_t>(blockIdx.x) * n;
    h += off;
    p += off;
    const float scale = rms_scale(block_sumsq(p, n, red), n, eps);
    // (x * 1.0f is x: out_scale 1 is the plain residual add)
    for (int i = threadIdx.x; i < n; i += kThreads) h[i] = (h[i] + p[i] * scale * w[i]) * out_scale;
}

// h *= out_scale over ntok rows of n values (Gemma 4's layer output scale, src/model.cpp:1178-1181).
__global__ void k_pre_scale(float* __restrict__ h, float out_scale, size_t count) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < count) h[i] *= out_scale;
}

// Gemma 4's per-layer embedding inputs of token t (src/model.cpp:905-925), a workgroup per
// (layer, token): slice (l, t) of in ([ntok][layers][dim], the per_layer_model_proj rows of the
// scaled embedding) scaled by proj_scale, RMS-normed with norm, plus the token's row of the
// per-layer table times table_scale, times 0.70710678.
__global__ __launch_bounds__(kThreads) void k_pre_ple_inputs(float* __restrict__ in, Packed table, const float* __restrict__ norm,
                                                             const int* __restrict__ seq, int pos0, int layers, int dim,
                                                             float proj_scale, float table_scale, float eps) {
    __shared__ double red[4];
    const int l = blockIdx.x, t = blockIdx.y;
    float* slice = in + (static_cast<size_t>(t) * layers + l) * dim;
    const uint32_t tok = static_cast<uint32_t>(seq[pos0 + t]);
    for (int i = threadIdx.x; i < dim; i += kThreads) slice[i] = slice[i] * proj_scale;
    __syncthreads();
    const float scale = rms_scale(block_sumsq(slice, dim, red), dim, eps);
    for (int i = threadIdx.x; i < dim; i += kThreads) {
        const float row = dequant_elem(table, tok, static_cast<uint32_t>(l * dim + i));
        slice[i] = (slice[i] * scale * norm[i] + row * table_scale) * 0.70710678f;
    }
}

// g[t][i] = gelu(g[t][i]) * in[t * in_stride + i] over ntok rows of n (gelu_mul_f32, src/kernels_f32.cpp:291-296).
__global__ void k_pre_gelu_mul(float* __restrict__ g, const float* __restrict__ in, int n, int in_stride, int ntok) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<size_t>(n) * ntok) return;
    const size_t t = i / n, c = i - t * n;
    g[i] = gelu_mul(g[i], in[t * in_stride + c]);
}

// LFM2 short convolution over ntok tokens at positions pos0 .. (src/model.cpp:935-969): for each
// token in order, bx = b * x is stored (fp16) at its position, then out = c * sum over the last
// `taps` positions, oldest first, of w[d][k] * bx (positions before 0 are zero state).  A thread
// a channel walks the tokens in order, so each bx it reads was stored before (by itself or by an
// earlier call).  bcx rows are [b | c | x], 3 n values each.
__global__ __launch_bounds__(kThreads) void k_pre_conv(const float* __restrict__ bcx, uint16_t* __restrict__ cache,
                                                       const float* __restrict__ w, int taps, int pos0, int n, int ntok,
                                                       float* __restrict__ out) {
    const int d = blockIdx.x * kThreads + threadIdx.x;
    if (d >= n) return;
    for (int t = 0; t < ntok; ++t) {
        const float* r = bcx + static_cast<size_t>(t) * 3 * n;
        const int pos = pos0 + t;
        cache[static_cast<size_t>(pos) * n + d] = f2h(r[2 * n + d] * r[d]);
        float acc = 0.0f;
        for (int k = 0; k < taps; ++k) {
            if (pos + k + 1 < taps) continue;
            acc += w[d * taps + k] * h2f(cache[static_cast<size_t>(pos + k + 1 - taps) * n + d]);
        }
        out[static_cast<size_t>(t) * n + d] = acc * r[n + d];
    }
}

// logits = cap * tanh(logits / cap) (src/model.cpp:1206-1208).
__global__ void k_softcap(float* __restrict__ x, size_t n, float cap) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) x[i] = cap * ref_tanhf(x[i] / cap);
}

// Q/K norms, RoPE, and the K/V cache rows of token t (grid: tokens x kv heads);
// the normed, rotated queries go back to q.  The same steps as the token
// path's attention prologue (attn_load_raw, attn_finish_prologue), with an LDS
// footprint of this token's rows only, so many workgroups share a CU.
constexpr int kRopeMaxHeads = 16;  // query heads a kv head (as the token path's AttnLds)
struct RopeLds {
    alignas(16) float q[kRopeMaxHeads * 128];
    float kcur[128], vcur[128];
    float rope[128];  // this position's RoPE row, loaded with the rows
};
__global__ __launch_bounds__(kThreads) void k_pre_rope(PreAttnArgs p) {
    __shared__ RopeLds s;
    const int t = blockIdx.x, kv = blockIdx.y, pos = p.pos0 + t, tid = threadIdx.x;
    const AttnArgs& g = p.a;
    const int hpk = g.heads / g.kv_heads, hd = g.head_dim;
    float* q = p.q + static_cast<size_t>(t) * p.qstride + kv * hpk * hd;
    const float* k = p.k + static_cast<size_t>(t) * p.kvstride + kv * hd;
    const float* v = p.v + static_cast<size_t>(t) * p.kvstride + kv * hd;
    for (int i = tid; i < hpk * hd; i += kThreads) s.q[i] = q[i];
    for (int i = tid; i < hd; i += kThreads) {
        s.kcur[i] = k[i];
        s.vcur[i] = g.vbias != nullptr ? v[i] + g.vbias[kv * hd + i] : v[i];
    }
    const float* rope_row = g.rope != nullptr ? g.rope + static_cast<size_t>(pos) * g.rope_dim : nullptr;
    if (rope_row != nullptr)  // the table row beside the rows: one round trip, not two
        for (int i = tid; i < g.rope_dim; i += kThreads) s.rope[i] = rope_row[i];
    __syncthreads();
    const float* rope = rope_row != nullptr ? s.rope : nullptr;
    for (int h = tid >> 6; h <= hpk; h += kThreads / 64) {  // a wave a head; the last is the key
        if (h < hpk) head_norm_rope(s.q + h * hd, g.qbias != nullptr ? g.qbias + (kv * hpk + h) * hd : nullptr, g.qnorm, rope, hd, g.rope_dim, g.neox, g.eps);
        else head_norm_rope(s.kcur, g.kbias != nullptr ? g.kbias + kv * hd : nullptr, g.knorm, rope, hd, g.rope_dim, g.neox, g.eps);
    }
    __syncthreads();
    // the cache rows, fp16 (store_f16, src/kernels_f32.cpp:248-250)
    uint16_t* kr = g.kcache + (static_cast<size_t>(kv) * g.ctx + pos) * hd;
    uint16_t* vr = g.vcache + (static_cast<size_t>(kv) * g.ctx + pos) * hd;
    for (int i = 2 * tid; i < hd; i += 2 * kThreads) {
        *reinterpret_cast<uint32_t*>(kr + i) = f2h(s.kcur[i]) | (static_cast<uint32_t>(f2h(s.kcur[i + 1])) << 16);
        *reinterpret_cast<uint32_t*>(vr + i) = f2h(s.vcur[i]) | (static_cast<uint32_t>(f2h(s.vcur[i + 1])) << 16);
    }
    for (int i = tid; i < hpk * hd; i += kThreads) q[i] = s.q[i];
}

// Attention of token t over positions 0 .. pos0 + t, in the reference's order.
__global__ __launch_bounds__(kThreads) void k_pre_attn(PreAttnArgs p) {
    __shared__ AttnLds s;
    const int t = blockIdx.x, kv = blockIdx.y, pos = p.pos0 + t;
    const AttnArgs& g = p.a;
    const int hpk = g.heads / g.kv_heads, hd = g.head_dim;
    const float* q = p.q + static_cast<size_t>(t) * p.qstride + kv * hpk * hd;
    for (int i = threadIdx.x; i < hpk * hd; i += kThreads) s.q[i] = q[i];
    const uint16_t* kr = g.kcache + (static_cast<size_t>(kv) * g.ctx + pos) * hd;
    const uint16_t* vr = g.vcache + (static_cast<size_t>(kv) * g.ctx + pos) * hd;
    for (int i = threadIdx.x; i < hd; i += kThreads) {
        s.kcur[i] = h2f(kr[i]);
        s.vcur[i] = h2f(vr[i]);
    }
    __syncthreads();
    const PlainOut o{p.out + static_cast<size_t>(t) * p.qstride, nullptr, nullptr};
    // a sliding layer sees positions start .. pos (src/model.cpp:1084-1085): its cache rows from start on
    const int start = g.window > 0 && pos + 1 > g.window ? pos + 1 - g.window : 0;
    if (start == 0) {
        attn_exact(g, s, kv, pos + 1, o);
        return;
    }
    AttnArgs gw = g;
    gw.kcache += static_cast<size_t>(start) * hd;
    gw.vcache += static_cast<size_t>(start) * hd;
    attn_exact(gw, s, kv, pos + 1 - start, o);
}

// Attention of a block of tokens over one key/value head, in the reference's
// order per query row (the same arithmetic as attn_exact): a workgroup takes
// kPaRows query rows (8 / hpk tokens x the hpk query heads of kv head
// blockIdx.y), so each staged key or value chunk serves all of them.  Scores
// for every visible position go to LDS (causal: token t sees positions up to
// pos0 + t), then softmax a row a wave, then value sums in position order, one
// (row, dimension) chain a lane.  The cache holds every position (k_pre_rope
// wrote this prompt's rows).
constexpr int kPaRows = 8;
constexpr int kPaMaxL = kExactMax;

struct PaLds {
    alignas(16) float q[kPaRows * 128];
    alignas(16) float sc[kPaRows * (kPaMaxL + 4)];
    alignas(16) uint16_t kv[2][kSplit * 128];
    double red[kPaRows];
};

// A cache chunk (kSplit positions of one head) through registers: loaded with
// ordinary 16-byte loads, then written to LDS in chunk_issue's layout, so the
// loads of the next chunk are in flight while the current one is computed.
struct PaChunk {
    uint4 v0, v1, v2, v3;  // pieces k * kThreads + threadIdx.x, k = 0..3 (kSplit * hd / 8 <= 4 * kThreads)
};
__device__ __forceinline__ uint4 pa_piece(const uint8_t* src, int i, int pieces, int P, int mask) {
    const int j = i < pieces ? i : pieces - 1;  // past the chunk: a copy, not stored
    const int p = j / P, c = (j - p * P) ^ (p & mask);
    return *reinterpret_cast<const uint4*>(src + (static_cast<size_t>(p) * P + c) * 16);
}
__device__ __forceinline__ void pa_chunk_load(PaChunk& r, const uint16_t* base, int p0, int n_pos, int hd, bool swz) {
    const int P = kv_pieces(hd), mask = swz ? kv_mask(hd) : 0, pieces = n_pos * P, t = static_cast<int>(threadIdx.x);
    const uint8_t* src = reinterpret_cast<const uint8_t*>(base + static_cast<size_t>(p0) * hd);
    r.v0 = pa_piece(src, t, pieces, P, mask);
    r.v1 = pa_piece(src, kThreads + t, pieces, P, mask);
    if (kSplit * hd / 8 > 2 * kThreads) {
        r.v2 = pa_piece(src, 2 * kThreads + t, pieces, P, mask);
        r.v3 = pa_piece(src, 3 * kThreads + t, pieces, P, mask);
    }
}
__device__ __forceinline__ void pa_chunk_store(const PaChunk& r, uint16_t* lds, int n_pos, int hd) {
    const int pieces = n_pos * kv_pieces(hd), t = static_cast<int>(threadIdx.x);
    uint4* dst = reinterpret_cast<uint4*>(lds);
    if (t < pieces) dst[t] = r.v0;
    if (kThreads + t < pieces) dst[kThreads + t] = r.v1;
    if (2 * kThreads + t < pieces) dst[2 * kThreads + t] = r.v2;
    if (3 * kThreads + t < pieces) dst[3 * kThreads + t] = r.v3;
}

// score_lane's arithmetic (dot_f32, src/kernels_f32.cpp:229-246: 16 lane
// partials, then their sum in order, times nothing yet) with each product q k
// one mul_h, so the key halves need no separate conversion.
template <int PER>
__device__ __forceinline__ float pa_score(const float* q, const uint16_t* chunk, int p, int P, int mask) {
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
        for (int j = 0; j < 16; ++j) lane[j] += (j & 1) ? mul_h<true>(qv[j], kw[j >> 1]) : mul_h<false>(qv[j], kw[j >> 1]);
    }
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) sum += lane[j];
    return sum;
}

template <int PER>
__device__ __forceinline__ void pa_scores(const PreAttnArgs& p, PaLds& s, int rows, int tpb, int hpk, int L, int tb0, int Ls,
                                          const uint16_t* kbase) {
    constexpr int hd = PER * 16, P = hd / 8, mask = P - 1;
    const int nchunks = (L + kSplit - 1) / kSplit;
    PaChunk r;
    pa_chunk_load(r, kbase, 0, L < kSplit ? L : kSplit, hd, true);
    for (int c = 0; c < nchunks; ++c) {
        // buffer c & 1 last held chunk c - 2, consumed before the barrier of chunk c - 1
        pa_chunk_store(r, s.kv[c & 1], L - c * kSplit < kSplit ? L - c * kSplit : kSplit, hd);
        if (c + 1 < nchunks) {
            const int p1 = (c + 1) * kSplit;
            pa_chunk_load(r, kbase, p1, L - p1 < kSplit ? L - p1 : kSplit, hd, true);  // in flight during chunk c
        }
        __syncthreads();  // chunk c staged
        const uint16_t* buf = s.kv[c & 1];
        const int p0 = c * kSplit;
        for (int i = threadIdx.x; i < rows * kSplit; i += kThreads) {
            const int row = i / kSplit, pp = i - row * kSplit, pos = p0 + pp;
            const int tpos = p.pos0 + tb0 + row / hpk;  // the row's token position: it sees 0 .. tpos
            if (pos <= tpos && pos < L) s.sc[row * Ls + pos] = pa_score<PER>(s.q + row * hd, buf, pp, P, mask) * p.a.scale;
        }
    }
    __syncthreads();
}

// Value sums of the block's rows: thread t owns dimension d = t % hd of rows
// t / hd, + kThreads / hd, ... (NCH chains).  The chains run in lockstep
// over the positions, so each value v[q][d] is read once for all of them and
// their adds are independent; each chain still adds its terms in position
// order (0 + w_0 v_0 + w_1 v_1 + ...), stopping at its row's last visible
// position.
template <int NCH>
__device__ __forceinline__ void pa_values(const PreAttnArgs& p, PaLds& s, int rows, int hpk, int L, int tb0, int Ls,
                                          const uint16_t* vbase, PaChunk& r) {
    const int hd = p.a.head_dim, t = threadIdx.x, d = t % hd, rstep = kThreads / hd, r0 = t / hd;
    float acc[NCH];
    int lr[NCH];
    const float* wrow[NCH];
    int lmin = kPaMaxL, lmax = 0;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        acc[k] = 0.0f;
        const int row = r0 + k * rstep < rows ? r0 + k * rstep : rows - 1;  // past the block: a copy, not stored
        lr[k] = p.pos0 + tb0 + row / hpk + 1;  // positions the row sees
        wrow[k] = s.sc + row * Ls;
        lmin = lr[k] < lmin ? lr[k] : lmin;
        lmax = lr[k] > lmax ? lr[k] : lmax;
    }
    const int nchunks = (L + kSplit - 1) / kSplit;
    for (int c = 0; c < nchunks; ++c) {
        // r holds value chunk c (chunk 0 was loaded before the softmax)
        pa_chunk_store(r, s.kv[c & 1], L - c * kSplit < kSplit ? L - c * kSplit : kSplit, hd);
        if (c + 1 < nchunks) {
            const int q1 = (c + 1) * kSplit;
            pa_chunk_load(r, vbase, q1, L - q1 < kSplit ? L - q1 : kSplit, hd, false);
        }
        __syncthreads();  // value chunk c staged (and, for c = 0, the weights are final)
        const uint16_t* vcol = s.kv[c & 1] + d;
        const int q0 = c * kSplit;
        const int nall = lmin - q0 < 0 ? 0 : (lmin - q0 < kSplit ? lmin - q0 : kSplit);  // every chain takes these
        const int nany = lmax - q0 < 0 ? 0 : (lmax - q0 < kSplit ? lmax - q0 : kSplit);
        int q = 0;
        for (; q + 4 <= nall; q += 4) {
            const uint32_t v0 = vcol[(q + 0) * hd], v1 = vcol[(q + 1) * hd];  // halves, widened by mul_h
            const uint32_t v2 = vcol[(q + 2) * hd], v3 = vcol[(q + 3) * hd];
#pragma unroll
            for (int k = 0; k < NCH; ++k) {
                const float4 w4 = *reinterpret_cast<const float4*>(wrow[k] + q0 + q);
                float a = acc[k];
                a += mul_h<false>(w4.x, v0); a += mul_h<false>(w4.y, v1); a += mul_h<false>(w4.z, v2); a += mul_h<false>(w4.w, v3);
                acc[k] = a;
            }
        }
        for (; q < nany; ++q) {
            const uint32_t v = vcol[q * hd];
#pragma unroll
            for (int k = 0; k < NCH; ++k)
                if (q0 + q < lr[k]) acc[k] += mul_h<false>(wrow[k][q0 + q], v);
        }
    }
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int row = r0 + k * rstep;
        if (row < rows) {
            const int tt = row / hpk, gq = row - tt * hpk;
            p.out[static_cast<size_t>(tb0 + tt) * p.qstride + (blockIdx.y * hpk + gq) * hd + d] = acc[k];
        }
    }
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 8))) void k_pre_attn_blk(PreAttnArgs p, int ntok) {
    __shared__ PaLds s;
    const AttnArgs& g = p.a;
    const int hpk = g.heads / g.kv_heads, hd = g.head_dim, kv = blockIdx.y;
    const int tpb = kPaRows / hpk, tb0 = blockIdx.x * tpb;
    const int ntb = ntok - tb0 < tpb ? ntok - tb0 : tpb, rows = ntb * hpk;
    const int L = p.pos0 + tb0 + ntb;  // positions the block's last token sees
    const int Ls = (L + 3) & ~3;
    const int t = threadIdx.x, wave = t >> 6, wl = t & 63;
    exp_tab_fill();  // ordered before the softmax by the barriers between
    for (int i = t; i < rows * hd; i += kThreads) {  // q rows: row = token * hpk + head
        const int row = i / hd, d = i - row * hd, tt = row / hpk, gq = row - tt * hpk;
        s.q[i] = p.q[static_cast<size_t>(tb0 + tt) * p.qstride + (kv * hpk + gq) * hd + d];
    }
    const uint16_t* kbase = g.kcache + static_cast<size_t>(kv) * g.ctx * hd;
    const uint16_t* vbase = g.vcache + static_cast<size_t>(kv) * g.ctx * hd;
    __syncthreads();
    if (hd == 128) pa_scores<8>(p, s, rows, tpb, hpk, L, tb0, Ls, kbase);
    else if (hd == 64) pa_scores<4>(p, s, rows, tpb, hpk, L, tb0, Ls, kbase);
    else pa_scores<2>(p, s, rows, tpb, hpk, L, tb0, Ls, kbase);
    // first value chunk in flight while the softmax runs
    PaChunk rv;
    pa_chunk_load(rv, vbase, 0, L < kSplit ? L : kSplit, hd, false);
    // ---- softmax, a row a wave: max, e = expf(s - max), double sum, w = e * (float)(1 / sum)
    for (int row = wave; row < rows; row += kThreads / 64) {
        const int Lr = p.pos0 + tb0 + row / hpk + 1;
        float* sc = s.sc + row * Ls;
        float m = -INFINITY;
        for (int q = wl; q < Lr; q += 64) m = fmaxf(m, sc[q]);
        m = wave_max(m);
        double part = 0.0;
        for (int q = wl; q < Lr; q += 64) {
            const float e = ref_expf_s(sc[q] - m);
            sc[q] = e;
            part += static_cast<double>(e);
        }
        const float scale = static_cast<float>(1.0 / wave_sum(part));
        for (int q = wl; q < Lr; q += 64) sc[q] *= scale;
    }
    // ---- value sums in position order: chains (row, d), kThreads / hd rows a pass
    if (hd == 128) pa_values<kPaRows * 128 / kThreads>(p, s, rows, hpk, L, tb0, Ls, vbase, rv);
    else if (hd == 64) pa_values<kPaRows * 64 / kThreads>(p, s, rows, hpk, L, tb0, Ls, vbase, rv);
    else pa_values<kPaRows * 32 / kThreads>(p, s, rows, hpk, L, tb0, Ls, vbase, rv);
}

// ---------------------------------------------------------------- exact attention, lane per position

// The reference's attention for a block of tokens (the same arithmetic as
// attn_exact), arranged so that no key or value is staged: a workgroup takes R
// query rows (R / hpk tokens x the hpk query heads of kv head blockIdx.y).
// Scores: a lane per position holds that position's key row in registers
// (loaded from the cache directly) and takes every row's dot_f32 against it,
// the query read as a broadcast; so a key is read once for all R rows and the
// only per-score work is the 16-lane dot itself.  Softmax: a row a wave.
// Values: a lane per (pair of dimensions, rows g, g + RG, ...), each value
// pair read straight from the cache once for all of the lane's rows; every
// chain adds its terms in position order, as weighted_sum_f32 does.
constexpr int kPxRows = 16;

// Causal attention blocks grow with their token index, and workgroups w,
// w + kKqCus, ... share a compute unit when the grid is resident at once.  So
// block ids are dealt heaviest first in a snake (round r of kKqCus ids takes
// the next kKqCus blocks, reversed on odd rounds): each unit's blocks then sum
// to about the same work.  Block k of the heavy-first order is token block
// nx - 1 - k / ny of kv head k % ny.
__device__ __forceinline__ void snake_block(int id, int nx, int ny, int& y, int& x) {
    const int r = id / kKqCus, c = id - r * kKqCus;
    const int k = r * kKqCus + ((r & 1) ? kKqCus - 1 - c : c);
    const int n = nx * ny;
    const int kk = k < n ? k : id;  // a partial last round: ids past n keep their own order
    x = nx - 1 - kk / ny;
    y = kk - (kk / ny) * ny;
}
template <int HD, int R, int LMAX>
struct PxLds {
    alignas(16) float q[R * HD];
    alignas(16) float sc[R * (LMAX + 4)];
};

template <int HD, int R, int LMAX>
__global__ __launch_bounds__(kThreads) void k_pre_attn_rows(PreAttnArgs p, int ntok) {
    __shared__ PxLds<HD, R, LMAX> s;
    constexpr int PER = HD / 16, NW = HD / 8;  // dot terms a lane partial; 16-byte pieces a key row
    const AttnArgs& g = p.a;
    const int hpk = g.heads / g.kv_heads, tpb = R / hpk;
    int kv, xb;
    snake_block(static_cast<int>(blockIdx.x), (ntok + tpb - 1) / tpb, g.kv_heads, kv, xb);
    const int tb0 = xb * tpb;
    const int ntb = ntok - tb0 < tpb ? ntok - tb0 : tpb, rows = ntb * hpk;
    const int first = p.pos0 + tb0;  // the block's first token's position
    const int L = first + ntb;       // positions the block's last token sees
    const int Ls = (L + 3) & ~3;
    const int t = threadIdx.x, wave = t >> 6, wl = t & 63;
    exp_tab_fill();  // ordered before the softmax by the barriers between
    for (int i = t; i < rows * HD; i += kThreads) {  // q rows: row = token * hpk + head
        const int row = i / HD, d = i - row * HD, tt = row / hpk, gq = row - tt * hpk;
        s.q[i] = p.q[static_cast<size_t>(tb0 + tt) * p.qstride + (kv * hpk + gq) * HD + d];
    }
    const uint16_t* kbase = g.kcache + static_cast<size_t>(kv) * g.ctx * HD;
    const uint16_t* vbase = g.vcache + static_cast<size_t>(kv) * g.ctx * HD;
    __syncthreads();
    // ---- scores: score_p = dot_f32(q, k_p) * scale, a lane per position
    for (int p0 = 0; p0 < L; p0 += kThreads) {
        const int pos = p0 + t;
        if (pos < L) {
            uint32_t kw[HD / 2];
            const uint4* krow = reinterpret_cast<const uint4*>(kbase + static_cast<size_t>(pos) * HD);
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const uint4 v = krow[w];
                kw[4 * w] = v.x; kw[4 * w + 1] = v.y; kw[4 * w + 2] = v.z; kw[4 * w + 3] = v.w;
            }
            // rows in token order: token tt sees positions 0 .. first + tt
            for (int tt = (pos > first ? pos - first : 0); tt < ntb; ++tt) {
                for (int gq = 0; gq < hpk; ++gq) {
                    const int row = tt * hpk + gq;
                    const float* q = s.q + row * HD;
                    // the lane partials start at their first product, not at 0 + it: they
                    // differ only by a zero's sign, which the 0 + ... of the final sum removes
                    float lane[16];
#pragma unroll
                    for (int m = 0; m < PER; ++m) {
                        const float4* q4 = reinterpret_cast<const float4*>(q + 16 * m);
                        const float4 qa = q4[0], qb = q4[1], qc = q4[2], qd = q4[3];
                        const float qv[16] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w,
                                              qc.x, qc.y, qc.z, qc.w, qd.x, qd.y, qd.z, qd.w};
#pragma unroll
                        for (int j = 0; j < 16; ++j) {
                            const float pr = (j & 1) ? mul_h<true>(qv[j], kw[8 * m + (j >> 1)]) : mul_h<false>(qv[j], kw[8 * m + (j >> 1)]);
                            lane[j] = m == 0 ? pr : lane[j] + pr;
                        }
                    }
                    float sum = 0.0f;
#pragma unroll
                    for (int j = 0; j < 16; ++j) sum += lane[j];
                    s.sc[row * Ls + pos] = sum * g.scale;
                }
            }
        }
    }
    __syncthreads();
    // ---- softmax, a row a wave: max, e = expf(s - max), double sum, w = e * (float)(1 / sum)
    // A sliding layer's row sees positions start .. Lr - 1 (src/model.cpp:1084-1088): the weights
    // before start are set to zero, so the value sums below add +0 until start and then the
    // same terms in the same order as from start.
    for (int row = wave; row < rows; row += kThreads / 64) {
        const int Lr = first + row / hpk + 1;
        const int start = g.window > 0 && Lr > g.window ? Lr - g.window : 0;
        float* sc = s.sc + row * Ls;
        float m = -INFINITY;
        for (int q = start + wl; q < Lr; q += 64) m = fmaxf(m, sc[q]);
        m = wave_max(m);
        double part = 0.0;
        for (int q = start + wl; q < Lr; q += 64) {
            const float e = ref_expf_s(sc[q] - m);
            sc[q] = e;
            part += static_cast<double>(e);
        }
        const float scale = static_cast<float>(1.0 / wave_sum(part));
        for (int q = start + wl; q < Lr; q += 64) sc[q] *= scale;
        for (int q = wl; q < start; q += 64) sc[q] = 0.0f;
    }
    __syncthreads();
    // ---- value sums in position order: lane = (dimension pair dp, rows rg, rg + RG, ...)
    constexpr int DP = HD / 2, RG = kThreads / DP, NR = R / RG;
    const int dp = t % DP, rg = t / DP;
    float acc0[NR], acc1[NR];
    int lr[NR];
    const float* wrow[NR];
    int lmin = L, lmax = 0;
#pragma unroll
    for (int k = 0; k < NR; ++k) {
        acc0[k] = acc1[k] = 0.0f;
        const int row = rg + k * RG < rows ? rg + k * RG : rows - 1;  // past the block: a copy, not stored
        lr[k] = first + row / hpk + 1;
        wrow[k] = s.sc + row * Ls;
        lmin = lr[k] < lmin ? lr[k] : lmin;
        lmax = lr[k] > lmax ? lr[k] : lmax;
    }
    const uint32_t* vcol = reinterpret_cast<const uint32_t*>(vbase) + dp;  // value pair (2 dp, 2 dp + 1) of row 0
    // positions every chain takes, in batches of B: the next batch's loads are
    // issued before the current batch's adds (two register sets, ping-pong),
    // so a batch waits for no load but the one issued a batch earlier
    constexpr int B = 16;
    const int nb = lmin / B;
    uint32_t va[B], vb[B];
    auto load = [&](uint32_t* v, int q0) {
#pragma unroll
        for (int u = 0; u < B; ++u) v[u] = vcol[static_cast<size_t>(q0 + u) * DP];
    };
    auto adds = [&](const uint32_t* v, int q0) {
#pragma unroll
        for (int k = 0; k < NR; ++k) {
            float a0 = acc0[k], a1 = acc1[k];
#pragma unroll
            for (int u4 = 0; u4 < B; u4 += 4) {
                const float4 w4 = *reinterpret_cast<const float4*>(wrow[k] + q0 + u4);
                const float w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    a0 += mul_h<false>(w[u], v[u4 + u]);
                    a1 += mul_h<true>(w[u], v[u4 + u]);
                }
            }
            acc0[k] = a0;
            acc1[k] = a1;
        }
    };
    if (nb > 0) load(va, 0);
    int b = 0;
    for (; b + 2 <= nb; b += 2) {
        load(vb, (b + 1) * B);
        adds(va, b * B);
        if (b + 2 < nb) load(va, (b + 2) * B);
        adds(vb, (b + 1) * B);
    }
    if (b < nb) adds(va, b * B);
    int q = nb * B;
    for (; q < lmax; ++q) {
        const uint32_t v = vcol[static_cast<size_t>(q) * DP];
#pragma unroll
        for (int k = 0; k < NR; ++k)
            if (q < lr[k]) {
                const float w = wrow[k][q];
                acc0[k] += mul_h<false>(w, v);
                acc1[k] += mul_h<true>(w, v);
            }
    }
#pragma unroll
    for (int k = 0; k < NR; ++k) {
        const int row = rg + k * RG;
        if (row < rows) {
            const int tt = row / hpk, gq = row - tt * hpk;
            float* o = p.out + static_cast<size_t>(tb0 + tt) * p.qstride + (kv * hpk + gq) * HD + 2 * dp;
            *reinterpret_cast<float2*>(o) = make_float2(acc0[k], acc1[k]);
        }
    }
    // The O projection's activation blocks: token tt's hpk heads of this kv head are values
    // kv * 256 .. kv * 256 + 255 of its row, one whole block, quantised here (as k_pre_quant_blocks
    // does from the stored rows) instead of by a separate launch.  s.q is free: its last reads
    // (the scores) are behind the softmax's barriers.
    if (p.qout.qs != nullptr && hpk * HD == 256) {
#pragma unroll
        for (int k = 0; k < NR; ++k) {
            const int row = rg + k * RG;
            if (row < rows) *reinterpret_cast<float2*>(s.q + row * HD + 2 * dp) = make_float2(acc0[k], acc1[k]);
        }
        __syncthreads();
        for (int tt = wave; tt < ntb; tt += kThreads / 64) {
            const float4 x = *reinterpret_cast<const float4*>(s.q + tt * 256 + 4 * wl);
            const float v[4] = {x.x, x.y, x.z, x.w};
            if (p.q8k) pre_quant_block<true>(v, tb0 + tt, kv, p.qbits, p.qout);
            else pre_quant_block<false>(v, tb0 + tt, kv, p.qbits, p.qout);
        }
    }
}

// ---------------------------------------------------------------- long-prompt attention on MFMA

// Opt-in (BRISK_HIP_PREFILL_ATTN=mfma), for prompts of kFaMinTok tokens or
// more: causal attention with the products on v_mfma_f32_16x16x32_f16, flash
// style (a running max and sum per query row, so no score row is stored).
// This is not the reference's summation order, so it is not bit-identical:
// each f32 operand is carried as two halves, x = hi + lo / 4096 with
// hi = f16(x) (probabilities scaled by 2^14 first, so small ones stay normal
// f16: the MFMA reads f16 subnormals as zero), and the lo products go to their
// own accumulators, so the products keep fp32 rounding.  The attention output
// then differs from the reference's by fp32 reordering only, but the next
// projection re-quantises it to int8, and one rounding that tips the other way
// moves later layers by a quantisation step: on small random-weight models
// logits can move by ~0.1.  The exact-order kernels above stay the default.
//
// A workgroup takes 64 query rows (64 / hpk tokens x the hpk query heads of kv
// head blockIdx.y), 16 a wave, and walks the visible positions in chunks of 32
// staged through LDS (keys row-major and XOR-swizzled, values transposed).
// Per wave and chunk, with g = lane / 16 and lane l % 16 = the wave's row r:
//   S^T = K Q^T:  A = keys (16 positions x head_dim), B = the query rows, so
//                 D puts positions 4 g + i (+ 16) of row r in lane l: the row
//                 is lane-local and its max needs two cross-lane steps.
//   O^T += V^T P^T: A = values transposed (16 dims x 32 positions), B = P^T,
//                 whose 8 k-slots per lane are exactly the 8 probabilities
//                 the lane holds (positions 4 g .. + 3 and 16 + 4 g .. + 3),
//                 so P never leaves registers; D puts dims 4 g + i of row r
//                 in lane l.
constexpr int kFaRows = 64;
constexpr int kFaPos = 32;
constexpr int kFaMinTok = 64;
constexpr int kFaVtRow = kFaPos + 8;  // halves a transposed value row (80 bytes: conflict-free 16-row reads)
constexpr float kFaPUp = 16384.0f;    // probabilities are scaled by this (<= 2^14) before the f16 split

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

template <int HD>
struct FaLds {
    alignas(16) uint16_t k[2][kFaPos * HD];
    alignas(16) uint16_t vt[2][HD * kFaVtRow];
};

// 16-byte piece p of key row `pos` in the staged chunk: XOR-swizzled so the 16
// rows one A fragment reads fall in distinct banks
template <int HD>
__device__ __forceinline__ int fa_kslot(int pos, int p) {
    constexpr int P = HD / 8, SH = HD >= 128 ? 0 : (HD == 64 ? 1 : 2);
    return pos * P + (p ^ ((pos >> SH) & (P - 1)));
}

template <int HD>
struct FaChunk {
    static constexpr int N = kFaPos * HD / 8 / kThreads;  // 16-byte pieces a thread, keys and values each
    uint4 k[N], v[N];
};

template <int HD>
__device__ __forceinline__ void fa_load(FaChunk<HD>& r, const uint16_t* kb, const uint16_t* vb, int p0, int L) {
    constexpr int P = HD / 8;
#pragma unroll
    for (int u = 0; u < FaChunk<HD>::N; ++u) {
        const int j = u * kThreads + static_cast<int>(threadIdx.x), p = j % P;
        // past the context: a copy of its last row (finite, and weighted by 0)
        const int pos = p0 + j / P < L ? p0 + j / P : L - 1;
        r.k[u] = *reinterpret_cast<const uint4*>(kb + static_cast<size_t>(pos) * HD + p * 8);
        r.v[u] = *reinterpret_cast<const uint4*>(vb + static_cast<size_t>(pos) * HD + p * 8);
    }
}

template <int HD>
__device__ __forceinline__ void fa_store(const FaChunk<HD>& r, FaLds<HD>& s, int buf) {
    constexpr int P = HD / 8;
#pragma unroll
    for (int u = 0; u < FaChunk<HD>::N; ++u) {
        const int j = u * kThreads + static_cast<int>(threadIdx.x), pos = j / P, p = j % P;
        reinterpret_cast<uint4*>(s.k[buf])[fa_kslot<HD>(pos, p)] = r.k[u];
        const uint32_t w[4] = {r.v[u].x, r.v[u].y, r.v[u].z, r.v[u].w};
        uint16_t* col = s.vt[buf] + (p * 8) * kFaVtRow + pos;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            col[(2 * e) * kFaVtRow] = static_cast<uint16_t>(w[e] & 0xFFFF);
            col[(2 * e + 1) * kFaVtRow] = static_cast<uint16_t>(w[e] >> 16);
        }
    }
}

// x = hi + lo / 4096: the low half is scaled up so it stays a normal
// f16 (the MFMA treats f16 subnormal inputs as zero) for all but tiny x
constexpr float kFaLoUp = 4096.0f, kFaLoDown = 1.0f / 4096.0f;
__device__ __forceinline__ void fa_split(const float* x, v8h& hi, v8h& lo) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const _Float16 h = static_cast<_Float16>(x[j]);
        hi[j] = h;
        lo[j] = static_cast<_Float16>((x[j] - static_cast<float>(h)) * kFaLoUp);
    }
}

__device__ __forceinline__ v4f fa_mfma(const v8h& a, const v8h& b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <int HD>
__global__ __launch_bounds__(kThreads) void k_pre_attn_fa(PreAttnArgs p, int ntok) {
    __shared__ FaLds<HD> s;
    constexpr int KS = HD / 32, DT = HD / 16;
    const AttnArgs& g = p.a;
    const int hpk = g.heads / g.kv_heads, tpb = kFaRows / hpk;
    int kv, xb;
    snake_block(static_cast<int>(blockIdx.x), (ntok + tpb - 1) / tpb, g.kv_heads, kv, xb);
    const int tb0 = xb * tpb;
    const int ntb = ntok - tb0 < tpb ? ntok - tb0 : tpb;
    const int L = p.pos0 + tb0 + ntb;  // positions the block's last token sees
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 15, gq4 = lane >> 4;
    const int row = wave * 16 + r;
    const int tt = row / hpk < ntb ? row / hpk : ntb - 1;  // past the prompt: a copy of its last token, not stored
    const int head = kv * hpk + row % hpk;
    const int lim = p.pos0 + tb0 + tt;  // the row sees positions 0 .. lim
    const int wlast = p.pos0 + tb0 + ((wave * 16 + 15) / hpk < ntb ? (wave * 16 + 15) / hpk : ntb - 1);
    const int wchunks = wlast / kFaPos + 1, nchunks = (L + kFaPos - 1) / kFaPos;

    const uint16_t* kb = g.kcache + static_cast<size_t>(kv) * g.ctx * HD;
    const uint16_t* vb = g.vcache + static_cast<size_t>(kv) * g.ctx * HD;
    FaChunk<HD> ch;
    fa_load<HD>(ch, kb, vb, 0, L);

    // this lane's query row, d = 32 ks + 8 g .. + 7, as hi / lo halves
    v8h qh[KS], ql[KS];
    {
        const float* q = p.q + static_cast<size_t>(tb0 + tt) * p.qstride + head * HD;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const float4 a = *reinterpret_cast<const float4*>(q + 32 * ks + 8 * gq4);
            const float4 b = *reinterpret_cast<const float4*>(q + 32 * ks + 8 * gq4 + 4);
            const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            fa_split(x, qh[ks], ql[ks]);
        }
    }
    v4f o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, lsum = 0.0f;
    const float scale = g.scale;

    for (int c = 0; c < nchunks; ++c) {
        const int buf = c & 1;
        fa_store<HD>(ch, s, buf);  // buffer c & 1 last held chunk c - 2, read before the barrier of chunk c - 1
        if (c + 1 < nchunks) fa_load<HD>(ch, kb, vb, (c + 1) * kFaPos, L);
        __syncthreads();
        if (c >= wchunks) continue;  // every row of this wave is past this chunk
        const int p0 = c * kFaPos;
        // scores S^T: tile t covers positions p0 + 16 t .. + 15
        v4f sc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            v4f acc = {0.0f, 0.0f, 0.0f, 0.0f}, accl = acc;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const v8h kf = *reinterpret_cast<const v8h*>(
                    reinterpret_cast<const uint4*>(s.k[buf]) + fa_kslot<HD>(16 * t + r, 4 * ks + gq4));
                acc = fa_mfma(kf, qh[ks], acc);
                accl = fa_mfma(kf, ql[ks], accl);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[t][i] = acc[i] + accl[i] * kFaLoDown;
        }
        // online softmax over the row's 8 positions in this lane and the row's other 3 lanes
        float sv[8];
        float cmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int pos = p0 + 16 * (j >> 2) + 4 * gq4 + (j & 3);
            sv[j] = pos <= lim ? sc[j >> 2][j & 3] * scale : -INFINITY;
            cmax = fmaxf(cmax, sv[j]);
        }
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
        const float mn = fmaxf(m, cmax);  // finite: chunk 0 holds position 0, which every row sees
        const float alpha = __expf(m - mn);
        m = mn;
        // probabilities scaled by 2^14 (<= 16384) so that small ones stay normal f16; the sum too
        float pv[8], psum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            pv[j] = __expf(sv[j] - mn) * kFaPUp;
            psum += pv[j];
        }
        lsum = lsum * alpha + psum;
        v8h ph, pl;
        fa_split(pv, ph, pl);
        // O^T += V^T P^T: A = values of dims 16 dt + r at positions 4 g .. + 3 and 16 + 4 g .. + 3
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const uint16_t* vr = s.vt[buf] + (16 * dt + r) * kFaVtRow + 4 * gq4;
            const uint2 a0 = *reinterpret_cast<const uint2*>(vr);
            const uint2 a1 = *reinterpret_cast<const uint2*>(vr + 16);
            const v8h vf = __builtin_bit_cast(v8h, make_uint4(a0.x, a0.y, a1.x, a1.y));
            v4f acc = o[dt] * alpha, accl = {0.0f, 0.0f, 0.0f, 0.0f};
            acc = fa_mfma(vf, ph, acc);
            accl = fa_mfma(vf, pl, accl);
#pragma unroll
            for (int i = 0; i < 4; ++i) o[dt][i] = acc[i] + accl[i] * kFaLoDown;
        }
    }
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    if (row / hpk < ntb) {
        const float inv = 1.0f / lsum;
        float* out = p.out + static_cast<size_t>(tb0 + tt) * p.qstride + head * HD + 4 * gq4;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const v4f v = o[dt] * inv;
            *reinterpret_cast<float4*>(out + 16 * dt) = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
}

// ---------------------------------------------------------------- launchers

// The expanded-plane GEMM: 4 waves (128 rows) a workgroup when that still gives every compute unit
// two workgroups, else 2 waves, else 1.  At one wave a SIMD a CU holds four waves either way; smaller
// workgroups couple fewer waves at each super-block's barrier (down on configs[2]: 59 us with 4
// waves a workgroup, 50 with 2 or 1).
template <int MODE, bool KM>
static void mmx_launch(const MmArgs& g, hipStream_t s) {
    const int tt = (g.ntok + 31) / 32;
    auto tiles = [&](int w) { return static_cast<int>((g.m.rows + 32 * w - 1) / (32 * w)) * tt; };
    if (tiles(4) >= 2 * kKqCus) hipLaunchKernelGGL((k_mmx<MODE, 1, 4, KM>), dim3(tiles(4)), dim3(256), 0, s, g);
    else if (tiles(2) >= 2 * kKqCus) hipLaunchKernelGGL((k_mmx<MODE, 1, 2, KM>), dim3(tiles(2)), dim3(128), 0, s, g);
    else hipLaunchKernelGGL((k_mmx<MODE, 1, 1, KM>), dim3(tiles(1)), dim3(64), 0, s, g);
}

template <int MODE>
static hipError_t mm_dispatch(const MmArgs& g, hipStream_t s) {
    const int tok = 16 * (g.m.type == kQ4_K || g.m.type == kQ5_K || g.m.type == kQ6_K ? mm_groups<kQ4_K>() : mm_groups<kQ4_0>());
    const dim3 grid((g.m.rows + kRowsPerWg - 1) / kRowsPerWg, (g.ntok + tok - 1) / tok);
    // K-quants: the widest token tile (64, 32 or 16 tokens) that still gives a workgroup to every CU
    const int row_tiles = static_cast<int>((g.m.rows + 63) / 64);
    int kq_g = 4;
    while (kq_g > 1 && row_tiles * ((g.ntok + 16 * kq_g - 1) / (16 * kq_g)) < kKqCus) kq_g /= 2;
    const dim3 kq_grid(row_tiles, (g.ntok + 16 * kq_g - 1) / (16 * kq_g));
    switch (g.m.type) {
        case kQ4_0: hipLaunchKernelGGL((k_mm<kQ4_0, MODE>), grid, dim3(kThreads), 0, s, g); break;
        case kQ4_1: hipLaunchKernelGGL((k_mm<kQ4_1, MODE>), grid, dim3(kThreads), 0, s, g); break;
        case kQ5_0: hipLaunchKernelGGL((k_mm<kQ5_0, MODE>), grid, dim3(kThreads), 0, s, g); break;
        case kQ8_0: hipLaunchKernelGGL((k_mm<kQ8_0, MODE>), grid, dim3(kThreads), 0, s, g); break;
        case kQ5_K:
            if (g.qx != nullptr) mmx_launch<MODE, true>(g, s);
            else hipLaunchKernelGGL((k_mm<kQ5_K, MODE>), grid, dim3(kThreads), 0, s, g);
            break;
        case kQ4_K:
            if (g.qx != nullptr) {
                mmx_launch<MODE, true>(g, s);
                break;
            }
            if (kq_g == 4) hipLaunchKernelGGL((k_mmk<kQ4_K, MODE, 4>), kq_grid, dim3(kThreads), 0, s, g, g);
            else if (kq_g == 2) hipLaunchKernelGGL((k_mmk<kQ4_K, MODE, 2>), kq_grid, dim3(kThreads), 0, s, g, g);
            else hipLaunchKernelGGL((k_mmk<kQ4_K, MODE, 1>), kq_grid, dim3(kThreads), 0, s, g, g);
            break;
        case kQ6_K:
            if (g.qx != nullptr) {
                mmx_launch<MODE, false>(g, s);
                break;
            }
            if (kq_g == 4) hipLaunchKernelGGL((k_mmk<kQ6_K, MODE, 4>), kq_grid, dim3(kThreads), 0, s, g, g);
            else if (kq_g == 2) hipLaunchKernelGGL((k_mmk<kQ6_K, MODE, 2>), kq_grid, dim3(kThreads), 0, s, g, g);
            else hipLaunchKernelGGL((k_mmk<kQ6_K, MODE, 1>), kq_grid, dim3(kThreads), 0, s, g, g);
            break;
        case kTQ2_0: hipLaunchKernelGGL((k_mm<kTQ2_0, MODE>), grid, dim3(kThreads), 0, s, g); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// BRISK_HIP_PAIR_SPLIT=1: Q4_K gate and up as two launches (the gate rows stored, then read back).
static bool pair_split() {
    const char* e = std::getenv("BRISK_HIP_PAIR_SPLIT");
    return e != nullptr && std::string(e) == "1";
}

hipError_t launch_mm(const MmArgs& g, int mode, hipStream_t s) {
    if (g.ntok <= 0) return hipSuccess;
    // rows of whole 256-value chunks; the 32-value-block formats (k_mm) also take a partial last chunk
    const bool small_blocks = g.m.type == kQ4_0 || g.m.type == kQ4_1 || g.m.type == kQ5_0 || g.m.type == kQ8_0;
    if ((g.m.cols % kChunkCols != 0 && !(small_blocks && g.m.cols % 32 == 0)) || g.x.stride % kChunkCols != 0 ||
        static_cast<size_t>(g.x.stride) < g.m.cols)
        return hipErrorInvalidValue;
    if (mode == kMmPair && (g.m2.type != g.m.type || g.m2.rows != g.m.rows || g.m2.cols != g.m.cols)) return hipErrorInvalidValue;
    switch (mode) {
        case kMmStore: return mm_dispatch<kMmStore>(g, s);
        case kMmAdd: return mm_dispatch<kMmAdd>(g, s);
        case kMmPair: {
            if (g.m.type == kQ4_K && g.qx == nullptr && g.qx2 == nullptr && !pair_split()) {  // one fused launch
                const int row_tiles = static_cast<int>((g.m.rows + 63) / 64);
                int kq_g = 4;
                while (kq_g > 1 && row_tiles * ((g.ntok + 16 * kq_g - 1) / (16 * kq_g)) < kKqCus) kq_g /= 2;
                const dim3 grid(row_tiles, (g.ntok + 16 * kq_g - 1) / (16 * kq_g));
                if (kq_g == 4) hipLaunchKernelGGL(k_mmk_pair<4>, grid, dim3(kThreads), 0, s, g);
                else if (kq_g == 2) hipLaunchKernelGGL(k_mmk_pair<2>, grid, dim3(kThreads), 0, s, g);
                else hipLaunchKernelGGL(k_mmk_pair<1>, grid, dim3(kThreads), 0, s, g);
                return hipGetLastError();
            }
            // the gate rows into out, then up with the gated epilogue
            const hipError_t e = mm_dispatch<kMmStore>(g, s);
            if (e != hipSuccess) return e;
            MmArgs up = g;
            up.m = g.m2;
            up.qx = g.qx2;
            up.qxd = g.qxd2;
            up.qxm = g.qxm2;
            return mm_dispatch<kMmGated>(up, s);
        }
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_mm_two(const MmArgs& a, const MmArgs& b, hipStream_t s) {
    if (a.ntok <= 0) return hipSuccess;
    const bool fuse = a.m.type == kQ4_K && b.m.type == kQ4_K && a.m.cols == b.m.cols && a.qx == nullptr && b.qx == nullptr &&
                      a.ntok == b.ntok && a.x.qs == b.x.qs && a.m.cols % kChunkCols == 0 && a.x.stride % kChunkCols == 0;
    if (!fuse) {
        const hipError_t e = launch_mm(a, kMmStore, s);
        return e != hipSuccess ? e : launch_mm(b, kMmStore, s);
    }
    // the widest token tile that still gives a workgroup to every CU, over both matrices' row tiles
    const int row_tiles = static_cast<int>((a.m.rows + 63) / 64 + (b.m.rows + 63) / 64);
    int kq_g = 4;
    while (kq_g > 1 && row_tiles * ((a.ntok + 16 * kq_g - 1) / (16 * kq_g)) < kKqCus) kq_g /= 2;
    const dim3 grid(row_tiles, (a.ntok + 16 * kq_g - 1) / (16 * kq_g));
    if (kq_g == 4) hipLaunchKernelGGL((k_mmk<kQ4_K, kMmStore, 4, true>), grid, dim3(kThreads), 0, s, a, b);
    else if (kq_g == 2) hipLaunchKernelGGL((k_mmk<kQ4_K, kMmStore, 2, true>), grid, dim3(kThreads), 0, s, a, b);
    else hipLaunchKernelGGL((k_mmk<kQ4_K, kMmStore, 1, true>), grid, dim3(kThreads), 0, s, a, b);
    return hipGetLastError();
}

static bool mx_km(uint32_t type) { return type == kQ4_K || type == kQ5_K; }

bool mx_expanded(uint32_t type) {
    const char* off = std::getenv("BRISK_HIP_PREFILL_MX");  // "0": every format on the packed-plane GEMMs
    if (off != nullptr && std::string(off) == "0") return false;
    if (type == kQ6_K || type == kQ5_K) return true;
    const char* e = std::getenv("BRISK_HIP_PREFILL_Q4X");
    return type == kQ4_K && e != nullptr && std::string(e) == "1";
}

size_t mx_bytes(uint32_t type, uint32_t rows, uint32_t cols) {
    const size_t rp = (rows + kMxRows - 1) / kMxRows * kMxRows, nsb = cols / 256;
    const size_t q = rp * cols * 2, d = align256(rp * nsb * (mx_km(type) ? 2 : 1) * 4);
    return q + d + (mx_km(type) ? align256(rp * nsb * 8) : 0);
}

hipError_t launch_mx_expand(const Packed& m, void* mem, MxPlanes* out, hipStream_t s) {
    if ((m.type != kQ6_K && !mx_km(m.type)) || m.cols % 256 != 0) return hipErrorInvalidValue;
    const size_t rp = (m.rows + kMxRows - 1) / kMxRows * kMxRows, nsb = m.cols / 256;
    int8_t* qq = static_cast<int8_t*>(mem);
    float* dd = reinterpret_cast<float*>(qq + rp * m.cols * 2);
    uint8_t* mm = reinterpret_cast<uint8_t*>(dd) + align256(rp * nsb * 2 * 4);
    const size_t threads = rp / 32 * nsb * 512;
    const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
    if (m.type == kQ6_K) {
        hipLaunchKernelGGL(k_q6x_expand, grid, dim3(256), 0, s, m, qq, dd, static_cast<uint32_t>(rp / 32));
        mm = nullptr;
    } else {
        hipLaunchKernelGGL(k_kmx_expand, grid, dim3(256), 0, s, m, qq, dd, mm, static_cast<uint32_t>(rp / 32));
    }
    out->q = qq;
    out->d = dd;
    out->mn = mm;
    return hipGetLastError();
}

hipError_t launch_pre_quant(const float* x, int xstride, const float* w, float eps, int cols, int ntok, bool q8k, int bits,
                            const ActPlanar& out, hipStream_t s) {
    if (ntok <= 0) return hipSuccess;
    if (cols % 256 != 0) {  // a workgroup a row (rows of whole 32-value blocks, up to kMaxCols)
        hipLaunchKernelGGL(k_pre_quant, dim3(ntok), dim3(kThreads), 0, s, x, xstride, w, eps, cols, q8k ? 1 : 0, bits, out);
        return hipGetLastError();
    }
    if (w != nullptr) {
        if (q8k) hipLaunchKernelGGL(k_pre_quant_norm<true>, dim3(ntok), dim3(kThreads), 0, s, x, xstride, w, eps, cols, bits, out);
        else hipLaunchKernelGGL(k_pre_quant_norm<false>, dim3(ntok), dim3(kThreads), 0, s, x, xstride, w, eps, cols, bits, out);
    } else {
        const size_t waves = static_cast<size_t>(ntok) * (cols / 256);
        const dim3 grid(static_cast<unsigned>((waves + 3) / 4));
        if (q8k) hipLaunchKernelGGL(k_pre_quant_blocks<true>, grid, dim3(kThreads), 0, s, x, xstride, cols, bits, out, ntok);
        else hipLaunchKernelGGL(k_pre_quant_blocks<false>, grid, dim3(kThreads), 0, s, x, xstride, cols, bits, out, ntok);
    }
    return hipGetLastError();
}

hipError_t launch_pre_planar(const void* xq, int cols, int ntok, bool q8k, const ActPlanar& out, hipStream_t s) {
    if (ntok <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_pre_planar, dim3(ntok), dim3(64), 0, s, static_cast<const uint8_t*>(xq), cols, q8k ? 1 : 0, out);
    return hipGetLastError();
}

hipError_t launch_pre_embed(const Packed& m, const int* seq, int pos0, int ntok, float* h, float scale, hipStream_t s) {
    if (ntok <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_pre_embed, dim3(ntok), dim3(kThreads), 0, s, m, seq, pos0, h, scale);
    return hipGetLastError();
}

hipError_t launch_pre_post_add(float* h, const float* p, const float* w, float eps, int n, int ntok, hipStream_t s, float out_scale) {
    if (ntok <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_pre_post_add, dim3(ntok), dim3(kThreads), 0, s, h, p, w, eps, n, out_scale);
    return hipGetLastError();
}

hipError_t launch_pre_scale(float* h, float out_scale, int n, int ntok, hipStream_t s) {
    const size_t count = static_cast<size_t>(n) * ntok;
    if (count == 0) return hipSuccess;
    hipLaunchKernelGGL(k_pre_scale, dim3(static_cast<unsigned>((count + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, h, out_scale,
                       count);
    return hipGetLastError();
}

hipError_t launch_pre_ple_inputs(float* in, const Packed& table, const float* norm, const int* seq, int pos0, int ntok, int layers,
                                 int dim, float proj_scale, float table_scale, float eps, hipStream_t s) {
    if (ntok <= 0) return hipSuccess;
    if (layers < 1 || dim < 1 || static_cast<size_t>(layers) * dim != table.cols) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pre_ple_inputs, dim3(static_cast<unsigned>(layers), static_cast<unsigned>(ntok)), dim3(kThreads), 0, s, in,
                       table, norm, seq, pos0, layers, dim, proj_scale, table_scale, eps);
    return hipGetLastError();
}

hipError_t launch_pre_gelu_mul(float* g, const float* in, int n, int in_stride, int ntok, hipStream_t s) {
    const size_t count = static_cast<size_t>(n) * ntok;
    if (count == 0) return hipSuccess;
    hipLaunchKernelGGL(k_pre_gelu_mul, dim3(static_cast<unsigned>((count + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, g, in, n,
                       in_stride, ntok);
    return hipGetLastError();
}

hipError_t launch_pre_conv(const float* bcx, uint16_t* cache, const float* w, int taps, int pos0, int n, int ntok, float* out,
                           hipStream_t s) {
    if (ntok <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_pre_conv, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, bcx, cache,
                       w, taps, pos0, n, ntok, out);
    return hipGetLastError();
}

hipError_t launch_softcap(float* x, size_t n, float cap, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_softcap, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, x, n, cap);
    return hipGetLastError();
}

hipError_t launch_pre_attention(const PreAttnArgs& p, int ntok, hipStream_t s, bool* quantised) {
    if (quantised != nullptr) *quantised = false;
    if (ntok <= 0) return hipSuccess;
    const dim3 grid(ntok, p.a.kv_heads);
    if (p.a.heads / p.a.kv_heads > kRopeMaxHeads || p.a.head_dim > 128 || p.a.rope_dim > 128) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pre_rope, grid, dim3(kThreads), 0, s, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int hpk = p.a.heads / p.a.kv_heads, hd = p.a.head_dim;
    const int L = p.pos0 + ntok;
    const bool fa_ok = pre_attn_mfma_fits(hpk, hd);
    if (p.mfma && p.a.window == 0 && fa_ok && (ntok >= kFaMinTok || L * hpk > kExactScores)) {
        const dim3 fgrid(((ntok + kFaRows / hpk - 1) / (kFaRows / hpk)) * p.a.kv_heads);
        if (hd == 64) hipLaunchKernelGGL(k_pre_attn_fa<64>, fgrid, dim3(kThreads), 0, s, p, ntok);
        else hipLaunchKernelGGL(k_pre_attn_fa<128>, fgrid, dim3(kThreads), 0, s, p, ntok);
    } else if (!p.legacy && (hd == 64 || hd == 128) && hpk <= kPxRows && kPxRows % hpk == 0 && L <= kPaMaxL) {
        const dim3 xgrid(((ntok + kPxRows / hpk - 1) / (kPxRows / hpk)) * p.a.kv_heads);
        if (hd == 64) hipLaunchKernelGGL((k_pre_attn_rows<64, kPxRows, kPaMaxL>), xgrid, dim3(kThreads), 0, s, p, ntok);
        else hipLaunchKernelGGL((k_pre_attn_rows<128, kPxRows, kPaMaxL>), xgrid, dim3(kThreads), 0, s, p, ntok);
        if (quantised != nullptr) *quantised = p.qout.qs != nullptr && hpk * hd == 256;
    } else if (p.a.window == 0 && hpk <= kPaRows && (p.a.head_dim == 32 || p.a.head_dim == 64 || p.a.head_dim == 128) &&
        p.pos0 + ntok <= kPaMaxL) {
        const int tpb = kPaRows / hpk;
        hipLaunchKernelGGL(k_pre_attn_blk, dim3((ntok + tpb - 1) / tpb, p.a.kv_heads), dim3(kThreads), 0, s, p, ntok);
    } else if (L * hpk <= kExactScores) {
        hipLaunchKernelGGL(k_pre_attn, grid, dim3(kThreads), 0, s, p);
    } else {
        return hipErrorInvalidValue;  // no prefill attention for this shape (the session decodes it token by token)
    }
    return hipGetLastError();
}

}  // namespace bh
