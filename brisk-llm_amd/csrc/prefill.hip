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
// Q8_0: as stored; Q4_K: nibble 0..15 (the mins enter through the offsets);
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
    } else if (T == kQ4_K) {
        const uint32_t nsb = m.cols / 256, jj = j & 7;
        const size_t blk = static_cast<size_t>(row) * nsb + j / 8;
        const uint64_t w = ld8(m.p0 + blk * 128 + (jj >> 1) * 32 + kq);
        return (jj & 1) ? ((w >> 4) & (0x0F * kB01)) : (w & (0x0F * kB01));
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

// One wave: 16 rows x (16 * kGroups) tokens; a workgroup: 64 rows (4 waves) x the same tokens.
constexpr int kGroups = 4;
constexpr int kRowsPerWg = 64, kTokPerWg = 16 * kGroups;

// Per-lane accumulators of one matrix: [token group][row i].
struct MmAcc {
    float s[kGroups][4];
};

// The lane's outputs of W x for tokens t0 + 16 g + l % 16 and rows r0 + 4 (l / 16) + i.
template <uint32_t T>
__device__ __forceinline__ void mm_tile(const Packed& m, const ActPlanar& x, int ntok, uint32_t r0, int t0, MmAcc& acc) {
    const int lane = threadIdx.x & 63, kq = (lane >> 4) * 8;
    const uint32_t arow_raw = r0 + (lane & 15);
    const bool arow_ok = arow_raw < m.rows;
    const uint32_t arow = arow_ok ? arow_raw : m.rows - 1;
    uint32_t orow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t r = r0 + (lane >> 4) * 4 + i;
        orow[i] = r < m.rows ? r : m.rows - 1;  // clamped for the scale loads; not stored
    }
    int tok[kGroups];
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        const int t = t0 + 16 * g + (lane & 15);
        tok[g] = t < ntok ? t : ntok - 1;
    }
    const int8_t* xq = x.qs;
    const size_t xs = x.stride, ds = x.stride / 32, bss = x.stride / 16;
#pragma unroll
    for (int g = 0; g < kGroups; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc.s[g][i] = 0.0f;
    const v4i zero = {0, 0, 0, 0};

    if (T == kQ4_0 || T == kQ8_0) {
        const uint32_t nsub = m.cols / 32;
        const uint16_t* dw = reinterpret_cast<const uint16_t*>(m.p1);
        for (uint32_t j = 0; j < nsub; ++j) {
            const uint64_t a = arow_ok ? frag_a<T>(m, arow, j, kq) : 0ull;
            v4i d[kGroups];
#pragma unroll
            for (int g = 0; g < kGroups; ++g)
                d[g] = mfma(a, ld8(reinterpret_cast<const uint8_t*>(xq) + tok[g] * xs + j * 32 + kq), zero);
            float w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = h2f(dw[static_cast<size_t>(orow[i]) * nsub + j]);
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
                const float xd = x.d[tok[g] * ds + j];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc.s[g][i] += static_cast<float>(d[g][i]) * w[i] * xd;  // src/quant.cpp:445-482
            }
        }
    } else if (T == kQ4_K) {
        const uint32_t nsb = m.cols / 256;
        for (uint32_t sb = 0; sb < nsb; ++sb) {
            uint4 meta[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) meta[i] = *reinterpret_cast<const uint4*>(m.p1 + (static_cast<size_t>(orow[i]) * nsb + sb) * 16);
            int wsum[kGroups][4], osum[kGroups][4];
#pragma unroll
            for (int g = 0; g < kGroups; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i) wsum[g][i] = osum[g][i] = 0;
            for (uint32_t jj = 0; jj < 8; ++jj) {
                const uint32_t j = sb * 8 + jj;
                const uint64_t a = arow_ok ? frag_a<T>(m, arow, j, kq) : 0ull;
                int sc[4], mn[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t mw[4] = {meta[i].x, meta[i].y, meta[i].z, meta[i].w};
                    q4k_scale_min(reinterpret_cast<const uint8_t*>(mw) + 4, static_cast<int>(jj), sc[i], mn[i]);
                }
#pragma unroll
                for (int g = 0; g < kGroups; ++g) {
                    const v4i d = mfma(a, ld8(reinterpret_cast<const uint8_t*>(xq) + tok[g] * xs + j * 32 + kq), zero);
                    const int32_t* bs = x.bs + tok[g] * bss + sb * 16 + 2 * jj;
                    const int pair = bs[0] + bs[1];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        wsum[g][i] += sc[i] * d[i];
                        osum[g][i] += mn[i] * pair;
                    }
                }
            }
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
                const float xd = x.d[tok[g] * ds + sb];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float d = h2f(static_cast<uint16_t>(meta[i].x & 0xFFFF)), dmin = h2f(static_cast<uint16_t>(meta[i].x >> 16));
                    acc.s[g][i] += xd * (d * static_cast<float>(wsum[g][i]) - dmin * static_cast<float>(osum[g][i]));  // :500-521
                }
            }
        }
    } else if (T == kQ6_K) {
        const uint32_t nsb = m.cols / 256;
        const bool lo_half = lane < 32;  // lanes 0..31 hold k 0..15 of a sub-block, 32..63 hold k 16..31
        for (uint32_t sb = 0; sb < nsb; ++sb) {
            int wsum[kGroups][4];
#pragma unroll
            for (int g = 0; g < kGroups; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i) wsum[g][i] = 0;
            for (uint32_t jj = 0; jj < 8; ++jj) {
                const uint32_t j = sb * 8 + jj;
                const uint64_t a = arow_ok ? frag_a<T>(m, arow, j, kq) : 0ull;
                const uint64_t a0 = lo_half ? a : 0ull, a1 = lo_half ? 0ull : a;  // groups 2 jj and 2 jj + 1 of 16
                int s0[4], s1[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int8_t* sc = reinterpret_cast<const int8_t*>(m.p2 + (static_cast<size_t>(orow[i]) * nsb + sb) * 20);
                    s0[i] = sc[2 * jj];
                    s1[i] = sc[2 * jj + 1];
                }
#pragma unroll
                for (int g = 0; g < kGroups; ++g) {
                    const uint64_t b = ld8(reinterpret_cast<const uint8_t*>(xq) + tok[g] * xs + j * 32 + kq);
                    const v4i d0 = mfma(a0, b, zero), d1 = mfma(a1, b, zero);
#pragma unroll
                    for (int i = 0; i < 4; ++i) wsum[g][i] += s0[i] * d0[i] + s1[i] * d1[i];
                }
            }
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
                const float xd = x.d[tok[g] * ds + sb];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint8_t* mp = m.p2 + (static_cast<size_t>(orow[i]) * nsb + sb) * 20;
                    const float d = h2f(static_cast<uint16_t>(mp[16] | (mp[17] << 8)));
                    acc.s[g][i] += xd * d * static_cast<float>(wsum[g][i]);  // src/quant.cpp:549-563
                }
            }
        }
    } else {  // TQ2_0
        const uint32_t nsb = m.cols / 256;
        const bool lut16 = (m.flags & kFlagLut16) != 0;
        const uint16_t* dw = reinterpret_cast<const uint16_t*>(m.p1);
        for (uint32_t sb = 0; sb < nsb; ++sb) {
            v4i d[kGroups];
#pragma unroll
            for (int g = 0; g < kGroups; ++g) d[g] = zero;
            for (uint32_t jj = 0; jj < 8; ++jj) {  // the block's int32 sum over its 8 sub-blocks, exact
                const uint32_t j = sb * 8 + jj;
                const uint64_t a = arow_ok ? frag_a<T>(m, arow, j, kq) : 0ull;
#pragma unroll
                for (int g = 0; g < kGroups; ++g)
                    d[g] = mfma(a, ld8(reinterpret_cast<const uint8_t*>(xq) + tok[g] * xs + j * 32 + kq), d[g]);
            }
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
                const float xd = x.d[tok[g] * ds + sb];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float w = h2f(dw[static_cast<size_t>(orow[i]) * nsb + sb]);
                    const float a = static_cast<float>(d[g][i]);
                    acc.s[g][i] += lut16 ? a * w * xd : xd * w * a;  // src/quant.cpp:789-802 / :580-596
                }
            }
        }
    }
}

// out[t * ostride + r] (=, += or the gated pair) for a 64-row x 64-token tile.
template <uint32_t T, int MODE>
__global__ __launch_bounds__(kThreads) void k_mm(MmArgs g) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t r0 = blockIdx.x * kRowsPerWg + wave * 16;
    const int t0 = blockIdx.y * kTokPerWg;
    if (r0 >= g.m.rows) return;
    MmAcc a;
    mm_tile<T>(g.m, g.x, g.ntok, r0, t0, a);
    MmAcc u;
    if (MODE == kMmPair) mm_tile<T>(g.m2, g.x, g.ntok, r0, t0, u);
#pragma unroll
    for (int gi = 0; gi < kGroups; ++gi) {
        const int t = t0 + 16 * gi + (lane & 15);
        if (t >= g.ntok) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = r0 + (lane >> 4) * 4 + i;
            if (r >= g.m.rows) continue;
            float* o = g.out + static_cast<size_t>(t) * g.ostride + r;
            const float v = a.s[gi][i];
            if (MODE == kMmStore) {
                *o = v;
            } else if (MODE == kMmAdd) {
                *o = *o + v;  // h += proj (src/model.cpp:1111, :1162)
            } else {
                const float up = u.s[gi][i];
                if (g.relu2) {
                    const float q = v > 0.0f ? v : 0.0f;
                    *o = q * q * up;  // src/model.cpp:1134-1138
                } else {
                    *o = v / (1.0f + ref_expf(-v)) * up;  // src/kernels_f32.cpp:287-289
                }
            }
        }
    }
}

// ---------------------------------------------------------------- per-token work

// Embedding rows of seq[pos0 + t] (embedding_row, src/model.cpp:27-70).
__global__ void k_pre_embed(Packed m, const int* __restrict__ seq, int pos0, float* __restrict__ h) {
    const int t = blockIdx.x;
    const uint32_t tok = static_cast<uint32_t>(seq[pos0 + t]);
    float* row = h + static_cast<size_t>(t) * m.cols;
    for (uint32_t e = threadIdx.x; e < m.cols; e += blockDim.x) row[e] = dequant_elem(m, tok, e);
}

// Q/K norms, RoPE, and the K/V cache rows of token t (grid: tokens x kv heads);
// the normed, rotated queries go back to q.
__global__ __launch_bounds__(kThreads) void k_pre_rope(PreAttnArgs p) {
    __shared__ AttnLds s;
    const int t = blockIdx.x, kv = blockIdx.y, pos = p.pos0 + t;
    AttnArgs g = p.a;
    g.q = p.q + static_cast<size_t>(t) * p.qstride;
    g.k = p.k + static_cast<size_t>(t) * p.kvstride;
    g.v = p.v + static_cast<size_t>(t) * p.kvstride;
    attn_load_raw<PlainIO>(g, s, kv, true);
    attn_finish_prologue<false>(g, s, kv, pos, true, true);
    const int hpk = g.heads / g.kv_heads, hd = g.head_dim;
    float* q = p.q + static_cast<size_t>(t) * p.qstride + kv * hpk * hd;
    for (int i = threadIdx.x; i < hpk * hd; i += kThreads) q[i] = s.q[i];
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
    attn_exact(g, s, kv, pos + 1, o);
}

// ---------------------------------------------------------------- launchers

template <int MODE>
static hipError_t mm_dispatch(const MmArgs& g, hipStream_t s) {
    const dim3 grid((g.m.rows + kRowsPerWg - 1) / kRowsPerWg, (g.ntok + kTokPerWg - 1) / kTokPerWg);
    switch (g.m.type) {
        case kQ4_0: hipLaunchKernelGGL((k_mm<kQ4_0, MODE>), grid, dim3(kThreads), 0, s, g); break;
        case kQ8_0: hipLaunchKernelGGL((k_mm<kQ8_0, MODE>), grid, dim3(kThreads), 0, s, g); break;
        case kQ4_K: hipLaunchKernelGGL((k_mm<kQ4_K, MODE>), grid, dim3(kThreads), 0, s, g); break;
        case kQ6_K: hipLaunchKernelGGL((k_mm<kQ6_K, MODE>), grid, dim3(kThreads), 0, s, g); break;
        case kTQ2_0: hipLaunchKernelGGL((k_mm<kTQ2_0, MODE>), grid, dim3(kThreads), 0, s, g); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_mm(const MmArgs& g, int mode, hipStream_t s) {
    if (g.ntok <= 0) return hipSuccess;
    if (mode == kMmPair && (g.m2.type != g.m.type || g.m2.rows != g.m.rows || g.m2.cols != g.m.cols)) return hipErrorInvalidValue;
    switch (mode) {
        case kMmStore: return mm_dispatch<kMmStore>(g, s);
        case kMmAdd: return mm_dispatch<kMmAdd>(g, s);
        case kMmPair: return mm_dispatch<kMmPair>(g, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_pre_quant(const float* x, int xstride, const float* w, float eps, int cols, int ntok, bool q8k, int bits,
                            const ActPlanar& out, hipStream_t s) {
    if (ntok <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_pre_quant, dim3(ntok), dim3(kThreads), 0, s, x, xstride, w, eps, cols, q8k ? 1 : 0, bits, out);
    return hipGetLastError();
}

hipError_t launch_pre_planar(const void* xq, int cols, int ntok, bool q8k, const ActPlanar& out, hipStream_t s) {
    if (ntok <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_pre_planar, dim3(ntok), dim3(64), 0, s, static_cast<const uint8_t*>(xq), cols, q8k ? 1 : 0, out);
    return hipGetLastError();
}

hipError_t launch_pre_embed(const Packed& m, const int* seq, int pos0, int ntok, float* h, hipStream_t s) {
    if (ntok <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_pre_embed, dim3(ntok), dim3(kThreads), 0, s, m, seq, pos0, h);
    return hipGetLastError();
}

hipError_t launch_pre_attention(const PreAttnArgs& p, int ntok, hipStream_t s) {
    if (ntok <= 0) return hipSuccess;
    const dim3 grid(ntok, p.a.kv_heads);
    hipLaunchKernelGGL(k_pre_rope, grid, dim3(kThreads), 0, s, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_pre_attn, grid, dim3(kThreads), 0, s, p);
    return hipGetLastError();
}

}  // namespace bh
