// Token-loop kernels for gfx950 (CDNA4): one workgroup of 256 threads
// (4 waves of 64) per tile throughout.
//
// The forward step of the reference's Session::eval_batch (src/model.cpp:867-1212)
// maps onto these launches per layer:
//   k_qkv      attn_norm -> Q8 quantise -> Q/K/V rows of one head -> (Q/K norm) ->
//              RoPE -> q out / fp16 K,V cache write              (:996-1046)
//   k_attn / k_attn_combine   split-K decode attention             (:1050-1093)
//   k_gemv     (sub-norm) -> quantise -> O rows -> residual add     (:1095-1111)
//   k_gateup   ffn_norm -> quantise -> gate+up rows -> SiLU / relu^2 gate (:1111-1143)
//   k_gemv     (sub-norm) -> quantise -> down rows -> residual add  (:1144-1162)
// then k_gemv (output_norm -> output rows) and k_argmax.
#include "launch.h"

namespace bh {

// ============================================================== repack (load time)

// GGUF blocks -> planes (layout.h).  One thread per block; bytes inside each run unchanged.
__global__ void k_pack(uint32_t type, const uint8_t* __restrict__ src, size_t blocks, uint8_t* __restrict__ p0,
                       uint8_t* __restrict__ p1, uint8_t* __restrict__ p2) {
    const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    switch (type) {
        case kQ4_0: {
            const uint8_t* s = src + b * 18;
            p1[2 * b] = s[0]; p1[2 * b + 1] = s[1];
            for (int i = 0; i < 16; ++i) p0[b * 16 + i] = s[2 + i];
            break;
        }
        case kQ8_0: {
            const uint8_t* s = src + b * 34;
            p1[2 * b] = s[0]; p1[2 * b + 1] = s[1];
            for (int i = 0; i < 32; ++i) p0[b * 32 + i] = s[2 + i];
            break;
        }
        case kQ4_K: {  // {d, dmin, scales[12]} then qs[128]
            const uint8_t* s = src + b * 144;
            for (int i = 0; i < 16; ++i) p1[b * 16 + i] = s[i];
            for (int i = 0; i < 128; ++i) p0[b * 128 + i] = s[16 + i];
            break;
        }
        case kQ6_K: {  // ql[128], qh[64], scales[16], d
            const uint8_t* s = src + b * 210;
            for (int i = 0; i < 128; ++i) p0[b * 128 + i] = s[i];
            for (int i = 0; i < 64; ++i) p1[b * 64 + i] = s[128 + i];
            for (int i = 0; i < 18; ++i) p2[b * 20 + i] = s[192 + i];
            p2[b * 20 + 18] = 0; p2[b * 20 + 19] = 0;
            break;
        }
        case kTQ2_0: {  // qs[64], d
            const uint8_t* s = src + b * 66;
            for (int i = 0; i < 64; ++i) p0[b * 64 + i] = s[i];
            p1[2 * b] = s[64]; p1[2 * b + 1] = s[65];
            break;
        }
        default: break;
    }
}

// ============================================================== activation preparation

// The activation row of a tile: x, or rms_norm(x, w) when w is given, quantised to
// the family `m` takes, into LDS.  Ends with a barrier.
__device__ inline void prepare_act(const Packed& m, const float* x, const float* w, float eps, int cols, ActLds& a,
                                   double* red) {
    float scale = 1.0f;
    if (w != nullptr) scale = rms_scale(block_sumsq(x, cols, red), cols, eps);
    if (takes_q8_k(m.type)) act_q8_k(x, w, scale, cols, act_bits(m), a);
    else act_q8_0(x, w, scale, cols, a);
    __syncthreads();
}

constexpr int kTermCap = 8448;  // floats of LDS for per-block terms of one tile

// ============================================================== ABI: quantise, matvec

__global__ void k_quant_q8_0(const float* __restrict__ x, uint8_t* __restrict__ out, size_t count) {
    __shared__ ActLds a;
    const size_t off = static_cast<size_t>(blockIdx.x) * kMaxCols;
    const int len = static_cast<int>(count - off < kMaxCols ? count - off : kMaxCols);
    act_q8_0(x + off, nullptr, 1.0f, len, a);
    __syncthreads();
    const int8_t* xs = reinterpret_cast<const int8_t*>(a.xs);
    for (int b = threadIdx.x; b < len / 32; b += kThreads) {
        uint8_t* o = out + (off / 32 + b) * 34;
        const uint16_t d = f2h(a.xd[b]);
        o[0] = static_cast<uint8_t>(d); o[1] = static_cast<uint8_t>(d >> 8);
        for (int i = 0; i < 32; ++i) o[2 + i] = static_cast<uint8_t>(xs[b * 32 + i]);
    }
}

__global__ void k_quant_q8_k(const float* __restrict__ x, uint8_t* __restrict__ out, size_t count, int bits) {
    __shared__ ActLds a;
    const size_t off = static_cast<size_t>(blockIdx.x) * kMaxCols;
    const int len = static_cast<int>(count - off < kMaxCols ? count - off : kMaxCols);
    act_q8_k(x + off, nullptr, 1.0f, len, bits, a);
    __syncthreads();
    const int8_t* xs = reinterpret_cast<const int8_t*>(a.xs);
    for (int b = threadIdx.x; b < len / 256; b += kThreads) {
        uint8_t* o = out + (off / 256 + b) * 292;
        *reinterpret_cast<float*>(o) = a.xd[b];
        for (int i = 0; i < 256; ++i) o[4 + i] = static_cast<uint8_t>(xs[b * 256 + i]);
        for (int g = 0; g < 16; ++g) *reinterpret_cast<int16_t*>(o + 260 + 2 * g) = static_cast<int16_t>(a.xsum[b * 16 + g]);
    }
}

// KernelSet::matvec / matmul (src/kernels.h:19-25) on GGUF-layout quantised
// activations: out[t * out_stride + r] = dot(row r, x row t).  Grid (tiles, n).
__global__ void k_matvec_q8(Packed m, int R, const uint8_t* __restrict__ xq, float* __restrict__ out, size_t out_stride) {
    __shared__ ActLds a;
    __shared__ float terms[kTermCap];
    __shared__ float sums[64];
    const int t = blockIdx.y;
    if (takes_q8_k(m.type)) act_from_q8_k(xq + static_cast<size_t>(t) * (m.cols / 256) * 292, m.cols, a);
    else act_from_q8_0(xq + static_cast<size_t>(t) * (m.cols / 32) * 34, m.cols, a);
    __syncthreads();
    const uint32_t row0 = blockIdx.x * R;
    tile_rowsums(m, row0, R, a, terms, sums);
    if (threadIdx.x < static_cast<uint32_t>(R) && row0 + threadIdx.x < m.rows)
        out[t * out_stride + row0 + threadIdx.x] = sums[threadIdx.x];
}

// ============================================================== generic GEMV

// Up to three matrices sharing one activation row (the reference's fused
// multiply, src/model.cpp:551-653).  Epilogue: store, or add into out (the
// residual update h += W x, src/model.cpp:1111 and :1162).
__global__ void k_gemv(GemvArgs g) {
    __shared__ ActLds a;
    __shared__ float terms[kTermCap];
    __shared__ float sums[64];
    __shared__ double red[4];
    int tile = blockIdx.x, i = 0;
    while (i < g.n - 1 && tile >= g.t[i].tiles) tile -= g.t[i++].tiles;
    const GemvTarget& tg = g.t[i];
    prepare_act(tg.m, g.x, g.normw, g.eps, static_cast<int>(tg.m.cols), a, red);
    const uint32_t row0 = static_cast<uint32_t>(tile) * tg.R;
    tile_rowsums(tg.m, row0, tg.R, a, terms, sums);
    const uint32_t r = threadIdx.x;
    if (r < static_cast<uint32_t>(tg.R) && row0 + r < tg.m.rows) {
        if (g.add) tg.out[row0 + r] += sums[r];
        else tg.out[row0 + r] = sums[r];
    }
}

// ============================================================== Q/K/V with norms, RoPE, cache write

// One head's rows per workgroup: blocks [0, heads) are query heads, then key
// heads, then value heads.  Per head (src/model.cpp:1020-1046): optional
// RMS norm over head_dim (q_norm / k_norm), RoPE from the host-built table
// (build_rope, src/model.cpp:880-894, one row of head_dim floats per position),
// then q to `qout`, K and V to the fp16 caches at position *pos.
__global__ void k_qkv(QkvArgs g) {
    __shared__ ActLds a;
    __shared__ float terms[kTermCap];
    __shared__ float vals[256];
    __shared__ double red[4];
    const int hd = g.head_dim;
    int h = blockIdx.x, kind = 0;  // 0 = q, 1 = k, 2 = v
    if (h >= g.heads) { h -= g.heads; kind = 1; }
    if (kind == 1 && h >= g.kv_heads) { h -= g.kv_heads; kind = 2; }
    const Packed& m = kind == 0 ? g.q : kind == 1 ? g.k : g.v;
    prepare_act(m, g.x, g.normw, g.eps, static_cast<int>(m.cols), a, red);
    const int sub = hd > 64 ? 64 : hd;
    for (int r0 = 0; r0 < hd; r0 += sub) tile_rowsums(m, static_cast<uint32_t>(h * hd + r0), sub, a, terms, vals + r0);
    const int pos = *g.pos;
    const int t = threadIdx.x;
    if (kind == 2) {
        if (t < hd) g.vcache[(static_cast<size_t>(h) * g.ctx + pos) * hd + t] = f2h(vals[t]);
        return;
    }
    const float* nw = kind == 0 ? g.qnorm : g.knorm;
    float v = t < hd ? vals[t] : 0.0f;
    if (nw != nullptr) {
        const float s = rms_scale(block_sumsq(vals, hd, red), hd, g.eps);
        if (t < hd) v = v * s * nw[t];
        __syncthreads();
        if (t < hd) vals[t] = v;
        __syncthreads();
    }
    // apply_rope (src/model.cpp:104-115)
    const float* rope = g.rope + static_cast<size_t>(pos) * hd;
    const int half = hd / 2;
    if (t < half) {
        const float c = rope[2 * t], s = rope[2 * t + 1];
        const int ia = g.neox ? t : 2 * t, ib = g.neox ? t + half : 2 * t + 1;
        const float x0 = vals[ia], x1 = vals[ib];
        const float ra = x0 * c - x1 * s, rb = x0 * s + x1 * c;
        if (kind == 0) {
            g.qout[h * hd + ia] = ra;
            g.qout[h * hd + ib] = rb;
        } else {
            uint16_t* kr = g.kcache + (static_cast<size_t>(h) * g.ctx + pos) * hd;
            kr[ia] = f2h(ra);
            kr[ib] = f2h(rb);
        }
    }
}

// ============================================================== gate/up + activation

// Rows [i0, i0 + R) of the gate and of the up matrix in one workgroup, then
// act[i] = silu(gate) * up (src/kernels_f32.cpp:287-289: g / (1 + exp(-g)) * u)
// or, for BitNet, max(g, 0)^2 * up (src/model.cpp:1134-1138).
__global__ void k_gateup(GateUpArgs g) {
    __shared__ ActLds a;
    __shared__ float terms[kTermCap];
    __shared__ float sg[64], su[64];
    __shared__ double red[4];
    prepare_act(g.gate, g.x, g.normw, g.eps, static_cast<int>(g.gate.cols), a, red);
    const uint32_t row0 = blockIdx.x * g.R;
    tile_rowsums(g.gate, row0, g.R, a, terms, sg);
    tile_rowsums(g.up, row0, g.R, a, terms, su);
    const uint32_t r = threadIdx.x;
    if (r < static_cast<uint32_t>(g.R) && row0 + r < g.gate.rows) {
        const float gv = sg[r], uv = su[r];
        float out;
        if (g.relu2) {
            const float q = gv > 0.0f ? gv : 0.0f;
            out = q * q * uv;
        } else {
            out = gv / (1.0f + ref_expf(-gv)) * uv;
        }
        g.act[row0 + r] = out;
    }
}

// ============================================================== attention (decode)

constexpr int kSplit = 64;        // positions per split in the split-K path
constexpr int kExactMax = 512;    // contexts up to this length take the exact-order path

// The reference's attention for one token (src/model.cpp:1050-1093 with the
// portable kernels of src/kernels_f32.cpp:229-284), operation for operation,
// for the query heads of key/value head `kv`:
//   score_p = dot_f32(q, k_p) * scale, dot_f32 being 16 lane partials over
//             i = j (mod 16) in order, then 0 + lane 0 + ... + lane 15;
//   softmax: max, e_p = expf(s_p - max), sum of e_p in double, w_p = e_p * (float)(1 / sum);
//   out    = 0 + w_0 v_0 + w_1 v_1 + ... in position order (weighted_sum_f32's axpy).
// The one grouping that differs is the double sum, whose rounding reaches the
// float scale only when terms below 2^-20 of the sum lose bits.
__device__ void attn_exact(const AttnArgs& g, int kv, int L, float* qs, float* sc) {
    const int hd = g.head_dim, hpk = g.heads / g.kv_heads, t = threadIdx.x;
    const int lane16 = t & 15, pgrp = t >> 4, per = hd / 16;
    const uint16_t* kbase = g.kcache + static_cast<size_t>(kv) * g.ctx * hd;
    for (int p = pgrp; p < L; p += kThreads / 16) {
        const uint16_t* kr = kbase + static_cast<size_t>(p) * hd;
        float k[8];
        for (int m = 0; m < per; ++m) k[m] = h2f(kr[lane16 + 16 * m]);
        for (int gq = 0; gq < hpk; ++gq) {
            float lane = 0.0f;
            for (int m = 0; m < per; ++m) lane += qs[gq * hd + lane16 + 16 * m] * k[m];
            float sum = 0.0f;
            for (int j = 0; j < 16; ++j) sum += __shfl(lane, (t & ~15) + j, 64);
            if (lane16 == 0) sc[gq * kExactMax + p] = sum * g.scale;
        }
    }
    __syncthreads();
    __shared__ float wmax[16];
    __shared__ double wsum[16][4];
    const int wave = t >> 6, wl = t & 63;
    for (int gq = 0; gq < hpk; ++gq) {
        float m = -INFINITY;
        for (int p = t; p < L; p += kThreads) m = fmaxf(m, sc[gq * kExactMax + p]);
        m = wave_max(m);
        if (wl == 0) wsum[gq][wave] = static_cast<double>(m);
    }
    __syncthreads();
    if (t < hpk) wmax[t] = static_cast<float>(fmax(fmax(wsum[t][0], wsum[t][1]), fmax(wsum[t][2], wsum[t][3])));
    __syncthreads();
    for (int gq = 0; gq < hpk; ++gq) {
        double part = 0.0;
        for (int p = t; p < L; p += kThreads) {
            const float e = ref_expf(sc[gq * kExactMax + p] - wmax[gq]);
            sc[gq * kExactMax + p] = e;
            part += static_cast<double>(e);
        }
        part = wave_sum(part);
        __syncthreads();
        if (wl == 0) wsum[gq][wave] = part;
    }
    __syncthreads();
    for (int gq = 0; gq < hpk; ++gq) {
        const double sum = ((wsum[gq][0] + wsum[gq][1]) + wsum[gq][2]) + wsum[gq][3];
        const float scale = static_cast<float>(1.0 / sum);
        for (int p = t; p < L; p += kThreads) sc[gq * kExactMax + p] *= scale;
    }
    __syncthreads();
    const uint16_t* vbase = g.vcache + static_cast<size_t>(kv) * g.ctx * hd;
    for (int c = t; c < hpk * hd; c += kThreads) {
        const int gq = c / hd, d = c % hd;
        const float* w = sc + gq * kExactMax;
        float acc = 0.0f;
        int p = 0;
        for (; p + 4 <= L; p += 4) {
            const float v0 = h2f(vbase[static_cast<size_t>(p) * hd + d]);
            const float v1 = h2f(vbase[static_cast<size_t>(p + 1) * hd + d]);
            const float v2 = h2f(vbase[static_cast<size_t>(p + 2) * hd + d]);
            const float v3 = h2f(vbase[static_cast<size_t>(p + 3) * hd + d]);
            acc += w[p] * v0;
            acc += w[p + 1] * v1;
            acc += w[p + 2] * v2;
            acc += w[p + 3] * v3;
        }
        for (; p < L; ++p) acc += w[p] * h2f(vbase[static_cast<size_t>(p) * hd + d]);
        g.out[(kv * hpk + gq) * hd + d] = acc;
    }
}

// Split-K (flash-decoding) partials for contexts longer than kExactMax: each
// workgroup scores a split of kSplit positions for all the key/value head's
// query heads and keeps (max, sum of exp, exp-weighted value sum); the last
// workgroup of the head to finish merges the splits with the log-sum-exp
// rescale.  Same mathematics as the reference, different rounding order.
__device__ void attn_split(const AttnArgs& g, int kv, int split, int L, float* qs, float* sc, float* red) {
    const int hd = g.head_dim, hpk = g.heads / g.kv_heads, t = threadIdx.x;
    const int start = split * kSplit;
    const int lane16 = t & 15, pgrp = t >> 4, per = hd / 16;
    const uint16_t* kbase = g.kcache + static_cast<size_t>(kv) * g.ctx * hd;
    for (int pi = pgrp; pi < kSplit; pi += 16) {
        const int p = start + pi;
        float k[8];
        for (int m = 0; m < per; ++m) k[m] = p < L ? h2f(kbase[static_cast<size_t>(p) * hd + lane16 + 16 * m]) : 0.0f;
        for (int gq = 0; gq < hpk; ++gq) {
            float s = 0.0f;
            for (int m = 0; m < per; ++m) s += qs[gq * hd + lane16 + 16 * m] * k[m];
            s += __shfl_xor(s, 1, 64);
            s += __shfl_xor(s, 2, 64);
            s += __shfl_xor(s, 4, 64);
            s += __shfl_xor(s, 8, 64);
            if (lane16 == 0) sc[gq * kSplit + pi] = p < L ? s * g.scale : -INFINITY;
        }
    }
    __syncthreads();
    const int wave = t >> 6, lane = t & 63;
    __shared__ float ml[16][2];
    for (int gq = wave; gq < hpk; gq += 4) {
        const float sv = sc[gq * kSplit + lane];
        const float mx = wave_max(sv);
        const float e = (start + lane < L) ? ref_expf(sv - mx) : 0.0f;
        const float l = wave_sum(e);
        sc[gq * kSplit + lane] = e;
        if (lane == 0) { ml[gq][0] = mx; ml[gq][1] = l; }
    }
    __syncthreads();
    const int nparts = kThreads / hd, part = t / hd, d = t % hd;
    float acc[16];
    for (int gq = 0; gq < 16; ++gq) acc[gq] = 0.0f;
    const uint16_t* vbase = g.vcache + static_cast<size_t>(kv) * g.ctx * hd;
    const int cnt = L - start < kSplit ? L - start : kSplit;
    for (int pi = part; pi < cnt; pi += nparts) {
        const float v = h2f(vbase[static_cast<size_t>(start + pi) * hd + d]);
        for (int gq = 0; gq < hpk; ++gq) acc[gq] += sc[gq * kSplit + pi] * v;
    }
    for (int gq = 0; gq < hpk; ++gq) red[(part * hpk + gq) * hd + d] = acc[gq];
    __syncthreads();
    for (int i = t; i < hpk * hd; i += kThreads) {
        const int gq = i / hd, dd = i % hd;
        float sum = 0.0f;
        for (int pp = 0; pp < nparts; ++pp) sum += red[(pp * hpk + gq) * hd + dd];
        const size_t slot = static_cast<size_t>(kv * hpk + gq) * g.max_splits + split;
        g.part_acc[slot * hd + dd] = sum;
        if (dd == 0) {
            g.part_ml[slot * 2] = ml[gq][0];
            g.part_ml[slot * 2 + 1] = ml[gq][1];
        }
    }
    // the last split of this key/value head to finish merges them all
    __shared__ bool last;
    __threadfence();
    __syncthreads();
    const int ns = (L + kSplit - 1) / kSplit;
    if (t == 0) last = atomicAdd(g.tickets + kv, 1u) == static_cast<unsigned>(ns - 1);
    __syncthreads();
    if (!last) return;
    __threadfence();
    for (int i = t; i < hpk * hd; i += kThreads) {
        const int gq = i / hd, dd = i % hd;
        const size_t base = static_cast<size_t>(kv * hpk + gq) * g.max_splits;
        float M = -INFINITY;
        for (int s2 = 0; s2 < ns; ++s2) M = fmaxf(M, __builtin_nontemporal_load(g.part_ml + (base + s2) * 2));
        float num = 0.0f, den = 0.0f;
        for (int s2 = 0; s2 < ns; ++s2) {
            const float f = ref_expf(__builtin_nontemporal_load(g.part_ml + (base + s2) * 2) - M);
            den += __builtin_nontemporal_load(g.part_ml + (base + s2) * 2 + 1) * f;
            num += __builtin_nontemporal_load(g.part_acc + (base + s2) * hd + dd) * f;
        }
        g.out[(kv * hpk + gq) * hd + dd] = num / den;
    }
    if (t == 0) g.tickets[kv] = 0u;
}

// Grid (kv_heads, max_splits).  The context length comes from the device
// position, so one captured launch serves every step.
__global__ void k_attn(AttnArgs g) {
    __shared__ float qs[16 * 128];
    __shared__ float sc[16 * kExactMax];           // exact path: [head][position]; split path: [head][kSplit]
    __shared__ float red[4096];                    // (256 / head_dim) parts x 16 heads x head_dim
    const int kv = blockIdx.x, split = blockIdx.y;
    const int L = *g.pos + 1;
    const int hd = g.head_dim, hpk = g.heads / g.kv_heads;
    const bool exact = L <= kExactMax;
    if (exact ? split != 0 : split * kSplit >= L) return;
    for (int i = threadIdx.x; i < hpk * hd; i += kThreads) qs[i] = g.q[kv * hpk * hd + i];
    __syncthreads();
    if (exact) attn_exact(g, kv, L, qs, sc);
    else attn_split(g, kv, split, L, qs, sc, red);
}

// ============================================================== embedding, argmax, position

// embedding_row (src/model.cpp:27-70): dequantise row *token of the packed embedding.
__global__ void k_embed(Packed m, const int* __restrict__ seq, const int* __restrict__ pos, float* __restrict__ h) {
    const uint32_t r = static_cast<uint32_t>(seq[*pos]);
    const uint32_t cols = m.cols;
    for (uint32_t e = threadIdx.x; e < cols; e += kThreads) {
        float y = 0.0f;
        switch (m.type) {
            case kQ8_0: {
                const size_t blk = static_cast<size_t>(r) * (cols / 32) + e / 32;
                const float d = h2f(reinterpret_cast<const uint16_t*>(m.p1)[blk]);
                y = static_cast<float>(static_cast<int8_t>(m.p0[blk * 32 + e % 32])) * d;
                break;
            }
            case kQ4_0: {
                const size_t blk = static_cast<size_t>(r) * (cols / 32) + e / 32;
                const float d = h2f(reinterpret_cast<const uint16_t*>(m.p1)[blk]);
                const int i = e % 32;
                const uint8_t q = m.p0[blk * 16 + (i & 15)];
                y = static_cast<float>((i < 16 ? (q & 0x0F) : (q >> 4)) - 8) * d;
                break;
            }
            case kQ4_K: {
                const size_t blk = static_cast<size_t>(r) * (cols / 256) + e / 256;
                const uint8_t* meta = m.p1 + blk * 16;
                const float d = h2f(static_cast<uint16_t>(meta[0] | (meta[1] << 8)));
                const float dmin = h2f(static_cast<uint16_t>(meta[2] | (meta[3] << 8)));
                const int i = e % 256, chunk = i / 64, hi = (i % 64) >= 32, j = i % 32;
                int sc, mn;
                q4k_scale_min(meta + 4, 2 * chunk + hi, sc, mn);
                const float d1 = d * static_cast<float>(sc), m1 = dmin * static_cast<float>(mn);
                const uint8_t q = m.p0[blk * 128 + chunk * 32 + j];
                y = d1 * static_cast<float>(hi ? (q >> 4) : (q & 0xF)) - m1;
                break;
            }
            case kQ6_K: {
                const size_t blk = static_cast<size_t>(r) * (cols / 256) + e / 256;
                const int i = e % 256, half = i / 128, w = i % 128, quarter = w / 32, l = w % 32;
                const uint8_t* ql = m.p0 + blk * 128 + half * 64;
                const uint8_t* qh = m.p1 + blk * 64 + half * 32;
                const uint8_t* meta = m.p2 + blk * 20;
                const int lo = (quarter & 1) ? ql[l + 32] : ql[l];
                const int nib = quarter >= 2 ? (lo >> 4) : (lo & 0xF);
                const int q = (nib | (((qh[l] >> (2 * quarter)) & 3) << 4)) - 32;
                const float d = h2f(static_cast<uint16_t>(meta[16] | (meta[17] << 8)));
                y = d * static_cast<float>(static_cast<int8_t>(meta[i / 16])) * static_cast<float>(q);
                break;
            }
            default: {  // TQ2_0
                const size_t blk = static_cast<size_t>(r) * (cols / 256) + e / 256;
                const int i = e % 256;
                const int c = (m.p0[blk * 64 + (i / 128) * 32 + i % 32] >> (2 * ((i % 128) / 32))) & 3;
                y = static_cast<float>(c - 1) * h2f(reinterpret_cast<const uint16_t*>(m.p1)[blk]);
                break;
            }
        }
        h[e] = y;
    }
}

// Greedy pick (Sampler::sample at temperature <= 0, src/sampler.cpp:11-13):
// the first index of the largest logit.  Each workgroup reduces a chunk; the
// last one to finish (atomic ticket) reduces the partials in index order,
// writes the token, advances the position if asked, and re-arms the ticket.
__device__ __forceinline__ void better(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

__global__ void k_argmax(ArgmaxArgs g) {
    __shared__ float sv[4];
    __shared__ int si[4];
    __shared__ bool last;
    const int chunk = (g.n + gridDim.x - 1) / gridDim.x;
    const int b0 = blockIdx.x * chunk, b1 = b0 + chunk < g.n ? b0 + chunk : g.n;
    float v = -INFINITY;
    int idx = 0x7FFFFFFF;
    for (int i = b0 + threadIdx.x; i < b1; i += kThreads) better(v, idx, g.logits[i], i);
    for (int o = 32; o > 0; o >>= 1) better(v, idx, __shfl_xor(v, o, 64), __shfl_xor(idx, o, 64));
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = v; si[threadIdx.x >> 6] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) better(v, idx, sv[w], si[w]);
        g.part_v[blockIdx.x] = v;
        g.part_i[blockIdx.x] = idx;
        __threadfence();
        last = atomicAdd(g.ticket, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    v = -INFINITY;
    idx = 0x7FFFFFFF;
    for (int b = threadIdx.x; b < static_cast<int>(gridDim.x); b += kThreads) {
        const float pv = __builtin_nontemporal_load(g.part_v + b);
        const int pi = __builtin_nontemporal_load(g.part_i + b);
        better(v, idx, pv, pi);
    }
    for (int o = 32; o > 0; o >>= 1) better(v, idx, __shfl_xor(v, o, 64), __shfl_xor(idx, o, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = v; si[threadIdx.x >> 6] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) better(v, idx, sv[w], si[w]);
        const int p = *g.pos;
        // positions below *g.fixed hold the caller's tokens (a prompt being evaluated): keep them
        if (p + 1 < g.seq_len && p + 1 >= *g.fixed) g.seq[p + 1] = idx;
        if (g.advance) *g.pos = p + 1;
        *g.ticket = 0u;
    }
}

// expf as the token loop computes it (ref_expf), for the parity tests.
__global__ void k_expf(const float* __restrict__ x, float* __restrict__ y, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] = ref_expf(x[i]);
}

hipError_t launch_expf(const float* x, float* y, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_expf, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

__global__ void k_advance(int* pos) {
    if (threadIdx.x == 0) *pos += 1;
}

// ============================================================== launchers

static inline unsigned cdiv(size_t a, size_t b) { return static_cast<unsigned>((a + b - 1) / b); }

hipError_t launch_pack(uint32_t type, const void* src, size_t rows, size_t cols, const Packed& dst, hipStream_t s) {
    const size_t blocks = rows * (cols / block_elems(type));
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(k_pack, dim3(cdiv(blocks, 256)), dim3(256), 0, s, type, static_cast<const uint8_t*>(src), blocks,
                       const_cast<uint8_t*>(dst.p0), const_cast<uint8_t*>(dst.p1), const_cast<uint8_t*>(dst.p2));
    return hipGetLastError();
}

hipError_t launch_quantize(int kind, const float* x, void* out, size_t count, int bits, hipStream_t s) {
    if (count == 0) return hipSuccess;
    if (kind == 0) hipLaunchKernelGGL(k_quant_q8_0, dim3(cdiv(count, kMaxCols)), dim3(kThreads), 0, s, x, static_cast<uint8_t*>(out), count);
    else hipLaunchKernelGGL(k_quant_q8_k, dim3(cdiv(count, kMaxCols)), dim3(kThreads), 0, s, x, static_cast<uint8_t*>(out), count, bits);
    return hipGetLastError();
}

int pick_rows_per_tile(uint32_t type, size_t rows, size_t cols) {
    const size_t units = cols / block_elems(type);
    int R = 64;
    while (R > 1 && static_cast<size_t>(R) * (units + 1) > static_cast<size_t>(kTermCap)) R /= 2;
    while (R > 8 && (rows + R - 1) / R < 1024) R /= 2;
    return R;
}

hipError_t launch_matvec_q8(const Packed& m, const void* xq, size_t n, float* out, size_t out_stride, hipStream_t s) {
    const int R = pick_rows_per_tile(m.type, m.rows, m.cols);
    hipLaunchKernelGGL(k_matvec_q8, dim3(cdiv(m.rows, R), static_cast<unsigned>(n)), dim3(kThreads), 0, s, m, R,
                       static_cast<const uint8_t*>(xq), out, out_stride);
    return hipGetLastError();
}

hipError_t launch_gemv(GemvArgs g, hipStream_t s) {
    unsigned tiles = 0;
    for (int i = 0; i < g.n; ++i) {
        g.t[i].R = pick_rows_per_tile(g.t[i].m.type, g.t[i].m.rows, g.t[i].m.cols);
        g.t[i].tiles = static_cast<int>(cdiv(g.t[i].m.rows, g.t[i].R));
        tiles += static_cast<unsigned>(g.t[i].tiles);
    }
    hipLaunchKernelGGL(k_gemv, dim3(tiles), dim3(kThreads), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_qkv(const QkvArgs& g, hipStream_t s) {
    hipLaunchKernelGGL(k_qkv, dim3(g.heads + 2 * g.kv_heads), dim3(kThreads), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_gateup(GateUpArgs g, hipStream_t s) {
    const size_t units = g.gate.cols / block_elems(g.gate.type);
    int R = 64;
    while (R > 1 && static_cast<size_t>(R) * (units + 1) > static_cast<size_t>(kTermCap)) R /= 2;
    while (R > 8 && (g.gate.rows + R - 1) / R < 512) R /= 2;
    g.R = R;
    hipLaunchKernelGGL(k_gateup, dim3(cdiv(g.gate.rows, R)), dim3(kThreads), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& g, hipStream_t s) {
    hipLaunchKernelGGL(k_attn, dim3(g.kv_heads, g.max_splits), dim3(kThreads), 0, s, g);
    return hipGetLastError();
}

int attention_max_splits(int ctx) { return (ctx + kSplit - 1) / kSplit; }

hipError_t launch_embed(const Packed& m, const int* seq, const int* pos, float* h, hipStream_t s) {
    hipLaunchKernelGGL(k_embed, dim3(1), dim3(kThreads), 0, s, m, seq, pos, h);
    return hipGetLastError();
}

hipError_t launch_argmax(const ArgmaxArgs& g, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax, dim3(kArgmaxBlocks), dim3(kThreads), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_advance(int* pos, hipStream_t s) {
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, pos);
    return hipGetLastError();
}

}  // namespace bh
