// Token-loop kernels for gfx950 (CDNA4): one workgroup of 256 threads
// (4 waves of 64) per tile throughout.
//
// The forward step of the reference's Session::eval_batch (src/model.cpp:867-1212)
// maps onto these launches per layer:
//   k_gemv     attn_norm -> Q8 quantise -> Q, K, V rows                (:996-1015)
//   k_attn     Q/K norms, RoPE, fp16 K/V cache write, attention         (:1020-1093)
//   k_gemv     (sub-norm) -> quantise -> O rows -> residual add         (:1095-1111)
//   k_gateup   ffn_norm -> quantise -> gate+up rows -> SiLU / relu^2    (:1111-1143)
//   k_gemv     (sub-norm) -> quantise -> down rows -> residual add      (:1144-1162)
// then k_head: output_norm -> output rows -> logits and the greedy pick.
#include "phases.h"

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
        case kQ4_1: {  // d, m, qs[16]
            const uint8_t* s = src + b * 20;
            p1[2 * b] = s[0]; p1[2 * b + 1] = s[1];
            p2[2 * b] = s[2]; p2[2 * b + 1] = s[3];
            for (int i = 0; i < 16; ++i) p0[b * 16 + i] = s[4 + i];
            break;
        }
        case kQ5_0: {  // d, qh[4], qs[16]
            const uint8_t* s = src + b * 22;
            p1[2 * b] = s[0]; p1[2 * b + 1] = s[1];
            for (int i = 0; i < 4; ++i) p2[b * 4 + i] = s[2 + i];
            for (int i = 0; i < 16; ++i) p0[b * 16 + i] = s[6 + i];
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
            for (int j = 0; j < 8; ++j) {  // q4_k_scale_min decoded once (src/quant.h:256-264)
                int sc, mn;
                q4k_scale_min(s + 4, j, sc, mn);
                p2[b * 16 + j] = static_cast<uint8_t>(sc);
                p2[b * 16 + 8 + j] = static_cast<uint8_t>(mn);
            }
            break;
        }
        case kQ5_K: {  // {d, dmin, scales[12]}, qh[32], qs[128]
            const uint8_t* s = src + b * 176;
            for (int i = 0; i < 16; ++i) p1[b * 16 + i] = s[i];
            for (int i = 0; i < 128; ++i) p0[b * 128 + i] = s[48 + i];
            for (int j = 0; j < 8; ++j) {
                int sc, mn;
                q4k_scale_min(s + 4, j, sc, mn);
                p2[b * 48 + j] = static_cast<uint8_t>(sc);
                p2[b * 48 + 8 + j] = static_cast<uint8_t>(mn);
            }
            for (int i = 0; i < 32; ++i) p2[b * 48 + 16 + i] = s[16 + i];
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

constexpr int kMinTiles = 256;  // spread every matrix over at least one workgroup per CU

// ============================================================== ABI: quantise, matvec

__global__ __launch_bounds__(kThreads) void k_quant_q8_0(const float* __restrict__ x, uint8_t* __restrict__ out, size_t count) {
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

__global__ __launch_bounds__(kThreads) void k_quant_q8_k(const float* __restrict__ x, uint8_t* __restrict__ out, size_t count, int bits) {
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
template <uint32_t T>
__global__ __launch_bounds__(kThreads) void k_matvec_q8(Packed m, int R, const uint8_t* __restrict__ xq, float* __restrict__ out, size_t out_stride) {
    __shared__ ActLds a;
    __shared__ __align__(16) float terms[kTermCap];
    __shared__ float sums[64];
    Tile<T> tile;
    tile.load(m, blockIdx.x * R, R);
    const int t = blockIdx.y;
    if (takes_q8_k(T)) act_from_q8_k(xq + static_cast<size_t>(t) * (m.cols / 256) * 292, m.cols, a);
    else act_from_q8_0(xq + static_cast<size_t>(t) * (m.cols / 32) * 34, m.cols, a);
    __syncthreads();
    tile.sums(m, a, terms, sums);
    const uint32_t row0 = blockIdx.x * R;
    if (threadIdx.x < static_cast<uint32_t>(R) && row0 + threadIdx.x < m.rows)
        out[t * out_stride + row0 + threadIdx.x] = sums[threadIdx.x];
}

// ============================================================== GEMV (decode)

// Up to three matrices of one format sharing one activation row (the
// reference's fused multiply, src/model.cpp:551-653).  Weight loads are issued
// first; the activation prologue (rms_norm + quantisation of x, when normw is
// given) runs while they are in flight.  Epilogue: store, or add into out (the
// residual update h += W x, src/model.cpp:1111 and :1162).
template <uint32_t T>
__global__ __launch_bounds__(kThreads) void k_gemv(GemvArgs g) {
    __shared__ ActLds a;
    __shared__ __align__(16) float terms[kTermCap];
    __shared__ float sums[64];
    __shared__ double red[4];
    int tile_id = blockIdx.x, i = 0;
    while (i < g.n - 1 && tile_id >= g.t[i].tiles) tile_id -= g.t[i++].tiles;
    const GemvTarget& tg = g.t[i];
    const int cols = static_cast<int>(tg.m.cols);
    ActRegs ar;
    act_issue(ar, g.x, g.normw, cols);
    Tile<T> tile;
    tile.load(tg.m, static_cast<uint32_t>(tile_id) * tg.R, tg.R);
    act_finish(ar, g.x, g.normw, g.eps, cols, takes_q8_k(T), act_bits(tg.m), a, red);
    tile.sums(tg.m, a, terms, sums);
    const uint32_t r = threadIdx.x, row = tile.row0 + r;
    if (r < static_cast<uint32_t>(tg.R) && row < tg.m.rows) {
        if (g.gelu_in != nullptr) tg.out[row] = gelu_mul(sums[r], g.gelu_in[row]);
        else if (g.add) tg.out[row] += sums[r];
        else tg.out[row] = sums[r];
    }
}

// Rows [i0, i0 + R) of the gate and of the up matrix in one workgroup, then
// act[i] = silu(gate) * up (src/kernels_f32.cpp:287-289: g / (1 + exp(-g)) * u)
// or, for BitNet, max(g, 0)^2 * up (src/model.cpp:1134-1138).
template <uint32_t T>
__global__ __launch_bounds__(kThreads) void k_gateup(GateUpArgs g) {
    __shared__ ActLds a;
    __shared__ __align__(16) float terms[kTermCap];
    __shared__ float sg[64], su[64];
    __shared__ double red[4];
    const uint32_t row0 = blockIdx.x * g.R;
    const int cols = static_cast<int>(g.gate.cols);
    ActRegs ar;
    act_issue(ar, g.x, g.normw, cols);
    Tile<T, (Unit<T>::kMaxPerThread + 1) / 2> tg, tu;
    tg.load(g.gate, row0, g.R);
    tu.load(g.up, row0, g.R);
    act_finish(ar, g.x, g.normw, g.eps, cols, takes_q8_k(T), act_bits(g.gate), a, red);
    tg.sums(g.gate, a, terms, sg);
    tu.sums(g.up, a, terms, su);
    const uint32_t r = threadIdx.x;
    if (r < static_cast<uint32_t>(g.R) && row0 + r < g.gate.rows) {
        const float gv = sg[r], uv = su[r];
        float out;
        if (g.relu2) {
            const float q = gv > 0.0f ? gv : 0.0f;
            out = q * q * uv;
        } else if (g.gelu) {
            out = gelu_mul(gv, uv);
        } else {
            out = gv / (1.0f + ref_expf(-gv)) * uv;
        }
        g.act[row0 + r] = out;
    }
}

// ============================================================== output projection + greedy pick

// output_norm -> quantise -> output rows (src/model.cpp:1201-1205) -> logits,
// and each workgroup's best (logit, index) folded into the step's pick key with
// an atomicMax -- issued only when it would raise the key, so most workgroups
// issue none.  The pick stays pending until finalize_pick (next kernel on).
template <uint32_t T>
__global__ __launch_bounds__(kThreads) void k_head(HeadArgs g) {
    __shared__ ActLds a;
    __shared__ __align__(16) float terms[kTermCap];
    __shared__ float sums[64];
    __shared__ double red[4];
    const int cols = static_cast<int>(g.m.cols);
    ActRegs ar;
    act_issue(ar, g.x, g.normw, cols);
    Tile<T> tile;
    tile.load(g.m, blockIdx.x * g.R, g.R);
    act_finish(ar, g.x, g.normw, g.eps, cols, takes_q8_k(T), act_bits(g.m), a, red);
    tile.sums(g.m, a, terms, sums);
    const uint32_t r = threadIdx.x, row = tile.row0 + r;
    if (threadIdx.x < 64) {  // R <= 64: the first wave holds the tile's rows
        unsigned long long key = 0;
        if (r < static_cast<uint32_t>(g.R) && row < g.m.rows) {
            float v = sums[r];
            if (g.softcap != 0.0f) v = g.softcap * ref_tanhf(v / g.softcap);  // src/model.cpp:1206-1209
            if (g.logits != nullptr) g.logits[row] = v;
            key = pick_key(v, row);
        }
        key = wave_max_u64(key);
        if (threadIdx.x == 0) {
            const unsigned long long cur = __hip_atomic_load(g.key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (key > cur) atomicMax(g.key, key);
        }
    }
}

// Turns a pending pick into the next token (one thread): seq[pos + 1] = token
// unless the caller supplied that position, pos + 1, key re-armed.  Returns
// the position now current.
__device__ int finalize_pick(const PickState& p) {
    const unsigned long long key = __hip_atomic_load(p.key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int pos = *p.pos;
    if (key != 0ull) {
        const int token = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(key & 0xFFFFFFFFu));
        if (pos + 1 < p.seq_len && pos + 1 >= *p.fixed) p.seq[pos + 1] = token;
        pos += 1;
        *p.pos = pos;
        __hip_atomic_store(p.key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return pos;
}

__global__ void k_finalize(PickState p) {
    if (threadIdx.x == 0) finalize_pick(p);
}

// ============================================================== attention (decode)

// Grid (kv_heads, max_splits).  The context length comes from the device
// position, so one captured launch serves every step.
__global__ __launch_bounds__(kThreads) void k_attn(AttnArgs g) {
    __shared__ AttnLds s;
    __shared__ bool last;
    const int kv = blockIdx.x, split = blockIdx.y;
    // A sliding layer sees positions start .. pos (src/model.cpp:1084-1085): the cache
    // rows and the RoPE table are taken from `start` on, and positions counted from there.
    const int pos_abs = *g.pos, start = g.window > 0 && pos_abs + 1 > g.window ? pos_abs + 1 - g.window : 0;
    if (start > 0) {
        const size_t shift = static_cast<size_t>(start) * g.head_dim;
        g.kcache += shift;
        g.vcache += shift;
        if (g.rope != nullptr) g.rope += static_cast<size_t>(start) * g.rope_dim;
    }
    const int pos = pos_abs - start, L = pos + 1;
    // exact-order attention at every length when the global score buffer is given
    const bool exact = attn_is_exact(L, g.heads / g.kv_heads) || g.gsc != nullptr;
    if (exact ? split != 0 : split * kSplit >= L) return;
    attn_prologue<PlainIO>(g, s, kv, pos, exact || split == pos / kSplit);
    const PlainOut o{g.out, g.part_acc, g.part_ml};
    if (exact) {
        attn_exact(g, s, kv, L, o);
        return;
    }
    attn_split_partial(g, s, kv, split, L, o);
    // the last split of this key/value head to finish merges them all
    __threadfence();
    __syncthreads();
    const int ns = (L + kSplit - 1) / kSplit;
    if (threadIdx.x == 0) last = atomicAdd(g.tickets + kv, 1u) == static_cast<unsigned>(ns - 1);
    __syncthreads();
    if (!last) return;
    __threadfence();
    attn_split_combine(g, kv, L, o);
    if (threadIdx.x == 0) g.tickets[kv] = 0u;
}

// ============================================================== embedding, argmax, position

// embedding_row (src/model.cpp:27-70): dequantise row *token of the packed embedding.
// Starts a step: finalizes the previous step's pick, if one is pending, then
// dequantises the row of token seq[pos].
// Gemma's rows are then multiplied by sqrt(embd) (src/model.cpp:899-901; scale 1 elsewhere).
__global__ __launch_bounds__(kThreads) void k_embed(Packed m, PickState ps, float* __restrict__ h, float scale) {
    __shared__ int tok;
    if (threadIdx.x == 0) tok = ps.seq[finalize_pick(ps)];
    __syncthreads();
    const uint32_t r = static_cast<uint32_t>(tok);
    for (uint32_t e = threadIdx.x; e < m.cols; e += kThreads) {
        const float v = dequant_elem(m, r, e);
        h[e] = scale != 1.0f ? v * scale : v;
    }
}

// h = (h + rms_norm(p, w)) * out_scale (src/model.cpp:1113-1121, :1153-1160, :1172-1176; x * 1.0f
// is x, so out_scale 1 is the plain residual add): one workgroup.
__global__ __launch_bounds__(kThreads) void k_post_add(float* __restrict__ h, const float* __restrict__ p,
                                                       const float* __restrict__ w, float eps, int n, float out_scale) {
    __shared__ double red[4];
    const float scale = rms_scale(block_sumsq(p, n, red), n, eps);
    for (int i = threadIdx.x; i < n; i += kThreads) h[i] = (h[i] + p[i] * scale * w[i]) * out_scale;
}

// h *= out_scale (src/model.cpp:1178-1181).
__global__ void k_scale(float* __restrict__ h, float out_scale, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] *= out_scale;
}

// Gemma 4's per-layer embedding inputs (src/model.cpp:905-925), one workgroup per layer's slice:
// the slice scaled by 1/sqrt(embd) (stored, as the reference scales it in place), RMS-normed with
// per_layer_proj_norm, plus the token's row of per_layer_token_embd times sqrt(dim), times 0.70710678.
__global__ __launch_bounds__(kThreads) void k_ple_inputs(float* __restrict__ in, Packed table, const float* __restrict__ norm,
                                                         const int* __restrict__ seq, const int* __restrict__ pos, int dim,
                                                         float proj_scale, float table_scale, float eps) {
    __shared__ double red[4];
    const int l = blockIdx.x;
    float* slice = in + static_cast<size_t>(l) * dim;
    const uint32_t tok = static_cast<uint32_t>(seq[*pos]);
    for (int i = threadIdx.x; i < dim; i += kThreads) slice[i] = slice[i] * proj_scale;
    __syncthreads();
    const float scale = rms_scale(block_sumsq(slice, dim, red), dim, eps);
    for (int i = threadIdx.x; i < dim; i += kThreads) {
        const float row = dequant_elem(table, tok, static_cast<uint32_t>(l * dim + i));
        slice[i] = (slice[i] * scale * norm[i] + row * table_scale) * 0.70710678f;
    }
}


// LFM2 short convolution (src/model.cpp:935-969): bx = b * x, kept per position as
// fp16 (store_f16); out = c * sum over the last `taps` positions, oldest first, of
// w[d][k] * bx (read back from the fp16 cache; positions before 0 are zero state).
// One thread per channel: the thread that stores bx[pos][d] is the one that reads it.
__global__ __launch_bounds__(kThreads) void k_conv(const float* __restrict__ bcx, uint16_t* __restrict__ cache,
                                                   const float* __restrict__ w, int taps, const int* __restrict__ pos_p,
                                                   int n, float* __restrict__ out) {
    const int d = blockIdx.x * kThreads + threadIdx.x;
    if (d >= n) return;
    const int pos = *pos_p;
    cache[static_cast<size_t>(pos) * n + d] = f2h(bcx[2 * n + d] * bcx[d]);
    float acc = 0.0f;
    for (int k = 0; k < taps; ++k) {
        if (pos + k + 1 < taps) continue;
        acc += w[d * taps + k] * h2f(cache[static_cast<size_t>(pos + k + 1 - taps) * n + d]);
    }
    out[d] = acc * bcx[n + d];
}

// Qwen3.5 Gated DeltaNet, Session::forward_recurrent (src/model.cpp:754-865) for one
// token: one workgroup per head h, thread j owning channel j of the head's q, k and v
// and row j (value j) of its state.
//   conv: x_c = SiLU(sum over taps i, oldest first, of w[c][i] in_i[c]), in_taps-1 the
//         token's own attn_qkv row, the others the ring's (zero before position 0);
//   q = x_q q_scale / sqrt(sum x_q^2 + eps), k = x_k / sqrt(sum x_k^2 + eps), each sum
//         float and sequential (one lane each);
//   decay = exp(softplus(alpha + dt) a), beta = sigmoid(beta);
//   S[j][i] = S[j][i] decay; d_j = (v_j - sum_i S[j][i] k_i) beta;
//   S[j][i] += k_i d_j; o_j = sum_i S[j][i] q_i   (both sums sequential in i);
//   out = rms_norm(o, ssm_norm) SiLU(z).
// The state is key-major ([i][j]), so a step of i reads and writes one contiguous row
// across the lanes; it lives in two halves by position parity, so the half a token read
// is still the state before that token (the reference's snapshot, src/model.cpp:798-812).

// The LDS of one recurrence workgroup.
struct SsmLds {
    float qs[kThreads], ks[kThreads];
    float inv[2];
    double red[4];
};

// A thread's conv state for its q, k and v channels, held in registers and right-aligned in
// fixed slots (every index a constant): the taps' weights at w[c][8 - taps ..], oldest first (the
// newest, for the token's own rows, at slot 7), and the last taps - 1 inputs at win[c][8 - taps ..],
// oldest first (zero before position 0).
constexpr int kSsmMaxTaps = 8;
struct SsmConv {
    float w[3][kSsmMaxTaps];
    float win[3][kSsmMaxTaps - 1];
};

// The conv state of thread j (a channel of head h) before the token at pos, from the weights and
// the ring (slot p % taps holds position p's rows).
template <int DIM>
__device__ __forceinline__ void ssm_conv_load(const SsmArgs& g, int h, int pos, SsmConv& cv) {
    const int j = threadIdx.x, taps = g.taps;
    if (j >= DIM) return;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const int ch = c * g.heads * DIM + h * DIM + j;
#pragma unroll
        for (int k = 0; k < kSsmMaxTaps; ++k) {
            const int i = k - (kSsmMaxTaps - taps);  // the tap in slot k
            cv.w[c][k] = i >= 0 ? g.conv_w[static_cast<size_t>(ch) * taps + i] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < kSsmMaxTaps - 1; ++k) {
            const int i = k - (kSsmMaxTaps - taps), p = pos - (taps - 1) + i;  // input i, at position p
            cv.win[c][k] = i >= 0 && p >= 0 ? g.ring[static_cast<size_t>(p % taps) * g.qkv_dim + ch] : 0.0f;
        }
    }
}

// One token of head h (a step of Session::forward_recurrent) whose attn_qkv rows for thread j's
// channels are cur[] and gate row z: the conv over the window and cur (which then joins the
// window), the norms, the delta update of the thread's state row (row[], in place) and the gated
// norm; returns the output of channel j (0 for threads j >= DIM).  Every thread of the workgroup
// calls it (it holds barriers).
// The step's per-head constants (dt bias, A, the gated norm's weight of channel j), read once
// ahead of a token loop.
struct SsmConst {
    float dt, a, norm;
};
template <int DIM>
__device__ __forceinline__ SsmConst ssm_const(const SsmArgs& g, int h) {
    return SsmConst{g.dt[h], g.a[h], g.norm[threadIdx.x < DIM ? threadIdx.x : 0]};
}

// A workgroup barrier that orders LDS only (the step's threads share nothing else): loads of
// global memory issued before it (the next token's rows) stay in flight.
__device__ __forceinline__ void ssm_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int DIM>
__device__ __forceinline__ float ssm_step(const SsmArgs& g, SsmLds& s, int h, const float (&cur)[3], SsmConv& cv, float z,
                                          float alpha_in, float beta_in, float (&row)[DIM], const SsmConst& kc) {
    const int j = threadIdx.x, taps = g.taps;
    float v = 0.0f;
    if (j < DIM) {
#pragma unroll
        for (int c = 0; c < 3; ++c) {  // q, k, v channels of head h
            float acc = 0.0f;  // the taps in order, oldest first (the slots before the first tap skipped)
#pragma unroll
            for (int k = 0; k < kSsmMaxTaps - 1; ++k)
                if (k >= kSsmMaxTaps - taps) acc = acc + cv.w[c][k] * cv.win[c][k];
            acc = acc + cv.w[c][kSsmMaxTaps - 1] * cur[c];
#pragma unroll
            for (int k = 0; k < kSsmMaxTaps - 2; ++k) cv.win[c][k] = cv.win[c][k + 1];  // the window moves on
            cv.win[c][kSsmMaxTaps - 2] = cur[c];
            const float x = acc / (1.0f + ref_expf(-acc));
            if (c == 0) s.qs[j] = x;
            else if (c == 1) s.ks[j] = x;
            else v = x;
        }
    }
    ssm_barrier();
    if (j == 0 || j == 64) {  // the two L2 sums, one lane of two waves
        const float* src = j == 0 ? s.qs : s.ks;
        float sum = 0.0f;
        for (int i = 0; i < DIM; ++i) sum += src[i] * src[i];
        s.inv[j == 0 ? 0 : 1] = (j == 0 ? g.q_scale : 1.0f) / sqrtf(sum + g.eps);
    }
    ssm_barrier();
    if (j < DIM) {
        s.qs[j] = s.qs[j] * s.inv[0];
        s.ks[j] = s.ks[j] * s.inv[1];
    }
    const float alpha = alpha_in + kc.dt;
    const float softplus = alpha > 20.0f ? alpha : ref_log1pf(ref_expf(alpha));
    const float decay = ref_expf(softplus * kc.a);
    const float beta = 1.0f / (1.0f + ref_expf(-beta_in));
    ssm_barrier();
    float o = 0.0f;
    if (j < DIM) {
        float sk = 0.0f;
#pragma unroll
        for (int i = 0; i < DIM; ++i) {
            row[i] = row[i] * decay;
            sk = sk + row[i] * s.ks[i];
        }
        const float d = (v - sk) * beta;
#pragma unroll
        for (int i = 0; i < DIM; ++i) {
            row[i] = row[i] + s.ks[i] * d;
            o = o + row[i] * s.qs[i];
        }
    }
    double sq = j < DIM ? static_cast<double>(o * o) : 0.0;
    sq = wave_sum(sq);
    if ((j & 63) == 0) s.red[j >> 6] = sq;
    ssm_barrier();
    const float scale = rms_scale(((s.red[0] + s.red[1]) + s.red[2]) + s.red[3], DIM, g.eps);
    float out = 0.0f;
    if (j < DIM) {
        const float gate = z / (1.0f + ref_expf(-z));
        out = o * scale * kc.norm * gate;
    }
    ssm_barrier();  // the LDS is the next token's
    return out;
}

// The attn_qkv rows of thread j's three channels of head h, from a token's row.
template <int DIM>
__device__ __forceinline__ void ssm_cur(const SsmArgs& g, int h, const float* qkv_t, float (&cur)[3]) {
    const int j = threadIdx.x < DIM ? threadIdx.x : 0;
#pragma unroll
    for (int c = 0; c < 3; ++c) cur[c] = qkv_t[c * g.heads * DIM + h * DIM + j];
}

// The state row of thread j in half `half`, or zero at position 0 (a new or restarted sequence).
template <int DIM>
__device__ __forceinline__ void ssm_row_load(const SsmArgs& g, int h, int half, bool fresh, float (&row)[DIM]) {
    const int j = threadIdx.x;
    const float* src = g.state + (static_cast<size_t>(half) * g.heads + h) * DIM * DIM + j;
#pragma unroll
    for (int i = 0; i < DIM; ++i) row[i] = fresh || j >= DIM ? 0.0f : src[static_cast<size_t>(i) * DIM];
}
template <int DIM>
__device__ __forceinline__ void ssm_row_store(const SsmArgs& g, int h, int half, const float (&row)[DIM]) {
    const int j = threadIdx.x;
    if (j >= DIM) return;
    float* dst = g.state + (static_cast<size_t>(half) * g.heads + h) * DIM * DIM + j;
#pragma unroll
    for (int i = 0; i < DIM; ++i) dst[static_cast<size_t>(i) * DIM] = row[i];
}

// Decode, state sizes 64 and 128: the thread's state row in registers, loaded by one batch of
// loads (in flight during the conv and the norms), the token at *pos read from half pos & 1 and
// written to the other.
template <int DIM>
__global__ __launch_bounds__(kThreads) void k_ssm(SsmArgs g) {
    __shared__ SsmLds s;
    const int h = blockIdx.x, pos = *g.pos, j = threadIdx.x;
    float row[DIM];
    ssm_row_load<DIM>(g, h, pos & 1, pos == 0, row);
    SsmConv cv;
    ssm_conv_load<DIM>(g, h, pos, cv);
    float cur[3];
    ssm_cur<DIM>(g, h, g.qkv, cur);
    const float z = g.z[h * DIM + (j < DIM ? j : 0)];
    const float out = ssm_step<DIM>(g, s, h, cur, cv, z, g.ab[h], g.ab[g.heads + h], row, ssm_const<DIM>(g, h));
    ssm_row_store<DIM>(g, h, (pos + 1) & 1, row);
    if (j < DIM) {
        g.out[h * DIM + j] = out;
#pragma unroll
        for (int c = 0; c < 3; ++c) g.ring[static_cast<size_t>(pos % g.taps) * g.qkv_dim + c * g.heads * DIM + h * DIM + j] = cur[c];
    }
}

// Prefill, state sizes 64 and 128: the ntok tokens at positions pos0 .. in order, the state row in
// registers throughout.  Token t's rows are qkv[t * qkv_dim ..], z[t * heads * DIM ..], alpha
// ab[t * ab_stride + h] and beta ab[t * ab_stride + heads + h]; outputs out[t * heads * DIM ..].
// The half of the last token's parity keeps the state before it (the reference's snapshot,
// src/model.cpp:798-812), the other half the state after it.
template <int DIM>
__global__ __launch_bounds__(kThreads) void k_pre_ssm(SsmArgs g, int pos0, int ntok, int ab_stride) {
    __shared__ SsmLds s;
    const int h = blockIdx.x, inner = g.heads * DIM, j = threadIdx.x, taps = g.taps;
    float row[DIM];
    ssm_row_load<DIM>(g, h, pos0 & 1, pos0 == 0, row);
    SsmConv cv;
    ssm_conv_load<DIM>(g, h, pos0, cv);
    const SsmConst kc = ssm_const<DIM>(g, h);
    // token t's rows, z and gates, loaded while token t - 1 steps (the step's barriers leave them in flight)
    struct In {
        float cur[3], z, a, b;
    };
    auto load_in = [&](int t, In& in) {
        ssm_cur<DIM>(g, h, g.qkv + static_cast<size_t>(t) * g.qkv_dim, in.cur);
        in.z = g.z[static_cast<size_t>(t) * inner + h * DIM + (j < DIM ? j : 0)];
        const float* ab = g.ab + static_cast<size_t>(t) * ab_stride;
        in.a = ab[h];
        in.b = ab[g.heads + h];
    };
    In in;
    load_in(0, in);
    for (int t = 0; t < ntok; ++t) {
        const int pos = pos0 + t;
        if (t + 1 == ntok) ssm_row_store<DIM>(g, h, pos & 1, row);
        In next = in;
        if (t + 1 < ntok) load_in(t + 1, next);
        const float out = ssm_step<DIM>(g, s, h, in.cur, cv, in.z, in.a, in.b, row, kc);
        if (j < DIM) g.out[static_cast<size_t>(t) * inner + h * DIM + j] = out;
        in = next;
    }
    ssm_row_store<DIM>(g, h, (pos0 + ntok) & 1, row);
    // the ring: the batch's last taps positions' rows (older slots keep theirs)
    if (j < DIM)
        for (int t = ntok - taps > 0 ? ntok - taps : 0; t < ntok; ++t)
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                const int ch = c * inner + h * DIM + j;
                g.ring[static_cast<size_t>((pos0 + t) % taps) * g.qkv_dim + ch] = g.qkv[static_cast<size_t>(t) * g.qkv_dim + ch];
            }
}

// Decode, any state size up to 256: the state read twice from memory.
__global__ __launch_bounds__(kThreads) void k_ssm_any(SsmArgs g) {
    __shared__ float qs[kThreads], ks[kThreads];
    __shared__ float inv[2];
    __shared__ double red[4];
    const int h = blockIdx.x, j = threadIdx.x, dim = g.dim, taps = g.taps, qkv = g.qkv_dim;
    const int pos = *g.pos, k_off = g.heads * dim;
    const size_t plane = static_cast<size_t>(dim) * dim;
    const float* sin = g.state + (static_cast<size_t>(pos & 1) * g.heads + h) * plane + j;
    float* sout = g.state + (static_cast<size_t>((pos + 1) & 1) * g.heads + h) * plane + j;
    const bool fresh = pos == 0;  // the zero state of a new or restarted sequence
    float v = 0.0f;
    if (j < dim) {
        for (int c = 0; c < 3; ++c) {  // q, k, v channels of head h
            const int ch = c * k_off + h * dim + j;
            const float cur = g.qkv[ch];
            const float* w = g.conv_w + static_cast<size_t>(ch) * taps;
            float acc = 0.0f;
            for (int i = 0; i < taps; ++i) {
                const int p = pos - (taps - 1) + i;
                const float in = i == taps - 1 ? cur : p < 0 ? 0.0f : g.ring[static_cast<size_t>(p % taps) * qkv + ch];
                acc = acc + w[i] * in;
            }
            g.ring[static_cast<size_t>(pos % taps) * qkv + ch] = cur;  // the slot of position pos - taps, read by no one
            const float x = acc / (1.0f + ref_expf(-acc));
            if (c == 0) qs[j] = x;
            else if (c == 1) ks[j] = x;
            else v = x;
        }
    }
    __syncthreads();
    if (j == 0 || j == 64) {  // the two L2 sums, one lane of two waves
        const float* src = j == 0 ? qs : ks;
        float sum = 0.0f;
        for (int i = 0; i < dim; ++i) sum += src[i] * src[i];
        inv[j == 0 ? 0 : 1] = (j == 0 ? g.q_scale : 1.0f) / sqrtf(sum + g.eps);
    }
    __syncthreads();
    if (j < dim) {
        qs[j] = qs[j] * inv[0];
        ks[j] = ks[j] * inv[1];
    }
    const float alpha = g.ab[h] + g.dt[h];
    const float softplus = alpha > 20.0f ? alpha : ref_log1pf(ref_expf(alpha));
    const float decay = ref_expf(softplus * g.a[h]);
    const float beta = 1.0f / (1.0f + ref_expf(-g.ab[g.heads + h]));
    __syncthreads();
    float o = 0.0f;
    if (j < dim) {
        float sk = 0.0f;
#pragma unroll 8
        for (int i = 0; i < dim; ++i) {
            const float si = (fresh ? 0.0f : sin[static_cast<size_t>(i) * dim]) * decay;
            sk = sk + si * ks[i];
        }
        const float d = (v - sk) * beta;
#pragma unroll 8
        for (int i = 0; i < dim; ++i) {
            float si = (fresh ? 0.0f : sin[static_cast<size_t>(i) * dim]) * decay;
            si = si + ks[i] * d;
            sout[static_cast<size_t>(i) * dim] = si;
            o = o + si * qs[i];
        }
    }
    double sq = j < dim ? static_cast<double>(o * o) : 0.0;
    sq = wave_sum(sq);
    if ((j & 63) == 0) red[j >> 6] = sq;
    __syncthreads();
    const float scale = rms_scale(((red[0] + red[1]) + red[2]) + red[3], dim, g.eps);
    if (j < dim) {
        const float z = g.z[h * dim + j];
        const float gate = z / (1.0f + ref_expf(-z));
        g.out[h * dim + j] = o * scale * g.norm[j] * gate;
    }
}

// Qwen3.5's query projection holds each head's query rows followed by its gate rows
// (src/model.cpp:1002-1012).
__global__ void k_qgate_split(const float* __restrict__ qg, float* __restrict__ q, float* __restrict__ gate, int hd, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int h = i / hd, d = i - h * hd;
    q[i] = qg[2 * h * hd + d];
    gate[i] = qg[2 * h * hd + hd + d];
}

// att *= 1 / (1 + exp(-gate)) (src/model.cpp:1102-1108).
__global__ void k_sigmoid_gate(float* __restrict__ att, const float* __restrict__ gate, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) att[i] = att[i] * (1.0f / (1.0f + ref_expf(-gate[i])));
}

// log1pf as the recurrence computes it (ref_log1pf), for the parity tests.
__global__ void k_log1pf(const float* __restrict__ x, float* __restrict__ y, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] = ref_log1pf(x[i]);
}

// ---------------------------------------------------------------- plain attention
//
// The reference's attention for one token (src/model.cpp:1019-1093 with the portable
// kernels of src/kernels_f32.cpp:229-284) in three kernels, for head sizes the LDS-resident
// attention does not take (up to 512) and for layers that read another layer's cache:
//   prologue (a wave per query head and per key/value head): bias, RMS norm and RoPE of each
//            query head into qn; of each key head, V's bias (and Gemma 4's weightless V norm),
//            and the fp16 K/V rows at pos;
//   scores   (a workgroup per query head and 64 positions, a lane per position):
//            dot_f32(q, k_p) * scale, 16 lane partials over i = j (mod 16) in order, then
//            0 + lane 0 + ... + lane 15;
//   values   (a wave per head and 64 output dimensions): the head's softmax (max,
//            e_p = expf(s_p - max), their sum in double, w_p = e_p * (float)(1 / sum)), then
//            for each output dimension 0 + w_0 v_0 + w_1 v_1 + ... in position order.
// A sliding layer's token sees positions [L - window, L) (src/model.cpp:1084-1085).

__device__ __forceinline__ int plain_start(const AttnArgs& g, int L) { return g.window > 0 && L > g.window ? L - g.window : 0; }

// One wave a head: wave h < heads forms query head h (bias, norm, RoPE) into qn; wave heads + kv
// forms key/value head kv (bias, norm, RoPE; V's bias and weightless norm) and stores its fp16 rows.
// A query head's raw rows are q[h * q_stride ..] (q_stride 2 * head_dim: Qwen3.5's query|gate rows).
__global__ __launch_bounds__(64) void k_plain_prologue(AttnArgs g) {
    __shared__ float a[kPlainMaxHead], b[kPlainMaxHead];
    const int hd = g.head_dim, lane = threadIdx.x, pos = *g.pos;
    const int qs = g.q_stride != 0 ? g.q_stride : hd;
    const float* rope = g.rope != nullptr ? g.rope + static_cast<size_t>(pos) * g.rope_dim : nullptr;
    const int w = blockIdx.x;
    if (w < g.heads) {
        for (int i = lane; i < hd; i += 64) a[i] = g.q[static_cast<size_t>(w) * qs + i];
        head_norm_rope(a, g.qbias != nullptr ? g.qbias + w * hd : nullptr, g.qnorm, rope, hd, g.rope_dim, g.neox, g.eps);
        for (int i = lane; i < hd; i += 64) g.qn[w * hd + i] = a[i];
        return;
    }
    const int kv = w - g.heads;
    for (int i = lane; i < hd; i += 64) {
        a[i] = g.k[kv * hd + i];
        b[i] = g.vbias != nullptr ? g.v[kv * hd + i] + g.vbias[kv * hd + i] : g.v[kv * hd + i];
    }
    head_norm_rope(a, g.kbias != nullptr ? g.kbias + kv * hd : nullptr, g.knorm, rope, hd, g.rope_dim, g.neox, g.eps);
    if (g.vnorm) {  // rms_norm(v) with no weight (src/model.cpp:1041)
        double sq = 0.0;
        for (int i = lane; i < hd; i += 64) sq += static_cast<double>(b[i] * b[i]);
        const float scale = rms_scale(wave_sum(sq), hd, g.eps);
        for (int i = lane; i < hd; i += 64) b[i] = b[i] * scale;
    }
    uint16_t* kr = g.kcache + (static_cast<size_t>(kv) * g.ctx + pos) * hd;
    uint16_t* vr = g.vcache + (static_cast<size_t>(kv) * g.ctx + pos) * hd;
    for (int i = lane; i < hd; i += 64) {
        kr[i] = f2h(a[i]);
        vr[i] = f2h(b[i]);
    }
}

// A workgroup per (query head, 64 positions), a lane per position.
__global__ __launch_bounds__(64) void k_plain_scores(AttnArgs g) {
    __shared__ float q[kPlainMaxHead];
    const int h = blockIdx.x, hd = g.head_dim, hpk = g.heads / g.kv_heads, kv = h / hpk, lane = threadIdx.x;
    const int L = *g.pos + 1, start = plain_start(g, L);
    const int p0 = start + static_cast<int>(blockIdx.y) * 64;
    if (p0 >= L) return;  // the grid covers the longest context
    for (int i = lane; i < hd; i += 64) q[i] = g.qn[h * hd + i];
    __syncthreads();
    const int p = p0 + lane;
    if (p >= L) return;
    const uint16_t* kr = g.kcache + (static_cast<size_t>(kv) * g.ctx + p) * hd;
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
    for (int b0 = 0; b0 < hd; b0 += 128) {  // eight 16-wide blocks' loads issued together
        uint4 kk[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) kk[u] = b0 + 8 * u < hd ? *reinterpret_cast<const uint4*>(kr + b0 + 8 * u) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int blk = 0; blk < 8; ++blk) {
            if (b0 + 16 * blk >= hd) break;
            const uint32_t kw[8] = {kk[2 * blk].x, kk[2 * blk].y, kk[2 * blk].z, kk[2 * blk].w,
                                    kk[2 * blk + 1].x, kk[2 * blk + 1].y, kk[2 * blk + 1].z, kk[2 * blk + 1].w};
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint16_t hv = static_cast<uint16_t>((j & 1) ? (kw[j >> 1] >> 16) : (kw[j >> 1] & 0xFFFF));
                acc[j] += q[b0 + 16 * blk + j] * h2f(hv);
            }
        }
    }
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) sum += acc[j];
    g.gsc[static_cast<size_t>(h) * g.ctx + p] = sum * g.scale;
}

// A wave per (head, 64 output dimensions): the head's softmax (each wave of the head computes the
// same weights: max, e_p = expf(s_p - max), their double sum, e_p * (float)(1 / sum)), held in LDS
// when the window fits it and recomputed per position otherwise; then a lane per output dimension
// sums w_p v_p[d] in position order, its loads issued 32 positions at a time.  Qwen3.5's sigmoid
// gate (src/model.cpp:1102-1108) is applied to the sums.
__global__ __launch_bounds__(64) void k_plain_values(AttnArgs g) {
    __shared__ float wl[kPlainLdsW];
    const int h = blockIdx.x, hd = g.head_dim, hpk = g.heads / g.kv_heads, kv = h / hpk, lane = threadIdx.x;
    const int L = *g.pos + 1, start = plain_start(g, L), n = L - start;
    const float* sc = g.gsc + static_cast<size_t>(h) * g.ctx + start;
    float m = -INFINITY;
    for (int p = lane; p < n; p += 64) m = fmaxf(m, sc[p]);
    m = wave_max(m);
    const bool in_lds = n <= kPlainLdsW;
    double part = 0.0;
    for (int p = lane; p < n; p += 64) {
        const float e = ref_expf(sc[p] - m);
        if (in_lds) wl[p] = e;
        part += static_cast<double>(e);
    }
    const float scale = static_cast<float>(1.0 / wave_sum(part));
    if (in_lds)
        for (int p = lane; p < n; p += 64) wl[p] = wl[p] * scale;
    __syncthreads();
    const int d = static_cast<int>(blockIdx.y) * 64 + lane;
    if (d >= hd) return;
    const uint16_t* vv = g.vcache + static_cast<size_t>(kv) * g.ctx * hd + static_cast<size_t>(start) * hd + d;
    auto weight = [&](int p) { return in_lds ? wl[p] : ref_expf(sc[p] - m) * scale; };
    constexpr int kB = 32;
    float a = 0.0f;
    int p = 0;
    for (; p + kB <= n; p += kB) {  // loads first, then the adds in position order
        float vf[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) vf[u] = h2f(vv[static_cast<size_t>(p + u) * hd]);
#pragma unroll
        for (int u = 0; u < kB; ++u) a += weight(p + u) * vf[u];
    }
    for (; p < n; ++p) a += weight(p) * h2f(vv[static_cast<size_t>(p) * hd]);
    if (g.gate != nullptr) a = a * (1.0f / (1.0f + ref_expf(-g.gate[static_cast<size_t>(h) * g.gate_stride + d])));
    g.out[h * hd + d] = a;
}

// The plain attention for the ntok tokens of a prompt (positions pos0 ..), each token's steps
// those of the decode kernels above: a prologue wave per (token, head), then a workgroup per
// (token, query head) that forms the scores of every visible position in LDS (a thread per
// position), runs the softmax on one wave (the decode kernels' grouping) and sums the values (a
// thread per output dimension).  Contexts up to kPlainLdsW positions.
__global__ __launch_bounds__(64) void k_pre_plain_prologue(PrePlainArgs p) {
    __shared__ float a[kPlainMaxHead], b[kPlainMaxHead];
    const AttnArgs& g = p.a;
    const int t = blockIdx.x, w = blockIdx.y, hd = g.head_dim, lane = threadIdx.x, pos = p.pos0 + t;
    const int qs = g.q_stride != 0 ? g.q_stride : hd;
    const float* rope = g.rope != nullptr ? g.rope + static_cast<size_t>(pos) * g.rope_dim : nullptr;
    if (w < g.heads) {
        const float* q = g.q + static_cast<size_t>(t) * p.q_tok + static_cast<size_t>(w) * qs;
        for (int i = lane; i < hd; i += 64) a[i] = q[i];
        head_norm_rope(a, g.qbias != nullptr ? g.qbias + w * hd : nullptr, g.qnorm, rope, hd, g.rope_dim, g.neox, g.eps);
        for (int i = lane; i < hd; i += 64) g.qn[(static_cast<size_t>(t) * g.heads + w) * hd + i] = a[i];
        return;
    }
    const int kv = w - g.heads;
    const float* k = g.k + static_cast<size_t>(t) * p.kv_tok + kv * hd;
    const float* v = g.v + static_cast<size_t>(t) * p.kv_tok + kv * hd;
    for (int i = lane; i < hd; i += 64) {
        a[i] = k[i];
        b[i] = g.vbias != nullptr ? v[i] + g.vbias[kv * hd + i] : v[i];
    }
    head_norm_rope(a, g.kbias != nullptr ? g.kbias + kv * hd : nullptr, g.knorm, rope, hd, g.rope_dim, g.neox, g.eps);
    if (g.vnorm) {
        double sq = 0.0;
        for (int i = lane; i < hd; i += 64) sq += static_cast<double>(b[i] * b[i]);
        const float scale = rms_scale(wave_sum(sq), hd, g.eps);
        for (int i = lane; i < hd; i += 64) b[i] = b[i] * scale;
    }
    uint16_t* kr = g.kcache + (static_cast<size_t>(kv) * g.ctx + pos) * hd;
    uint16_t* vr = g.vcache + (static_cast<size_t>(kv) * g.ctx + pos) * hd;
    for (int i = lane; i < hd; i += 64) {
        kr[i] = f2h(a[i]);
        vr[i] = f2h(b[i]);
    }
}

__global__ __launch_bounds__(kThreads) void k_pre_plain_attn(PrePlainArgs p) {
    __shared__ float q[kPlainMaxHead];
    __shared__ float wl[kPlainLdsW];
    const AttnArgs& g = p.a;
    const int t = blockIdx.x, h = blockIdx.y, hd = g.head_dim, hpk = g.heads / g.kv_heads, kv = h / hpk, tid = threadIdx.x;
    const int L = p.pos0 + t + 1, start = plain_start(g, L), n = L - start;
    for (int i = tid; i < hd; i += kThreads) q[i] = g.qn[(static_cast<size_t>(t) * g.heads + h) * hd + i];
    __syncthreads();
    const uint16_t* kbase = g.kcache + (static_cast<size_t>(kv) * g.ctx + start) * hd;
    for (int pp = tid; pp < n; pp += kThreads) {  // dot_f32 order: 16 lane partials, then their sum
        const uint16_t* kr = kbase + static_cast<size_t>(pp) * hd;
        float acc[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
        for (int b0 = 0; b0 < hd; b0 += 16) {
            const uint4 k0 = *reinterpret_cast<const uint4*>(kr + b0), k1 = *reinterpret_cast<const uint4*>(kr + b0 + 8);
            const uint32_t kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint16_t hv = static_cast<uint16_t>((j & 1) ? (kw[j >> 1] >> 16) : (kw[j >> 1] & 0xFFFF));
                acc[j] += q[b0 + j] * h2f(hv);
            }
        }
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) sum += acc[j];
        wl[pp] = sum * g.scale;
    }
    __syncthreads();
    if (tid < 64) {  // the softmax on one wave, as k_plain_values runs it
        float m = -INFINITY;
        for (int pp = tid; pp < n; pp += 64) m = fmaxf(m, wl[pp]);
        m = wave_max(m);
        double part = 0.0;
        for (int pp = tid; pp < n; pp += 64) {
            const float e = ref_expf(wl[pp] - m);
            wl[pp] = e;
            part += static_cast<double>(e);
        }
        const float scale = static_cast<float>(1.0 / wave_sum(part));
        for (int pp = tid; pp < n; pp += 64) wl[pp] = wl[pp] * scale;
    }
    __syncthreads();
    constexpr int kChains = kPlainMaxHead / kThreads;
    const uint16_t* vbase = g.vcache + (static_cast<size_t>(kv) * g.ctx + start) * hd;
#pragma unroll
    for (int c = 0; c < kChains; ++c) {
        const int d = tid + c * kThreads;
        if (d >= hd) break;
        const uint16_t* vv = vbase + d;
        constexpr int kB = 32;
        float acc = 0.0f;
        int pp = 0;
        for (; pp + kB <= n; pp += kB) {  // loads first, then the adds in position order
            float vf[kB];
#pragma unroll
            for (int u = 0; u < kB; ++u) vf[u] = h2f(vv[static_cast<size_t>(pp + u) * hd]);
#pragma unroll
            for (int u = 0; u < kB; ++u) acc += wl[pp + u] * vf[u];
        }
        for (; pp < n; ++pp) acc += wl[pp] * h2f(vv[static_cast<size_t>(pp) * hd]);
        if (g.gate != nullptr)
            acc = acc * (1.0f / (1.0f + ref_expf(-g.gate[static_cast<size_t>(t) * p.q_tok + static_cast<size_t>(h) * g.gate_stride + d])));
        g.out[static_cast<size_t>(t) * g.heads * hd + h * hd + d] = acc;
    }
}

// tanhf as the Gemma epilogues compute it (ref_tanhf), for the parity tests.
__global__ void k_tanhf(const float* __restrict__ x, float* __restrict__ y, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] = ref_tanhf(x[i]);
}

// expf as the token loop computes it (ref_expf), for the parity tests.
__global__ void k_expf(const float* __restrict__ x, float* __restrict__ y, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] = ref_expf(x[i]);
}

// The short exact divisions of device.h against IEEE division, over every
// input: bad[0] counts div127 mismatches (finite a >= 0), bad[1] rcp_rn
// mismatches (finite d != 0), bad[2] hardware f2h against the bit-level
// conversion (every float), bad[3] mul_h against the product of the widened
// half (every float).
__global__ void k_div_selftest(unsigned long long* bad) {
    const unsigned long long stride = static_cast<unsigned long long>(gridDim.x) * blockDim.x;
    unsigned long long n127 = 0, nrcp = 0;
    for (unsigned long long j = static_cast<unsigned long long>(blockIdx.x) * blockDim.x + threadIdx.x; j < (1ull << 32); j += stride) {
        const uint32_t i = static_cast<uint32_t>(j);
        if ((i & 0x7F800000u) == 0x7F800000u) continue;  // inf, NaN
        const float x = __uint_as_float(i);
        if ((i >> 31) == 0 && __float_as_uint(div127(x)) != __float_as_uint(__fdiv_rn(x, 127.0f))) ++n127;
        if ((i & 0x7FFFFFFFu) != 0 && __float_as_uint(rcp_rn(x)) != __float_as_uint(__fdiv_rn(1.0f, x))) ++nrcp;
    }
    if (n127 != 0) atomicAdd(bad, n127);
    if (nrcp != 0) atomicAdd(bad + 1, nrcp);
    unsigned long long nh = 0;
    for (unsigned long long j = static_cast<unsigned long long>(blockIdx.x) * blockDim.x + threadIdx.x; j < (1ull << 32); j += stride) {
        const float x = __uint_as_float(static_cast<uint32_t>(j));
        if (f2h(x) != f2h_bits(x)) ++nh;
    }
    if (nh != 0) atomicAdd(bad + 2, nh);
    // mul_h against the widened product: every float q, with a half drawn from
    // q's bits (every half is met about 65536 times), low and high
    unsigned long long nm = 0;
    for (unsigned long long j = static_cast<unsigned long long>(blockIdx.x) * blockDim.x + threadIdx.x; j < (1ull << 32); j += stride) {
        const uint32_t i = static_cast<uint32_t>(j);
        const float q = __uint_as_float(i);
        const uint32_t w = (i * 2654435761u) ^ (i >> 7);
        const float lo = q * h2f(static_cast<uint16_t>(w & 0xFFFF)), hi = q * h2f(static_cast<uint16_t>(w >> 16));
        const float mlo = mul_h<false>(q, w), mhi = mul_h<true>(q, w);
        const bool nan = lo != lo;  // NaN payloads may differ; NaN must stay NaN
        if (nan ? mlo == mlo : __float_as_uint(mlo) != __float_as_uint(lo)) ++nm;
        if ((hi != hi) ? mhi == mhi : __float_as_uint(mhi) != __float_as_uint(hi)) ++nm;
    }
    if (nm != 0) atomicAdd(bad + 3, nm);
}

// The int8 MFMA rate this device sustains: every wave runs independent
// accumulator chains of one int8 MFMA shape (8 of v_mfma_i32_16x16x64_i8, the
// prefill GEMMs' instruction, or 4 of v_mfma_i32_32x32x32_i8; 8192 multiply-adds
// a chain step either way... the 32x32 shape does 32768) on register operands,
// so nothing but the matrix cores bounds it.  out receives a checksum that
// keeps the work alive.
typedef int v4i_mb __attribute__((ext_vector_type(4)));
typedef int v16i_mb __attribute__((ext_vector_type(16)));
template <int kShape>  // 0: v_mfma_i32_16x16x64_i8, 1: v_mfma_i32_32x32x32_i8
__global__ __launch_bounds__(kThreads) void k_mfma_rate(int iters, int* out) {
    const int lane = threadIdx.x & 63;
    const v4i_mb a = {lane, lane * 3, lane * 5, lane * 7}, b = {lane * 11, lane * 13, 17, lane};
    int sum = 0;
    if (kShape == 0) {
        v4i_mb acc[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] = v4i_mb{k, 0, 0, 0};
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[k] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[k], 0, 0, 0);
#pragma unroll
        for (int k = 0; k < 8; ++k) sum += acc[k][0] + acc[k][1] + acc[k][2] + acc[k][3];
    } else {
        v16i_mb acc[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            acc[k] = v16i_mb{};
            acc[k][0] = k;
        }
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[k], 0, 0, 0);
#pragma unroll
        for (int k = 0; k < 4; ++k) sum += acc[k][0] + acc[k][5] + acc[k][10] + acc[k][15];
    }
    if (sum == 0x7FFFFFFF) out[0] = sum;  // practically never: keeps the chains without a store per wave
    if (threadIdx.x == 0 && blockIdx.x == 0) out[1] = sum;
}

hipError_t launch_mfma_rate(int shape, int blocks, int iters, int* out, hipStream_t s) {
    if (shape == 0) hipLaunchKernelGGL(k_mfma_rate<0>, dim3(blocks), dim3(kThreads), 0, s, iters, out);
    else hipLaunchKernelGGL(k_mfma_rate<1>, dim3(blocks), dim3(kThreads), 0, s, iters, out);
    return hipGetLastError();
}

hipError_t launch_div_selftest(unsigned long long* bad, hipStream_t s) {
    hipLaunchKernelGGL(k_div_selftest, dim3(8192), dim3(256), 0, s, bad);
    return hipGetLastError();
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

// Unit (row r, block b) of a packed 32-value-block matrix to unit (b, r) of
// `dst`: the same planes, block-major ([cols/32][rows] units), so the units of
// one block column across every row are contiguous.  Value runs and scales are
// copied unchanged (Q4_0, Q4_1, Q5_0, Q8_0).
__global__ void k_unit_transpose(Packed src, uint8_t* __restrict__ p0, uint8_t* __restrict__ p1, uint8_t* __restrict__ p2,
                                 uint32_t run, uint32_t extra) {
    const size_t units = src.cols / 32, total = static_cast<size_t>(src.rows) * units;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const size_t r = i / units, b = i - r * units, o = b * src.rows + r;
        for (uint32_t k = 0; k < run; k += 16)
            *reinterpret_cast<uint4*>(p0 + o * run + k) = *reinterpret_cast<const uint4*>(src.p0 + i * run + k);
        reinterpret_cast<uint16_t*>(p1)[o] = reinterpret_cast<const uint16_t*>(src.p1)[i];
        if (extra == 2) reinterpret_cast<uint16_t*>(p2)[o] = reinterpret_cast<const uint16_t*>(src.p2)[i];
        if (extra == 4) reinterpret_cast<uint32_t*>(p2)[o] = reinterpret_cast<const uint32_t*>(src.p2)[i];
    }
}

hipError_t launch_unit_transpose(const Packed& src, const Packed& dst, hipStream_t s) {
    uint32_t run = 0, extra = 0;
    switch (src.type) {
        case kQ4_0: run = 16; break;
        case kQ4_1: run = 16; extra = 2; break;
        case kQ5_0: run = 16; extra = 4; break;
        case kQ8_0: run = 32; break;
        default: return hipErrorInvalidValue;
    }
    const size_t total = static_cast<size_t>(src.rows) * (src.cols / 32);
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_unit_transpose, dim3(static_cast<unsigned>(cdiv(total, 256) < 4096 ? cdiv(total, 256) : 4096)), dim3(256), 0, s,
                       src, const_cast<uint8_t*>(dst.p0), const_cast<uint8_t*>(dst.p1), const_cast<uint8_t*>(dst.p2), run, extra);
    return hipGetLastError();
}

hipError_t launch_quantize(int kind, const float* x, void* out, size_t count, int bits, hipStream_t s) {
    if (count == 0) return hipSuccess;
    if (kind == 0) hipLaunchKernelGGL(k_quant_q8_0, dim3(cdiv(count, kMaxCols)), dim3(kThreads), 0, s, x, static_cast<uint8_t*>(out), count);
    else hipLaunchKernelGGL(k_quant_q8_k, dim3(cdiv(count, kMaxCols)), dim3(kThreads), 0, s, x, static_cast<uint8_t*>(out), count, bits);
    return hipGetLastError();
}

// Rows per tile: the largest power of two up to 64 whose units fit the
// per-thread register budget and the LDS term buffer, then smaller until the
// matrix spans at least kMinTiles workgroups.
int pick_rows_per_tile(uint32_t type, size_t rows, size_t cols) {
    int max_per_thread = 0;
    switch (type) {
        case kQ4_0: max_per_thread = Unit<kQ4_0>::kMaxPerThread; break;
        case kQ4_1: max_per_thread = Unit<kQ4_1>::kMaxPerThread; break;
        case kQ5_0: max_per_thread = Unit<kQ5_0>::kMaxPerThread; break;
        case kQ8_0: max_per_thread = Unit<kQ8_0>::kMaxPerThread; break;
        case kQ4_K: max_per_thread = Unit<kQ4_K>::kMaxPerThread; break;
        case kQ5_K: max_per_thread = Unit<kQ5_K>::kMaxPerThread; break;
        case kQ6_K: max_per_thread = Unit<kQ6_K>::kMaxPerThread; break;
        default: max_per_thread = Unit<kTQ2_0>::kMaxPerThread; break;
    }
    const size_t units = cols / block_elems(type);
    int R = 64;
    while (R > 1 && (static_cast<size_t>(R) * units > static_cast<size_t>(max_per_thread) * kThreads ||
                     static_cast<size_t>(R) * term_stride(static_cast<uint32_t>(units)) > static_cast<size_t>(kTermCap)))
        R /= 2;
    while (R > 1 && (rows + R - 1) / R < static_cast<size_t>(kMinTiles)) R /= 2;
    return R;
}

// Instantiates kernel K for the weight type at run time.
#define BH_DISPATCH(type, K, ...)                                                           \
    switch (type) {                                                                        \
        case kQ4_0: hipLaunchKernelGGL(K<kQ4_0>, __VA_ARGS__); break;                       \
        case kQ4_1: hipLaunchKernelGGL(K<kQ4_1>, __VA_ARGS__); break;                       \
        case kQ5_0: hipLaunchKernelGGL(K<kQ5_0>, __VA_ARGS__); break;                       \
        case kQ8_0: hipLaunchKernelGGL(K<kQ8_0>, __VA_ARGS__); break;                       \
        case kQ4_K: hipLaunchKernelGGL(K<kQ4_K>, __VA_ARGS__); break;                       \
        case kQ5_K: hipLaunchKernelGGL(K<kQ5_K>, __VA_ARGS__); break;                       \
        case kQ6_K: hipLaunchKernelGGL(K<kQ6_K>, __VA_ARGS__); break;                       \
        case kTQ2_0: hipLaunchKernelGGL(K<kTQ2_0>, __VA_ARGS__); break;                     \
        default: return hipErrorInvalidValue;                                              \
    }

hipError_t launch_matvec_q8(const Packed& m, const void* xq, size_t n, float* out, size_t out_stride, hipStream_t s) {
    const int R = pick_rows_per_tile(m.type, m.rows, m.cols);
    BH_DISPATCH(m.type, k_matvec_q8, dim3(cdiv(m.rows, R), static_cast<unsigned>(n)), dim3(kThreads), 0, s, m, R,
                static_cast<const uint8_t*>(xq), out, out_stride);
    return hipGetLastError();
}

hipError_t launch_gemv(GemvArgs g, hipStream_t s) {
    if (g.gelu_in != nullptr && (g.n != 1 || g.add)) return hipErrorInvalidValue;
    unsigned tiles = 0;
    for (int i = 0; i < g.n; ++i) {
        if (g.t[i].m.type != g.t[0].m.type) return hipErrorInvalidValue;
        g.t[i].R = pick_rows_per_tile(g.t[i].m.type, g.t[i].m.rows, g.t[i].m.cols);
        g.t[i].tiles = static_cast<int>(cdiv(g.t[i].m.rows, g.t[i].R));
        tiles += static_cast<unsigned>(g.t[i].tiles);
    }
    BH_DISPATCH(g.t[0].m.type, k_gemv, dim3(tiles), dim3(kThreads), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_gateup(GateUpArgs g, hipStream_t s) {
    if (g.gate.type != g.up.type) return hipErrorInvalidValue;
    // two tiles (gate, up) per workgroup: each within half the per-thread budget
    g.R = pick_rows_per_tile(g.gate.type, g.gate.rows, g.gate.cols * 2);
    BH_DISPATCH(g.gate.type, k_gateup, dim3(cdiv(g.gate.rows, g.R)), dim3(kThreads), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_head(HeadArgs g, hipStream_t s) {
    g.R = pick_rows_per_tile(g.m.type, g.m.rows, g.m.cols);
    BH_DISPATCH(g.m.type, k_head, dim3(cdiv(g.m.rows, g.R)), dim3(kThreads), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& g, hipStream_t s) {
    hipLaunchKernelGGL(k_attn, dim3(g.kv_heads, g.max_splits), dim3(kThreads), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_attention_plain(const AttnArgs& g, hipStream_t s) {
    const int hpk = g.kv_heads > 0 ? g.heads / g.kv_heads : 0;
    if (g.head_dim < 16 || g.head_dim > kPlainMaxHead || g.head_dim % 16 != 0 || hpk < 1 || hpk > 16 ||
        hpk * g.kv_heads != g.heads || g.qn == nullptr || g.gsc == nullptr)
        return hipErrorInvalidValue;
    const unsigned pos_blocks = static_cast<unsigned>((g.ctx + 63) / 64);  // the most any position needs
    hipLaunchKernelGGL(k_plain_prologue, dim3(static_cast<unsigned>(g.heads + (g.no_kv ? 0 : g.kv_heads))), dim3(64), 0, s, g);
    hipLaunchKernelGGL(k_plain_scores, dim3(static_cast<unsigned>(g.heads), pos_blocks), dim3(64), 0, s, g);
    hipLaunchKernelGGL(k_plain_values, dim3(static_cast<unsigned>(g.heads), static_cast<unsigned>(g.head_dim / 64 + (g.head_dim % 64 != 0))),
                       dim3(64), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_pre_attention_plain(const PrePlainArgs& p, hipStream_t s) {
    const AttnArgs& g = p.a;
    const int hpk = g.kv_heads > 0 ? g.heads / g.kv_heads : 0;
    if (g.head_dim < 16 || g.head_dim > kPlainMaxHead || g.head_dim % 16 != 0 || hpk < 1 || hpk > 16 ||
        hpk * g.kv_heads != g.heads || g.qn == nullptr || p.ntok < 1 || p.pos0 < 0 || !pre_plain_fits(p.pos0 + p.ntok))
        return hipErrorInvalidValue;
    // a layer reading another layer's cache (no_kv) forms its queries only
    hipLaunchKernelGGL(k_pre_plain_prologue, dim3(static_cast<unsigned>(p.ntok), static_cast<unsigned>(g.heads + (g.no_kv ? 0 : g.kv_heads))),
                       dim3(64), 0, s, p);
    hipLaunchKernelGGL(k_pre_plain_attn, dim3(static_cast<unsigned>(p.ntok), static_cast<unsigned>(g.heads)), dim3(kThreads), 0, s, p);
    return hipGetLastError();
}

int attention_max_splits(int ctx) { return (ctx + kSplit - 1) / kSplit; }

hipError_t launch_post_add(float* h, const float* p, const float* w, float eps, int n, hipStream_t s, float out_scale) {
    hipLaunchKernelGGL(k_post_add, dim3(1), dim3(kThreads), 0, s, h, p, w, eps, n, out_scale);
    return hipGetLastError();
}

hipError_t launch_scale(float* h, float out_scale, int n, hipStream_t s) {
    hipLaunchKernelGGL(k_scale, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, h, out_scale, n);
    return hipGetLastError();
}

hipError_t launch_ple_inputs(float* in, const Packed& table, const float* norm, const int* seq, const int* pos, int layers,
                             int dim, float proj_scale, float table_scale, float eps, hipStream_t s) {
    if (layers < 1 || dim < 1 || static_cast<size_t>(layers) * dim != table.cols) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_ple_inputs, dim3(static_cast<unsigned>(layers)), dim3(kThreads), 0, s, in, table, norm, seq, pos, dim,
                       proj_scale, table_scale, eps);
    return hipGetLastError();
}

hipError_t launch_ssm(const SsmArgs& g, hipStream_t s) {
    if (g.dim < 1 || g.dim > kThreads || g.heads < 1 || g.taps < 2 || g.taps > 8 || g.qkv_dim != 3 * g.heads * g.dim)
        return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(g.heads)), block(kThreads);
    if (g.dim == 64) hipLaunchKernelGGL(k_ssm<64>, grid, block, 0, s, g);
    else if (g.dim == 128) hipLaunchKernelGGL(k_ssm<128>, grid, block, 0, s, g);
    else hipLaunchKernelGGL(k_ssm_any, grid, block, 0, s, g);
    return hipGetLastError();
}

hipError_t launch_pre_ssm(const SsmArgs& g, int pos0, int ntok, int ab_stride, hipStream_t s) {
    if (!pre_ssm_fits(g.dim) || g.heads < 1 || g.taps < 2 || g.taps > 8 || g.qkv_dim != 3 * g.heads * g.dim || ntok < 1 || pos0 < 0)
        return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(g.heads)), block(kThreads);
    if (g.dim == 64) hipLaunchKernelGGL(k_pre_ssm<64>, grid, block, 0, s, g, pos0, ntok, ab_stride);
    else hipLaunchKernelGGL(k_pre_ssm<128>, grid, block, 0, s, g, pos0, ntok, ab_stride);
    return hipGetLastError();
}

hipError_t launch_qgate_split(const float* qg, float* q, float* gate, int heads, int hd, hipStream_t s) {
    const int n = heads * hd;
    hipLaunchKernelGGL(k_qgate_split, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, qg, q,
                       gate, hd, n);
    return hipGetLastError();
}

hipError_t launch_sigmoid_gate(float* att, const float* gate, int n, hipStream_t s) {
    hipLaunchKernelGGL(k_sigmoid_gate, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, att,
                       gate, n);
    return hipGetLastError();
}

hipError_t launch_log1pf(const float* x, float* y, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_log1pf, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

hipError_t launch_conv(const float* bcx, uint16_t* cache, const float* w, int taps, const int* pos, int n, float* out,
                       hipStream_t s) {
    hipLaunchKernelGGL(k_conv, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, bcx, cache, w,
                       taps, pos, n, out);
    return hipGetLastError();
}

hipError_t launch_tanhf(const float* x, float* y, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_tanhf, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

hipError_t launch_embed(const Packed& m, const PickState& ps, float* h, float scale, hipStream_t s) {
    hipLaunchKernelGGL(k_embed, dim3(1), dim3(kThreads), 0, s, m, ps, h, scale);
    return hipGetLastError();
}

hipError_t launch_finalize(const PickState& ps, hipStream_t s) {
    hipLaunchKernelGGL(k_finalize, dim3(1), dim3(64), 0, s, ps);
    return hipGetLastError();
}

hipError_t launch_advance(int* pos, hipStream_t s) {
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, pos);
    return hipGetLastError();
}

}  // namespace bh
