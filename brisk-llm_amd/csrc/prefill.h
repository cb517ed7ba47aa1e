// Batched prefill (prefill.hip): argument blocks and launchers.
#pragma once

#include <hip/hip_runtime.h>

#include "launch.h"

namespace bh {

// Activations quantised per token: int8 values [T][stride], scales
// [T][stride / 32] (Q8_0: per 32 values; Q8_K: per 256), int32 sums
// [T][stride / 16] (Q8_0: per 32; Q8_K: the bsums per 16).
struct ActPlanar {
    int8_t* qs;
    float* d;
    int32_t* bs;
    int stride;  // values per token row (>= the widest input, a multiple of 256)
};

enum { kMmStore = 0, kMmAdd = 1, kMmPair = 2, kMmGated = 3 };

struct MmArgs {
    Packed m;        // the weight matrix (rows x cols)
    Packed m2;       // kMmPair: the up matrix (same shape and format as m, the gate)
    ActPlanar x;     // ntok quantised rows of m.cols values
    int ntok;
    float* out;      // out[t * ostride + r]
    int ostride;
    int relu2;       // kMmPair: BitNet's squared-ReLU gate instead of SiLU
    int gelu;        // kMmPair: Gemma's GELU (tanh form) gate instead of SiLU
    // Q6_K / Q4_K / Q5_K: the expanded planes of m (and m2) from launch_mx_expand, or null (the
    // packed-plane GEMMs)
    const int8_t* qx;
    const float* qxd;
    const uint8_t* qxm;
    const int8_t* qx2;
    const float* qxd2;
    const uint8_t* qxm2;
};

// A matrix's expanded planes: int8 lo and hi weights, float scales (and dmins), and the
// K-quants' sub-block mins (null for Q6_K).
struct MxPlanes {
    const int8_t* q = nullptr;
    const float* d = nullptr;
    const uint8_t* mn = nullptr;
};

// Rows the widest workgroup of the expanded-plane GEMM computes; the planes pad rows to it.
constexpr int kMxRows = 128;
// Formats the prefill multiplies from expanded planes: Q6_K and Q5_K; Q4_K when
// BRISK_HIP_PREFILL_Q4X=1 (its packed-plane GEMM folds the scales without them); none when
// BRISK_HIP_PREFILL_MX=0.
bool mx_expanded(uint32_t type);
// Bytes of a Q6_K, Q4_K or Q5_K matrix's expanded planes.
size_t mx_bytes(uint32_t type, uint32_t rows, uint32_t cols);
// Writes the expanded planes of m into mem (mx_bytes of it); *out points into mem.
hipError_t launch_mx_expand(const Packed& m, void* mem, MxPlanes* out, hipStream_t s);

struct PreAttnArgs {
    AttnArgs a;      // layer, shape and cache (a.q/k/v/pos/out unused)
    float* q;        // [T][qstride] raw, then normed and rotated by k_pre_rope
    const float* k;  // [T][kvstride]
    const float* v;
    float* out;      // [T][qstride] attention output
    int qstride, kvstride;
    int pos0;        // position of token 0
    int legacy;      // 1: the staged-chunk exact kernel (k_pre_attn_blk) in place of k_pre_attn_rows
    int mfma;        // 1: prompts of kFaMinTok tokens or more take the MFMA attention (not order-exact)
    // When qout.qs is set and the launch takes k_pre_attn_rows with heads-per-kv x head_dim = 256,
    // that kernel also writes each (token, kv head)'s output as the 256-value activation block kv of
    // qout (Q8_K when q8k, else Q8_0; qbits as act_bits), and launch_pre_attention reports it in
    // *quantised.  Otherwise qout is untouched and the caller quantises out itself.
    ActPlanar qout;
    int q8k, qbits;
};

// Shapes the MFMA prefill attention (opt-in) takes: 64 query rows a workgroup.
inline bool pre_attn_mfma_fits(int hpk, int head_dim) {
    return hpk >= 1 && hpk <= 64 && 64 % hpk == 0 && (head_dim == 64 || head_dim == 128);
}

hipError_t launch_mm(const MmArgs& g, int mode, hipStream_t s);
// Two store GEMMs of one activation (Q and K): one launch when both are packed-plane Q4_K of one
// width, else launch_mm of each.
hipError_t launch_mm_two(const MmArgs& a, const MmArgs& b, hipStream_t s);
// The GEMMs take rows whose length is a multiple of this many values (one staged chunk).
constexpr int kMmChunkCols = 256;
hipError_t launch_pre_quant(const float* x, int xstride, const float* w, float eps, int cols, int ntok, bool q8k, int bits,
                            const ActPlanar& out, hipStream_t s);
hipError_t launch_pre_planar(const void* xq, int cols, int ntok, bool q8k, const ActPlanar& out, hipStream_t s);
hipError_t launch_pre_embed(const Packed& m, const int* seq, int pos0, int ntok, float* h, float scale, hipStream_t s);
// h[t] += rms_norm(p[t], w) for the ntok rows of n values (Gemma's post-norms)
// h[t] = (h[t] + rms_norm(p[t], w)) * out_scale (Gemma 4's per-layer embedding with its output scale)
hipError_t launch_pre_post_add(float* h, const float* p, const float* w, float eps, int n, int ntok, hipStream_t s,
                               float out_scale = 1.0f);
// h *= out_scale over ntok rows of n values
hipError_t launch_pre_scale(float* h, float out_scale, int n, int ntok, hipStream_t s);
// Gemma 4's per-layer embedding inputs of tokens seq[pos0 ..] (src/model.cpp:905-925): in is [ntok][layers][dim]
hipError_t launch_pre_ple_inputs(float* in, const Packed& table, const float* norm, const int* seq, int pos0, int ntok, int layers,
                                 int dim, float proj_scale, float table_scale, float eps, hipStream_t s);
// g[t][i] = gelu(g[t][i]) * in[t * in_stride + i], ntok rows of n
hipError_t launch_pre_gelu_mul(float* g, const float* in, int n, int in_stride, int ntok, hipStream_t s);
// LFM2's short convolution for ntok tokens at positions pos0 ..: bcx [ntok][3 n] in, out [ntok][n]
hipError_t launch_pre_conv(const float* bcx, uint16_t* cache, const float* w, int taps, int pos0, int n, int ntok, float* out,
                           hipStream_t s);
// x[i] = cap tanh(x[i] / cap) (Gemma's final logit soft-capping)
hipError_t launch_softcap(float* x, size_t n, float cap, hipStream_t s);
hipError_t launch_pre_attention(const PreAttnArgs& p, int ntok, hipStream_t s, bool* quantised = nullptr);

}  // namespace bh
