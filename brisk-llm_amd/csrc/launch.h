// Host-side launchers of the token-loop kernels and their argument blocks.
#pragma once

#include <hip/hip_runtime.h>

#include "device.h"
#include "layout.h"

namespace bh {

constexpr int kSplit = 64;          // attention positions per split / per LDS chunk
constexpr int kExactMax = 512;      // contexts up to this length take the exact-order attention
constexpr int kExactScores = 4096;  // ... when heads-per-kv x length fits this many LDS scores
__host__ __device__ inline bool attn_is_exact(int L, int hpk) { return L <= kExactMax && L * hpk <= kExactScores; }

struct GemvTarget {
    Packed m;
    float* out;
    int R;      // rows per tile (set by the launcher)
    int tiles;  // tiles of this target (set by the launcher)
};

struct GemvArgs {
    GemvTarget t[4];
    int n;                // targets
    const float* x;       // activation row (f32)
    const float* normw;   // rms_norm weight applied to x first, or null
    float eps;
    int add;              // 1: out += W x (residual), 0: out = W x
    const float* gelu_in; // non-null: out[r] = gelu(W x)[r] * gelu_in[r] (gelu_mul_f32; Gemma 4's per-layer gate)
};

struct GateUpArgs {
    Packed gate, up;
    int R;
    const float* x;
    const float* normw;   // ffn_norm
    float eps;
    int relu2;            // BitNet squared-ReLU gate
    int gelu;             // Gemma GELU (tanh form) gate
    float* act;
};

struct AttnArgs {
    const float* q;       // this token's raw projections (before norms and RoPE): [heads][head_dim]
    const float* k;       // [kv_heads][head_dim]
    const float* v;
    const float* qnorm;   // per-head q/k RMS weights (Qwen3) or null
    const float* knorm;
    const float* qbias;   // projection biases added to the raw q, k, v (Qwen2) or null
    const float* kbias;   // ([heads][head_dim], [kv_heads][head_dim], ditto)
    const float* vbias;
    const float* rope;    // [max_context][rope_dim] cos, sin pairs; null on a layer without RoPE (SmolLM3)
    int rope_dim;         // dimensions rotated (the head's first rope_dim; Phi-3 rotates part of it)
    float eps;
    int neox;
    int window;           // a sliding layer's last `window` positions (Gemma 3); 0: every position
    uint16_t* kcache;     // this layer's [kv_heads][ctx][head_dim]
    uint16_t* vcache;
    const int* pos;
    int ctx, head_dim, heads, kv_heads;
    float scale;
    float* part_acc;      // [heads][max_splits][head_dim]
    float* part_ml;       // [heads][max_splits][2]
    int max_splits;
    unsigned* tickets;    // [kv_heads], zero between launches (the merging workgroup re-arms its own)
    // exact attention past the LDS score limit: the scores in global memory, [kv_heads][hpk][ctx]
    // (null: such contexts take the split attention)
    float* gsc;
    float* out;           // [heads][head_dim]
    // the plain attention (launch_attention_plain) only:
    float* qn;            // [heads][head_dim]: the normed and rotated queries
    int vnorm;            // V RMS-normalised without weight before the cache (Gemma 4)
    int no_kv;            // the layer reads another layer's cache and stores no rows (Gemma 4's shared K/V)
    int q_stride;         // floats from one query head's raw rows to the next (0: head_dim)
    const float* gate;    // the output times sigmoid(gate[h * gate_stride + d]) (Qwen3.5), or null
    int gate_stride;
    unsigned long long* stamps;  // optional profiling: key/value head 0's wall clock at sub-phase ends
};

// One token of a Qwen3.5 Gated DeltaNet layer after its projections (src/model.cpp:754-865).
struct SsmArgs {
    const float* qkv;     // this token's attn_qkv rows [q | k | v] before the conv (qkv_dim)
    const float* z;       // attn_gate rows [heads][dim]
    const float* ab;      // ssm_alpha rows [heads], then ssm_beta rows [heads]
    const float* conv_w;  // ssm_conv1d [qkv_dim][taps]
    const float* a;       // ssm_a [heads]
    const float* dt;      // ssm_dt.bias [heads]
    const float* norm;    // ssm_norm [dim]
    float* ring;          // [taps][qkv_dim]: slot p % taps holds position p's attn_qkv rows
    float* state;         // [2][heads][dim (key i)][dim (value j)]: position p reads half p & 1, writes the other
    const int* pos;
    float* out;           // [heads][dim]
    int heads, dim, taps, qkv_dim;
    float eps, q_scale;
};

// The pending greedy pick and the sequence state it updates.
struct PickState {
    unsigned long long* key;   // 0 = no pick pending; else the ordered (logit, index) key of the best row
    int* pos;                  // position of the token the current step processes
    int* seq;                  // token sequence by position
    int seq_len;
    const int* fixed;          // seq[0, *fixed) are caller tokens a pick must not overwrite
};

struct HeadArgs {
    Packed m;             // output projection
    int R;
    const float* x;
    const float* normw;   // output_norm
    float eps;
    float* logits;        // or null
    unsigned long long* key;   // the step's pick key (PickState::key)
    float softcap;        // logits = c tanh(logits / c) before the pick (Gemma); 0: none
};

hipError_t launch_pack(uint32_t type, const void* src, size_t rows, size_t cols, const Packed& dst, hipStream_t s);
// Block-major copy of a packed Q4_0 / Q4_1 / Q5_0 / Q8_0 matrix (dst planes sized as src's).
hipError_t launch_unit_transpose(const Packed& src, const Packed& dst, hipStream_t s);
hipError_t launch_quantize(int kind, const float* x, void* out, size_t count, int bits, hipStream_t s);
hipError_t launch_matvec_q8(const Packed& m, const void* xq, size_t n, float* out, size_t out_stride, hipStream_t s);
hipError_t launch_gemv(GemvArgs g, hipStream_t s);
hipError_t launch_gateup(GateUpArgs g, hipStream_t s);
hipError_t launch_attention(const AttnArgs& g, hipStream_t s);
// The reference's attention for one token by three plain kernels (prologue, scores, softmax with
// values), for any head size up to 512 (a multiple of 16): scores and weights in gsc
// ([heads][ctx]), the queries in qn.
hipError_t launch_attention_plain(const AttnArgs& g, hipStream_t s);
constexpr int kPlainMaxHead = 512;
constexpr int kPlainLdsW = 8192;  // the weights a plain-attention softmax keeps in LDS
// The plain attention for a prompt's ntok tokens at positions pos0 .. (every token's rows and
// outputs at the strides below; the queries' gate, when given, at a.gate + t * q_tok).
struct PrePlainArgs {
    AttnArgs a;    // a.q, a.k, a.v: token 0's raw rows; a.qn: [ntok][heads][head_dim]; a.out: [ntok][heads * head_dim]
    int pos0, ntok;
    int q_tok, kv_tok;  // floats from one token's raw query (key/value) rows to the next
};
inline bool pre_plain_fits(int positions) { return positions <= kPlainLdsW; }
hipError_t launch_pre_attention_plain(const PrePlainArgs& p, hipStream_t s);
hipError_t launch_embed(const Packed& m, const PickState& ps, float* h, float scale, hipStream_t s);
// h = (h + rms_norm(p, w)) * out_scale over n values (Gemma's post-attention / post-feed-forward
// norm with out_scale 1; Gemma 4's per-layer embedding with the layer's output scale).
hipError_t launch_post_add(float* h, const float* p, const float* w, float eps, int n, hipStream_t s, float out_scale = 1.0f);
// h *= out_scale (Gemma 4's layer output scale without per-layer embeddings).
hipError_t launch_scale(float* h, float out_scale, int n, hipStream_t s);
// Gemma 4's per-layer embedding inputs of the token seq[*pos] (src/model.cpp:905-925): for each
// layer l, slice l of in (the per_layer_model_proj rows of the scaled embedding) becomes
// (rms_norm(slice * proj_scale, norm) + table[tok][l * dim ..] * table_scale) * 0.70710678.
hipError_t launch_ple_inputs(float* in, const Packed& table, const float* norm, const int* seq, const int* pos, int layers,
                             int dim, float proj_scale, float table_scale, float eps, hipStream_t s);
hipError_t launch_finalize(const PickState& ps, hipStream_t s);
hipError_t launch_head(HeadArgs g, hipStream_t s);
hipError_t launch_advance(int* pos, hipStream_t s);
hipError_t launch_expf(const float* x, float* y, size_t n, hipStream_t s);
hipError_t launch_tanhf(const float* x, float* y, size_t n, hipStream_t s);
// LFM2's short convolution of the token at *pos: bc = [b | c | x] rows, cache [ctx][n] fp16,
// w [n][taps]; out = c * sum_k w[d][k] bx[pos + k + 1 - taps] with bx = b * x stored at pos.
hipError_t launch_conv(const float* bcx, uint16_t* cache, const float* w, int taps, const int* pos, int n, float* out,
                       hipStream_t s);
// Qwen3.5: one recurrent layer's conv, delta-rule state update and gated norm (one workgroup a head).
hipError_t launch_ssm(const SsmArgs& g, hipStream_t s);
// Qwen3.5 prefill: the recurrence over ntok tokens at positions pos0 .. in one launch (state sizes
// 64 and 128): g.qkv [ntok][qkv_dim], g.z [ntok][heads * dim], alpha and beta of token t at
// g.ab[t * ab_stride + h] and g.ab[t * ab_stride + heads + h], out [ntok][heads * dim].
hipError_t launch_pre_ssm(const SsmArgs& g, int pos0, int ntok, int ab_stride, hipStream_t s);
inline bool pre_ssm_fits(int dim) { return dim == 64 || dim == 128; }
// Qwen3.5 attention: [heads][q | gate] rows split into q and gate; att *= sigmoid(gate).
hipError_t launch_qgate_split(const float* qg, float* q, float* gate, int heads, int hd, hipStream_t s);
hipError_t launch_sigmoid_gate(float* att, const float* gate, int n, hipStream_t s);
hipError_t launch_log1pf(const float* x, float* y, size_t n, hipStream_t s);
hipError_t launch_div_selftest(unsigned long long* bad, hipStream_t s);
hipError_t launch_mfma_rate(int shape, int blocks, int iters, int* out, hipStream_t s);
int attention_max_splits(int ctx);
int pick_rows_per_tile(uint32_t type, size_t rows, size_t cols);

}  // namespace bh
