/* brisk_hip — the C ABI of the MI355X (gfx950) token loop for brisk-llm.
 *
 * Plain pointers and sizes only.  Two layers:
 *
 *  1. Kernel level: the counterpart of the reference's kernel dispatch ABI,
 *     `KernelSet{Matvec, Matmul, Prepare, PreparedBytes}` (src/kernels.h:19-39),
 *     on device memory and a HIP stream (passed as void*; NULL = default stream).
 *     Used by the parity tests to pin the HIP arithmetic against the reference's
 *     scalar dot products (src/quant.cpp:445-596).
 *
 *  2. Session level: the counterpart of `class Engine` (src/engine.h:13-37) as
 *     the reference's `Session` (src/model.h:223-310) and `MetalSession`
 *     (src/metal/metal_session.h:21-37) implement it: eval / eval_all /
 *     rollback / position, over the weights of a `Model(file, repack = false)`
 *     (src/model.cpp:303-530) passed as a table of GGUF-layout tensors.
 *
 * Every call returns 0 on success or a negative BRISK_HIP_E* code; the message,
 * worded as the reference words the same failure where it has one (e.g.
 * "model: context length exceeded", src/model.cpp:704-736), is then available
 * from brisk_hip_last_error() on the calling thread.  Session calls are
 * synchronous: results are in host memory when they return.  A session is not
 * reentrant (like Engine): one caller at a time.
 */
#ifndef BRISK_HIP_H
#define BRISK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BRISK_HIP_ABI_VERSION 3

enum {
    BRISK_HIP_OK = 0,
    BRISK_HIP_EINVAL = -1,    /* bad argument, shape or model (std::runtime_error in the reference) */
    BRISK_HIP_ENODEV = -2,    /* no usable GPU */
    BRISK_HIP_EHIP = -3,      /* a HIP runtime call failed */
    BRISK_HIP_ENOMEM = -4     /* device allocation failed */
};

/* Tensor types: the ggml numbers a GGUF file uses (src/gguf.h:22-27). */
enum {
    BRISK_HIP_F32 = 0,
    BRISK_HIP_Q4_0 = 2,
    BRISK_HIP_Q4_1 = 3,
    BRISK_HIP_Q5_0 = 6,
    BRISK_HIP_Q8_0 = 8,
    BRISK_HIP_Q4_K = 12,
    BRISK_HIP_Q5_K = 13,
    BRISK_HIP_Q6_K = 14,
    BRISK_HIP_TQ2_0 = 35
};

/* Model families on this path (Architecture, src/model.h:21-32). */
enum {
    BRISK_HIP_ARCH_QWEN3 = 0,
    BRISK_HIP_ARCH_LLAMA = 1,
    BRISK_HIP_ARCH_BITNET = 2,
    BRISK_HIP_ARCH_QWEN2 = 3,   /* Q/K/V projection biases, no Q/K norms */
    BRISK_HIP_ARCH_SMOLLM3 = 4, /* Llama-shaped; every fourth layer attends without RoPE */
    BRISK_HIP_ARCH_GEMMA3 = 5,  /* Q/K norms, post-norms, GELU gate, sliding-window layers, scaled embeddings */
    BRISK_HIP_ARCH_PHI3 = 6,    /* fused QKV and gate/up tensors, partial rotary, LongRoPE factors */
    BRISK_HIP_ARCH_LFM2 = 7,    /* short-convolution layers (those with blk.N.shortconv.* tensors) between attention layers */
    BRISK_HIP_ARCH_QWEN35 = 8,  /* Gated DeltaNet layers (those with blk.N.ssm_a) between gated attention layers */
    BRISK_HIP_ARCH_GEMMA4 = 9   /* Gemma 3 plus per-layer embeddings, K/V sharing, wider global heads, unscaled scores */
};

/* The fields of ModelConfig (src/model.h:36-60) this path reads. */
typedef struct {
    int arch;
    uint32_t vocab, embd, layers, heads, kv_heads, head_dim, ff, context_length;
    float rope_base, rms_epsilon;
    /* Gemma 3 (zero for the other families; ModelConfig, src/model.h:63-71): */
    uint32_t sliding_window; /* layers with l % 6 != 5 see only the last this-many positions; 0: none */
    float rope_base_local;   /* those layers' RoPE base (rope.freq_base_swa) */
    float rope_scale;        /* the other layers' position scale, 1 / rope.scaling.factor; 0 reads as 1 */
    float final_softcap;     /* logits = c tanh(logits / c); 0: none */
    /* RoPE details (src/model.h:48-62); zero reads as the default: */
    uint32_t rope_dim;       /* dimensions rotated, the first of each head (Phi-3); 0: the head size */
    float rope_attn_factor;  /* cos and sin scaled by it (Phi-3 LongRoPE); 0 reads as 1 */
    uint32_t rope_original_context; /* past it, rope_factors_long.weight replaces rope_factors_short.weight */
    uint32_t conv_taps;      /* LFM2's short-convolution width (shortconv.l_cache), 2 to 8; 0 elsewhere */
    /* ModelConfig's flags (src/model.h:45-110); zero reads as the family's value: */
    int32_t rope_neox;       /* 1: RoPE pairs (i, i + rotated / 2) ("NeoX"); 2: adjacent pairs (2 i, 2 i + 1) */
    uint32_t no_rope_step;   /* every no_rope_step-th layer attends without RoPE (SmolLM3: 4); 0xFFFFFFFF: none */
    float embedding_scale;   /* the embedding rows are multiplied by it (Gemma: sqrt(embd)) */
    int32_t gelu;            /* 1: GELU (tanh) gating (Gemma); 2: SiLU / the family's */
    /* Qwen3.5's Gated DeltaNet layers (ModelConfig, src/model.h:100-109); zero elsewhere: */
    uint32_t ssm_state;      /* ssm.state_size: a head's state is ssm_state x ssm_state, at most 256 */
    uint32_t ssm_k_heads;    /* ssm.group_count */
    uint32_t ssm_v_heads;    /* ssm.time_step_rank (equal to ssm_k_heads) */
    uint32_t ssm_inner;      /* ssm.inner_size = ssm_v_heads x ssm_state */
    uint32_t ssm_conv;       /* ssm.conv_kernel: the causal conv's width, 2 to 8 */
    /* Gemma 4 (ModelConfig, src/model.h:76-118); zero / NULL elsewhere.  head_dim, kv_heads and
     * ff hold the largest of the layers' values; the tables are read during create only: */
    uint32_t head_dim_local;        /* the sliding layers' head size; 0: head_dim */
    uint32_t kv_from_start;         /* layers from this one on read an earlier layer's K/V (kv_layer_of); 0: none */
    uint32_t ple_dim;               /* the per-layer embedding width; 0: none */
    float attention_scale;          /* the score scale; 0: 1 / sqrt(the layer's head size) */
    int32_t value_norm;             /* 1: V is RMS-normalised, without weight, before the cache */
    const uint8_t* sliding_pattern; /* [layers], 1 = sliding; NULL: with sliding_window, every layer but each sixth */
    const uint32_t* ff_dims;        /* [layers] feed-forward widths; NULL: ff everywhere */
    const uint32_t* kv_head_counts; /* [layers] key/value heads; NULL: kv_heads everywhere */
} brisk_hip_config;

/* One model tensor in GGUF layout (host memory, e.g. the file's mmap):
 * matrices are rows x cols blocks as stored (GGUF dims {cols, rows}),
 * vectors have rows = 1 and type BRISK_HIP_F32.  Names are the GGUF names the
 * reference's loader reads (token_embd.weight, blk.N.attn_q.weight, ...). */
typedef struct {
    const char* name;
    int type;
    uint64_t rows, cols;
    const void* data;
} brisk_hip_tensor;

typedef struct brisk_hip_session brisk_hip_session;

/* Device bytes a session takes, by part (MemoryEstimate, src/memory.h:13-20). */
typedef struct {
    size_t weights;  /* the repacked matrices and the norm vectors */
    size_t cache;    /* the fp16 K/V caches for the context */
    size_t scratch;  /* activations, hand-off words, attention partials, RoPE table, prefill buffers, logits */
    size_t total;
} brisk_hip_memory;

const char* brisk_hip_last_error(void);
int brisk_hip_abi_version(void);
int brisk_hip_device_count(int* count);

/* ---------------------------------------------------------------- kernel level */

/* Device bytes of a matrix after the load-time repack (counterpart of
 * KernelSet::PreparedBytes, src/kernels.h:31-32, for weights). */
size_t brisk_hip_packed_bytes(int type, size_t rows, size_t cols);

/* Repacks rows x cols GGUF blocks (device memory) into the coalesced HBM layout
 * at `packed` (brisk_hip_packed_bytes bytes).  Replaces the reference's
 * load-time repacks (src/model.cpp:481-525). */
int brisk_hip_pack(int type, const void* gguf_blocks, size_t rows, size_t cols, void* packed, void* stream);

/* quantize_q8_0 / quantize_q8_k(bits) (src/quant.h:202-203, src/quant.cpp:115-194):
 * `count` floats -> GGUF BlockQ8_0 (34 B) / BlockQ8_K (292 B) rows, bit-exact. */
int brisk_hip_quantize_q8_0(const float* x, void* out, size_t count, void* stream);
int brisk_hip_quantize_q8_k(const float* x, void* out, size_t count, int bits, void* stream);

/* KernelSet::matvec and ::matmul (src/kernels.h:19-25): out[t*out_stride + r] =
 * dot(row r, activation row t) over a packed matrix and pre-quantised
 * activations (Q8_0 rows for Q4_0/Q8_0, Q8_K rows for Q4_K/Q6_K/TQ2_0).  Each
 * output is bit-identical to the reference's generic kernels. `flags`: bit 0
 * selects, for TQ2_0, the x86 TQ2_0x16 arithmetic (src/quant.cpp:789-802).
 * Rows of any width (src/kernels.cpp:13-30); rows wider than 8192 must be
 * whole 256-value blocks.  For n > 1, and for rows wider than 8192, matmul
 * allocates a scratch block for the call: the planar activation rows, and for
 * Q6_K and Q5_K the matrix's expanded weight planes (about 2 bytes a weight),
 * as a session's batched prefill holds them. */
int brisk_hip_matvec(int type, int flags, const void* packed, size_t rows, size_t cols, const void* xq, float* out,
                     void* stream);
int brisk_hip_matmul(int type, int flags, const void* packed, size_t rows, size_t cols, const void* xq, size_t n,
                     float* out, size_t out_stride, void* stream);

/* brisk_hip_matmul without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, hosts that forbid hipMalloc).  For n > 1 (or
 * rows wider than 8192) the activation rows are staged in a static device buffer of 4 MiB, one
 * per GPU, held until the process ends (n x ceil(cols / 256) x 256 x 1.375
 * bytes must fit, e.g. 372 rows of 8192 columns; larger requests fail with
 * BRISK_HIP_EINVAL).  Outputs are identical to brisk_hip_matmul's.  The call
 * does not synchronise: the buffer is reused by the next call on that GPU, so
 * calls on one GPU that overlap (other streams, other threads) race. */
int brisk_hip_matmul_noalloc(int type, int flags, const void* packed, size_t rows, size_t cols, const void* xq, size_t n,
                             float* out, size_t out_stride, void* stream);

/* The decode GEMV of the token loop: quantises the f32 row x in-kernel (after
 * rms_norm with weight `norm_w` and `eps` when norm_w is non-null), then
 * out = W x, or out += W x when `accumulate` (the residual update).  Rows of
 * at most 8192 values (the row is held in LDS). */
int brisk_hip_gemv(int type, int flags, const void* packed, size_t rows, size_t cols, const float* x,
                   const float* norm_w, float eps, float* out, int accumulate, void* stream);

/* expf exactly as the reference's host libm computes it (glibc's expf, which
 * softmax_f32 and silu_mul_f32 call: src/kernels_f32.cpp:276-289); the token
 * loop's softmax and SiLU use the same device routine.  y[i] = expf(x[i]). */
int brisk_hip_expf(const float* x, float* y, size_t n, void* stream);

/* tanhf exactly as the reference's host libm computes it (glibc 2.35's, which
 * gelu_mul_f32 and the final logit softcap call: src/kernels_f32.cpp:291-296,
 * src/model.cpp:1206-1209); the Gemma epilogues use the same device routine.
 * y[i] = tanhf(x[i]). */
int brisk_hip_tanhf(const float* x, float* y, size_t n, void* stream);

/* log1pf exactly as the reference's host libm computes it (glibc 2.35's, the
 * softplus of Qwen3.5's recurrence, src/model.cpp:827).  No counterpart in the
 * reference's API: it exposes the device routine for parity tests.
 * y[i] = log1pf(x[i]). */
int brisk_hip_log1pf(const float* x, float* y, size_t n, void* stream);

/* Self-test of the shortcuts the device arithmetic takes: the two short
 * divisions of the activation quantisation (a / 127 for a >= 0, and 1 / d),
 * each compared with IEEE division on every finite input it can take, and the
 * hardware float-to-half conversion, compared with the reference's bit-level
 * conversion (src/quant.cpp:87-113) on every float, and the mixed-precision
 * multiply of a float by a half (the attention's q k and w v products) against
 * the product of the widened half, on every float.  mismatches[0..3] receive
 * the counts (all 0 when the shortcuts are exact).  Test support; no
 * counterpart in the reference. */
int brisk_hip_div_selftest(unsigned long long* mismatches);

/* The int8 matrix-core rate this device sustains (TOP/s): independent MFMA
 * chains a wave on register operands, four workgroups a compute unit, timed
 * with HIP events.  shape 0: v_mfma_i32_16x16x64_i8 (the prefill GEMMs'
 * instruction), 1: v_mfma_i32_32x32x32_i8.  The measured ceiling the prefill
 * GEMMs' MFMA fraction is read against.  Measurement support; no counterpart
 * in the reference. */
int brisk_hip_mfma_rate(int shape, double* int8_tops);

/* ---------------------------------------------------------------- session level */

/* What a session of these tensors and context would take on the device
 * (estimate_memory, src/memory.cpp:46-96, for HBM instead of host RAM):
 * computed from the shapes alone, nothing is allocated.  max_context as for
 * brisk_hip_session_create. */
int brisk_hip_session_estimate(const brisk_hip_config* config, const brisk_hip_tensor* tensors, size_t n_tensors,
                               size_t max_context, brisk_hip_memory* out);

/* Free and total device memory of `device` (available_memory,
 * src/memory.cpp:98-116, for HBM). */
int brisk_hip_device_memory(int device, size_t* free_bytes, size_t* total_bytes);

/* Engine construction, as `MetalSession(model, file bytes, max_context)`
 * (src/main.cpp:206): copies and repacks every tensor to the GPU `device`.
 * max_context 0 = the model's context length; otherwise min of both.
 * Before allocating, the estimate (plus a 256 MB margin) is checked against
 * the device's free memory, as check_memory (src/memory.cpp:118-135) does for
 * RAM: BRISK_HIP_ENOMEM with a message naming the shortfall, unless
 * BRISK_NO_MEMORY_CHECK is set. */
int brisk_hip_session_create(const brisk_hip_config* config, const brisk_hip_tensor* tensors, size_t n_tensors,
                             size_t max_context, int device, brisk_hip_session** out);
void brisk_hip_session_destroy(brisk_hip_session* s);

/* Engine::eval (src/engine.h:17-21): appends tokens, writes the last token's
 * vocab logits to `logits` (host; may be NULL to skip the copy). */
int brisk_hip_session_eval(brisk_hip_session* s, const int32_t* tokens, size_t n, float* logits);

/* Engine::eval_all (src/engine.h:23-26): 1..64 tokens, logits of every token ([n][vocab], host). */
int brisk_hip_session_eval_all(brisk_hip_session* s, const int32_t* tokens, size_t n, float* logits);

/* eval followed by the greedy pick on the device (Sampler::sample at
 * temperature 0, src/sampler.cpp:11-13: first index of the max); no logits copy. */
int brisk_hip_session_eval_greedy(brisk_hip_session* s, const int32_t* tokens, size_t n, int32_t* next);

/* cmd_generate's greedy loop (src/main.cpp:220-299) with the loop on the
 * device: eval(prompt), then n_gen picks, each evaluated but the last.
 * out[n_gen] receives the picked ids. */
int brisk_hip_session_generate(brisk_hip_session* s, const int32_t* prompt, size_t n_prompt, size_t n_gen, int32_t* out);

/* The body of that loop on its own: n more greedy steps, each evaluating the
 * pending pick (the one the previous eval / decode chose) and picking the next;
 * out[n] (may be NULL) receives the n new picks.  No host round trip between
 * steps.  Needs a prior eval; advances position() by n. */
int brisk_hip_session_decode(brisk_hip_session* s, size_t n, int32_t* out);

/* Engine::rollback / position (src/engine.h:28-31). */
int brisk_hip_session_rollback(brisk_hip_session* s, size_t position);
size_t brisk_hip_session_position(const brisk_hip_session* s);
size_t brisk_hip_session_max_context(const brisk_hip_session* s);

/* Device pointer and size of layer `layer`'s fp16 key (value = 0) or value (1)
 * cache, laid out [kv_head][max_context][head_dim] as the reference's
 * (src/model.cpp:984-991).  With brisk_hip_session_set_position it lets a
 * caller install a pre-filled cache (no Engine counterpart).  BRISK_HIP_EINVAL
 * for a layer without one (an LFM2 short-convolution layer). */
int brisk_hip_session_kv_cache(brisk_hip_session* s, int layer, int value, void** device_ptr, size_t* bytes);
int brisk_hip_session_set_position(brisk_hip_session* s, size_t position);

/* The session's HIP stream (hipStream_t), for timing with events. */
void* brisk_hip_session_stream(brisk_hip_session* s);

/* Profiling: with BRISK_HIP_TRACE set when the session was created, the
 * persistent loop records a 100 MHz wall-clock stamp at the start and after
 * every grid barrier of its last launch; copies up to n stamps, returns the
 * count copied (0 when tracing is off). */
size_t brisk_hip_session_trace(brisk_hip_session* s, unsigned long long* out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
