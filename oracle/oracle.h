/* TEST INFRASTRUCTURE ONLY — the CPU oracle for the HIP token loop.
 *
 * A plain-C restatement of the reference's CPU path (roticv/brisk-llm,
 * src/quant.cpp, src/kernels.cpp, src/kernels_f32.cpp portable branch,
 * src/model.cpp Session::eval_batch) for the three families the benchmark
 * configs use (qwen3, llama, bitnet).  It is only ever used as the checker by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg; the product
 * path never links or calls it.
 *
 * Pinning: every function is checked against the reference itself (the
 * compiled oracle/_ref library) bit for bit in tests/test_oracle.py, plus the
 * known-answer and exhaustive tests of the reference's tests/kernels_test.cpp
 * restated there.  No function here is "parity unpinned".
 */
#ifndef BRISK_ORACLE_H
#define BRISK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor types (src/gguf.h:22-27). */
enum { OR_F32 = 0, OR_Q4_0 = 2, OR_Q4_1 = 3, OR_Q5_0 = 6, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14, OR_TQ2_0 = 35 };
/* Architectures of src/model.h:21-32 that the configs use. */
enum { OR_QWEN3 = 0, OR_LLAMA = 1, OR_BITNET = 2, OR_QWEN2 = 3, OR_SMOLLM3 = 4, OR_GEMMA3 = 5, OR_PHI3 = 6, OR_LFM2 = 7, OR_QWEN35 = 8, OR_GEMMA4 = 9 };

typedef struct {
    int arch;
    int embd, layers, heads, kv_heads, head_dim, ff, vocab;
    float rope_base, eps;
    int max_context;
    /* Gemma 3 (src/model.cpp:170-176, :286); zero elsewhere */
    int sliding_window;
    float rope_base_local, rope_scale, final_softcap;
    /* RoPE details (src/model.h:48-62): rotated dims (0: head size), cos/sin factor (0: 1), and
     * Phi-3's LongRoPE switch-over context */
    int rope_dim;
    float rope_attn_factor;
    int rope_original_context;
    int conv_taps; /* LFM2 short-convolution width */
    /* Qwen3.5 Gated DeltaNet layers (src/model.h:100-109): state size, key and value heads,
     * inner width (value heads x state), conv width; the layers with blk.N.ssm_a are recurrent */
    int ssm_state, ssm_k_heads, ssm_v_heads, ssm_inner, ssm_conv;
    /* Gemma 4 (src/model.cpp:189-226, src/model.h:76-118); zero / NULL elsewhere: the sliding
     * layers' head size (0: head_dim), the first layer reading another's K/V (0: none), the
     * per-layer embedding width, the score scale (0: 1 / sqrt(head size)), V's weightless norm,
     * and per-layer tables (NULL: every sixth layer global; ff and kv_heads everywhere) */
    int head_dim_local, kv_from_start, ple_dim, value_norm;
    float attention_scale;
    const uint8_t* sliding_pattern;
    const int32_t* ff_dims;
    const int32_t* kv_head_counts;
} oracle_config;

/* One tensor of the model: `rows` x `cols` (vectors: rows = 1), GGUF bytes. */
typedef struct {
    const char* name;
    int type;
    uint64_t rows, cols;
    const void* data;
} oracle_tensor;

float or_half_to_float(uint16_t h);
uint16_t or_float_to_half(float f);
void or_quantize_q8_0(const float* x, void* out, size_t count);
void or_quantize_q8_k(const float* x, void* out, size_t count, int bits);
/* Row dot products, over `blocks` blocks.  `type` is a tensor type; for TQ2_0
 * `lut16` selects the x86 load-time TQ2_0x16 arithmetic (7-bit activations). */
float or_dot(int type, int lut16, const void* w_row, const void* x, size_t blocks);
void or_matvec(int type, const void* w, size_t rows, size_t cols, const void* x, float* out);
void or_dequantize(int type, const void* blocks, float* out, size_t count);
void or_repack_tq2_0x16(const void* in, size_t rows, size_t blocks, void* out);
float or_dot_f32(const float* a, const float* b, size_t n);
void or_softmax(float* x, size_t n);
void or_rms_norm(const float* x, const float* w, float eps, float* out, size_t n);
/* glibc expf over a batch, and the check of the HIP loop's restatement of it. */
void or_expf_batch(const float* x, float* y, size_t n);
uint64_t or_expf_check(uint32_t stride, uint64_t* checked);
void or_tanhf_batch(const float* x, float* y, size_t n);
uint64_t or_tanhf_check(uint32_t stride, uint64_t* checked);
/* glibc log1pf over a batch, and the check of the HIP recurrence's restatement of it. */
void or_log1pf_batch(const float* x, float* y, size_t n);
uint64_t or_log1pf_check(uint32_t stride, uint64_t* checked);
/* Activation bits a matrix of `type` with `rows` rows takes on x86 (src/model.cpp:496-503, src/quant.cpp:144). */
int or_activation_bits(int type, size_t rows);

typedef struct oracle_session oracle_session;
oracle_session* or_session_create(const oracle_config* cfg, const oracle_tensor* tensors, size_t n_tensors);
void or_session_destroy(oracle_session* s);
/* eval / eval_all of src/model.cpp:704-727: logits of the last token (all_logits = 0) or of every token.
 * Qwen3.5: each call leaves the snapshot of the recurrent states before its last token
 * (src/model.cpp:798-812), which or_session_rollback restores or, for any other earlier
 * position, replaces by a restart at position 0 (src/model.cpp:735-751). */
int or_session_eval(oracle_session* s, const int32_t* tokens, size_t n, int all_logits, float* out);
size_t or_session_position(const oracle_session* s);
int or_session_rollback(oracle_session* s, size_t position);
/* Direct access to layer l's fp16 caches [kv_head][max_context][head_dim], to pre-fill them. */
uint16_t* or_session_kv(oracle_session* s, int layer, int value);
void or_session_set_position(oracle_session* s, size_t position);
const char* or_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
