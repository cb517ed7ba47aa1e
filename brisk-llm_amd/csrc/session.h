// Host-side state of one device-resident sequence (see session.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/brisk_hip.h"
#include "launch.h"
#include "loop.h"
#include "prefill.h"

namespace bh {

// An error with the C ABI status it maps to.
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& what) : std::runtime_error(what), code(c) {}
};

struct DeviceMatrix {
    Packed p{};
    void* mem = nullptr;
    // Q6_K, Q5_K (Q4_K on request): the batched prefill's expanded planes (launch_mx_expand), made at
    // the first prefill
    void* xmem = nullptr;
    MxPlanes x{};
    DeviceMatrix() = default;
    DeviceMatrix(const DeviceMatrix&) = delete;
    DeviceMatrix& operator=(const DeviceMatrix&) = delete;
    DeviceMatrix(DeviceMatrix&& o) noexcept : p(o.p), mem(o.mem), xmem(o.xmem), x(o.x) {
        o.mem = nullptr;
        o.xmem = nullptr;
    }
    ~DeviceMatrix();
};

struct Layer {
    DeviceMatrix q, k, v, o, gate, up, down;
    const float* attn_norm = nullptr;
    const float* q_norm = nullptr;
    const float* k_norm = nullptr;
    const float* attn_sub_norm = nullptr;
    const float* ffn_norm = nullptr;
    const float* ffn_sub_norm = nullptr;
    const float* q_bias = nullptr;  // projection biases (Qwen2 and some Llama-shaped models), all or none
    const float* k_bias = nullptr;
    const float* v_bias = nullptr;
    bool rope = true;               // false: the layer attends without RoPE (SmolLM3's every fourth)
    const float* attn_post_norm = nullptr;  // Gemma: norms of the attention and feed-forward outputs
    const float* ffn_post_norm = nullptr;
    bool slides = false;            // Gemma: a sliding-window layer (local RoPE base)
    // the layer's head size, key/value heads and width (Gemma 4 varies them per layer), and the
    // layer whose K/V cache it reads (itself, or for Gemma 4's shared layers an earlier one)
    int hd = 0, kvh = 0, ff = 0, kv_src = 0;
    bool v_is_k = false;            // Gemma 4: no V projection, K's raw rows serve as V
    DeviceMatrix ple_gate, ple_proj; // Gemma 4's per-layer embedding (src/model.cpp:403-407)
    const float* ple_post_norm = nullptr;
    float out_scale = 1.0f;         // layer_output_scale
    DeviceMatrix conv_in, conv_out; // LFM2 short-convolution layer: in_proj (3 embd rows), out_proj
    const float* conv_w = nullptr;  // [embd][taps]; non-null marks a convolution layer
    uint16_t* conv_cache = nullptr; // bx per position, fp16 [ctx][embd]
    // Qwen3.5 Gated DeltaNet layer (src/model.cpp:343-358); ssm_a non-null marks it
    DeviceMatrix ssm_qkv, ssm_gate, ssm_alpha, ssm_beta, ssm_out;
    const float* ssm_a = nullptr;
    const float* ssm_dt = nullptr;
    const float* ssm_conv_w = nullptr;  // [qkv_dim][conv]
    const float* ssm_norm = nullptr;
    float* ssm_ring = nullptr;          // [conv][qkv_dim]: slot p % conv holds position p's attn_qkv rows
    float* ssm_state = nullptr;         // [2][heads][state (key)][state (value)], halves by position parity
};

// Device bytes a session of these tensors would allocate (see Session's constructor).
brisk_hip_memory estimate_session(const brisk_hip_config& cfg, const brisk_hip_tensor* tensors, size_t n, size_t max_context);

class Session {
public:
    static constexpr int kPrefillTokens = 512;  // batched prefill: buffers for this many tokens, allocated on first use
    Session(const brisk_hip_config& cfg, const brisk_hip_tensor* tensors, size_t n, size_t max_context, int device);
    ~Session();
    Session(const Session&) = delete;
    Session& operator=(const Session&) = delete;

    void eval(const int32_t* tokens, size_t n, float* logits);
    void eval_all(const int32_t* tokens, size_t n, float* logits);
    int32_t eval_greedy(const int32_t* tokens, size_t n);
    void generate(const int32_t* prompt, size_t n_prompt, size_t n_gen, int32_t* out);
    void decode(size_t n, int32_t* out);
    void rollback(size_t position);
    void set_position(size_t position);
    size_t position() const { return position_; }
    size_t max_context() const { return max_ctx_; }
    bool uses_loop() const { return loop_kernel_ != nullptr; }
    size_t trace(unsigned long long* out, size_t n);
    void kv_cache(int layer, int value, void** ptr, size_t* bytes);
    hipStream_t stream() const { return stream_; }
    int device() const { return device_; }

private:
    void* alloc(size_t bytes);
    void record_step(bool full);
    hipGraphExec_t capture(bool full);
    void step(bool full);
    void validate(const int32_t* tokens, size_t n) const;
    void stage(const int32_t* tokens, size_t n);
    void stage(const int32_t* tokens, size_t n, size_t device_pos);
    int32_t picked();
    void debug_layer(uint32_t l);
    PickState pick_state() const;
    void finish();
    void setup_loop();
    void run_loop(size_t pos0, size_t n_steps, size_t first_full, size_t fixed);
    void check_loop_error();
    bool use_prefill(size_t n) const;
    void ensure_prefill();
    void prefill_layers(size_t pos0, int T);
    bool neox() const;
    bool gemma() const { return cfg_.arch == BRISK_HIP_ARCH_GEMMA3 || cfg_.arch == BRISK_HIP_ARCH_GEMMA4; }
    bool lfm2() const { return cfg_.arch == BRISK_HIP_ARCH_LFM2; }
    bool qwen35() const { return cfg_.arch == BRISK_HIP_ARCH_QWEN35; }
    bool gemma4() const { return cfg_.arch == BRISK_HIP_ARCH_GEMMA4; }
    void evaluated();
    void prefill_quant(const float* x, int xstride, const float* w, int cols, int T, const DeviceMatrix& consumer);

    brisk_hip_config cfg_;
    int device_;
    hipStream_t stream_ = nullptr;
    size_t max_ctx_ = 0;
    size_t position_ = 0;
    size_t weight_bytes_ = 0;
    std::vector<void*> owned_;
    DeviceMatrix embd_, out_own_;
    const DeviceMatrix* out_ = nullptr;
    const float* out_norm_ = nullptr;
    std::vector<Layer> layers_;
    std::vector<uint16_t*> kcache_, vcache_;
    std::vector<size_t> kv_bytes_;  // per layer (0: no cache of its own)
    float *h_ = nullptr, *q_ = nullptr, *att_ = nullptr, *act_ = nullptr, *logits_ = nullptr, *rope_ = nullptr;
    float *part_acc_ = nullptr, *part_ml_ = nullptr, *k_ = nullptr, *v_ = nullptr;
    float* rope_local_ = nullptr;  // Gemma 3 sliding layers' RoPE table
    float* proj_ = nullptr;        // Gemma: a projection's output before its post-norm
    float* conv_buf_ = nullptr;    // LFM2: in_proj's [b | c | x] rows
    // Qwen3.5: the recurrent layers' projections, the attention layers' query|gate rows and gates
    float *ssm_qkv_ = nullptr, *ssm_z_ = nullptr, *ssm_ab_ = nullptr, *qg_ = nullptr, *agate_ = nullptr;
    // Qwen3.5: the recurrent states can step back to snap_pos_ (the last evaluated token's
    // position, whose input state is still held) while snap_ok_
    bool snap_ok_ = false;
    size_t snap_pos_ = 0;
    // the plain attention (launch_attention_plain): head sizes past 128, or BRISK_HIP_ATTN=plain
    bool plain_attn_ = false;
    float *plain_q_ = nullptr, *plain_sc_ = nullptr;
    // Gemma 4's per-layer embeddings: table, projection of the embedding, its norm; the token's inputs
    DeviceMatrix ple_tok_, ple_proj_;
    const float* ple_norm_ = nullptr;
    float *ple_in_ = nullptr, *ple_g_ = nullptr;
    float embd_scale_ = 1.0f;      // Gemma: sqrt(embd) (src/model.cpp:286)
    int rope_dim_ = 0;             // dimensions the RoPE table rotates (its row stride)
    unsigned long long* key_ = nullptr;
    unsigned* ticket_ = nullptr;
    int* pos_ = nullptr;
    int* seq_ = nullptr;
    int max_splits_ = 0;
    bool use_graphs_ = true;
    // persistent loop
    const void* loop_kernel_ = nullptr;
    int loop_grid_ = 0;
    bool loop_cooperative_ = false;  // BRISK_HIP_COOPERATIVE: launch the loop cooperatively
    LoopArgs loop_{};
    LayerDev* layers_dev_ = nullptr;
    unsigned* loop_done_ = nullptr;
    unsigned long long* tagged_ = nullptr;
    size_t tagged_words_ = 0;
    size_t launches_ = 0;
    int* loop_error_ = nullptr;
    unsigned long long* trace_ = nullptr;
    static constexpr size_t kTraceSlots = 1 << 20;
    bool debug_ = false;
    bool prefill_on_ = true;
    bool prefill_shapes_ = true;   // every matrix's rows a whole number of the batched GEMM's chunks
    bool prefill_mfma_ = false;    // BRISK_HIP_PREFILL_ATTN=mfma
    bool prefill_legacy_ = false;  // BRISK_HIP_PREFILL_ATTN=staged
    float *pre_h_ = nullptr, *pre_q_ = nullptr, *pre_k_ = nullptr, *pre_v_ = nullptr, *pre_att_ = nullptr, *pre_act_ = nullptr;
    void* host_io_ = nullptr;  // pinned staging for token and logits copies (host_buf)
    size_t host_io_bytes_ = 0;
    void* host_buf(size_t bytes);
    void fetch_logits(float* out, const float* dev, size_t rows);
    float* pre_proj_ = nullptr;  // Gemma: a projection's rows before their post-norm; LFM2: conv outputs
    float* pre_conv_ = nullptr;  // LFM2: in_proj rows [b | c | x]
    // Qwen3.5: the recurrence's projections [T][qkv], [T][inner], [T][alpha | beta]; the query|gate rows
    float *pre_sqkv_ = nullptr, *pre_sz_ = nullptr, *pre_sab_ = nullptr, *pre_qg_ = nullptr;
    float *pre_ple_ = nullptr, *pre_pleg_ = nullptr;  // Gemma 4: per-layer embedding inputs and gate rows
    ActPlanar pre_x_{};
    ActPlanar wide_x_{};  // feed-forward rows past kMaxCols: the down projection's quantised input (one token)
    float* all_logits_ = nullptr;  // eval_all's [64][vocab] logits, allocated on first use
    hipGraphExec_t graph_layers_ = nullptr, graph_full_ = nullptr;
};

}  // namespace bh
