// TEST INFRASTRUCTURE ONLY — never part of the product path.
//
// A C-ABI shim over the reference's own CPU engine, built from the reference's
// sources where they lie (/root/reference/src) by oracle/Makefile into
// oracle/_ref/libbrisk_ref.so.  Only tests/, tests/golden/ scripts,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, as the
// checker or as the timed CPU baseline.
//
// The calls mirror what the reference's CLI does:
//   ref_open      ~ cmd_generate's MappedFile + GgufFile::parse + Model(file, repack = !gpu)
//                   + Session(model, threads, max_context)   (src/main.cpp:178-212)
//   ref_generate  ~ the greedy loop of cmd_generate           (src/main.cpp:220-299)
//   ref_eval / ref_eval_all / ref_rollback ~ Engine           (src/engine.h:13-37)
// plus the kernel-level entry points of src/quant.h and src/kernels.h that the
// parity tests pin the HIP kernels against.
#include <algorithm>
#include <cmath>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "engine.h"
#include "gguf.h"
#include "kernels.h"
#include "kernels_f32.h"
#include "mapped_file.h"
#include "model.h"
#include "quant.h"

namespace {

thread_local std::string g_error;

struct RefHandle {
    brisk::MappedFile mapped;
    brisk::GgufFile file;
    std::unique_ptr<brisk::Model> model;
    std::unique_ptr<brisk::Session> session;
    explicit RefHandle(const std::string& path) : mapped(path), file(brisk::GgufFile::parse(mapped.bytes())) {}
};

template <typename F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

}  // namespace

extern "C" {

const char* ref_last_error(void) { return g_error.c_str(); }

void* ref_open(const char* path, int threads, size_t max_context) {
    RefHandle* h = nullptr;
    const int rc = guarded([&] {
        auto owned = std::make_unique<RefHandle>(path);
        owned->model = std::make_unique<brisk::Model>(owned->file, /*repack=*/true);
        owned->session = std::make_unique<brisk::Session>(*owned->model, static_cast<std::size_t>(std::max(threads, 1)), max_context);
        h = owned.release();
    });
    return rc == 0 ? h : nullptr;
}

void ref_close(void* handle) { delete static_cast<RefHandle*>(handle); }

uint32_t ref_vocab(void* handle) { return static_cast<RefHandle*>(handle)->model->config().vocab_size; }

// The reference's parse of the file's metadata (ModelConfig, src/model.h:34-125, filled by
// src/model.cpp:161-301), for pinning the Python binding's own parse against it.
struct RefConfig {
    uint32_t arch, vocab, embd, layers, heads, kv_heads, head_dim, ff, context;
    float rope_base, eps;
    int32_t rope_neox;
    uint32_t rope_dim, rope_original_context;
    float rope_attn_factor;
    uint32_t sliding_window;
    float rope_base_local, rope_scale, embedding_scale, final_softcap;
    int32_t gelu;
    uint32_t conv_taps, no_rope_step;
    uint32_t n_rope_factors, n_factors_short, n_factors_long;
    uint64_t conv_layers;  // bit l: layer l is a short-convolution layer (layers 0..63)
    uint32_t ssm_state, ssm_k_heads, ssm_v_heads, ssm_inner, ssm_conv;
    int32_t attention_gate;
    uint64_t recurrent_layers;  // bit l: layer l is a Gated DeltaNet layer (layers 0..63)
    uint32_t head_dim_local, kv_from_start, ple_dim;
    float attention_scale;
    int32_t value_norm;
    uint64_t sliding_layers;    // bit l: layer_slides(l) (layers 0..63)
    uint32_t head_dim_of[64], kv_heads_of[64], ff_of[64], kv_layer_of[64];
};

int ref_config(void* handle, RefConfig* out) {
    return guarded([&] {
        const brisk::ModelConfig& c = static_cast<RefHandle*>(handle)->model->config();
        RefConfig r{};
        r.arch = static_cast<uint32_t>(c.architecture);
        r.vocab = c.vocab_size; r.embd = c.embedding_dim; r.layers = c.layer_count; r.heads = c.head_count;
        r.kv_heads = c.kv_head_count; r.head_dim = c.head_dim; r.ff = c.feed_forward_dim; r.context = c.context_length;
        r.rope_base = c.rope_base; r.eps = c.rms_epsilon; r.rope_neox = c.rope_neox ? 1 : 0;
        r.rope_dim = c.rope_dim_of(); r.rope_original_context = c.rope_original_context; r.rope_attn_factor = c.rope_attn_factor;
        r.sliding_window = c.sliding_window; r.rope_base_local = c.rope_base_local; r.rope_scale = c.rope_scale;
        r.embedding_scale = c.embedding_scale; r.final_softcap = c.final_softcap; r.gelu = c.gelu ? 1 : 0;
        r.conv_taps = c.conv_taps; r.no_rope_step = c.no_rope_step;
        r.n_rope_factors = static_cast<uint32_t>(c.rope_factors.size());
        r.n_factors_short = static_cast<uint32_t>(c.rope_factors_short.size());
        r.n_factors_long = static_cast<uint32_t>(c.rope_factors_long.size());
        for (std::size_t l = 0; l < c.layer_count && l < 64; ++l)
            if (c.layer_is_conv(l)) r.conv_layers |= uint64_t{1} << l;
        r.ssm_state = c.ssm_state; r.ssm_k_heads = c.ssm_k_heads; r.ssm_v_heads = c.ssm_v_heads;
        r.ssm_inner = c.ssm_inner; r.ssm_conv = c.ssm_conv; r.attention_gate = c.attention_gate ? 1 : 0;
        for (std::size_t l = 0; l < c.layer_count && l < 64; ++l)
            if (c.layer_is_recurrent(l)) r.recurrent_layers |= uint64_t{1} << l;
        r.head_dim_local = c.head_dim_local; r.kv_from_start = c.kv_from_start; r.ple_dim = c.ple_dim;
        r.attention_scale = c.attention_scale; r.value_norm = c.value_norm ? 1 : 0;
        for (std::size_t l = 0; l < c.layer_count && l < 64; ++l) {
            if (c.layer_slides(l)) r.sliding_layers |= uint64_t{1} << l;
            r.head_dim_of[l] = c.head_dim_of(l);
            r.kv_heads_of[l] = c.kv_head_count_of(l);
            r.ff_of[l] = c.ff_dim_of(l);
            r.kv_layer_of[l] = static_cast<uint32_t>(c.kv_layer_of(l));
        }
        *out = r;
    });
}

size_t ref_position(void* handle) { return static_cast<RefHandle*>(handle)->session->position(); }

int ref_rollback(void* handle, size_t position) {
    return guarded([&] { static_cast<RefHandle*>(handle)->session->rollback(position); });
}

// Last-token logits of eval(tokens) into out[vocab].
int ref_eval(void* handle, const int32_t* tokens, size_t n, float* out) {
    return guarded([&] {
        auto* h = static_cast<RefHandle*>(handle);
        const auto logits = h->session->eval(std::span<const brisk::Token>(tokens, n));
        std::memcpy(out, logits.data(), logits.size() * sizeof(float));
    });
}

// All n rows of eval_all(tokens) into out[n * vocab].
// Engine::log_likelihood (src/engine.cpp:10-33) on the CPU Session.
int ref_log_likelihood(void* handle, const int32_t* tokens, size_t n, double* out) {
    return guarded([&] { *out = static_cast<RefHandle*>(handle)->session->log_likelihood(std::span<const brisk::Token>(tokens, n)); });
}

int ref_eval_all(void* handle, const int32_t* tokens, size_t n, float* out) {
    return guarded([&] {
        auto* h = static_cast<RefHandle*>(handle);
        const auto logits = h->session->eval_all(std::span<const brisk::Token>(tokens, n));
        std::memcpy(out, logits.data(), logits.size() * sizeof(float));
    });
}

// The greedy loop of cmd_generate (src/main.cpp:220-299) on token ids:
// logits = eval(prompt); then n_gen times: next = first index of the max
// (Sampler::sample at temperature 0, src/sampler.cpp:11-13), record it, and
// evaluate it unless it is the last one.  gaps[i] = top-1 minus top-2 logit of
// the distribution token i was picked from (may be null).  Timing fields as
// src/main.cpp:312-318: prefill seconds and generation seconds.
int ref_generate(void* handle, const int32_t* prompt, size_t n_prompt, size_t n_gen, int32_t* out_ids, float* gaps,
                 double* prefill_s, double* gen_s) {
    return guarded([&] {
        auto* h = static_cast<RefHandle*>(handle);
        using Clock = std::chrono::steady_clock;
        const auto t0 = Clock::now();
        std::span<const float> logits = h->session->eval(std::span<const brisk::Token>(prompt, n_prompt));
        const auto t1 = Clock::now();
        for (size_t i = 0; i < n_gen; ++i) {
            const auto best = std::max_element(logits.begin(), logits.end());
            const auto next = static_cast<brisk::Token>(best - logits.begin());
            out_ids[i] = next;
            if (gaps != nullptr) {
                float second = -INFINITY;
                for (size_t v = 0; v < logits.size(); ++v) {
                    if (static_cast<brisk::Token>(v) != next) second = std::max(second, logits[v]);
                }
                gaps[i] = *best - second;
            }
            if (i + 1 == n_gen) break;
            logits = h->session->eval(next);
        }
        const auto t2 = Clock::now();
        *prefill_s = std::chrono::duration<double>(t1 - t0).count();
        *gen_s = std::chrono::duration<double>(t2 - t1).count();
    });
}

// --- kernel level (src/quant.h, src/kernels.h) ---

float ref_half_to_float(uint16_t h) { return brisk::half_to_float(h); }
uint16_t ref_float_to_half(float f) { return brisk::float_to_half(f); }

void ref_quantize_q8_0(const float* x, void* out, size_t count) {
    brisk::quantize_q8_0(x, static_cast<brisk::BlockQ8_0*>(out), count);
}
void ref_quantize_q8_k(const float* x, void* out, size_t count, int bits) {
    brisk::quantize_q8_k(x, static_cast<brisk::BlockQ8_K*>(out), count, bits);
}

// Formats by the ggml tensor-type numbers a GGUF file uses (src/gguf.h:22-27);
// 1016 stands for the load-time TQ2_0x16 layout.
static brisk::WeightFormat format_of(int type) {
    switch (type) {
        case 2: return brisk::WeightFormat::Q4_0;
        case 3: return brisk::WeightFormat::Q4_1;
        case 6: return brisk::WeightFormat::Q5_0;
        case 8: return brisk::WeightFormat::Q8_0;
        case 12: return brisk::WeightFormat::Q4_K;
        case 13: return brisk::WeightFormat::Q5_K;
        case 14: return brisk::WeightFormat::Q6_K;
        case 35: return brisk::WeightFormat::TQ2_0;
        case 1016: return brisk::WeightFormat::TQ2_0x16;
        default: throw std::runtime_error("ref shim: unsupported format " + std::to_string(type));
    }
}

// KernelSet::matvec / matmul of the generic kernels (src/kernels.cpp:129-163) on
// pre-quantised activations.
int ref_matvec(int type, const void* w, size_t rows, size_t cols, const void* x, float* out) {
    return guarded([&] { brisk::kernels::kernels_for(format_of(type)).matvec(w, rows, cols, x, out); });
}
int ref_matmul(int type, const void* w, size_t rows, size_t cols, const void* x, size_t n, float* out, size_t out_stride) {
    return guarded([&] { brisk::kernels::kernels_for(format_of(type)).matmul(w, rows, cols, x, n, out, out_stride); });
}

void ref_repack_tq2_0x16(const void* in, size_t rows, size_t blocks, void* out) {
    brisk::repack_tq2_0x16_scalar(static_cast<const brisk::BlockTQ2_0*>(in), rows, blocks, static_cast<brisk::BlockTQ2_0x16*>(out));
}

// Dequantised rows (src/quant.h:209-218), for the tolerance checks.
int ref_dequantize(int type, const void* blocks, float* out, size_t count) {
    return guarded([&] {
        switch (format_of(type)) {
            case brisk::WeightFormat::Q4_0: brisk::dequantize_q4_0(static_cast<const brisk::BlockQ4_0*>(blocks), out, count); break;
            case brisk::WeightFormat::Q8_0: brisk::dequantize_q8_0(static_cast<const brisk::BlockQ8_0*>(blocks), out, count); break;
            case brisk::WeightFormat::Q4_1: brisk::dequantize_q4_1(static_cast<const brisk::BlockQ4_1*>(blocks), out, count); break;
            case brisk::WeightFormat::Q5_0: brisk::dequantize_q5_0(static_cast<const brisk::BlockQ5_0*>(blocks), out, count); break;
            case brisk::WeightFormat::Q5_K: brisk::dequantize_q5_k(static_cast<const brisk::BlockQ5_K*>(blocks), out, count); break;
            case brisk::WeightFormat::Q4_K: brisk::dequantize_q4_k(static_cast<const brisk::BlockQ4_K*>(blocks), out, count); break;
            case brisk::WeightFormat::Q6_K: brisk::dequantize_q6_k(static_cast<const brisk::BlockQ6_K*>(blocks), out, count); break;
            case brisk::WeightFormat::TQ2_0: brisk::dequantize_tq2_0(static_cast<const brisk::BlockTQ2_0*>(blocks), out, count); break;
            default: throw std::runtime_error("ref shim: no dequantiser");
        }
    });
}

// The attention kernels of src/kernels_f32.h (portable branch) for one query.
void ref_softmax(float* x, size_t n) { brisk::kernels::softmax_f32(std::span<float>(x, n)); }
float ref_dot_f32(const float* a, const float* b, size_t n) { return brisk::kernels::dot_f32(a, b, n); }

}  // extern "C"
