// HipSession: brisk-llm's Engine (src/engine.h:13-37) over the MI355X token
// loop of include/brisk_hip.h.  This is the binding a maintainer adds to the
// reference tree as src/hip/hip_session.h; it is written against the
// reference's own headers (engine.h, model.h) and compiles with them
// (oracle/Makefile builds it into a test library).
//
// Construction mirrors MetalSession(model, file bytes, max_context)
// (src/main.cpp:206): `model` comes from Model(file, /*repack=*/false), so every
// matrix is in its GGUF layout, and the session copies and repacks the weights
// to HBM, keeping no pointer into the mapping afterwards.
#pragma once

#include <cstddef>
#include <cstdint>
#include <span>
#include <stdexcept>
#include <string>
#include <vector>

#include "brisk_hip.h"
#include "engine.h"
#include "model.h"

namespace brisk {

class HipSession final : public Engine {
public:
    HipSession(const Model& model, std::span<const std::byte> /*file*/, std::size_t max_context, int device = 0)
        : vocab_(model.config().vocab_size) {
        const ModelConfig& c = model.config();
        brisk_hip_config cfg{};
        switch (c.architecture) {  // the families on this path (src/model.h:20-31)
            case Architecture::Qwen3: cfg.arch = BRISK_HIP_ARCH_QWEN3; break;
            case Architecture::Llama: cfg.arch = BRISK_HIP_ARCH_LLAMA; break;
            case Architecture::BitNet: cfg.arch = BRISK_HIP_ARCH_BITNET; break;
            case Architecture::Qwen2: cfg.arch = BRISK_HIP_ARCH_QWEN2; break;
            case Architecture::SmolLM3: cfg.arch = BRISK_HIP_ARCH_SMOLLM3; break;
            case Architecture::Gemma3: cfg.arch = BRISK_HIP_ARCH_GEMMA3; break;
            case Architecture::Phi3: cfg.arch = BRISK_HIP_ARCH_PHI3; break;
            case Architecture::LFM2: cfg.arch = BRISK_HIP_ARCH_LFM2; break;
            case Architecture::Qwen35: cfg.arch = BRISK_HIP_ARCH_QWEN35; break;
            case Architecture::Gemma4: cfg.arch = BRISK_HIP_ARCH_GEMMA4; break;
            default: throw std::runtime_error("hip: this architecture is not on the GPU path");
        }
        // ModelConfig (src/model.h:36-125)
        cfg.vocab = c.vocab_size;
        cfg.embd = c.embedding_dim;
        cfg.layers = c.layer_count;
        cfg.heads = c.head_count;
        cfg.kv_heads = c.kv_head_count;
        cfg.head_dim = c.head_dim;
        cfg.ff = c.feed_forward_dim;
        cfg.context_length = c.context_length;
        cfg.rope_base = c.rope_base;
        cfg.rms_epsilon = c.rms_epsilon;
        cfg.sliding_window = c.sliding_window;
        cfg.rope_base_local = c.rope_base_local;
        cfg.rope_scale = c.rope_scale;
        cfg.final_softcap = c.final_softcap;
        cfg.rope_dim = c.rope_dim;
        cfg.rope_attn_factor = c.rope_attn_factor;
        cfg.rope_original_context = c.rope_original_context;
        cfg.conv_taps = c.conv_taps;
        cfg.rope_neox = c.rope_neox ? 1 : 2;
        cfg.no_rope_step = c.no_rope_step == 0 ? 0xFFFFFFFFu : c.no_rope_step;
        cfg.embedding_scale = c.embedding_scale;
        cfg.gelu = c.gelu ? 1 : 2;
        cfg.ssm_state = c.ssm_state;
        cfg.ssm_k_heads = c.ssm_k_heads;
        cfg.ssm_v_heads = c.ssm_v_heads;
        cfg.ssm_inner = c.ssm_inner;
        cfg.ssm_conv = c.ssm_conv;
        cfg.head_dim_local = c.head_dim_local;
        cfg.kv_from_start = c.kv_from_start;
        cfg.ple_dim = c.ple_dim;
        cfg.attention_scale = c.attention_scale;
        cfg.value_norm = c.value_norm ? 1 : 0;
        cfg.sliding_pattern = c.sliding_pattern.empty() ? nullptr : c.sliding_pattern.data();
        cfg.ff_dims = c.ff_dims.empty() ? nullptr : c.ff_dims.data();
        cfg.kv_head_counts = c.architecture != Architecture::Gemma4 || c.kv_head_counts.empty() ? nullptr : c.kv_head_counts.data();
        for (std::size_t l = 0; l < c.layer_count && c.architecture != Architecture::Gemma4; ++l)
            if (c.kv_head_count_of(l) != 0 && c.kv_head_count_of(l) != c.kv_head_count)
                throw std::runtime_error("hip: attention layers with different key/value head counts are not on the GPU path");

        // The tensor table, under the GGUF names the session reads, from the model's
        // accessors (src/model.h:141-195) and the config's RoPE factor vectors.
        names_.reserve(32 + 32 * static_cast<std::size_t>(c.layer_count));
        add_matrix("token_embd.weight", model.token_embedding());
        const Matrix& out = model.output_projection();
        if (out.bytes.data() != model.token_embedding().bytes.data() || out.f32.data() != model.token_embedding().f32.data())
            add_matrix("output.weight", out);  // else tied to the embedding (src/model.cpp:328-330)
        add_vector(c.architecture == Architecture::LFM2 ? "token_embd_norm.weight" : "output_norm.weight", model.output_norm());
        add_vector("rope_freqs.weight", c.rope_factors);
        add_vector("rope_factors_short.weight", c.rope_factors_short);
        add_vector("rope_factors_long.weight", c.rope_factors_long);
        if (c.ple_dim != 0) {  // Gemma 4's per-layer embeddings
            add_matrix("per_layer_token_embd.weight", model.ple_token_embedding());
            add_matrix("per_layer_model_proj.weight", model.ple_model_proj());
            add_vector("per_layer_proj_norm.weight", model.ple_proj_norm());
        }
        for (std::size_t l = 0; l < c.layer_count; ++l) {
            const Model::Layer& L = model.layers()[l];
            const std::string b = "blk." + std::to_string(l) + ".";
            add_vector(b + "attn_norm.weight", L.attention_norm);
            if (c.layer_is_recurrent(l)) {  // Qwen3.5 Gated DeltaNet
                add_matrix(b + "attn_qkv.weight", L.ssm_qkv);
                add_matrix(b + "attn_gate.weight", L.ssm_gate);
                add_matrix(b + "ssm_alpha.weight", L.ssm_alpha);
                add_matrix(b + "ssm_beta.weight", L.ssm_beta);
                add_vector(b + "ssm_a", L.ssm_a);
                add_vector(b + "ssm_dt.bias", L.ssm_dt_bias);
                add_vector(b + "ssm_conv1d.weight", L.ssm_conv_weight);
                add_vector(b + "ssm_norm.weight", L.ssm_norm);
                add_matrix(b + "ssm_out.weight", L.ssm_out);
            } else if (c.layer_is_conv(l)) {  // LFM2 short convolution
                add_matrix(b + "shortconv.in_proj.weight", L.conv_in);
                add_matrix(b + "shortconv.out_proj.weight", L.conv_out);
                add_vector(b + "shortconv.conv.weight", L.conv_weight);
            } else {
                add_matrix(b + "attn_q.weight", L.query);  // Phi-3: row views of attn_qkv (src/model.cpp:370-380)
                add_matrix(b + "attn_k.weight", L.key);
                add_matrix(b + "attn_v.weight", L.value);
                add_vector(b + "attn_q_norm.weight", L.query_norm);
                add_vector(b + "attn_k_norm.weight", L.key_norm);
                add_vector(b + "attn_q.bias", L.query_bias);
                add_vector(b + "attn_k.bias", L.key_bias);
                add_vector(b + "attn_v.bias", L.value_bias);
                add_vector(b + "attn_sub_norm.weight", L.attention_sub_norm);
                add_matrix(b + "attn_output.weight", L.attention_output);
                add_vector(b + "post_attention_norm.weight", L.attention_post_norm);
            }
            // Qwen3.5 names the feed-forward norm post_attention_norm (src/model.cpp:418)
            add_vector(b + (c.architecture == Architecture::Qwen35 ? "post_attention_norm.weight" : "ffn_norm.weight"),
                       L.feed_forward_norm);
            add_matrix(b + "ffn_gate.weight", L.gate);  // Phi-3: row views of ffn_up
            add_matrix(b + "ffn_up.weight", L.up);
            add_vector(b + "ffn_sub_norm.weight", L.feed_forward_sub_norm);
            add_matrix(b + "ffn_down.weight", L.down);
            add_vector(b + "post_ffw_norm.weight", L.feed_forward_post_norm);
            add_matrix(b + "inp_gate.weight", L.ple_gate);
            add_matrix(b + "proj.weight", L.ple_proj);
            add_vector(b + "post_norm.weight", L.ple_post_norm);
            if (L.out_scale != 1.0f) add_vector(b + "layer_output_scale.weight", std::span<const float>(&L.out_scale, 1));
        }
        for (std::size_t i = 0; i < table_.size(); ++i) table_[i].name = names_[i].c_str();
        check(brisk_hip_session_create(&cfg, table_.data(), table_.size(), max_context, device, &s_));
        logits_.resize(Engine::kMaxScoredTokens * static_cast<std::size_t>(vocab_));
    }
    ~HipSession() override { brisk_hip_session_destroy(s_); }
    HipSession(const HipSession&) = delete;
    HipSession& operator=(const HipSession&) = delete;

    using Engine::eval;  // eval(Token)
    std::span<const float> eval(std::span<const Token> tokens) override {
        check(brisk_hip_session_eval(s_, tokens.data(), tokens.size(), logits_.data()));
        return {logits_.data(), vocab_};
    }
    std::span<const float> eval_all(std::span<const Token> tokens) override {
        check(brisk_hip_session_eval_all(s_, tokens.data(), tokens.size(), logits_.data()));
        return {logits_.data(), tokens.size() * vocab_};
    }
    void rollback(std::size_t position) override { check(brisk_hip_session_rollback(s_, position)); }
    std::size_t position() const override { return brisk_hip_session_position(s_); }

    // cmd_generate's greedy loop at temperature 0 (src/main.cpp:220-299) with the picks kept on the
    // GPU: eval(prompt), then out.size() picks, each evaluated but the last.
    void generate_greedy(std::span<const Token> prompt, std::span<Token> out) {
        check(brisk_hip_session_generate(s_, prompt.data(), prompt.size(), out.size(), out.data()));
    }

private:
    static void check(int rc) {
        if (rc != BRISK_HIP_OK) throw std::runtime_error(brisk_hip_last_error());
    }
    // ggml type numbers of the formats a Model(file, repack = false) holds (src/quant.h:16)
    static int ggml_type(WeightFormat f) {
        switch (f) {
            case WeightFormat::F32: return BRISK_HIP_F32;
            case WeightFormat::Q4_0: return BRISK_HIP_Q4_0;
            case WeightFormat::Q4_1: return BRISK_HIP_Q4_1;
            case WeightFormat::Q5_0: return BRISK_HIP_Q5_0;
            case WeightFormat::Q8_0: return BRISK_HIP_Q8_0;
            case WeightFormat::Q4_K: return BRISK_HIP_Q4_K;
            case WeightFormat::Q5_K: return BRISK_HIP_Q5_K;
            case WeightFormat::Q6_K: return BRISK_HIP_Q6_K;
            case WeightFormat::TQ2_0: return BRISK_HIP_TQ2_0;
            default: throw std::runtime_error("hip: load the model with Model(file, /*repack=*/false)");
        }
    }
    void add_matrix(std::string name, const Matrix& m) {
        if (m.rows == 0) return;
        const void* data = m.format == WeightFormat::F32 ? static_cast<const void*>(m.f32.data()) : static_cast<const void*>(m.bytes.data());
        names_.push_back(std::move(name));
        table_.push_back({nullptr, ggml_type(m.format), m.rows, m.cols, data});
    }
    void add_vector(std::string name, std::span<const float> v) {
        if (v.empty()) return;
        names_.push_back(std::move(name));
        table_.push_back({nullptr, BRISK_HIP_F32, 1, v.size(), v.data()});
    }

    brisk_hip_session* s_ = nullptr;
    std::size_t vocab_;
    std::vector<float> logits_;
    std::vector<std::string> names_;
    std::vector<brisk_hip_tensor> table_;
};

}  // namespace brisk
