// TEST INFRASTRUCTURE ONLY — never part of the product path.
//
// A C-ABI shim that drives the drop-in binding (brisk-llm_amd/binding/hip_session.h,
// class HipSession : Engine) exactly as the reference's own code drives an Engine,
// built by oracle/Makefile from the reference's sources where they lie into
// oracle/_ref/libhip_engine.so, linked against libbrisk_hip.so.  Only tests/ load it.
//
//   he_open        ~ MappedFile + GgufFile::parse + Model(file, repack = false) + HipSession
//                    (the MetalSession construction of src/main.cpp:206, src/server.cpp:243)
//   he_generate    ~ cmd_generate's greedy loop over Engine::eval (src/main.cpp:287-299)
//   he_speculative ~ cmd_generate --draft: Speculator over the HipSession target with a
//                    LookupDrafter or a CPU ModelDrafter (src/main.cpp:236-276, src/speculative.cpp)
//   he_serve_prefill ~ the server's prefix reuse: rollback to the common prefix, eval the rest
//                    (src/server.cpp:380-395), after the warm-up pass (src/server.cpp:258-265)
//   he_log_likelihood ~ Engine::log_likelihood over eval_all (src/engine.cpp:10-33)
#include <algorithm>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "engine.h"
#include "gguf.h"
#include "hip_session.h"
#include "mapped_file.h"
#include "model.h"
#include "speculative.h"

namespace {

thread_local std::string g_error;

struct Handle {
    brisk::MappedFile mapped;
    brisk::GgufFile file;
    std::unique_ptr<brisk::Model> model;
    std::unique_ptr<brisk::HipSession> session;
    std::vector<brisk::Token> cached;  // the server's tokens already in the cache
    explicit Handle(const std::string& path) : mapped(path), file(brisk::GgufFile::parse(mapped.bytes())) {}
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

brisk::Token argmax(std::span<const float> logits) {  // Sampler::sample at temperature 0 (src/sampler.cpp:10-13)
    return static_cast<brisk::Token>(std::max_element(logits.begin(), logits.end()) - logits.begin());
}

}  // namespace

extern "C" {

const char* he_last_error(void) { return g_error.c_str(); }

void* he_open(const char* path, size_t max_context) {
    Handle* h = nullptr;
    const int rc = guarded([&] {
        auto owned = std::make_unique<Handle>(path);
        owned->model = std::make_unique<brisk::Model>(owned->file, /*repack=*/false);
        owned->session = std::make_unique<brisk::HipSession>(*owned->model, owned->mapped.bytes(), max_context);
        h = owned.release();
    });
    return rc == 0 ? h : nullptr;
}

void he_close(void* handle) { delete static_cast<Handle*>(handle); }

size_t he_position(void* handle) { return static_cast<Handle*>(handle)->session->position(); }

int he_rollback(void* handle, size_t position) {
    return guarded([&] { static_cast<Handle*>(handle)->session->rollback(position); });
}

int he_eval(void* handle, const int32_t* tokens, size_t n, float* out) {
    return guarded([&] {
        const auto logits = static_cast<Handle*>(handle)->session->eval(std::span<const brisk::Token>(tokens, n));
        std::copy(logits.begin(), logits.end(), out);
    });
}

int he_eval_all(void* handle, const int32_t* tokens, size_t n, float* out) {
    return guarded([&] {
        const auto logits = static_cast<Handle*>(handle)->session->eval_all(std::span<const brisk::Token>(tokens, n));
        std::copy(logits.begin(), logits.end(), out);
    });
}

int he_generate(void* handle, const int32_t* prompt, size_t n_prompt, size_t n_gen, int32_t* out) {
    return guarded([&] {
        brisk::Engine& engine = *static_cast<Handle*>(handle)->session;
        std::span<const float> logits = engine.eval(std::span<const brisk::Token>(prompt, n_prompt));
        for (size_t i = 0; i < n_gen; ++i) {
            out[i] = argmax(logits);
            if (i + 1 < n_gen) logits = engine.eval(out[i]);
        }
    });
}

int he_generate_greedy(void* handle, const int32_t* prompt, size_t n_prompt, size_t n_gen, int32_t* out) {
    return guarded([&] {
        static_cast<Handle*>(handle)->session->generate_greedy(std::span<const brisk::Token>(prompt, n_prompt),
                                                               std::span<brisk::Token>(out, n_gen));
    });
}

// draft_path NULL: the lookup drafter; else a CPU ModelDrafter of that GGUF (threads CPU threads).
int he_speculative(void* handle, const char* draft_path, int threads, const int32_t* prompt, size_t n_prompt, size_t n_gen,
                   size_t draft_tokens, int32_t* out, size_t* stats) {
    return guarded([&] {
        Handle& h = *static_cast<Handle*>(handle);
        brisk::Engine& target = *h.session;
        const std::vector<brisk::Token> p(prompt, prompt + n_prompt);
        std::unique_ptr<brisk::MappedFile> dm;
        std::unique_ptr<brisk::GgufFile> df;
        std::unique_ptr<brisk::Model> dmodel;
        std::unique_ptr<brisk::Drafter> drafter;
        if (draft_path == nullptr) {
            drafter = std::make_unique<brisk::LookupDrafter>();
        } else {
            dm = std::make_unique<brisk::MappedFile>(draft_path);
            df = std::make_unique<brisk::GgufFile>(brisk::GgufFile::parse(dm->bytes()));
            dmodel = std::make_unique<brisk::Model>(*df);
            drafter = std::make_unique<brisk::ModelDrafter>(*dmodel, static_cast<std::size_t>(std::max(threads, 1)),
                                                            n_prompt + n_gen + 80);
        }
        target.eval(std::span<const brisk::Token>(p));
        drafter->observe(p);
        target.rollback(p.size() - 1);
        brisk::Speculator spec(target, *drafter, p.back(), draft_tokens);
        size_t got = 0;
        while (got < n_gen)
            for (const brisk::Token t : spec.step()) {
                if (got == n_gen) break;
                out[got++] = t;
            }
        const brisk::SpeculativeStats& st = spec.stats();
        stats[0] = st.rounds; stats[1] = st.plain; stats[2] = st.drafted; stats[3] = st.accepted;
    });
}

// The server's turn: after the warm-up pass (eval of one token, rollback to 0) at construction,
// each request rolls back to the longest common prefix with the cached tokens and evaluates the
// rest (at least its last token again); *reused receives the prefix length.
int he_serve_warmup(void* handle, int32_t first) {
    return guarded([&] {
        Handle& h = *static_cast<Handle*>(handle);
        h.session->eval(first);
        h.session->rollback(0);
        h.cached.clear();
    });
}

int he_serve_prefill(void* handle, const int32_t* prompt, size_t n, float* out, size_t* reused) {
    return guarded([&] {
        Handle& h = *static_cast<Handle*>(handle);
        const std::vector<brisk::Token> p(prompt, prompt + n);
        size_t common = 0;
        while (common < p.size() && common < h.cached.size() && p[common] == h.cached[common]) ++common;
        if (common == p.size()) --common;
        h.session->rollback(common);
        common = h.session->position();
        *reused = common;
        const auto logits = h.session->eval(std::span<const brisk::Token>(p).subspan(common));
        h.cached = p;
        std::copy(logits.begin(), logits.end(), out);
    });
}

// A served turn's reply tokens join the cache as the server's generate loop evaluates them.
int he_serve_extend(void* handle, const int32_t* tokens, size_t n, float* out) {
    return guarded([&] {
        Handle& h = *static_cast<Handle*>(handle);
        for (size_t i = 0; i < n; ++i) {
            const auto logits = h.session->eval(tokens[i]);
            h.cached.push_back(tokens[i]);
            if (i + 1 == n) std::copy(logits.begin(), logits.end(), out);
        }
    });
}

int he_log_likelihood(void* handle, const int32_t* tokens, size_t n, double* out) {
    return guarded([&] { *out = static_cast<Handle*>(handle)->session->log_likelihood(std::span<const brisk::Token>(tokens, n)); });
}

}  // extern "C"
