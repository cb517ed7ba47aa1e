// HipSession: the device-resident token loop behind the C ABI.
//
// Counterpart of the reference's Session / MetalSession (src/model.h:223-310,
// src/metal/metal_session.h:21-37).  Differences in mechanism, not in result:
//  * weights are copied once to HBM and repacked into planes (layout.h);
//  * the token sequence and the position live in device memory: the embedding
//    kernel reads seq[pos], the argmax kernel writes seq[pos + 1] and advances
//    pos, so one decode step is a fixed launch sequence, captured once as a
//    hipGraph and replayed per token with no host round trip;
//  * two step graphs: "layers" (a prompt token whose logits nobody reads, as
//    eval_batch computes only the last token's logits, src/model.cpp:1201-1205)
//    and "full" (layers + output projection + greedy pick).
#include "session.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

namespace bh {

// The expanded planes of m (or nulls) as a GEMM's first / second matrix.
static void set_mx(MmArgs& g, const DeviceMatrix& m) {
    g.qx = m.x.q; g.qxd = m.x.d; g.qxm = m.x.mn;
}
static void set_mx2(MmArgs& g, const DeviceMatrix& m) {
    g.qx2 = m.x.q; g.qxd2 = m.x.d; g.qxm2 = m.x.mn;
}

namespace {

[[noreturn]] void model_fail(const std::string& what) { throw Error(BRISK_HIP_EINVAL, "model: " + what); }

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        throw Error(e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation ? BRISK_HIP_ENOMEM : BRISK_HIP_EHIP,
                    std::string("hip: ") + what + ": " + hipGetErrorString(e));
    }
}

// Host -> device uploads of the model's bytes through two pinned chunks.  The
// host copies chunk i + 1 out of the caller's (usually memory-mapped) tensor
// bytes while the DMA engine moves chunk i, so the transfer overlaps the host
// reads instead of going through the runtime's pageable path, one blocking
// copy at a time.  The host copy of a chunk is split over a few threads (a
// single thread's memcpy from the page cache is slower than the link).  The
// reference's loader maps the file and reads the tensors in place
// (src/mapped_file.cpp:88-102); this is the device-side counterpart.
class Uploader {
public:
    static constexpr size_t kChunk = size_t{32} << 20;
    explicit Uploader(hipStream_t s) : s_(s) {
        for (int k = 0; k < 2; ++k) {
            if (hipHostMalloc(&buf_[k], kChunk, hipHostMallocDefault) != hipSuccess) buf_[k] = nullptr;
            if (hipEventCreateWithFlags(&ev_[k], hipEventDisableTiming) != hipSuccess) ev_[k] = nullptr;
        }
        // BRISK_HIP_PAGEABLE_UPLOAD=1: the runtime's pageable copies (for comparison)
        pinned_ = buf_[0] != nullptr && buf_[1] != nullptr && ev_[0] != nullptr && ev_[1] != nullptr &&
                  std::getenv("BRISK_HIP_PAGEABLE_UPLOAD") == nullptr;
        const unsigned hw = std::thread::hardware_concurrency();
        threads_ = static_cast<int>(std::min(8u, std::max(1u, hw)));
    }
    ~Uploader() {
        (void)hipStreamSynchronize(s_);
        for (int k = 0; k < 2; ++k) {
            if (buf_[k] != nullptr) (void)hipHostFree(buf_[k]);
            if (ev_[k] != nullptr) (void)hipEventDestroy(ev_[k]);
        }
    }
    Uploader(const Uploader&) = delete;
    Uploader& operator=(const Uploader&) = delete;

    // Enqueues dst[0, bytes) = src[0, bytes) on the stream; src may be reused on return.
    void copy(void* dst, const void* src, size_t bytes) {
        if (!pinned_) {  // no pinned memory: the runtime's blocking pageable copy
            check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s_), "hipMemcpy(upload)");
            check(hipStreamSynchronize(s_), "upload sync");
            return;
        }
        for (size_t off = 0; off < bytes; off += kChunk) {
            const size_t n = std::min(kChunk, bytes - off);
            const int k = next_;
            next_ ^= 1;
            if (used_[k]) check(hipEventSynchronize(ev_[k]), "upload wait");  // the chunk's previous DMA is done
            host_copy(buf_[k], static_cast<const uint8_t*>(src) + off, n);
            check(hipMemcpyAsync(static_cast<uint8_t*>(dst) + off, buf_[k], n, hipMemcpyHostToDevice, s_), "hipMemcpy(upload)");
            check(hipEventRecord(ev_[k], s_), "hipEventRecord(upload)");
            used_[k] = true;
        }
    }
    bool pinned() const { return pinned_; }

private:
    void host_copy(void* dst, const uint8_t* src, size_t n) const {
        constexpr size_t kMinPerThread = size_t{2} << 20;
        const int t = static_cast<int>(std::min<size_t>(threads_, std::max<size_t>(1, n / kMinPerThread)));
        if (t <= 1) {
            std::memcpy(dst, src, n);
            return;
        }
        const size_t per = (n / t + 63) & ~static_cast<size_t>(63);
        std::vector<std::thread> pool;
        pool.reserve(t - 1);
        for (int i = 1; i < t; ++i) {
            const size_t a = std::min(n, per * i), b = std::min(n, per * (i + 1));
            if (a < b) pool.emplace_back([=] { std::memcpy(static_cast<uint8_t*>(dst) + a, src + a, b - a); });
        }
        std::memcpy(dst, src, std::min(n, per));
        for (auto& th : pool) th.join();
    }

    hipStream_t s_;
    void* buf_[2] = {nullptr, nullptr};
    hipEvent_t ev_[2] = {nullptr, nullptr};
    bool used_[2] = {false, false};
    int next_ = 0;
    int threads_ = 1;
    bool pinned_ = false;
};

}  // namespace

DeviceMatrix::~DeviceMatrix() {
    if (mem != nullptr) (void)hipFree(mem);
    if (xmem != nullptr) (void)hipFree(xmem);
}

// The sizes the constructor (and the first prefill / eval_all) allocate, from the
// shapes alone: estimate_memory's parts (src/memory.cpp:46-96) for this backend.
brisk_hip_memory estimate_session(const brisk_hip_config& cfg, const brisk_hip_tensor* tensors, size_t n, size_t max_context) {
    brisk_hip_memory m{};
    size_t staging = 0;
    for (size_t i = 0; i < n; ++i) {
        const brisk_hip_tensor& t = tensors[i];
        if (t.type == BRISK_HIP_F32) {
            m.weights += t.rows * t.cols * 4;
        } else if (block_elems(t.type) != 0) {
            m.weights += packed_bytes(t.type, t.rows, t.cols);
            staging = std::max<size_t>(staging, t.rows * (t.cols / block_elems(t.type)) * gguf_block_bytes(t.type));
        }
    }
    const size_t ctx = max_context == 0 ? cfg.context_length : std::min<size_t>(max_context, cfg.context_length);
    const size_t e = cfg.embd, hd = cfg.head_dim, qd = static_cast<size_t>(cfg.heads) * hd,
                 kvd = static_cast<size_t>(cfg.kv_heads) * hd, ff = cfg.ff;
    // per layer, as estimate_memory counts it (src/memory.cpp:59-68): an LFM2 short-convolution
    // layer (one with blk.N.shortconv.* tensors) holds ctx bx rows of embd halves, every other
    // layer its K and V caches
    size_t conv_layers = 0;
    if (cfg.arch == BRISK_HIP_ARCH_LFM2)
        for (size_t i = 0; i < n; ++i) {
            const std::string name = tensors[i].name != nullptr ? tensors[i].name : "";
            const std::string suffix = ".shortconv.in_proj.weight";
            if (name.size() > suffix.size() && name.compare(name.size() - suffix.size(), suffix.size(), suffix) == 0) ++conv_layers;
        }
    conv_layers = std::min<size_t>(conv_layers, cfg.layers);
    // a Qwen3.5 Gated DeltaNet layer (one with blk.N.ssm_a) holds its state in two halves and
    // the conv's last inputs (src/memory.cpp:62-63)
    size_t rec_layers = 0;
    const size_t ssm_qkv = 3 * static_cast<size_t>(cfg.ssm_v_heads) * cfg.ssm_state;
    if (cfg.arch == BRISK_HIP_ARCH_QWEN35)
        for (size_t i = 0; i < n; ++i) {
            const std::string name = tensors[i].name != nullptr ? tensors[i].name : "";
            const std::string suffix = ".ssm_a";
            if (name.size() > suffix.size() && name.compare(name.size() - suffix.size(), suffix.size(), suffix) == 0) ++rec_layers;
        }
    rec_layers = std::min<size_t>(rec_layers, cfg.layers - conv_layers);
    m.cache = 2 * (static_cast<size_t>(cfg.layers) - conv_layers - rec_layers) * kvd * ctx * 2 + conv_layers * ctx * e * 2 +
              rec_layers * (2 * static_cast<size_t>(cfg.ssm_v_heads) * cfg.ssm_state * cfg.ssm_state + cfg.ssm_conv * ssm_qkv) * 4;
    if (cfg.arch == BRISK_HIP_ARCH_GEMMA4) {  // the layers' own caches at their own shapes (src/memory.cpp:59-68)
        m.cache = 0;
        for (uint32_t l = 0; l < cfg.layers; ++l) {
            const bool slides = cfg.sliding_pattern != nullptr ? cfg.sliding_pattern[l] != 0 : cfg.sliding_window != 0 && l % 6 != 5;
            if (cfg.kv_from_start != 0 && l >= cfg.kv_from_start) continue;
            const size_t hdl = cfg.head_dim_local != 0 && slides ? cfg.head_dim_local : hd;
            const size_t kvh = cfg.kv_head_counts != nullptr ? cfg.kv_head_counts[l] : cfg.kv_heads;
            m.cache += 2 * kvh * hdl * ctx * 2;
        }
    }
    const size_t splits = static_cast<size_t>(attention_max_splits(static_cast<int>(ctx)));
    size_t sc = (e + 2 * qd + ff + cfg.vocab + 2 * kvd) * 4;              // token-path activations, logits
    sc += static_cast<size_t>(cfg.heads) * splits * (hd + 2) * 4;          // attention partials
    sc += (ctx + 1) * 4 + ctx * hd * 4;                                    // token sequence, RoPE table
    if (hd > 128) sc += (qd + static_cast<size_t>(cfg.heads) * ctx) * 4;  // the plain attention's queries and scores
    if (cfg.arch == BRISK_HIP_ARCH_GEMMA3 || cfg.arch == BRISK_HIP_ARCH_GEMMA4) sc += ctx * hd * 4 + e * 4;  // local RoPE, post-norm input
    if (cfg.arch == BRISK_HIP_ARCH_GEMMA4)  // the plain attention, the per-layer embedding inputs and gate
        sc += (qd + static_cast<size_t>(cfg.heads) * ctx + static_cast<size_t>(cfg.ple_dim) * (cfg.layers + 1)) * 4;
    if (cfg.arch == BRISK_HIP_ARCH_LFM2) sc += 3 * e * 4;                  // conv rows
    if (cfg.arch == BRISK_HIP_ARCH_QWEN35)                                 // recurrence rows, query|gate rows, gates
        sc += (ssm_qkv + 2 * static_cast<size_t>(cfg.ssm_inner) + 2 * cfg.ssm_v_heads + 3 * qd) * 4;
    sc += (e + 2 * qd + 2 * kvd + ff + static_cast<size_t>(cfg.heads) * splits * (hd + 2) +
           static_cast<size_t>(cfg.heads) * ctx) * 8;                      // hand-off words (with the spread scores)
    const size_t T = Session::kPrefillTokens, widest = std::max(std::max(e, qd), ff), stride = (widest + 255) / 256 * 256;
    sc += T * (e + 2 * qd + 2 * kvd + ff) * 4 + T * stride * (1 + 4 / 32.0 + 4 / 16.0);  // prefill buffers
    if (cfg.arch == BRISK_HIP_ARCH_GEMMA3 || cfg.arch == BRISK_HIP_ARCH_LFM2) sc += T * e * 4;  // post-norm inputs, conv outputs
    if (cfg.arch == BRISK_HIP_ARCH_LFM2) sc += T * 3 * e * 4;                                   // prefill conv rows
    if (cfg.arch == BRISK_HIP_ARCH_GEMMA4)  // prefill per-layer embedding inputs and gate rows
        sc += T * static_cast<size_t>(cfg.ple_dim) * (cfg.layers + 1) * 4;
    if (cfg.arch == BRISK_HIP_ARCH_QWEN35)  // prefill recurrence rows, query|gate rows, the wider attention output
        sc += T * (5 * static_cast<size_t>(cfg.ssm_inner) + 2 * cfg.ssm_v_heads + 2 * qd) * 4;
    if (ff > static_cast<size_t>(kMaxCols)) sc += (ff + 255) / 256 * 256 * (1 + 4 / 32.0 + 4 / 16.0);  // wide down input
    sc += static_cast<size_t>(64) * cfg.vocab * 4;                         // eval_all logits
    for (size_t i = 0; i < n; ++i)  // the prefill's expanded layer matrices
        if (mx_expanded(static_cast<uint32_t>(tensors[i].type)) && tensors[i].name != nullptr &&
            std::strncmp(tensors[i].name, "blk.", 4) == 0 && tensors[i].rows > 1)
            sc += mx_bytes(static_cast<uint32_t>(tensors[i].type), static_cast<uint32_t>(tensors[i].rows),
                           static_cast<uint32_t>(tensors[i].cols));
    sc += staging + (64 << 10);                                            // load staging, small state
    {  // the token loop's block-major down copies and their term words (Session::setup_loop's push)
        size_t down_bytes = 0;
        bool fmt = cfg.ff % 32 == 0 && cfg.embd <= 4096 && cfg.arch != BRISK_HIP_ARCH_BITNET && cfg.arch != BRISK_HIP_ARCH_GEMMA3 &&
                   cfg.arch != BRISK_HIP_ARCH_GEMMA4 && cfg.arch != BRISK_HIP_ARCH_QWEN35 &&
                   cfg.arch != BRISK_HIP_ARCH_LFM2;
        for (size_t i = 0; i < n && fmt; ++i) {
            const std::string name = tensors[i].name != nullptr ? tensors[i].name : "";
            const auto ends = [&](const std::string& suffix) {
                return name.size() > suffix.size() && name.compare(name.size() - suffix.size(), suffix.size(), suffix) == 0;
            };
            const uint32_t ty = static_cast<uint32_t>(tensors[i].type);
            if (ends(".ffn_sub_norm.weight")) fmt = false;
            if (ends(".ffn_gate.weight") && takes_q8_k(ty)) fmt = false;
            if (ends(".ffn_down.weight")) {
                if (ty != kQ4_0 && ty != kQ4_1 && ty != kQ5_0 && ty != kQ8_0) fmt = false;
                else down_bytes += packed_bytes(ty, tensors[i].rows, tensors[i].cols);
            }
        }
        if (fmt) sc += down_bytes + static_cast<size_t>(cfg.ff / 32) * e * 8;
    }
    m.scratch = sc;
    m.total = m.weights + m.cache + m.scratch;
    return m;
}

static std::string gb(size_t bytes) {
    char buf[32];
    std::snprintf(buf, sizeof(buf), "%.2f GB", static_cast<double>(bytes) / (1024.0 * 1024.0 * 1024.0));
    return buf;
}

// Rotate-half RoPE for every family but the adjacent-pair Llama and SmolLM3 (src/model.cpp:167).
bool Session::neox() const {
    if (cfg_.rope_neox != 0) return cfg_.rope_neox == 1;  // the caller's ModelConfig::rope_neox
    return cfg_.arch != BRISK_HIP_ARCH_LLAMA && cfg_.arch != BRISK_HIP_ARCH_SMOLLM3;
}

Session::Session(const brisk_hip_config& cfg, const brisk_hip_tensor* tensors, size_t n, size_t max_context, int device)
    : cfg_(cfg), device_(device) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) throw Error(BRISK_HIP_ENODEV, "hip: no GPU device available");
    if (device < 0 || device >= count) throw Error(BRISK_HIP_ENODEV, "hip: no GPU device " + std::to_string(device));
    if (cfg.arch < BRISK_HIP_ARCH_QWEN3 || cfg.arch > BRISK_HIP_ARCH_GEMMA4) model_fail("unsupported architecture");
    if (cfg.arch == BRISK_HIP_ARCH_GEMMA4) {  // src/model.cpp:219-227, :275-291
        if (cfg.kv_from_start != 0 && cfg.kv_from_start < 2) model_fail("more shared K/V layers than layers");
        if (cfg.head_dim_local != 0 && (cfg.head_dim_local % 32 != 0 || cfg.head_dim_local > cfg.head_dim))
            model_fail("the sliding layers' head size must be a multiple of 32 no larger than the global one");
        for (uint32_t l = 0; l < cfg.layers; ++l) {
            const uint32_t kvh = cfg.kv_head_counts != nullptr ? cfg.kv_head_counts[l] : cfg.kv_heads;
            if (kvh == 0 || cfg.heads % kvh != 0) model_fail("head_count is not a multiple of head_count_kv");
            if (cfg.heads / kvh > 16) model_fail("more than 16 query heads per key/value head is not supported");
            if (kvh > cfg.kv_heads) model_fail("kv_heads must be the largest of the layers' key/value heads");
            if (cfg.ff_dims != nullptr && (cfg.ff_dims[l] == 0 || cfg.ff_dims[l] > cfg.ff))
                model_fail("ff must be the largest of the layers' feed-forward widths");
        }
    } else if (cfg.sliding_pattern != nullptr || cfg.ff_dims != nullptr || cfg.kv_head_counts != nullptr || cfg.ple_dim != 0 ||
               cfg.kv_from_start != 0 || cfg.head_dim_local != 0) {
        model_fail("per-layer shapes, shared K/V and per-layer embeddings are Gemma 4's only");
    }
    if (cfg.arch == BRISK_HIP_ARCH_QWEN35) {  // src/model.cpp:262-265, :675
        if (cfg.ssm_v_heads == 0 || cfg.ssm_inner % cfg.ssm_v_heads != 0 || cfg.ssm_inner / cfg.ssm_v_heads != cfg.ssm_state ||
            cfg.ssm_k_heads != cfg.ssm_v_heads || cfg.ssm_conv < 2 || cfg.ssm_conv > 8)
            model_fail("qwen35: unsupported DeltaNet shape (equal key and value heads of state_size values are supported)");
        if (cfg.ssm_state > 256) model_fail("qwen35: a DeltaNet state wider than 256 is not supported");
        if (cfg.ssm_inner > kMaxCols) model_fail("a row wider than 8192 is not supported");
    }
    if (cfg.arch == BRISK_HIP_ARCH_LFM2 && (cfg.conv_taps < 2 || cfg.conv_taps > 8)) model_fail("unsupported short-convolution width");
    if (cfg.rope_dim > cfg.head_dim || cfg.rope_dim % 2 != 0) model_fail("rope dimension count must be even and at most the head size");
    if (cfg.embd == 0 || cfg.layers == 0 || cfg.heads == 0 || cfg.kv_heads == 0 || cfg.ff == 0 || cfg.context_length == 0 ||
        cfg.vocab == 0)
        model_fail("a model dimension is zero");
    if (cfg.heads % cfg.kv_heads != 0) model_fail("head_count is not a multiple of head_count_kv");
    if (cfg.heads / cfg.kv_heads > 16) model_fail("more than 16 query heads per key/value head is not supported");
    if (cfg.kv_heads > 1000) model_fail("more than 1000 key/value heads is not supported");  // ticket slots
    if (cfg.head_dim == 0 || cfg.head_dim % 32 != 0 || cfg.head_dim > static_cast<uint32_t>(kPlainMaxHead))
        model_fail("head size must be a non-zero multiple of 32 up to 512");
    if (cfg.embd > kMaxCols || cfg.heads * cfg.head_dim > kMaxCols) model_fail("a row wider than 8192 is not supported");
    // feed-forward rows past kMaxCols: the down projection runs as a one-token GEMM over 256-value
    // chunks (its input quantised to a global buffer), which has no width limit
    if (cfg.ff > kMaxCols && cfg.ff % kMmChunkCols != 0)
        model_fail("a feed-forward row wider than 8192 must be whole 256-value blocks");
    {
        const char* at = std::getenv("BRISK_HIP_ATTN");
        // Gemma 4's layers differ in head size and may read another layer's cache: the plain attention
        plain_attn_ = cfg.head_dim > 128 || cfg.arch == BRISK_HIP_ARCH_GEMMA4 || (at != nullptr && std::string(at) == "plain");
    }
    check(hipSetDevice(device), "hipSetDevice");
    if (std::getenv("BRISK_NO_MEMORY_CHECK") == nullptr) {  // check_memory (src/memory.cpp:118-135), for HBM
        size_t free_b = 0, total_b = 0;
        check(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo");
        const brisk_hip_memory need = estimate_session(cfg, tensors, n, max_context);
        constexpr size_t margin = size_t{256} << 20;
        if (need.total + margin > free_b) {
            std::string hint = "a smaller model or quantisation";
            const size_t shortfall = need.total + margin - free_b;
            if (shortfall <= need.cache * 7 / 8) hint = "a shorter context (the cache is " + gb(need.cache) + "), or " + hint;
            throw Error(BRISK_HIP_ENOMEM, "hip: the session needs about " + gb(need.total) + " (" + gb(need.weights) + " weights, " +
                                              gb(need.cache) + " cache, " + gb(need.scratch) + " scratch) but " + gb(free_b) +
                                              " of device memory is free. Try " + hint +
                                              ", or set BRISK_NO_MEMORY_CHECK=1 to proceed regardless.");
        }
    }
    check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
    max_ctx_ = max_context == 0 ? cfg.context_length : std::min<size_t>(max_context, cfg.context_length);

    auto find = [&](const std::string& name) -> const brisk_hip_tensor* {
        for (size_t i = 0; i < n; ++i)
            if (tensors[i].name != nullptr && name == tensors[i].name) return &tensors[i];
        return nullptr;
    };
    // staging for the GGUF bytes of one matrix before its repack
    size_t staging_bytes = 0;
    for (size_t i = 0; i < n; ++i) {
        const brisk_hip_tensor& t = tensors[i];
        if (t.type != BRISK_HIP_F32) staging_bytes = std::max<size_t>(staging_bytes, t.rows * (t.cols / block_elems(t.type)) * gguf_block_bytes(t.type));
    }
    void* staging = nullptr;
    if (staging_bytes) check(hipMalloc(&staging, staging_bytes), "hipMalloc(staging)");
    // stream order keeps a matrix's upload after the previous matrix's repack out of `staging`
    Uploader up(stream_);

    // rows [row0, row0 + rows) of a matrix of `total` rows (Phi-3's fused tensors, load_matrix_rows,
    // src/model.cpp:370-380; a whole matrix otherwise)
    auto load_rows = [&](const std::string& name, size_t row0, size_t rows, size_t total, size_t cols, DeviceMatrix& m) {
        const brisk_hip_tensor* t = find(name);
        if (t == nullptr) model_fail("missing tensor '" + name + "'");
        if (t->rows != total || t->cols != cols) model_fail("tensor '" + name + "' has an unexpected shape");
        const uint32_t type = static_cast<uint32_t>(t->type);
        if (gguf_block_bytes(type) == 0) model_fail("tensor '" + name + "' has a type the HIP session does not take");
        if (cols % block_elems(type) != 0) model_fail("tensor '" + name + "' row length is not a multiple of its block size");
        size_t planes[3];
        plane_bytes(type, rows, cols, planes);
        check(hipMalloc(&m.mem, packed_bytes(type, rows, cols)), "hipMalloc(weights)");
        uint8_t* base = static_cast<uint8_t*>(m.mem);
        m.p = Packed{base, base + align256(planes[0]), base + align256(planes[0]) + align256(planes[1]),
                     static_cast<uint32_t>(rows), static_cast<uint32_t>(cols), type, 0u};
        // x86's load-time TQ2_0x16 layout (rows % 16 == 0) takes 7-bit activations (src/model.cpp:496-503)
        if (type == kTQ2_0 && rows % 16 == 0) m.p.flags |= kFlagLut16;
        const size_t row_bytes = (cols / block_elems(type)) * gguf_block_bytes(type), bytes = rows * row_bytes;
        up.copy(staging, static_cast<const uint8_t*>(t->data) + row0 * row_bytes, bytes);
        check(launch_pack(type, staging, rows, cols, m.p, stream_), "pack");
        weight_bytes_ += bytes;
    };
    auto load_matrix = [&](const std::string& name, size_t rows, size_t cols, DeviceMatrix& m) {
        load_rows(name, 0, rows, rows, cols, m);
    };
    auto load_vector = [&](const std::string& name, size_t count) -> float* {
        const brisk_hip_tensor* t = find(name);
        if (t == nullptr) model_fail("missing tensor '" + name + "'");
        if (t->rows * t->cols != count) model_fail("tensor '" + name + "' has an unexpected size");
        if (t->type != BRISK_HIP_F32) model_fail("tensor '" + name + "' is not F32");
        float* p = static_cast<float*>(alloc(count * sizeof(float)));
        up.copy(p, t->data, count * sizeof(float));
        return p;
    };

    const size_t e = cfg.embd, hd = cfg.head_dim, qd = static_cast<size_t>(cfg.heads) * hd, kvd = static_cast<size_t>(cfg.kv_heads) * hd;
    // ModelConfig's flags: the caller's values where given, else the family's (src/model.cpp:161-301)
    const uint32_t no_rope_step = cfg.no_rope_step == 0xFFFFFFFFu ? 0 : cfg.no_rope_step != 0 ? cfg.no_rope_step
                                : cfg.arch == BRISK_HIP_ARCH_SMOLLM3 ? 4 : 0;
    if (cfg.gelu != 0 && (cfg.gelu == 1) != gemma()) model_fail("GELU gating outside Gemma is not supported");
    if (cfg.embedding_scale != 0.0f && !gemma() && cfg.embedding_scale != 1.0f)
        model_fail("scaled embeddings outside Gemma are not supported");
    load_matrix("token_embd.weight", cfg.vocab, e, embd_);
    if (find("output.weight") != nullptr) {
        load_matrix("output.weight", cfg.vocab, e, out_own_);
        out_ = &out_own_;
    } else {
        out_ = &embd_;  // tied (src/model.cpp:328-330)
    }
    out_norm_ = load_vector(cfg.arch == BRISK_HIP_ARCH_LFM2 ? "token_embd_norm.weight" : "output_norm.weight", e);  // src/model.cpp:331
    if (cfg.ple_dim != 0) {  // Gemma 4's per-layer embeddings (src/model.cpp:319-324)
        const size_t pall = static_cast<size_t>(cfg.ple_dim) * cfg.layers;
        load_matrix("per_layer_token_embd.weight", cfg.vocab, pall, ple_tok_);
        load_matrix("per_layer_model_proj.weight", pall, e, ple_proj_);
        ple_norm_ = load_vector("per_layer_proj_norm.weight", cfg.ple_dim);
    }
    layers_.resize(cfg.layers);
    for (uint32_t l = 0; l < cfg.layers; ++l) {
        const std::string b = "blk." + std::to_string(l) + ".";
        Layer& L = layers_[l];
        L.attn_norm = load_vector(b + "attn_norm.weight", e);
        // ModelConfig's per-layer accessors (src/model.h:87-118)
        L.slides = gemma() && (cfg.sliding_pattern != nullptr ? cfg.sliding_pattern[l] != 0 : cfg.sliding_window != 0 && l % 6 != 5);
        L.hd = static_cast<int>(cfg.head_dim_local != 0 && L.slides ? cfg.head_dim_local : cfg.head_dim);
        L.kvh = static_cast<int>(cfg.kv_head_counts != nullptr ? cfg.kv_head_counts[l] : cfg.kv_heads);
        L.ff = static_cast<int>(cfg.ff_dims != nullptr ? cfg.ff_dims[l] : cfg.ff);
        L.kv_src = static_cast<int>(cfg.kv_from_start == 0 || l < cfg.kv_from_start ? l : cfg.kv_from_start - (L.slides ? 2 : 1));
        if (cfg.arch == BRISK_HIP_ARCH_QWEN35 && find(b + "ssm_a") != nullptr) {  // src/model.cpp:343-358
            const size_t qkv = 3 * static_cast<size_t>(cfg.ssm_v_heads) * cfg.ssm_state;
            load_matrix(b + "attn_qkv.weight", qkv, e, L.ssm_qkv);
            load_matrix(b + "attn_gate.weight", cfg.ssm_inner, e, L.ssm_gate);
            load_matrix(b + "ssm_alpha.weight", cfg.ssm_v_heads, e, L.ssm_alpha);
            load_matrix(b + "ssm_beta.weight", cfg.ssm_v_heads, e, L.ssm_beta);
            L.ssm_a = load_vector(b + "ssm_a", cfg.ssm_v_heads);
            L.ssm_dt = load_vector(b + "ssm_dt.bias", cfg.ssm_v_heads);
            L.ssm_conv_w = load_vector(b + "ssm_conv1d.weight", static_cast<size_t>(cfg.ssm_conv) * qkv);
            L.ssm_norm = load_vector(b + "ssm_norm.weight", cfg.ssm_state);
            load_matrix(b + "ssm_out.weight", e, cfg.ssm_inner, L.ssm_out);
            L.ffn_norm = load_vector(b + "post_attention_norm.weight", e);
            load_matrix(b + "ffn_gate.weight", cfg.ff, e, L.gate);
            load_matrix(b + "ffn_up.weight", cfg.ff, e, L.up);
            load_matrix(b + "ffn_down.weight", e, cfg.ff, L.down);
            if (takes_q8_k(L.gate.p.type) != takes_q8_k(L.up.p.type) || act_bits(L.gate.p) != act_bits(L.up.p))
                model_fail("fused multiply mixes activation widths");
            continue;
        }
        if (cfg.arch == BRISK_HIP_ARCH_LFM2 && find(b + "shortconv.in_proj.weight") != nullptr) {  // src/model.cpp:360-364
            load_matrix(b + "shortconv.in_proj.weight", 3 * e, e, L.conv_in);
            load_matrix(b + "shortconv.out_proj.weight", e, e, L.conv_out);
            L.conv_w = load_vector(b + "shortconv.conv.weight", static_cast<size_t>(cfg.conv_taps) * e);
            L.ffn_norm = load_vector(b + "ffn_norm.weight", e);
            load_matrix(b + "ffn_gate.weight", cfg.ff, e, L.gate);
            load_matrix(b + "ffn_up.weight", cfg.ff, e, L.up);
            load_matrix(b + "ffn_down.weight", e, cfg.ff, L.down);
            continue;
        }
        if (cfg.arch == BRISK_HIP_ARCH_PHI3 && find(b + "attn_qkv.weight") != nullptr) {  // Q|K|V rows of attn_qkv, gate|up rows of ffn_up
            load_rows(b + "attn_qkv.weight", 0, qd, qd + 2 * kvd, e, L.q);
            load_rows(b + "attn_qkv.weight", qd, kvd, qd + 2 * kvd, e, L.k);
            load_rows(b + "attn_qkv.weight", qd + kvd, kvd, qd + 2 * kvd, e, L.v);
            load_rows(b + "ffn_up.weight", 0, cfg.ff, 2 * static_cast<size_t>(cfg.ff), e, L.gate);
            load_rows(b + "ffn_up.weight", cfg.ff, cfg.ff, 2 * static_cast<size_t>(cfg.ff), e, L.up);
        } else {
            const size_t qdl = static_cast<size_t>(cfg.heads) * L.hd, kvdl = static_cast<size_t>(L.kvh) * L.hd;
            load_matrix(b + "attn_q.weight", qwen35() ? 2 * qdl : qdl, e, L.q);  // Qwen3.5: each head's query, then its gate
            if (L.kv_src == static_cast<int>(l)) {
                load_matrix(b + "attn_k.weight", kvdl, e, L.k);
                // Gemma 4 global layers may have no V projection: K serves as V (src/model.cpp:386-388)
                L.v_is_k = gemma4() && find(b + "attn_v.weight") == nullptr;
                if (!L.v_is_k) load_matrix(b + "attn_v.weight", kvdl, e, L.v);
            }
            load_matrix(b + "ffn_gate.weight", L.ff, e, L.gate);
            load_matrix(b + "ffn_up.weight", L.ff, e, L.up);
        }
        load_matrix(b + "attn_output.weight", e, static_cast<size_t>(cfg.heads) * L.hd, L.o);
        L.ffn_norm = load_vector(b + (qwen35() ? "post_attention_norm.weight" : "ffn_norm.weight"), e);  // src/model.cpp:418
        load_matrix(b + "ffn_down.weight", e, L.ff, L.down);
        if (cfg.arch == BRISK_HIP_ARCH_QWEN3 || gemma() || cfg.arch == BRISK_HIP_ARCH_LFM2 || qwen35()) {
            L.q_norm = load_vector(b + "attn_q_norm.weight", L.hd);
            if (L.kv_src == static_cast<int>(l)) L.k_norm = load_vector(b + "attn_k_norm.weight", L.hd);
        }
        if (cfg.ple_dim != 0) {  // src/model.cpp:403-407
            load_matrix(b + "inp_gate.weight", cfg.ple_dim, e, L.ple_gate);
            load_matrix(b + "proj.weight", e, cfg.ple_dim, L.ple_proj);
            L.ple_post_norm = load_vector(b + "post_norm.weight", e);
        }
        if (const brisk_hip_tensor* os = find(b + "layer_output_scale.weight")) {  // src/model.cpp:408-410
            if (os->type != BRISK_HIP_F32 || os->rows * os->cols != 1) model_fail("tensor '" + b + "layer_output_scale.weight' has an unexpected size");
            L.out_scale = *static_cast<const float*>(os->data);
        }
        if (cfg.arch == BRISK_HIP_ARCH_BITNET) {
            L.attn_sub_norm = load_vector(b + "attn_sub_norm.weight", e);
            L.ffn_sub_norm = load_vector(b + "ffn_sub_norm.weight", cfg.ff);
        }
        if (find(b + "attn_q.bias") != nullptr) {  // src/model.cpp:411-416
            L.q_bias = load_vector(b + "attn_q.bias", qd);
            L.k_bias = load_vector(b + "attn_k.bias", kvd);
            L.v_bias = load_vector(b + "attn_v.bias", kvd);
        }
        L.rope = no_rope_step == 0 || (l + 1) % no_rope_step != 0;  // layer_has_rope (src/model.h:110, src/model.cpp:168)
        if (gemma()) {  // src/model.cpp:399-402
            L.attn_post_norm = load_vector(b + "post_attention_norm.weight", e);
            L.ffn_post_norm = load_vector(b + "post_ffw_norm.weight", e);
        }
        // one activation row feeds Q, K and V: they must take the same width (src/model.cpp:584-590)
        const Packed& kp = L.k.mem != nullptr ? L.k.p : L.q.p;  // a shared layer projects Q only
        const Packed& vp = L.v.mem != nullptr ? L.v.p : kp;     // K serving as V
        if (takes_q8_k(L.q.p.type) != takes_q8_k(kp.type) || takes_q8_k(L.q.p.type) != takes_q8_k(vp.type) ||
            act_bits(L.q.p) != act_bits(kp) || act_bits(L.q.p) != act_bits(vp) ||
            takes_q8_k(L.gate.p.type) != takes_q8_k(L.up.p.type) || act_bits(L.gate.p) != act_bits(L.up.p))
            model_fail("fused multiply mixes activation widths");
    }
    check(hipStreamSynchronize(stream_), "upload sync");
    if (staging) check(hipFree(staging), "hipFree(staging)");
    // the per-layer tables live in the layers now; the caller's arrays are not kept
    cfg_.sliding_pattern = nullptr;
    cfg_.ff_dims = nullptr;
    cfg_.kv_head_counts = nullptr;

    // activations and state
    h_ = static_cast<float*>(alloc(e * 4));
    if (lfm2()) {
        conv_buf_ = static_cast<float*>(alloc(3 * e * 4));
        for (Layer& L : layers_)
            if (L.conv_w != nullptr) L.conv_cache = static_cast<uint16_t*>(alloc(max_ctx_ * e * 2));
    }
    if (qwen35()) {
        const size_t qkv = 3 * static_cast<size_t>(cfg.ssm_v_heads) * cfg.ssm_state;
        ssm_qkv_ = static_cast<float*>(alloc(qkv * 4));
        ssm_z_ = static_cast<float*>(alloc(static_cast<size_t>(cfg.ssm_inner) * 4));
        ssm_ab_ = static_cast<float*>(alloc(2 * static_cast<size_t>(cfg.ssm_v_heads) * 4));
        qg_ = static_cast<float*>(alloc(2 * qd * 4));
        agate_ = static_cast<float*>(alloc(qd * 4));
        for (Layer& L : layers_) {
            if (L.ssm_a == nullptr) continue;
            const size_t ring = static_cast<size_t>(cfg.ssm_conv) * qkv * 4,
                         state = 2 * static_cast<size_t>(cfg.ssm_v_heads) * cfg.ssm_state * cfg.ssm_state * 4;
            L.ssm_ring = static_cast<float*>(alloc(ring));
            L.ssm_state = static_cast<float*>(alloc(state));
            check(hipMemsetAsync(L.ssm_ring, 0, ring, stream_), "memset");
            check(hipMemsetAsync(L.ssm_state, 0, state, stream_), "memset");
        }
    }
    q_ = static_cast<float*>(alloc(qd * 4));
    att_ = static_cast<float*>(alloc(std::max<size_t>(qd, cfg.ssm_inner) * 4));
    act_ = static_cast<float*>(alloc(static_cast<size_t>(cfg.ff) * 4));
    if (cfg.ff > kMaxCols) {  // the wide down projection's quantised input, one token
        wide_x_.stride = static_cast<int>((cfg.ff + kMmChunkCols - 1) / kMmChunkCols * kMmChunkCols);
        wide_x_.qs = static_cast<int8_t*>(alloc(wide_x_.stride));
        wide_x_.d = static_cast<float*>(alloc((wide_x_.stride / 32) * 4));
        wide_x_.bs = static_cast<int32_t*>(alloc((wide_x_.stride / 16) * 4));
    }
    logits_ = static_cast<float*>(alloc(static_cast<size_t>(cfg.vocab) * 4));
    max_splits_ = attention_max_splits(static_cast<int>(max_ctx_));
    if (plain_attn_) {
        plain_q_ = static_cast<float*>(alloc(qd * 4));
        plain_sc_ = static_cast<float*>(alloc(static_cast<size_t>(cfg.heads) * max_ctx_ * 4));
    }
    part_acc_ = static_cast<float*>(alloc(static_cast<size_t>(cfg.heads) * max_splits_ * hd * 4));
    part_ml_ = static_cast<float*>(alloc(static_cast<size_t>(cfg.heads) * max_splits_ * 2 * 4));
    k_ = static_cast<float*>(alloc(kvd * 4));
    v_ = static_cast<float*>(alloc(kvd * 4));
    key_ = static_cast<unsigned long long*>(alloc(64));  // [0]: graph path; [2], [3]: loop (by step parity)
    check(hipMemsetAsync(key_, 0, 64, stream_), "memset");
    ticket_ = static_cast<unsigned*>(alloc(4096));
    pos_ = static_cast<int*>(alloc(64));
    seq_ = static_cast<int*>(alloc((max_ctx_ + 1) * 4));
    check(hipMemsetAsync(ticket_, 0, 4096, stream_), "memset");
    check(hipMemsetAsync(pos_, 0, 64, stream_), "memset");
    check(hipMemsetAsync(seq_, 0, (max_ctx_ + 1) * 4, stream_), "memset");
    kcache_.assign(cfg.layers, nullptr);
    vcache_.assign(cfg.layers, nullptr);
    kv_bytes_.assign(cfg.layers, 0);
    for (uint32_t l = 0; l < cfg.layers; ++l) {
        const Layer& L = layers_[l];
        if (L.conv_w != nullptr) continue;  // a short-convolution layer keeps its bx rows instead (LFM2)
        if (L.ssm_a != nullptr) continue;   // a recurrent layer keeps its state instead (Qwen3.5)
        if (L.kv_src != static_cast<int>(l)) {  // Gemma 4: the cache of an earlier layer of its kind (src/model.cpp:979-983)
            kcache_[l] = kcache_[L.kv_src];
            vcache_[l] = vcache_[L.kv_src];
            kv_bytes_[l] = kv_bytes_[L.kv_src];
            continue;
        }
        const size_t kv_bytes = static_cast<size_t>(L.kvh) * max_ctx_ * L.hd * 2;
        kcache_[l] = static_cast<uint16_t*>(alloc(kv_bytes));
        vcache_[l] = static_cast<uint16_t*>(alloc(kv_bytes));
        check(hipMemsetAsync(kcache_[l], 0, kv_bytes, stream_), "memset");
        check(hipMemsetAsync(vcache_[l], 0, kv_bytes, stream_), "memset");
        kv_bytes_[l] = kv_bytes;
    }
    if (cfg.ple_dim != 0) {
        ple_in_ = static_cast<float*>(alloc(static_cast<size_t>(cfg.ple_dim) * cfg.layers * 4));
        ple_g_ = static_cast<float*>(alloc(static_cast<size_t>(cfg.ple_dim) * 4));
    }

    // RoPE table, built on the host exactly as build_rope does (src/model.cpp:880-894):
    // theta_scale = base^(-2/dim); theta = pos * scale, multiplied by theta_scale per pair.
    // Gemma 3: the global layers' positions are scaled by 1 / rope.scaling.factor, the
    // sliding layers take their own base at scale 1 (src/model.cpp:893-894).
    // Per-frequency factors divide the angle (Llama 3's rope_freqs, Phi-3's LongRoPE short or,
    // past the original context, long factors: src/model.cpp:312-318, :691-694, :886-888) and
    // Phi-3's attention factor scales cos and sin; only the first rope_dim dimensions rotate.
    const size_t rd = cfg.rope_dim != 0 ? cfg.rope_dim : hd;
    rope_dim_ = static_cast<int>(rd);
    const float attn_factor = cfg.rope_attn_factor != 0.0f ? cfg.rope_attn_factor : 1.0f;
    const float* factors = nullptr;
    {
        std::vector<const char*> names = {"rope_freqs.weight"};
        if (cfg.arch == BRISK_HIP_ARCH_PHI3)
            names = {cfg.rope_original_context != 0 && max_ctx_ > cfg.rope_original_context ? "rope_factors_long.weight"
                                                                                            : "rope_factors_short.weight"};
        for (const char* nm : names) {
            const brisk_hip_tensor* t = find(nm);
            if (t == nullptr) continue;
            if (t->type != BRISK_HIP_F32 || t->rows * t->cols < rd / 2) model_fail(std::string("tensor '") + nm + "' has an unexpected size");
            factors = static_cast<const float*>(t->data);
        }
    }
    auto rope_table = [&](float base, float scale, size_t dim, const float* fac, float af) {
        std::vector<float> rope(max_ctx_ * dim);
        const float theta_scale = std::pow(base, -2.0f / static_cast<float>(dim));
        for (size_t p = 0; p < max_ctx_; ++p) {
            float theta = static_cast<float>(p) * scale;
            float* r = rope.data() + p * dim;
            for (size_t i = 0; i < dim / 2; ++i) {
                const float angle = fac != nullptr ? theta / fac[i] : theta;
                r[2 * i] = std::cos(angle) * af;
                r[2 * i + 1] = std::sin(angle) * af;
                theta *= theta_scale;
            }
        }
        float* d = static_cast<float*>(alloc(rope.size() * 4));
        check(hipMemcpy(d, rope.data(), rope.size() * 4, hipMemcpyHostToDevice), "hipMemcpy(rope)");
        return d;
    };
    rope_ = rope_table(cfg.rope_base, gemma() && cfg.rope_scale != 0.0f ? cfg.rope_scale : 1.0f, rd, factors, attn_factor);
    if (gemma()) {
        // the sliding layers' table at their own head size (Gemma 4's are narrower, src/model.cpp:875, :894)
        if (cfg.sliding_window != 0)
            rope_local_ = rope_table(cfg.rope_base_local, 1.0f, cfg.head_dim_local != 0 ? cfg.head_dim_local : hd, nullptr, 1.0f);
        proj_ = static_cast<float*>(alloc(e * 4));
        embd_scale_ = cfg.embedding_scale != 0.0f ? cfg.embedding_scale : std::sqrt(static_cast<float>(cfg.embd));
    }
    check(hipStreamSynchronize(stream_), "init sync");
    debug_ = std::getenv("BRISK_HIP_DEBUG") != nullptr;
    {
        const char* pf = std::getenv("BRISK_HIP_PREFILL");
        prefill_on_ = !(pf != nullptr && std::string(pf) == "0") && !debug_;
        // the batched GEMMs stage their rows in 256-value chunks; rows of 32-value blocks may end
        // inside the last one
        auto chunked = [](const Packed& p) {
            const bool small = p.type == kQ4_0 || p.type == kQ4_1 || p.type == kQ5_0 || p.type == kQ8_0;
            return p.cols % kMmChunkCols == 0 || (small && p.cols % 32 == 0 && p.cols <= static_cast<uint32_t>(kMaxCols));
        };
        for (const Layer& L : layers_)
            for (const DeviceMatrix* m : {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down, &L.conv_in, &L.conv_out, &L.ssm_qkv,
                                          &L.ssm_gate, &L.ssm_alpha, &L.ssm_beta, &L.ssm_out, &L.ple_gate, &L.ple_proj})
                if (m->mem != nullptr && !chunked(m->p)) prefill_shapes_ = false;
        if (!chunked(out_->p)) prefill_shapes_ = false;
        if (ple_proj_.mem != nullptr && !chunked(ple_proj_.p)) prefill_shapes_ = false;
        prefill_on_ = prefill_on_ && prefill_shapes_;
        const char* pa = std::getenv("BRISK_HIP_PREFILL_ATTN");  // "mfma": long prompts' attention on f16 MFMA
        prefill_mfma_ = pa != nullptr && std::string(pa) == "mfma";
        prefill_legacy_ = pa != nullptr && std::string(pa) == "staged";
    }
    setup_loop();
    use_graphs_ = std::getenv("BRISK_HIP_NO_GRAPH") == nullptr && !debug_;
    if (use_graphs_) {
        graph_layers_ = capture(false);
        graph_full_ = capture(true);
    }
}

Session::~Session() {
    // the stream's work (a loop launch, copies into the pinned staging buffer) is done before any
    // graph, allocation or the stream itself is released
    if (stream_) (void)hipStreamSynchronize(stream_);
    if (graph_layers_) (void)hipGraphExecDestroy(graph_layers_);
    if (graph_full_) (void)hipGraphExecDestroy(graph_full_);
    for (void* p : owned_) (void)hipFree(p);
    if (host_io_) (void)hipHostFree(host_io_);
    if (stream_) (void)hipStreamDestroy(stream_);
}

// Pinned host staging for the token and logits copies: a pageable copy goes through the
// runtime's own staging, a few hundred microseconds more for a row of logits.  Grown on demand.
void* Session::host_buf(size_t bytes) {
    if (bytes > host_io_bytes_) {
        if (host_io_) (void)hipHostFree(host_io_);
        host_io_ = nullptr;
        host_io_bytes_ = 0;
        check(hipHostMalloc(&host_io_, bytes, hipHostMallocDefault), "hipHostMalloc(staging)");
        host_io_bytes_ = bytes;
    }
    return host_io_;
}

void* Session::alloc(size_t bytes) {
    void* p = nullptr;
    check(hipMalloc(&p, bytes < 64 ? 64 : bytes), "hipMalloc");
    owned_.push_back(p);
    return p;
}

// One decode step at *pos_: embed seq[*pos_], every layer, then either the
// output projection + greedy pick (which advances *pos_) or a bare advance.
void Session::record_step(bool full) {
    check(launch_embed(embd_.p, pick_state(), h_, embd_scale_, stream_), "embed");
    const int e = static_cast<int>(cfg_.embd);
    if (cfg_.ple_dim != 0) {  // Gemma 4's per-layer embedding inputs (src/model.cpp:905-925)
        GemvArgs pa{};
        pa.n = 1; pa.t[0].m = ple_proj_.p; pa.t[0].out = ple_in_;
        pa.x = h_; pa.normw = nullptr; pa.eps = cfg_.rms_epsilon; pa.add = 0;
        check(launch_gemv(pa, stream_), "per-layer projection");
        check(launch_ple_inputs(ple_in_, ple_tok_.p, ple_norm_, seq_, pos_, static_cast<int>(cfg_.layers), static_cast<int>(cfg_.ple_dim),
                                1.0f / std::sqrt(static_cast<float>(cfg_.embd)), std::sqrt(static_cast<float>(cfg_.ple_dim)),
                                cfg_.rms_epsilon, stream_),
              "per-layer inputs");
    }
    for (uint32_t l = 0; l < cfg_.layers; ++l) {
        const Layer& L = layers_[l];
        if (L.conv_w != nullptr) {  // LFM2 short convolution in place of attention (src/model.cpp:935-969)
            GemvArgs ca{};
            ca.n = 1; ca.t[0].m = L.conv_in.p; ca.t[0].out = conv_buf_;
            ca.x = h_; ca.normw = L.attn_norm; ca.eps = cfg_.rms_epsilon; ca.add = 0;
            check(launch_gemv(ca, stream_), "conv in_proj");
            check(launch_conv(conv_buf_, L.conv_cache, L.conv_w, static_cast<int>(cfg_.conv_taps), pos_,
                              static_cast<int>(cfg_.embd), att_, stream_), "conv");
            GemvArgs co{};
            co.n = 1; co.t[0].m = L.conv_out.p; co.t[0].out = h_;
            co.x = att_; co.normw = nullptr; co.eps = cfg_.rms_epsilon; co.add = 1;
            check(launch_gemv(co, stream_), "conv out_proj");
        }
        if (L.ssm_a != nullptr) {  // Qwen3.5 Gated DeltaNet in place of attention (src/model.cpp:754-865)
            // attn_qkv, attn_gate, ssm_alpha and ssm_beta rows from attn_norm(h): one launch per weight format
            const DeviceMatrix* mats[4] = {&L.ssm_qkv, &L.ssm_gate, &L.ssm_alpha, &L.ssm_beta};
            float* outs[4] = {ssm_qkv_, ssm_z_, ssm_ab_, ssm_ab_ + cfg_.ssm_v_heads};
            GemvArgs ia{};
            ia.x = h_; ia.normw = L.attn_norm; ia.eps = cfg_.rms_epsilon; ia.add = 0;
            bool done[4] = {false, false, false, false};
            for (int i = 0; i < 4; ++i) {
                if (done[i]) continue;
                ia.n = 0;
                for (int j = i; j < 4; ++j) {
                    if (!done[j] && mats[j]->p.type == mats[i]->p.type) {
                        ia.t[ia.n].m = mats[j]->p;
                        ia.t[ia.n].out = outs[j];
                        ++ia.n;
                        done[j] = true;
                    }
                }
                check(launch_gemv(ia, stream_), "recurrence projections");
            }
            SsmArgs sa{};
            sa.qkv = ssm_qkv_; sa.z = ssm_z_; sa.ab = ssm_ab_; sa.conv_w = L.ssm_conv_w; sa.a = L.ssm_a; sa.dt = L.ssm_dt;
            sa.norm = L.ssm_norm; sa.ring = L.ssm_ring; sa.state = L.ssm_state; sa.pos = pos_; sa.out = att_;
            sa.heads = static_cast<int>(cfg_.ssm_v_heads); sa.dim = static_cast<int>(cfg_.ssm_state);
            sa.taps = static_cast<int>(cfg_.ssm_conv); sa.qkv_dim = 3 * sa.heads * sa.dim;
            sa.eps = cfg_.rms_epsilon; sa.q_scale = 1.0f / std::sqrt(static_cast<float>(cfg_.ssm_state));  // src/model.cpp:813
            check(launch_ssm(sa, stream_), "recurrence");
            GemvArgs so{};
            so.n = 1; so.t[0].m = L.ssm_out.p; so.t[0].out = h_;
            so.x = att_; so.normw = nullptr; so.eps = cfg_.rms_epsilon; so.add = 1;
            check(launch_gemv(so, stream_), "ssm_out");
        }
        // Q, K, V rows from attn_norm(h) (src/model.cpp:996-1015): one launch per weight format
        const bool own_kv = L.kv_src == static_cast<int>(l);
        if (L.conv_w == nullptr && L.ssm_a == nullptr) {
            // a shared layer (Gemma 4) projects Q only; K serving as V is projected once
            const DeviceMatrix* mats[3] = {&L.q, &L.k, &L.v};
            float* outs[3] = {qwen35() ? qg_ : q_, k_, v_};
            const int nm = !own_kv ? 1 : L.v_is_k ? 2 : 3;
            GemvArgs qa{};
            qa.x = h_; qa.normw = L.attn_norm; qa.eps = cfg_.rms_epsilon; qa.add = 0;
            bool done[3] = {false, false, false};
            for (int i = 0; i < nm; ++i) {
                if (done[i]) continue;
                qa.n = 0;
                for (int j = i; j < nm; ++j) {
                    if (!done[j] && mats[j]->p.type == mats[i]->p.type) {
                        qa.t[qa.n].m = mats[j]->p;
                        qa.t[qa.n].out = outs[j];
                        ++qa.n;
                        done[j] = true;
                    }
                }
                check(launch_gemv(qa, stream_), "qkv");
            }
            // Qwen3.5: the plain attention reads the query and gate rows in place; the others take them split
            if (qwen35() && !plain_attn_)
                check(launch_qgate_split(qg_, q_, agate_, static_cast<int>(cfg_.heads), static_cast<int>(cfg_.head_dim), stream_), "query gate");
        }

        if (L.conv_w == nullptr && L.ssm_a == nullptr) {
        AttnArgs aa{};
        aa.q = q_; aa.k = k_; aa.v = L.v_is_k ? k_ : v_; aa.qnorm = L.q_norm; aa.knorm = L.k_norm;
        aa.rope = !L.rope ? nullptr : L.slides ? rope_local_ : rope_;
        aa.window = L.slides ? static_cast<int>(cfg_.sliding_window) : 0;
        // the rotated width (src/model.cpp:1024): the sliding layer's head, else the rotary dimension within the head
        aa.rope_dim = L.slides ? L.hd : std::min(rope_dim_, L.hd);
        aa.qbias = L.q_bias; aa.kbias = L.k_bias; aa.vbias = L.v_bias;
        aa.eps = cfg_.rms_epsilon; aa.neox = neox();
        aa.kcache = kcache_[l]; aa.vcache = vcache_[l]; aa.pos = pos_;
        aa.ctx = static_cast<int>(max_ctx_); aa.head_dim = L.hd;
        aa.heads = static_cast<int>(cfg_.heads); aa.kv_heads = L.kvh;
        aa.vnorm = cfg_.value_norm; aa.no_kv = own_kv ? 0 : 1;
        // src/model.cpp:978: the family's scale, else 1 / sqrt(the layer's head size)
        aa.scale = cfg_.attention_scale != 0.0f ? cfg_.attention_scale : 1.0f / std::sqrt(static_cast<float>(L.hd));
        aa.part_acc = part_acc_; aa.part_ml = part_ml_; aa.max_splits = max_splits_;
        aa.tickets = ticket_ + 4; aa.out = att_;
        // scores past the LDS limit go to the split buffers: heads x ctx floats fit them
        // (heads x max_splits x head_dim, head_dim >= the split length)
        aa.gsc = cfg_.head_dim >= static_cast<uint32_t>(kSplit) ? part_acc_ : nullptr;
        if (plain_attn_) {
            aa.gsc = plain_sc_;
            aa.qn = plain_q_;
            if (qwen35()) {  // each head's query rows, then its gate rows (src/model.cpp:1002-1012)
                aa.q = qg_;
                aa.q_stride = 2 * L.hd;
                aa.gate = qg_ + L.hd;
                aa.gate_stride = 2 * L.hd;
            }
            check(launch_attention_plain(aa, stream_), "attention");
        } else {
            check(launch_attention(aa, stream_), "attention");
            if (qwen35()) check(launch_sigmoid_gate(att_, agate_, static_cast<int>(cfg_.heads * cfg_.head_dim), stream_), "attention gate");
        }

        // h += W_o att, or with a post-norm h += rms_norm(W_o att) (src/model.cpp:1113-1121)
        GemvArgs oa{};
        oa.n = 1; oa.t[0].m = L.o.p; oa.t[0].out = L.attn_post_norm ? proj_ : h_;
        oa.x = att_; oa.normw = L.attn_sub_norm; oa.eps = cfg_.rms_epsilon; oa.add = L.attn_post_norm ? 0 : 1;
        check(launch_gemv(oa, stream_), "attn_output");
        if (L.attn_post_norm) check(launch_post_add(h_, proj_, L.attn_post_norm, cfg_.rms_epsilon, static_cast<int>(cfg_.embd), stream_), "post norm");
        }

        GateUpArgs ga{};
        ga.gate = L.gate.p; ga.up = L.up.p; ga.x = h_; ga.normw = L.ffn_norm; ga.eps = cfg_.rms_epsilon;
        ga.relu2 = cfg_.arch == BRISK_HIP_ARCH_BITNET; ga.gelu = gemma(); ga.act = act_;
        check(launch_gateup(ga, stream_), "gate_up");

        if (L.ff > kMaxCols) {  // wider than the GEMV's activation buffer: quantised to wide_x_, then a one-token GEMM
            check(launch_pre_quant(act_, L.ff, L.ffn_sub_norm, cfg_.rms_epsilon, L.ff, 1, takes_q8_k(L.down.p.type), act_bits(L.down.p),
                                   wide_x_, stream_),
                  "ffn_down input");
            MmArgs dm{};
            dm.m = L.down.p; dm.x = wide_x_; dm.ntok = 1; dm.out = L.ffn_post_norm ? proj_ : h_; dm.ostride = e;
            check(launch_mm(dm, L.ffn_post_norm ? kMmStore : kMmAdd, stream_), "ffn_down");
        } else {
            GemvArgs da{};
            da.n = 1; da.t[0].m = L.down.p; da.t[0].out = L.ffn_post_norm ? proj_ : h_;
            da.x = act_; da.normw = L.ffn_sub_norm; da.eps = cfg_.rms_epsilon; da.add = L.ffn_post_norm ? 0 : 1;
            check(launch_gemv(da, stream_), "ffn_down");
        }
        if (L.ffn_post_norm) check(launch_post_add(h_, proj_, L.ffn_post_norm, cfg_.rms_epsilon, static_cast<int>(cfg_.embd), stream_), "post norm");
        if (cfg_.ple_dim != 0) {  // h = (h + norm(proj(gelu(gate h) * input l))) * scale (src/model.cpp:1163-1177)
            GemvArgs pg{};  // gelu(gate h) * input l, in the GEMV's epilogue
            pg.n = 1; pg.t[0].m = L.ple_gate.p; pg.t[0].out = ple_g_;
            pg.x = h_; pg.normw = nullptr; pg.eps = cfg_.rms_epsilon; pg.add = 0;
            pg.gelu_in = ple_in_ + static_cast<size_t>(l) * cfg_.ple_dim;
            check(launch_gemv(pg, stream_), "per-layer gate");
            GemvArgs pp{};
            pp.n = 1; pp.t[0].m = L.ple_proj.p; pp.t[0].out = proj_;
            pp.x = ple_g_; pp.normw = nullptr; pp.eps = cfg_.rms_epsilon; pp.add = 0;
            check(launch_gemv(pp, stream_), "per-layer projection");
            check(launch_post_add(h_, proj_, L.ple_post_norm, cfg_.rms_epsilon, e, stream_, L.out_scale), "per-layer norm");
        } else if (L.out_scale != 1.0f) {
            check(launch_scale(h_, L.out_scale, e, stream_), "layer scale");
        }
        if (debug_) debug_layer(l);
    }
    if (full) {
        HeadArgs ha{};
        ha.m = out_->p; ha.x = h_; ha.normw = out_norm_; ha.eps = cfg_.rms_epsilon; ha.logits = logits_;
        ha.key = key_; ha.softcap = gemma() ? cfg_.final_softcap : 0.0f;
        check(launch_head(ha, stream_), "output");
    } else {
        check(launch_advance(pos_, stream_), "advance");
    }
}

// Rows per tile for a phase of the loop: about one tile per workgroup, within
// the per-thread register budget and the LDS term buffer of every matrix in it.
static int loop_rows(const std::vector<const Packed*>& ms, int grid, bool head = false) {
    size_t rows = 0;
    for (const Packed* m : ms) rows += m->rows;
    // the most rows a tile can take (registers, LDS terms), then the fewest
    // rounds of tiles over the grid, then rows spread evenly over those rounds
    // (not rounded to a power of two: 3072 gate rows are 256 tiles of 12)
    size_t cap = 64;
    for (const Packed* m : ms) {
        const size_t units = m->cols / block_elems(m->type);
        cap = std::min(cap, static_cast<size_t>(loop_units_per_thread(m->type, head)) * kThreads / units);
        cap = std::min(cap, static_cast<size_t>(kTermCap) / term_stride(static_cast<uint32_t>(units)));
    }
    cap = std::max<size_t>(cap, 1);
    const size_t g = static_cast<size_t>(grid);
    const size_t rounds = (rows + g * cap - 1) / (g * cap);
    // full tiles when they take no more rounds: every unit of a full tile is in the matrix, so
    // its terms are formed without per-unit branches
    if ((rows + cap - 1) / cap <= g * rounds && rows % cap == 0) return static_cast<int>(cap);
    return static_cast<int>(std::max<size_t>(1, (rows + g * rounds - 1) / (g * rounds)));
}

static int tiles_of(const Packed& m, int R) { return static_cast<int>((m.rows + R - 1) / R); }

void Session::setup_loop() {
    const char* path = std::getenv("BRISK_HIP_PATH");
    if (path != nullptr && std::string(path) == "graph") return;
    if (debug_) return;
    // the loop's exact attentions hold at most 4 outputs a thread (heads per kv head x head size <= 1024)
    if ((cfg_.heads / cfg_.kv_heads) * cfg_.head_dim > 4 * kThreads) return;
    if (embd_.p.type != out_->p.type) return;  // the loop reads the embedding in its output's format
    if (gemma() || lfm2() || qwen35()) return;  // post-norms, windows, softcap, convolutions, recurrences: graph-path phases only
    if (plain_attn_) return;                    // the plain attention is a graph-path phase
    if (wide_x_.qs != nullptr) return;          // feed-forward rows past kMaxCols: the graph path's one-token GEMM
    const Layer& L0 = layers_[0];
    const void* k = find_loop_kernel(L0.q.p.type, L0.v.p.type, L0.o.p.type, L0.gate.p.type, L0.down.p.type, out_->p.type);
    if (k == nullptr) return;
    for (const Layer& L : layers_) {  // every layer must share layer 0's formats
        if (L.q.p.type != L0.q.p.type || L.k.p.type != L0.q.p.type || L.v.p.type != L0.v.p.type || L.o.p.type != L0.o.p.type ||
            L.gate.p.type != L0.gate.p.type || L.up.p.type != L0.gate.p.type || L.down.p.type != L0.down.p.type ||
            L.q.p.flags != L0.q.p.flags || L.v.p.flags != L0.v.p.flags || L.o.p.flags != L0.o.p.flags ||
            L.gate.p.flags != L0.gate.p.flags || L.down.p.flags != L0.down.p.flags)
            return;
    }
    // Every workgroup of the loop waits on others, so all of them must be resident at once: one
    // workgroup a compute unit, within the occupancy (below).  BRISK_HIP_COOPERATIVE=1 makes the
    // launch cooperative, so the runtime refuses a grid it cannot place whole (a device shared with
    // other work); by default a plain launch, whose bounded waits report such a case as an error.
    int cus = 0, per_cu = 0;
    if (const char* e = std::getenv("BRISK_HIP_COOPERATIVE")) {
        int coop = 0;
        check(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, device_), "hipDeviceGetAttribute");
        loop_cooperative_ = std::string(e) != "0";
        if (loop_cooperative_ && coop == 0) return;  // no cooperative launches: the one-kernel-per-phase path
    }
    check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device_), "hipDeviceGetAttribute");
    check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kThreads, 0), "hipOccupancy");
    if (cus <= 0 || per_cu < 1 || cus < static_cast<int>(cfg_.kv_heads)) return;
    {
        // the loop only where its attention keeps the reference's order at every length of the
        // context: the spread attention takes all of it, or the pooled exact attention does.  Other
        // sessions take the one-kernel-per-phase path, whose attention is order-exact at any length.
        const int heads = static_cast<int>(cfg_.heads), kvh = static_cast<int>(cfg_.kv_heads), hd = static_cast<int>(cfg_.head_dim);
        const int ctx = static_cast<int>(max_ctx_);
        bool spread_ok = loop_spread_fits(heads, kvh, hd, rope_dim_, cus) && loop_spread_covers(heads, kvh, hd, cus, ctx);
        if (const char* e = std::getenv("BRISK_HIP_SPREAD")) spread_ok = spread_ok && std::string(e) != "0";
        const bool pool_ok = loop_pool_covers(heads / kvh, ctx);
        if (!spread_ok && !pool_ok) return;
    }
    loop_grid_ = cus;  // one resident workgroup per CU: the barrier needs every workgroup resident
    loop_kernel_ = k;

    // the pushed feed-forward block (phase D writes the down terms of its activation block, phase F
    // adds them): down rows in a Q8_0-activation format, no ffn_sub norm, rows of at most 4096
    const uint32_t td = L0.down.p.type;
    const bool push_fmt = (td == kQ4_0 || td == kQ4_1 || td == kQ5_0 || td == kQ8_0) && !takes_q8_k(L0.gate.p.type) &&
                          L0.ffn_sub_norm == nullptr && cfg_.ff % 32 == 0 && cfg_.embd <= 4096 && cfg_.arch != BRISK_HIP_ARCH_BITNET;
    const char* push_env = std::getenv("BRISK_HIP_PUSH_FFN");
    const bool push = push_fmt && (push_env == nullptr || std::string(push_env) != "0");
    std::vector<Packed> down_t(cfg_.layers);
    if (push) {
        for (uint32_t l = 0; l < cfg_.layers; ++l) {
            const Packed& d = layers_[l].down.p;
            size_t planes[3];
            plane_bytes(d.type, d.rows, d.cols, planes);
            uint8_t* base = static_cast<uint8_t*>(alloc(packed_bytes(d.type, d.rows, d.cols)));
            down_t[l] = Packed{base, base + align256(planes[0]), base + align256(planes[0]) + align256(planes[1]), d.rows, d.cols, d.type,
                               d.flags};
            check(launch_unit_transpose(d, down_t[l], stream_), "transpose(down)");
        }
        check(hipStreamSynchronize(stream_), "transpose(down)");
    }

    std::vector<LayerDev> ld(cfg_.layers);
    for (uint32_t l = 0; l < cfg_.layers; ++l) {
        const Layer& L = layers_[l];
        ld[l] = LayerDev{L.q.p, L.k.p, L.v.p, L.o.p, L.gate.p, L.up.p, L.down.p, L.attn_norm, L.q_norm, L.k_norm,
                         L.attn_sub_norm, L.ffn_norm, L.ffn_sub_norm, L.q_bias, L.k_bias, L.v_bias, L.rope ? 1 : 0,
                         kcache_[l], vcache_[l], down_t[l]};
    }
    layers_dev_ = static_cast<LayerDev*>(alloc(ld.size() * sizeof(LayerDev)));
    check(hipMemcpy(layers_dev_, ld.data(), ld.size() * sizeof(LayerDev), hipMemcpyHostToDevice), "hipMemcpy(layers)");
    loop_done_ = static_cast<unsigned*>(alloc(64));
    loop_error_ = static_cast<int*>(alloc(64));
    {
        const size_t qd = static_cast<size_t>(cfg_.heads) * cfg_.head_dim, kvd = static_cast<size_t>(cfg_.kv_heads) * cfg_.head_dim;
        const size_t parts = static_cast<size_t>(cfg_.heads) * max_splits_;
        const size_t dterms = push ? static_cast<size_t>(cfg_.ff / 32) * cfg_.embd : 0;
        tagged_words_ = cfg_.embd + qd + 2 * kvd + qd + cfg_.ff + parts * cfg_.head_dim + parts * 2 +
                        static_cast<size_t>(cfg_.heads) * max_ctx_ + dterms;
        unsigned long long* w = static_cast<unsigned long long*>(alloc(tagged_words_ * 8));
        tagged_ = w;
        check(hipMemset(w, 0, tagged_words_ * 8), "memset(tagged)");
        loop_.ht = w; w += cfg_.embd;
        loop_.qt = w; w += qd;
        loop_.kt = w; w += kvd;
        loop_.vt = w; w += kvd;
        loop_.attt = w; w += qd;
        loop_.actt = w; w += cfg_.ff;
        loop_.pacct = w; w += parts * cfg_.head_dim;
        loop_.pmlt = w; w += parts * 2;
        loop_.sct = w; w += static_cast<size_t>(cfg_.heads) * max_ctx_;
        loop_.dtt = dterms ? w : nullptr;
    }
    if (std::getenv("BRISK_HIP_TRACE") != nullptr) trace_ = static_cast<unsigned long long*>(alloc(kTraceSlots * 8));
    check(hipMemset(loop_error_, 0, 64), "memset");

    LoopArgs& g = loop_;
    g.layers = layers_dev_;
    g.n_layers = static_cast<int>(cfg_.layers);
    g.embd = embd_.p;
    g.out = out_->p;
    g.out_norm = out_norm_;
    g.embd_dim = static_cast<int>(cfg_.embd);
    g.heads = static_cast<int>(cfg_.heads);
    g.kv_heads = static_cast<int>(cfg_.kv_heads);
    g.head_dim = static_cast<int>(cfg_.head_dim);
    g.ff = static_cast<int>(cfg_.ff);
    g.neox = neox();
    g.relu2 = cfg_.arch == BRISK_HIP_ARCH_BITNET;
    g.eps = cfg_.rms_epsilon;
    g.scale = 1.0f / std::sqrt(static_cast<float>(cfg_.head_dim));
    g.rope = rope_;
    g.rope_dim = rope_dim_;
    g.ctx = static_cast<int>(max_ctx_);
    g.logits = logits_;
    g.max_splits = max_splits_;
    g.done = loop_done_;
    g.keys = key_ + 2;
    g.pos_out = pos_;
    g.seq = seq_;
    g.seq_len = static_cast<int>(max_ctx_) + 1;
    g.error = loop_error_;
    const int G = loop_grid_;
    if (L0.q.p.type == L0.v.p.type) {
        const int R = loop_rows({&L0.q.p, &L0.k.p, &L0.v.p}, G);
        for (int i = 0; i < 3; ++i) g.R_qkv[i] = R;
    } else {
        const int R = loop_rows({&L0.q.p, &L0.k.p}, G);
        g.R_qkv[0] = g.R_qkv[1] = R;
        g.R_qkv[2] = loop_rows({&L0.v.p}, G);
    }
    g.tiles_qkv[0] = tiles_of(L0.q.p, g.R_qkv[0]);
    g.tiles_qkv[1] = tiles_of(L0.k.p, g.R_qkv[1]);
    g.tiles_qkv[2] = tiles_of(L0.v.p, g.R_qkv[2]);
    // with the spread attention, its stage-2 workgroups take no O or down tiles
    g.spread = loop_spread_fits(static_cast<int>(cfg_.heads), static_cast<int>(cfg_.kv_heads), static_cast<int>(cfg_.head_dim), rope_dim_, G) ? 1 : 0;
    if (const char* e = std::getenv("BRISK_HIP_SPREAD")) g.spread = g.spread && std::string(e) != "0";
    g.sp_slices = static_cast<int>(cfg_.head_dim) / 32;
    g.sp_hpk = static_cast<int>(cfg_.heads / cfg_.kv_heads);
    g.sp_n2 = static_cast<int>(cfg_.kv_heads) * g.sp_slices;
    g.sp_per_kv = (G - g.sp_n2) / static_cast<int>(cfg_.kv_heads);
    g.sp_all = g.spread && loop_spread_covers(static_cast<int>(cfg_.heads), static_cast<int>(cfg_.kv_heads), static_cast<int>(cfg_.head_dim),
                                              G, static_cast<int>(max_ctx_)) ? 1 : 0;
    // (only when every position of the context takes it: longer contexts run the split attention)
    g.c_first = g.spread && loop_spread_covers(static_cast<int>(cfg_.heads), static_cast<int>(cfg_.kv_heads), static_cast<int>(cfg_.head_dim),
                                               G, static_cast<int>(max_ctx_))
                    ? static_cast<int>(cfg_.kv_heads * (cfg_.head_dim / 32)) : 0;
    if (const char* e = std::getenv("BRISK_HIP_C_FIRST")) g.c_first = g.spread && std::string(e) != "0" ? g.c_first : 0;
    // with the pushed feed-forward block, its tasks get workgroups of their own (the stage-2
    // workgroups, then the last ones), so they request their weights while phase C runs
    const int tasks = push ? static_cast<int>(cfg_.ff / 32) : 0;
    g.n_c = G - g.c_first;
    if (push && tasks > g.c_first) g.n_c = std::max(G - tasks, std::min(G - g.c_first, 64));
    const int Gc = g.n_c;
    g.R_o = loop_rows({&L0.o.p}, Gc);
    g.tiles_o = tiles_of(L0.o.p, g.R_o);
    g.att_q8 = !takes_q8_k(L0.o.p.type) && L0.attn_sub_norm == nullptr &&
               ((cfg_.heads / cfg_.kv_heads) * cfg_.head_dim) % 32 == 0 ? 1 : 0;
    if (const char* e = std::getenv("BRISK_HIP_ATT_Q8")) g.att_q8 = g.att_q8 && std::string(e) != "0";
    g.R_gu = loop_rows({&L0.gate.p}, G);
    g.tiles_gu = tiles_of(L0.gate.p, g.R_gu);
    g.R_d = push ? g.R_o : loop_rows({&L0.down.p}, Gc);  // the pushed phase F takes phase C's rows
    {
        const int R = std::min(g.R_o, g.R_d);
        const int tiles = tiles_of(L0.o.p, R);
        g.own_h = ((tiles + Gc - 1) / Gc) * R <= kOwnRows ? 1 : 0;
        if (g.own_h) g.R_o = g.R_d = R;
    }
    g.tiles_o = tiles_of(L0.o.p, g.R_o);
    g.att_q8 = !takes_q8_k(L0.o.p.type) && L0.attn_sub_norm == nullptr &&
               ((cfg_.heads / cfg_.kv_heads) * cfg_.head_dim) % 32 == 0 ? 1 : 0;
    if (const char* e = std::getenv("BRISK_HIP_ATT_Q8")) g.att_q8 = g.att_q8 && std::string(e) != "0";
    g.tiles_d = tiles_of(L0.down.p, g.R_d);
    // the pushed phase F sums every owned row's ff / 32 terms in LDS: they must fit the term buffer
    const bool push_fits = static_cast<size_t>((g.tiles_o + Gc - 1) / Gc) * g.R_o * term_stride(cfg_.ff / 32) <= kTermCap;
    g.push_ffn = push && g.own_h && push_fits ? 1 : 0;
    if (!g.push_ffn && push) {  // not pushed after all: phase F tiles the down rows on their own
        g.R_d = loop_rows({&L0.down.p}, Gc);
        g.tiles_d = tiles_of(L0.down.p, g.R_d);
        g.own_h = 0;
    }
    {
        // the pushed phase D's tasks on the workgroups past those with O tiles, if there are enough
        // (the stage-2 attention workgroups, which finish phase B last, then take none); else from
        // the end of the grid round to the stage-2 workgroups
        const int c_wgs = std::min(g.tiles_o, g.n_c);
        g.d_first = G - g.c_first - c_wgs >= tasks ? g.c_first + c_wgs : (g.c_first + g.n_c) % G;
    }
    {
        // the resident attention: its workgroups (the spread attention's stage-2 tasks, the first
        // sp_n2) take no tiles of phases A, C, D and F, so their LDS holds the next layer's keys and
        // values between attentions; phase A's tiles are planned over the other workgroups
        const int hpk = static_cast<int>(cfg_.heads / cfg_.kv_heads);
        const int n2 = static_cast<int>(cfg_.heads) * std::max(1, static_cast<int>(cfg_.head_dim) / 64);
        bool ok = g.spread && n2 <= g.c_first && (cfg_.head_dim == 64 || cfg_.head_dim == 128) && hpk <= 4 &&
                  L0.q.p.type == L0.v.p.type && L0.q.p.type == L0.k.p.type && g.push_ffn && g.d_first >= n2 &&
                  g.d_first + tasks <= G && G - n2 >= 64;
        if (const char* e = std::getenv("BRISK_HIP_RESIDENT")) ok = ok && std::string(e) != "0";
        g.res_ok = ok ? 1 : 0;
        g.res_n = ok ? n2 : 0;
        g.a_touch = 0;
        if (ok) {
            // an h-row owner finishes phase F last; its phase-A tile's weight loads, issued then,
            // would hold its input poll back (loads complete in order), so it touches that tile
            // into L2 at the start of phase F, where it waits for the pushed terms anyway
            g.a_touch = g.own_h && g.push_ffn ? 1 : 0;
            if (const char* e = std::getenv("BRISK_HIP_A_TOUCH")) g.a_touch = g.a_touch && std::string(e) != "0";
            const int R = loop_rows({&L0.q.p, &L0.k.p, &L0.v.p}, G - n2);
            for (int i = 0; i < 3; ++i) g.R_qkv[i] = R;
            g.tiles_qkv[0] = tiles_of(L0.q.p, R);
            g.tiles_qkv[1] = tiles_of(L0.k.p, R);
            g.tiles_qkv[2] = tiles_of(L0.v.p, R);
        }
    }
    g.head_attn = static_cast<int>(cfg_.heads) <= G ? 1 : 0;
    if (const char* e = std::getenv("BRISK_HIP_HEAD_ATTN")) g.head_attn = g.head_attn && std::string(e) != "0";
    g.R_h = loop_rows({&out_->p}, G, true);
    g.tiles_h = tiles_of(out_->p, g.R_h);
}

// One launch of the persistent loop: n_steps steps from position pos0; steps
// from first_full on compute the output projection and the pick.
void Session::run_loop(size_t pos0, size_t n_steps, size_t first_full, size_t fixed) {
    LoopArgs g = loop_;
    g.pos0 = static_cast<int>(pos0);
    g.n_steps = static_cast<int>(n_steps);
    g.first_full = static_cast<int>(first_full);
    g.fixed = static_cast<int>(fixed);
    g.trace = trace_;
    g.trace_step = g.trace_layer = -1;
    if (const char* e = std::getenv("BRISK_HIP_TRACE_AT")) std::sscanf(e, "%d,%d", &g.trace_step, &g.trace_layer);
    // tags: 255 launch slots of 2^24 step/layer/phase indices; the words are
    // cleared each time the slots wrap, so a stale word never carries a live tag
    if (launches_ % 255 == 0) check(hipMemsetAsync(tagged_, 0, tagged_words_ * 8, stream_), "memset(tagged)");
    g.tag_base = static_cast<unsigned>(launches_ % 255 + 1) << 24;
    ++launches_;
    if (n_steps * cfg_.layers * 8 + 8 >= (1u << 24)) throw Error(BRISK_HIP_EINVAL, "hip: too many steps for one loop launch");
    check(hipMemsetAsync(loop_done_, 0, 64, stream_), "memset(done)");
    check(hipMemsetAsync(key_ + 2, 0, 16, stream_), "memset(keys)");
    check(launch_loop(loop_kernel_, g, loop_grid_, stream_, loop_cooperative_), "loop");
}

// BRISK_HIP_TRACE: workgroup 0's wall clock (100 MHz) after each barrier of the last loop launch.
size_t Session::trace(unsigned long long* out, size_t n) {
    if (trace_ == nullptr) return 0;
    n = std::min(n, kTraceSlots);
    check(hipMemcpy(out, trace_, n * 8, hipMemcpyDeviceToHost), "hipMemcpy(trace)");
    return n;
}

void Session::check_loop_error() {
    if (loop_kernel_ == nullptr) return;
    int err = 0;
    check(hipMemcpy(&err, loop_error_, 4, hipMemcpyDeviceToHost), "hipMemcpy(error)");
    if (err != 0) {
        (void)hipMemset(loop_error_, 0, 4);
        throw Error(BRISK_HIP_EHIP, "hip: token loop barrier timed out (a workgroup was not resident)");
    }
}

PickState Session::pick_state() const {
    return PickState{key_, pos_, seq_, static_cast<int>(max_ctx_) + 1, pos_ + 1};
}

// Ends a call: the last step's pick, still pending, becomes seq[pos + 1].
void Session::finish() { check(launch_finalize(pick_state(), stream_), "finalize"); }

hipGraphExec_t Session::capture(bool full) {
    hipGraph_t graph = nullptr;
    check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    try {
        record_step(full);
    } catch (...) {
        (void)hipStreamEndCapture(stream_, &graph);
        if (graph) (void)hipGraphDestroy(graph);
        throw;
    }
    check(hipStreamEndCapture(stream_, &graph), "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    check(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    check(hipGraphDestroy(graph), "hipGraphDestroy");
    return exec;
}

void Session::step(bool full) {
    if (use_graphs_) check(hipGraphLaunch(full ? graph_full_ : graph_layers_, stream_), "hipGraphLaunch");
    else record_step(full);
}

// BRISK_HIP_DEBUG: the reference's BRISK_CPU_DEBUG line (src/model.cpp:1183-1192) after
// each layer, for a layer-by-layer comparison with the CPU (steps then run uncaptured).
void Session::debug_layer(uint32_t l) {
    std::vector<float> h(cfg_.embd);
    int pos = 0;
    check(hipStreamSynchronize(stream_), "debug sync");
    check(hipMemcpy(h.data(), h_, h.size() * 4, hipMemcpyDeviceToHost), "debug copy");
    check(hipMemcpy(&pos, pos_, 4, hipMemcpyDeviceToHost), "debug copy");
    double sum = 0.0;
    float peak = 0.0f;
    for (const float v : h) {
        sum += std::fabs(v);
        peak = std::max(peak, std::fabs(v));
    }
    std::fprintf(stderr, "layer %u pos %d: max|h| %.4f mean|h| %.6f  h[0..3] %.5f %.5f %.5f %.5f\n", l, pos, peak,
                 sum / cfg_.embd, h[0], h[1], h[2], h[3]);
}

void Session::validate(const int32_t* tokens, size_t n) const {
    if (n == 0) throw Error(BRISK_HIP_EINVAL, "model: no tokens to evaluate");
    for (size_t i = 0; i < n; ++i)
        if (tokens[i] < 0 || static_cast<uint32_t>(tokens[i]) >= cfg_.vocab) throw Error(BRISK_HIP_EINVAL, "model: token id out of range");
    if (n > max_ctx_ - position_) throw Error(BRISK_HIP_EINVAL, "model: context length exceeded");
}

// Writes tokens to seq[position_ ..], syncs the device position to the host's and
// marks seq[0, position_ + n) as caller tokens (pos_[1]).
// rows x vocab logits from the device into out (when given) through the pinned staging; waits for the stream.
void Session::fetch_logits(float* out, const float* dev, size_t rows) {
    const size_t bytes = rows * static_cast<size_t>(cfg_.vocab) * 4;
    void* hb = out != nullptr ? host_buf(bytes) : nullptr;
    if (out != nullptr) check(hipMemcpyAsync(hb, dev, bytes, hipMemcpyDeviceToHost, stream_), "hipMemcpy(logits)");
    check(hipStreamSynchronize(stream_), "eval sync");
    if (out != nullptr) std::memcpy(out, hb, bytes);
}

void Session::stage(const int32_t* tokens, size_t n) { stage(tokens, n, position_); }

void Session::stage(const int32_t* tokens, size_t n, size_t device_pos) {
    int32_t* pin = static_cast<int32_t*>(host_buf(std::max<size_t>((n + 2) * 4, static_cast<size_t>(cfg_.vocab) * 4)));
    std::memcpy(pin, tokens, n * 4);
    pin[n] = static_cast<int32_t>(device_pos);
    pin[n + 1] = static_cast<int32_t>(position_ + n);
    check(hipMemcpyAsync(seq_ + position_, pin, n * 4, hipMemcpyHostToDevice, stream_), "hipMemcpy(tokens)");
    check(hipMemcpyAsync(pos_, pin + n, 8, hipMemcpyHostToDevice, stream_), "hipMemcpy(pos)");
    check(hipStreamSynchronize(stream_), "stage sync");  // the staging buffer is reused by the next copy
}

// Prompts of two or more tokens whose attention stays on the exact path go
// through the batched prefill (BRISK_HIP_PREFILL=0 turns it off).
bool Session::use_prefill(size_t n) const {
    // the exact-order prefill attention keeps every score of a token's query heads in LDS
    const bool exact_fits = (position_ + n) * (cfg_.heads / cfg_.kv_heads) <= static_cast<size_t>(kExactScores);
    const bool mfma_fits = prefill_mfma_ && pre_attn_mfma_fits(static_cast<int>(cfg_.heads / cfg_.kv_heads), static_cast<int>(cfg_.head_dim));
    // Gemma 3 (sliding layers, post-norms, GELU, soft-capped logits) and LFM2 (short convolutions)
    // take the exact attention only
    // Qwen3.5: the projections batched, the recurrence over the tokens in one launch (state sizes 64
    // and 128), the plain attention batched (contexts of its LDS window)
    if (qwen35())
        return prefill_on_ && n >= 2 && pre_ssm_fits(static_cast<int>(cfg_.ssm_state)) && pre_plain_fits(static_cast<int>(position_ + n));
    // the plain attention batched (contexts of its LDS window); Gemma 4's per-layer shapes and
    // per-layer embeddings take their prompts token by token
    if (plain_attn_) return prefill_on_ && n >= 2 && pre_plain_fits(static_cast<int>(position_ + n));
    if (gemma() || lfm2()) return prefill_on_ && n >= 2 && exact_fits && cfg_.head_dim <= 128;
    return prefill_on_ && n >= 2 && (exact_fits || mfma_fits);
}

void Session::ensure_prefill() {
    if (pre_h_ != nullptr) return;
    const size_t T = kPrefillTokens, e = cfg_.embd, qd = static_cast<size_t>(cfg_.heads) * cfg_.head_dim,
                 kvd = static_cast<size_t>(cfg_.kv_heads) * cfg_.head_dim, ff = cfg_.ff;
    pre_h_ = static_cast<float*>(alloc(T * e * 4));
    pre_q_ = static_cast<float*>(alloc(T * qd * 4));
    pre_k_ = static_cast<float*>(alloc(T * kvd * 4));
    pre_v_ = static_cast<float*>(alloc(T * kvd * 4));
    pre_att_ = static_cast<float*>(alloc(T * std::max<size_t>(qd, cfg_.ssm_inner) * 4));
    pre_act_ = static_cast<float*>(alloc(T * ff * 4));
    if (gemma() || lfm2()) pre_proj_ = static_cast<float*>(alloc(T * e * 4));  // post-norm inputs; conv outputs
    if (lfm2()) pre_conv_ = static_cast<float*>(alloc(T * 3 * e * 4));           // LFM2's [b | c | x] rows
    if (cfg_.ple_dim != 0) {  // Gemma 4's per-layer embedding inputs [T][layers][ple_dim] and gate rows
        pre_ple_ = static_cast<float*>(alloc(T * cfg_.ple_dim * cfg_.layers * 4));
        pre_pleg_ = static_cast<float*>(alloc(T * cfg_.ple_dim * 4));
    }
    if (qwen35()) {
        const size_t inner = cfg_.ssm_inner, heads = cfg_.ssm_v_heads;
        pre_sqkv_ = static_cast<float*>(alloc(T * 3 * inner * 4));
        pre_sz_ = static_cast<float*>(alloc(T * inner * 4));
        pre_sab_ = static_cast<float*>(alloc(T * 2 * heads * 4));
        pre_qg_ = static_cast<float*>(alloc(T * 2 * qd * 4));
    }
    const size_t widest = std::max(std::max(std::max(e, qd), ff), static_cast<size_t>(cfg_.ssm_inner));
    pre_x_.stride = static_cast<int>((widest + 255) / 256 * 256);
    pre_x_.qs = static_cast<int8_t*>(alloc(T * pre_x_.stride));
    pre_x_.d = static_cast<float*>(alloc(T * (pre_x_.stride / 32) * 4));
    pre_x_.bs = static_cast<int32_t*>(alloc(T * (pre_x_.stride / 16) * 4));
    for (Layer& L : layers_)
        for (DeviceMatrix* m : {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down, &L.conv_in, &L.conv_out, &L.ssm_qkv, &L.ssm_gate,
                                &L.ssm_alpha, &L.ssm_beta, &L.ssm_out, &L.ple_gate, &L.ple_proj})
            if (m->mem != nullptr && mx_expanded(m->p.type) && m->xmem == nullptr) {
                check(hipMalloc(&m->xmem, mx_bytes(m->p.type, m->p.rows, m->p.cols)), "hipMalloc(expanded planes)");
                check(launch_mx_expand(m->p, m->xmem, &m->x, stream_), "expand planes");
            }
}

// T rows of x (rms_norm'd by w when given), quantised for `consumer`'s activation format.
void Session::prefill_quant(const float* x, int xstride, const float* w, int cols, int T, const DeviceMatrix& consumer) {
    check(launch_pre_quant(x, xstride, w, cfg_.rms_epsilon, cols, T, takes_q8_k(consumer.p.type), act_bits(consumer.p), pre_x_,
                           stream_),
          "prefill quantise");
}

// Every layer for the T tokens seq[pos0 .. pos0 + T), as eval_batch runs a batch
// (src/model.cpp:867-1162): the hidden rows end in pre_h_.
void Session::prefill_layers(size_t pos0, int T) {
    const int e = static_cast<int>(cfg_.embd), qd = static_cast<int>(cfg_.heads * cfg_.head_dim),
              kvd = static_cast<int>(cfg_.kv_heads * cfg_.head_dim), ff = static_cast<int>(cfg_.ff);
    check(launch_pre_embed(embd_.p, seq_, static_cast<int>(pos0), T, pre_h_, embd_scale_, stream_), "prefill embed");
    if (cfg_.ple_dim != 0) {  // Gemma 4's per-layer embedding inputs (src/model.cpp:905-925)
        prefill_quant(pre_h_, e, nullptr, e, T, ple_proj_);
        MmArgs pg{};
        pg.x = pre_x_; pg.ntok = T; pg.m = ple_proj_.p; set_mx(pg, ple_proj_); pg.out = pre_ple_;
        pg.ostride = static_cast<int>(cfg_.ple_dim * cfg_.layers);
        check(launch_mm(pg, kMmStore, stream_), "prefill per-layer projection of the embedding");
        check(launch_pre_ple_inputs(pre_ple_, ple_tok_.p, ple_norm_, seq_, static_cast<int>(pos0), T, static_cast<int>(cfg_.layers),
                                    static_cast<int>(cfg_.ple_dim), 1.0f / std::sqrt(static_cast<float>(cfg_.embd)),
                                    std::sqrt(static_cast<float>(cfg_.ple_dim)), cfg_.rms_epsilon, stream_),
              "prefill per-layer inputs");
    }
    for (uint32_t l = 0; l < cfg_.layers; ++l) {
        const Layer& L = layers_[l];
        MmArgs g{};
        g.x = pre_x_;
        g.ntok = T;
        if (L.ssm_a != nullptr) {  // Qwen3.5 Gated DeltaNet (src/model.cpp:754-865)
            const int heads = static_cast<int>(cfg_.ssm_v_heads), inner = static_cast<int>(cfg_.ssm_inner), qkv = 3 * inner;
            const DeviceMatrix* mats[4] = {&L.ssm_qkv, &L.ssm_gate, &L.ssm_alpha, &L.ssm_beta};
            float* outs[4] = {pre_sqkv_, pre_sz_, pre_sab_, pre_sab_ + heads};
            const int strides[4] = {qkv, inner, 2 * heads, 2 * heads};
            const DeviceMatrix* quantised_for = nullptr;
            for (int i = 0; i < 4; ++i) {  // attn_norm(h) quantised once per activation format
                const DeviceMatrix& m = *mats[i];
                if (quantised_for == nullptr || takes_q8_k(m.p.type) != takes_q8_k(quantised_for->p.type) ||
                    act_bits(m.p) != act_bits(quantised_for->p)) {
                    prefill_quant(pre_h_, e, L.attn_norm, e, T, m);
                    quantised_for = &m;
                }
                g.m = m.p; set_mx(g, m); g.out = outs[i]; g.ostride = strides[i];
                check(launch_mm(g, kMmStore, stream_), "prefill recurrence projections");
            }
            SsmArgs sa{};
            sa.qkv = pre_sqkv_; sa.z = pre_sz_; sa.ab = pre_sab_; sa.conv_w = L.ssm_conv_w; sa.a = L.ssm_a; sa.dt = L.ssm_dt;
            sa.norm = L.ssm_norm; sa.ring = L.ssm_ring; sa.state = L.ssm_state; sa.pos = pos_; sa.out = pre_att_;
            sa.heads = heads; sa.dim = static_cast<int>(cfg_.ssm_state); sa.taps = static_cast<int>(cfg_.ssm_conv); sa.qkv_dim = qkv;
            sa.eps = cfg_.rms_epsilon; sa.q_scale = 1.0f / std::sqrt(static_cast<float>(cfg_.ssm_state));  // src/model.cpp:813
            check(launch_pre_ssm(sa, static_cast<int>(pos0), T, 2 * heads, stream_), "prefill recurrence");
            prefill_quant(pre_att_, inner, nullptr, inner, T, L.ssm_out);
            g.m = L.ssm_out.p; set_mx(g, L.ssm_out); g.out = pre_h_; g.ostride = e;
            check(launch_mm(g, kMmAdd, stream_), "prefill ssm_out");
        } else if (qwen35()) {  // Qwen3.5's gated attention: each head's query rows, then its gate rows
            prefill_quant(pre_h_, e, L.attn_norm, e, T, L.q);
            g.m = L.q.p; set_mx(g, L.q); g.out = pre_qg_; g.ostride = 2 * qd;
            check(launch_mm(g, kMmStore, stream_), "prefill q");
            g.m = L.k.p; set_mx(g, L.k); g.out = pre_k_; g.ostride = kvd;
            check(launch_mm(g, kMmStore, stream_), "prefill k");
            g.m = L.v.p; set_mx(g, L.v); g.out = pre_v_; g.ostride = kvd;
            check(launch_mm(g, kMmStore, stream_), "prefill v");
            PrePlainArgs pp{};
            AttnArgs& aa = pp.a;
            aa.q = pre_qg_; aa.k = pre_k_; aa.v = pre_v_; aa.qnorm = L.q_norm; aa.knorm = L.k_norm;
            aa.rope = rope_; aa.rope_dim = std::min(rope_dim_, L.hd); aa.eps = cfg_.rms_epsilon; aa.neox = neox();
            aa.kcache = kcache_[l]; aa.vcache = vcache_[l]; aa.ctx = static_cast<int>(max_ctx_); aa.head_dim = L.hd;
            aa.heads = static_cast<int>(cfg_.heads); aa.kv_heads = L.kvh;
            aa.scale = 1.0f / std::sqrt(static_cast<float>(L.hd));  // src/model.cpp:978
            aa.qn = pre_q_; aa.out = pre_att_;
            aa.q_stride = 2 * L.hd; aa.gate = pre_qg_ + L.hd; aa.gate_stride = 2 * L.hd;
            pp.pos0 = static_cast<int>(pos0); pp.ntok = T; pp.q_tok = 2 * qd; pp.kv_tok = kvd;
            check(launch_pre_attention_plain(pp, stream_), "prefill attention");
            prefill_quant(pre_att_, qd, nullptr, qd, T, L.o);
            g.m = L.o.p; set_mx(g, L.o); g.out = pre_h_; g.ostride = e;
            check(launch_mm(g, kMmAdd, stream_), "prefill o");
        } else if (L.conv_w != nullptr) {  // LFM2 short convolution in place of attention (src/model.cpp:935-969)
            prefill_quant(pre_h_, e, L.attn_norm, e, T, L.conv_in);
            g.m = L.conv_in.p; set_mx(g, L.conv_in); g.out = pre_conv_; g.ostride = 3 * e;
            check(launch_mm(g, kMmStore, stream_), "prefill conv in_proj");
            check(launch_pre_conv(pre_conv_, L.conv_cache, L.conv_w, static_cast<int>(cfg_.conv_taps), static_cast<int>(pos0), e, T,
                                  pre_proj_, stream_), "prefill conv");
            prefill_quant(pre_proj_, e, nullptr, e, T, L.conv_out);
            g.m = L.conv_out.p; set_mx(g, L.conv_out); g.out = pre_h_; g.ostride = e;
            check(launch_mm(g, kMmAdd, stream_), "prefill conv out_proj");
        } else {
            // Q, K, V of attn_norm(h) (src/model.cpp:996-1015), at the layer's head size and key/value
            // heads (Gemma 4: a shared layer projects Q only; K may serve as V)
            const int qdl = static_cast<int>(cfg_.heads) * L.hd, kvdl = L.kvh * L.hd;
            bool o_quantised = false;  // the attention wrote O's activation blocks
            const bool own_kv = L.kv_src == static_cast<int>(l);
            prefill_quant(pre_h_, e, L.attn_norm, e, T, L.q);
            g.m = L.q.p; set_mx(g, L.q); g.out = pre_q_; g.ostride = qdl;
            if (own_kv) {  // Q and K in one launch where their formats allow
                MmArgs gk = g;
                gk.m = L.k.p; set_mx(gk, L.k); gk.out = pre_k_; gk.ostride = kvdl;
                check(launch_mm_two(g, gk, stream_), "prefill q, k");
                if (!L.v_is_k) {
                    g.m = L.v.p; set_mx(g, L.v); g.out = pre_v_; g.ostride = kvdl;
                    check(launch_mm(g, kMmStore, stream_), "prefill v");
                }
            } else {
                check(launch_mm(g, kMmStore, stream_), "prefill q");
            }
            // norms, RoPE, cache rows, attention (:1020-1093)
            if (plain_attn_) {  // heads past 128 (or BRISK_HIP_ATTN=plain): the plain attention batched
                PrePlainArgs pp{};
                AttnArgs& aa = pp.a;
                aa.q = pre_q_; aa.k = pre_k_; aa.v = L.v_is_k ? pre_k_ : pre_v_; aa.qnorm = L.q_norm; aa.knorm = L.k_norm;
                aa.rope = !L.rope ? nullptr : L.slides ? rope_local_ : rope_;
                aa.window = L.slides ? static_cast<int>(cfg_.sliding_window) : 0;
                aa.rope_dim = L.slides ? L.hd : std::min(rope_dim_, L.hd);
                aa.qbias = L.q_bias; aa.kbias = L.k_bias; aa.vbias = L.v_bias;
                aa.eps = cfg_.rms_epsilon; aa.neox = neox();
                aa.kcache = kcache_[l]; aa.vcache = vcache_[l]; aa.ctx = static_cast<int>(max_ctx_); aa.head_dim = L.hd;
                aa.heads = static_cast<int>(cfg_.heads); aa.kv_heads = L.kvh;
                aa.vnorm = cfg_.value_norm; aa.no_kv = own_kv ? 0 : 1;
                // src/model.cpp:978: the family's scale, else 1 / sqrt(the layer's head size)
                aa.scale = cfg_.attention_scale != 0.0f ? cfg_.attention_scale : 1.0f / std::sqrt(static_cast<float>(L.hd));
                // the queries normed in place (one wave owns each token's head, reading it whole first)
                aa.qn = pre_q_; aa.out = pre_att_;
                pp.pos0 = static_cast<int>(pos0); pp.ntok = T; pp.q_tok = qdl; pp.kv_tok = kvdl;
                check(launch_pre_attention_plain(pp, stream_), "prefill attention");
            } else {
            PreAttnArgs pa{};
            pa.a.qnorm = L.q_norm; pa.a.knorm = L.k_norm; pa.a.eps = cfg_.rms_epsilon;
            pa.a.rope = !L.rope ? nullptr : L.slides ? rope_local_ : rope_;  // Gemma 3's sliding layers: the local base
            pa.a.window = L.slides ? static_cast<int>(cfg_.sliding_window) : 0;
            pa.a.rope_dim = L.slides ? static_cast<int>(cfg_.head_dim) : rope_dim_;
            pa.a.qbias = L.q_bias; pa.a.kbias = L.k_bias; pa.a.vbias = L.v_bias;
            pa.a.neox = neox();
            pa.a.kcache = kcache_[l]; pa.a.vcache = vcache_[l];
            pa.a.ctx = static_cast<int>(max_ctx_); pa.a.head_dim = static_cast<int>(cfg_.head_dim);
            pa.a.heads = static_cast<int>(cfg_.heads); pa.a.kv_heads = static_cast<int>(cfg_.kv_heads);
            pa.a.scale = 1.0f / std::sqrt(static_cast<float>(cfg_.head_dim));  // src/model.cpp:978
            pa.q = pre_q_; pa.k = pre_k_; pa.v = pre_v_; pa.out = pre_att_;
            pa.qstride = qd; pa.kvstride = kvd; pa.pos0 = static_cast<int>(pos0);
            pa.mfma = prefill_mfma_ ? 1 : 0;
            pa.legacy = prefill_legacy_ ? 1 : 0;
            if (L.attn_sub_norm == nullptr && qdl == qd) {  // the attention may quantise O's input itself
                pa.qout = pre_x_; pa.q8k = takes_q8_k(L.o.p.type) ? 1 : 0; pa.qbits = act_bits(L.o.p);
            }
            check(launch_pre_attention(pa, T, stream_, &o_quantised), "prefill attention");
            }
            // h += O (sub-normed) att (:1095-1111)
            if (!o_quantised) prefill_quant(pre_att_, qdl, L.attn_sub_norm, qdl, T, L.o);
            g.m = L.o.p; set_mx(g, L.o); g.out = L.attn_post_norm ? pre_proj_ : pre_h_; g.ostride = e;
            check(launch_mm(g, L.attn_post_norm ? kMmStore : kMmAdd, stream_), "prefill o");
            if (L.attn_post_norm)  // h += rms_norm(O att, post_attention_norm) (:1113-1121)
                check(launch_pre_post_add(pre_h_, pre_proj_, L.attn_post_norm, cfg_.rms_epsilon, e, T, stream_), "prefill post norm");
        }
        // act = silu(gate) * up of ffn_norm(h) (:1111-1143)
        prefill_quant(pre_h_, e, L.ffn_norm, e, T, L.gate);
        g.m = L.gate.p; g.m2 = L.up.p; set_mx(g, L.gate); set_mx2(g, L.up); g.out = pre_act_; g.ostride = ff; g.relu2 = cfg_.arch == BRISK_HIP_ARCH_BITNET;
        g.gelu = gemma();
        check(launch_mm(g, kMmPair, stream_), "prefill gate/up");
        // h += down (sub-normed) act (:1144-1162); Gemma 4's rows are the layer's width at stride ff
        prefill_quant(pre_act_, ff, L.ffn_sub_norm, L.ff, T, L.down);
        g.m = L.down.p; set_mx(g, L.down); g.out = L.ffn_post_norm ? pre_proj_ : pre_h_; g.ostride = e;
        g.relu2 = 0; g.gelu = 0;
        check(launch_mm(g, L.ffn_post_norm ? kMmStore : kMmAdd, stream_), "prefill down");
        if (L.ffn_post_norm)  // h += rms_norm(down act, post_ffw_norm) (:1153-1160)
            check(launch_pre_post_add(pre_h_, pre_proj_, L.ffn_post_norm, cfg_.rms_epsilon, e, T, stream_), "prefill post norm");
        if (cfg_.ple_dim != 0) {  // h = (h + norm(proj(gelu(gate h) * input l))) * scale (src/model.cpp:1163-1177)
            const int pd = static_cast<int>(cfg_.ple_dim), pall = pd * static_cast<int>(cfg_.layers);
            prefill_quant(pre_h_, e, nullptr, e, T, L.ple_gate);
            g.m = L.ple_gate.p; set_mx(g, L.ple_gate); g.out = pre_pleg_; g.ostride = pd;
            check(launch_mm(g, kMmStore, stream_), "prefill per-layer gate");
            check(launch_pre_gelu_mul(pre_pleg_, pre_ple_ + static_cast<size_t>(l) * pd, pd, pall, T, stream_), "prefill per-layer gelu");
            prefill_quant(pre_pleg_, pd, nullptr, pd, T, L.ple_proj);
            g.m = L.ple_proj.p; set_mx(g, L.ple_proj); g.out = pre_proj_; g.ostride = e;
            check(launch_mm(g, kMmStore, stream_), "prefill per-layer projection");
            check(launch_pre_post_add(pre_h_, pre_proj_, L.ple_post_norm, cfg_.rms_epsilon, e, T, stream_, L.out_scale),
                  "prefill per-layer norm");
        } else if (L.out_scale != 1.0f) {
            check(launch_pre_scale(pre_h_, L.out_scale, e, T, stream_), "prefill layer scale");
        }
    }
}

void Session::eval(const int32_t* tokens, size_t n, float* logits) {
    validate(tokens, n);
    if (use_prefill(n)) {
        ensure_prefill();
        // the device position is the last token's: the head's pick then lands in seq[position_ + n]
        stage(tokens, n, position_ + n - 1);
        int T = 0;
        for (size_t c = 0; c < n; c += kPrefillTokens) {
            T = static_cast<int>(std::min(n - c, static_cast<size_t>(kPrefillTokens)));
            prefill_layers(position_ + c, T);
        }
        HeadArgs ha{};  // output_norm + output rows of the last token (src/model.cpp:1195-1205)
        ha.m = out_->p; ha.x = pre_h_ + static_cast<size_t>(T - 1) * cfg_.embd; ha.normw = out_norm_;
        ha.eps = cfg_.rms_epsilon; ha.logits = logits_; ha.key = key_; ha.softcap = gemma() ? cfg_.final_softcap : 0.0f;
        check(launch_head(ha, stream_), "output");
        finish();
        fetch_logits(logits, logits_, 1);
        position_ += n;
        evaluated();
        return;
    }
    stage(tokens, n);
    if (uses_loop()) {
        run_loop(position_, n, n - 1, position_ + n);
    } else {
        for (size_t i = 0; i + 1 < n; ++i) step(false);
        step(true);
        finish();
    }
    fetch_logits(logits, logits_, 1);
    check_loop_error();
    position_ += n;
    evaluated();
}

void Session::eval_all(const int32_t* tokens, size_t n, float* logits) {
    if (n == 0 || n > 64) throw Error(BRISK_HIP_EINVAL, "model: eval_all takes 1 to 64 tokens");
    validate(tokens, n);
    if (use_prefill(n)) {
        // every row through the batched layers, then output_norm and the output rows
        // for all of them as one GEMM (the logits of eval_batch with all rows,
        // src/model.cpp:712-714, :1195-1205); the last row's head also leaves the
        // pending greedy pick, as eval does
        ensure_prefill();
        if (all_logits_ == nullptr) all_logits_ = static_cast<float*>(alloc(static_cast<size_t>(64) * cfg_.vocab * 4));
        stage(tokens, n, position_ + n - 1);
        const int T = static_cast<int>(n);
        prefill_layers(position_, T);
        prefill_quant(pre_h_, static_cast<int>(cfg_.embd), out_norm_, static_cast<int>(cfg_.embd), T, *out_);
        MmArgs g{};
        g.m = out_->p; g.x = pre_x_; g.ntok = T; g.out = all_logits_; g.ostride = static_cast<int>(cfg_.vocab);
        check(launch_mm(g, kMmStore, stream_), "eval_all output");
        if (gemma() && cfg_.final_softcap != 0.0f)  // every row's logits soft-capped (src/model.cpp:1206-1208)
            check(launch_softcap(all_logits_, n * cfg_.vocab, cfg_.final_softcap, stream_), "eval_all softcap");
        HeadArgs ha{};
        ha.m = out_->p; ha.x = pre_h_ + static_cast<size_t>(T - 1) * cfg_.embd; ha.normw = out_norm_;
        ha.eps = cfg_.rms_epsilon; ha.logits = nullptr; ha.key = key_; ha.softcap = gemma() ? cfg_.final_softcap : 0.0f;
        check(launch_head(ha, stream_), "output");
        finish();
        fetch_logits(logits, all_logits_, n);
        position_ += n;
        evaluated();
        return;
    }
    stage(tokens, n);
    const size_t row = static_cast<size_t>(cfg_.vocab) * 4;
    char* hb = static_cast<char*>(host_buf(n * row));
    for (size_t i = 0; i < n; ++i) {
        if (uses_loop()) {
            run_loop(position_ + i, 1, 0, position_ + n);
        } else {
            step(true);
            if (i + 1 == n) finish();
        }
        check(hipMemcpyAsync(hb + i * row, logits_, row, hipMemcpyDeviceToHost, stream_), "hipMemcpy(logits)");
    }
    check(hipStreamSynchronize(stream_), "eval_all sync");
    std::memcpy(logits, hb, n * row);
    check_loop_error();
    position_ += n;
    evaluated();
}

int32_t Session::picked() {
    int32_t next = 0;
    check(hipMemcpy(&next, seq_ + position_, 4, hipMemcpyDeviceToHost), "hipMemcpy(next)");
    return next;
}

int32_t Session::eval_greedy(const int32_t* tokens, size_t n) {
    eval(tokens, n, nullptr);
    return picked();  // the argmax of the last step wrote seq[position_]
}

void Session::generate(const int32_t* prompt, size_t n_prompt, size_t n_gen, int32_t* out) {
    if (n_gen == 0) return;
    validate(prompt, n_prompt);
    if (n_gen - 1 > max_ctx_ - position_ - n_prompt) throw Error(BRISK_HIP_EINVAL, "model: context length exceeded");
    eval(prompt, n_prompt, nullptr);
    const size_t first = position_;  // seq[first] holds the first pick
    // each further step embeds the previous pick (seq[pos]) and writes the next one
    if (uses_loop()) {
        if (n_gen > 1) run_loop(position_, n_gen - 1, 0, position_ + 1);
    } else {
        for (size_t i = 1; i < n_gen; ++i) step(true);
        finish();
    }
    check(hipMemcpyAsync(out, seq_ + first, n_gen * 4, hipMemcpyDeviceToHost, stream_), "hipMemcpy(ids)");
    check(hipStreamSynchronize(stream_), "generate sync");
    check_loop_error();
    position_ += n_gen - 1;
    evaluated();
}

void Session::decode(size_t n, int32_t* out) {
    if (n == 0) return;
    if (position_ == 0) throw Error(BRISK_HIP_EINVAL, "model: decode needs an evaluated token first");
    if (n > max_ctx_ - position_) throw Error(BRISK_HIP_EINVAL, "model: context length exceeded");
    const size_t first = position_ + 1;
    // the device position follows the host's (a rollback may have moved it); seq[position_] is the pending pick
    const int p[2] = {static_cast<int>(position_), static_cast<int>(position_ + 1)};
    check(hipMemcpyAsync(pos_, p, 8, hipMemcpyHostToDevice, stream_), "hipMemcpy(pos)");
    check(hipStreamSynchronize(stream_), "decode stage sync");  // the copy above reads stack memory
    if (uses_loop()) {
        run_loop(position_, n, 0, position_ + 1);
    } else {
        for (size_t i = 0; i < n; ++i) step(true);
        finish();
    }
    if (out != nullptr) check(hipMemcpyAsync(out, seq_ + first, n * 4, hipMemcpyDeviceToHost, stream_), "hipMemcpy(ids)");
    check(hipStreamSynchronize(stream_), "decode sync");
    check_loop_error();
    position_ += n;
    evaluated();
}

// After a call that evaluated tokens up to position_ - 1: the recurrent layers' input state of that
// last token is still held (the half of its parity), so rollback can step back to it, as it can to
// the reference's snapshot taken before a batch's last token (src/model.cpp:798-812).
void Session::evaluated() {
    snap_ok_ = qwen35() && position_ > 0;
    snap_pos_ = position_ - 1;
}

void Session::rollback(size_t position) {
    if (position > position_) throw Error(BRISK_HIP_EINVAL, "model: cannot roll forward");  // src/model.cpp:736
    if (qwen35() && position != position_) {
        // The recurrent states absorb every token: they step back to the last evaluated token's
        // input state, or start over at 0 (src/model.cpp:737-750).  At position 0 the recurrence
        // reads a zero state and the conv zero inputs, whatever the buffers hold.
        if (!(snap_ok_ && position == snap_pos_)) position = 0;
        snap_ok_ = false;
    }
    position_ = position;  // the caches keep their storage; later entries are overwritten
}

void Session::set_position(size_t position) {
    if (position > max_ctx_) throw Error(BRISK_HIP_EINVAL, "model: context length exceeded");
    if (qwen35() && position != 0) throw Error(BRISK_HIP_EINVAL, "model: a recurrent model cannot start past position 0");
    position_ = position;
    snap_ok_ = false;
}

void Session::kv_cache(int layer, int value, void** ptr, size_t* bytes) {
    if (layer < 0 || static_cast<uint32_t>(layer) >= cfg_.layers) throw Error(BRISK_HIP_EINVAL, "model: layer out of range");
    if (kcache_[layer] == nullptr) throw Error(BRISK_HIP_EINVAL, "model: layer has no key/value cache");
    *ptr = value ? static_cast<void*>(vcache_[layer]) : static_cast<void*>(kcache_[layer]);
    *bytes = kv_bytes_[layer];
}

}  // namespace bh
