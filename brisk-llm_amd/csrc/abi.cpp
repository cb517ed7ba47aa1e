// The extern "C" surface declared in include/brisk_hip.h.
#include <hip/hip_runtime.h>

#include <exception>
#include <mutex>
#include <new>
#include <string>

#include "prefill.h"
#include "session.h"

struct brisk_hip_session {
    bh::Session impl;
    template <typename... A>
    explicit brisk_hip_session(A&&... a) : impl(static_cast<A&&>(a)...) {}
};

// The no-alloc matmul's staging: the planar int8 activation rows (values,
// scales, sums) that brisk_hip_matmul otherwise hipMallocs per call.  One copy
// per GPU, held until the process ends; every no-alloc call on a GPU reuses it.
constexpr size_t kNoAllocScratch = size_t{4} << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratch];

namespace {

thread_local std::string g_error;

int set_error(int code, const std::string& what) {
    g_error = what;
    return code;
}

template <typename F>
int guarded(F&& f) {
    try {
        f();
        return BRISK_HIP_OK;
    } catch (const bh::Error& e) {
        return set_error(e.code, e.what());
    } catch (const std::bad_alloc&) {
        return set_error(BRISK_HIP_ENOMEM, "out of host memory");
    } catch (const std::exception& e) {
        return set_error(BRISK_HIP_EINVAL, e.what());
    }
}

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw bh::Error(BRISK_HIP_EHIP, std::string("hip: ") + what + ": " + hipGetErrorString(e));
}

bool known_type(int type) {
    return type == BRISK_HIP_Q4_0 || type == BRISK_HIP_Q4_1 || type == BRISK_HIP_Q5_0 || type == BRISK_HIP_Q8_0 ||
           type == BRISK_HIP_Q4_K || type == BRISK_HIP_Q5_K || type == BRISK_HIP_Q6_K || type == BRISK_HIP_TQ2_0;
}

bh::Packed packed_view(int type, int flags, const void* packed, size_t rows, size_t cols) {
    if (!known_type(type)) throw bh::Error(BRISK_HIP_EINVAL, "kernels: unsupported weight type " + std::to_string(type));
    if (cols == 0 || cols % bh::block_elems(static_cast<uint32_t>(type)) != 0)
        throw bh::Error(BRISK_HIP_EINVAL, "kernels: cols must be a non-zero multiple of the block size");
    if (cols > static_cast<size_t>(bh::kMaxCols) && cols % 256 != 0)
        throw bh::Error(BRISK_HIP_EINVAL, "kernels: rows wider than 8192 must be whole 256-value blocks");
    if (rows == 0 || rows > 0xFFFFFFFFu) throw bh::Error(BRISK_HIP_EINVAL, "kernels: bad row count");
    if (packed == nullptr) throw bh::Error(BRISK_HIP_EINVAL, "kernels: null weights");
    size_t planes[3];
    bh::plane_bytes(static_cast<uint32_t>(type), rows, cols, planes);
    const uint8_t* base = static_cast<const uint8_t*>(packed);
    bh::Packed p{base, base + bh::align256(planes[0]), base + bh::align256(planes[0]) + bh::align256(planes[1]),
                 static_cast<uint32_t>(rows), static_cast<uint32_t>(cols), static_cast<uint32_t>(type),
                 static_cast<uint32_t>(flags) & bh::kFlagLut16};
    if (type != BRISK_HIP_TQ2_0) p.flags = 0;
    return p;
}

// The device address of `scratch` on the current device.  The array's name is
// only a host-side handle: its address differs per GPU and comes from
// hipGetSymbolAddress, looked up once per device with that device current.
void* noalloc_scratch() {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* ptrs[kMaxDevices] = {};
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) throw bh::Error(BRISK_HIP_ENODEV, "kernels: device index out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (ptrs[dev] == nullptr) {
        void* ptr = nullptr;
        hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress");
        ptrs[dev] = ptr;
    }
    return ptrs[dev];
}

}  // namespace

extern "C" {

const char* brisk_hip_last_error(void) { return g_error.c_str(); }

int brisk_hip_abi_version(void) { return BRISK_HIP_ABI_VERSION; }

int brisk_hip_device_count(int* count) {
    return guarded([&] {
        int n = 0;
        const hipError_t e = hipGetDeviceCount(&n);
        *count = e == hipSuccess ? n : 0;
    });
}

size_t brisk_hip_packed_bytes(int type, size_t rows, size_t cols) {
    if (!known_type(type) || cols % bh::block_elems(static_cast<uint32_t>(type)) != 0) return 0;
    return bh::packed_bytes(static_cast<uint32_t>(type), rows, cols);
}

int brisk_hip_pack(int type, const void* gguf_blocks, size_t rows, size_t cols, void* packed, void* stream) {
    return guarded([&] {
        const bh::Packed p = packed_view(type, 0, packed, rows, cols);
        if (gguf_blocks == nullptr) throw bh::Error(BRISK_HIP_EINVAL, "kernels: null source");
        hip_check(bh::launch_pack(static_cast<uint32_t>(type), gguf_blocks, rows, cols, p, static_cast<hipStream_t>(stream)), "pack");
    });
}

int brisk_hip_quantize_q8_0(const float* x, void* out, size_t count, void* stream) {
    return guarded([&] {
        if (count % 32 != 0) throw bh::Error(BRISK_HIP_EINVAL, "kernels: count must be a multiple of 32");
        hip_check(bh::launch_quantize(0, x, out, count, 8, static_cast<hipStream_t>(stream)), "quantize_q8_0");
    });
}

int brisk_hip_quantize_q8_k(const float* x, void* out, size_t count, int bits, void* stream) {
    return guarded([&] {
        if (count % 256 != 0) throw bh::Error(BRISK_HIP_EINVAL, "kernels: count must be a multiple of 256");
        if (bits != 7 && bits != 8) throw bh::Error(BRISK_HIP_EINVAL, "kernels: bits must be 7 or 8");
        hip_check(bh::launch_quantize(1, x, out, count, bits, static_cast<hipStream_t>(stream)), "quantize_q8_k");
    });
}

int brisk_hip_matvec(int type, int flags, const void* packed, size_t rows, size_t cols, const void* xq, float* out, void* stream) {
    return brisk_hip_matmul(type, flags, packed, rows, cols, xq, 1, out, rows, stream);
}

int brisk_hip_matmul(int type, int flags, const void* packed, size_t rows, size_t cols, const void* xq, size_t n, float* out,
                     size_t out_stride, void* stream) {
    return guarded([&] {
        const bh::Packed p = packed_view(type, flags, packed, rows, cols);
        if (n == 0 || n > 65535) throw bh::Error(BRISK_HIP_EINVAL, "kernels: n must be 1..65535");
        if (out_stride < rows) throw bh::Error(BRISK_HIP_EINVAL, "kernels: out_stride < rows");
        const hipStream_t st = static_cast<hipStream_t>(stream);
        if (n == 1 && cols <= static_cast<size_t>(bh::kMaxCols)) {  // the GEMV holds the row in LDS
            hip_check(bh::launch_matvec_q8(p, xq, n, out, out_stride, st), "matmul");
            return;
        }
        // batches (and rows wider than the GEMV's buffer) take the int8 MFMA path of the prefill:
        // the GGUF activation rows are converted to its planar layout in a scratch allocation,
        // released when done
        const int stride = static_cast<int>((cols + 255) / 256 * 256);
        bh::ActPlanar x{};
        x.stride = stride;
        void* mem = nullptr;
        const size_t qb = n * static_cast<size_t>(stride), db = n * static_cast<size_t>(stride / 32) * 4,
                     bb = n * static_cast<size_t>(stride / 16) * 4;
        // a matrix the session's prefill holds expanded is expanded there too (launch_mx_expand)
        const size_t xb = bh::mx_expanded(p.type) ? bh::mx_bytes(p.type, p.rows, p.cols) : 0;
        const size_t ab = bh::align256(qb + db + bb);
        hip_check(hipMalloc(&mem, ab + xb), "hipMalloc");
        x.qs = static_cast<int8_t*>(mem);
        x.d = reinterpret_cast<float*>(static_cast<char*>(mem) + qb);
        x.bs = reinterpret_cast<int32_t*>(static_cast<char*>(mem) + qb + db);
        bh::MmArgs g{};
        hipError_t e = bh::launch_pre_planar(xq, static_cast<int>(cols), static_cast<int>(n), bh::takes_q8_k(p.type), x, st);
        if (e == hipSuccess && xb != 0) {
            bh::MxPlanes xp{};
            e = bh::launch_mx_expand(p, static_cast<char*>(mem) + ab, &xp, st);
            g.qx = xp.q; g.qxd = xp.d; g.qxm = xp.mn;
        }
        if (e == hipSuccess) {
            g.m = p; g.x = x; g.ntok = static_cast<int>(n); g.out = out; g.ostride = static_cast<int>(out_stride);
            e = bh::launch_mm(g, bh::kMmStore, st);
        }
        const hipError_t e2 = hipStreamSynchronize(st);
        (void)hipFree(mem);
        hip_check(e, "matmul");
        hip_check(e2, "matmul sync");
    });
}

int brisk_hip_matmul_noalloc(int type, int flags, const void* packed, size_t rows, size_t cols, const void* xq, size_t n,
                             float* out, size_t out_stride, void* stream) {
    return guarded([&] {
        const bh::Packed p = packed_view(type, flags, packed, rows, cols);
        if (n == 0 || n > 65535) throw bh::Error(BRISK_HIP_EINVAL, "kernels: n must be 1..65535");
        if (out_stride < rows) throw bh::Error(BRISK_HIP_EINVAL, "kernels: out_stride < rows");
        const hipStream_t st = static_cast<hipStream_t>(stream);
        if (n == 1 && cols <= static_cast<size_t>(bh::kMaxCols)) {  // the matvec takes no scratch
            hip_check(bh::launch_matvec_q8(p, xq, n, out, out_stride, st), "matmul");
            return;
        }
        const int stride = static_cast<int>((cols + 255) / 256 * 256);
        const size_t qb = n * static_cast<size_t>(stride), db = n * static_cast<size_t>(stride / 32) * 4,
                     bb = n * static_cast<size_t>(stride / 16) * 4;
        if (qb + db + bb > kNoAllocScratch)
            throw bh::Error(BRISK_HIP_EINVAL, "kernels: " + std::to_string(n) + " rows of " + std::to_string(cols) +
                                                  " columns need " + std::to_string(qb + db + bb) +
                                                  " bytes of scratch; the no-alloc matmul holds " +
                                                  std::to_string(kNoAllocScratch));
        char* mem = static_cast<char*>(noalloc_scratch());
        bh::ActPlanar x{};
        x.stride = stride;
        x.qs = reinterpret_cast<int8_t*>(mem);
        x.d = reinterpret_cast<float*>(mem + qb);
        x.bs = reinterpret_cast<int32_t*>(mem + qb + db);
        hip_check(bh::launch_pre_planar(xq, static_cast<int>(cols), static_cast<int>(n), bh::takes_q8_k(p.type), x, st),
                  "matmul");
        bh::MmArgs g{};
        g.m = p; g.x = x; g.ntok = static_cast<int>(n); g.out = out; g.ostride = static_cast<int>(out_stride);
        hip_check(bh::launch_mm(g, bh::kMmStore, st), "matmul");
    });
}

int brisk_hip_gemv(int type, int flags, const void* packed, size_t rows, size_t cols, const float* x, const float* norm_w, float eps,
                   float* out, int accumulate, void* stream) {
    return guarded([&] {
        if (cols > static_cast<size_t>(bh::kMaxCols))  // the fused norm reads the whole row from LDS
            throw bh::Error(BRISK_HIP_EINVAL, "kernels: gemv rows wider than 8192 are not supported (quantise, then matvec)");
        bh::GemvArgs g{};
        g.n = 1;
        g.t[0].m = packed_view(type, flags, packed, rows, cols);
        g.t[0].out = out;
        g.x = x;
        g.normw = norm_w;
        g.eps = eps;
        g.add = accumulate != 0;
        hip_check(bh::launch_gemv(g, static_cast<hipStream_t>(stream)), "gemv");
    });
}

int brisk_hip_expf(const float* x, float* y, size_t n, void* stream) {
    return guarded([&] { hip_check(bh::launch_expf(x, y, n, static_cast<hipStream_t>(stream)), "expf"); });
}

int brisk_hip_tanhf(const float* x, float* y, size_t n, void* stream) {
    return guarded([&] { hip_check(bh::launch_tanhf(x, y, n, static_cast<hipStream_t>(stream)), "tanhf"); });
}

int brisk_hip_log1pf(const float* x, float* y, size_t n, void* stream) {
    return guarded([&] { hip_check(bh::launch_log1pf(x, y, n, static_cast<hipStream_t>(stream)), "log1pf"); });
}

int brisk_hip_div_selftest(unsigned long long* mismatches) {
    return guarded([&] {
        unsigned long long* d = nullptr;
        hip_check(hipMalloc(&d, 32), "hipMalloc");
        hipError_t e = hipMemset(d, 0, 32);
        if (e == hipSuccess) e = bh::launch_div_selftest(d, nullptr);
        if (e == hipSuccess) e = hipMemcpy(mismatches, d, 32, hipMemcpyDeviceToHost);
        (void)hipFree(d);
        hip_check(e, "div selftest");
    });
}

int brisk_hip_mfma_rate(int shape, double* int8_tops) {
    return guarded([&] {
        if (int8_tops == nullptr || shape < 0 || shape > 1) throw bh::Error(BRISK_HIP_EINVAL, "mfma rate: bad argument");
        int dev = 0, cus = 0;
        hip_check(hipGetDevice(&dev), "hipGetDevice");
        hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
        int* d = nullptr;
        hip_check(hipMalloc(&d, 8), "hipMalloc");
        hipEvent_t e0 = nullptr, e1 = nullptr;
        const int blocks = 4 * cus, iters = 4096;
        hipError_t e = hipEventCreate(&e0);
        if (e == hipSuccess) e = hipEventCreate(&e1);
        if (e == hipSuccess) e = bh::launch_mfma_rate(shape, blocks, 64, d, nullptr);  // warm-up
        if (e == hipSuccess) e = hipEventRecord(e0, nullptr);
        if (e == hipSuccess) e = bh::launch_mfma_rate(shape, blocks, iters, d, nullptr);
        if (e == hipSuccess) e = hipEventRecord(e1, nullptr);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
        (void)hipFree(d);
        hip_check(e, "mfma rate");
        // multiply-adds (2 ops each) per wave and iteration: 8 x 16x16x64 or 4 x 32x32x32
        const double per_iter = shape == 0 ? 8.0 * 16 * 16 * 64 : 4.0 * 32 * 32 * 32;
        const double ops = static_cast<double>(blocks) * (bh::kThreads / 64) * iters * per_iter * 2;
        *int8_tops = ops / (ms * 1e-3) / 1e12;
    });
}

int brisk_hip_session_estimate(const brisk_hip_config* config, const brisk_hip_tensor* tensors, size_t n_tensors,
                               size_t max_context, brisk_hip_memory* out) {
    return guarded([&] {
        if (config == nullptr || out == nullptr || (tensors == nullptr && n_tensors != 0))
            throw bh::Error(BRISK_HIP_EINVAL, "session: null argument");
        *out = bh::estimate_session(*config, tensors, n_tensors, max_context);
    });
}

int brisk_hip_device_memory(int device, size_t* free_bytes, size_t* total_bytes) {
    return guarded([&] {
        if (free_bytes == nullptr || total_bytes == nullptr) throw bh::Error(BRISK_HIP_EINVAL, "device memory: null argument");
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count)
            throw bh::Error(BRISK_HIP_ENODEV, "hip: no GPU device " + std::to_string(device));
        hip_check(hipSetDevice(device), "hipSetDevice");
        hip_check(hipMemGetInfo(free_bytes, total_bytes), "hipMemGetInfo");
    });
}

int brisk_hip_session_create(const brisk_hip_config* config, const brisk_hip_tensor* tensors, size_t n_tensors, size_t max_context,
                             int device, brisk_hip_session** out) {
    return guarded([&] {
        if (config == nullptr || out == nullptr || (tensors == nullptr && n_tensors != 0))
            throw bh::Error(BRISK_HIP_EINVAL, "session: null argument");
        *out = nullptr;
        *out = new brisk_hip_session(*config, tensors, n_tensors, max_context, device);
    });
}

void brisk_hip_session_destroy(brisk_hip_session* s) { delete s; }

int brisk_hip_session_eval(brisk_hip_session* s, const int32_t* tokens, size_t n, float* logits) {
    return guarded([&] { s->impl.eval(tokens, n, logits); });
}

int brisk_hip_session_eval_all(brisk_hip_session* s, const int32_t* tokens, size_t n, float* logits) {
    return guarded([&] {
        if (logits == nullptr) throw bh::Error(BRISK_HIP_EINVAL, "session: null logits");
        s->impl.eval_all(tokens, n, logits);
    });
}

int brisk_hip_session_eval_greedy(brisk_hip_session* s, const int32_t* tokens, size_t n, int32_t* next) {
    return guarded([&] { *next = s->impl.eval_greedy(tokens, n); });
}

int brisk_hip_session_generate(brisk_hip_session* s, const int32_t* prompt, size_t n_prompt, size_t n_gen, int32_t* out) {
    return guarded([&] { s->impl.generate(prompt, n_prompt, n_gen, out); });
}

int brisk_hip_session_decode(brisk_hip_session* s, size_t n, int32_t* out) {
    return guarded([&] { s->impl.decode(n, out); });
}

int brisk_hip_session_rollback(brisk_hip_session* s, size_t position) {
    return guarded([&] { s->impl.rollback(position); });
}

size_t brisk_hip_session_position(const brisk_hip_session* s) { return s->impl.position(); }

size_t brisk_hip_session_max_context(const brisk_hip_session* s) { return s->impl.max_context(); }

int brisk_hip_session_kv_cache(brisk_hip_session* s, int layer, int value, void** device_ptr, size_t* bytes) {
    return guarded([&] { s->impl.kv_cache(layer, value, device_ptr, bytes); });
}

int brisk_hip_session_set_position(brisk_hip_session* s, size_t position) {
    return guarded([&] { s->impl.set_position(position); });
}

void* brisk_hip_session_stream(brisk_hip_session* s) { return static_cast<void*>(s->impl.stream()); }

size_t brisk_hip_session_trace(brisk_hip_session* s, unsigned long long* out, size_t n) {
    try {
        return s->impl.trace(out, n);
    } catch (const std::exception& e) {
        set_error(BRISK_HIP_EHIP, e.what());
        return 0;
    }
}

}  // extern "C"
