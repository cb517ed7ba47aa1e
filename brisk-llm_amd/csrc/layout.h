// HBM layout of repacked weight matrices (shared by host and device code).
//
// The GGUF blocks interleave a 2-byte scale with 16/32/128-byte value runs,
// which leaves the values off 16-byte alignment.  At load time each matrix is
// split into planes so every value run is a 16-byte aligned vector load and
// consecutive blocks of a row are consecutive in memory:
//
//   Q4_0   p0: nibbles  [rows][cols/32][16]    p1: d [rows][cols/32] (fp16)
//   Q4_1   p0: nibbles  [rows][cols/32][16]    p1: d, p2: m [rows][cols/32] (fp16 each)
//   Q5_0   p0: nibbles  [rows][cols/32][16]    p1: d [rows][cols/32] (fp16)  p2: qh [rows][cols/32] (u32)
//   Q8_0   p0: int8     [rows][cols/32][32]    p1: d [rows][cols/32] (fp16)
//   Q4_K   p0: nibbles  [rows][cols/256][128]  p1: {d, dmin, scales[12]} [rows][cols/256][16]
//          p2: the 8 sub-block scales then the 8 mins, decoded to bytes [rows][cols/256][16]
//   Q5_K   p0: nibbles  [rows][cols/256][128]  p1: {d, dmin, scales[12]} [rows][cols/256][16]
//          p2: decoded scales and mins (as Q4_K's) then qh[32] [rows][cols/256][48]
//   Q6_K   p0: ql       [rows][cols/256][128]  p1: qh [rows][cols/256][64]
//          p2: {int8 scales[16], d, pad} [rows][cols/256][20]
//   TQ2_0  p0: 2-bit    [rows][cols/256][64]   p1: d [rows][cols/256] (fp16)
//
// Bytes within each run are unchanged, so the byte total equals the GGUF size
// (plus 2 pad bytes per Q6_K block, the K-quants' decoded scale planes, and plane alignment).
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace bh {

// ggml tensor type numbers (src/gguf.h:22-27 of the reference)
enum : uint32_t { kF32 = 0, kQ4_0 = 2, kQ4_1 = 3, kQ5_0 = 6, kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kTQ2_0 = 35 };

// Packed::flags
enum : uint32_t {
    kFlagLut16 = 1,  // TQ2_0: x86 TQ2_0x16 arithmetic (7-bit activations, acc * d_w * d_x)
};

struct Packed {
    const uint8_t* p0;
    const uint8_t* p1;
    const uint8_t* p2;
    uint32_t rows, cols, type, flags;
};

__host__ __device__ constexpr inline uint32_t block_elems(uint32_t type) {
    return (type == kQ4_0 || type == kQ4_1 || type == kQ5_0 || type == kQ8_0) ? 32u : 256u;
}
__host__ __device__ inline bool takes_q8_k(uint32_t type) {
    return type == kQ4_K || type == kQ5_K || type == kQ6_K || type == kTQ2_0;
}
// Activation width the matrix takes: 7 bits for the x86 ternary layout (src/quant.cpp:144).
__host__ __device__ inline int act_bits(const Packed& m) { return (m.flags & kFlagLut16) ? 7 : 8; }

// Floats per row of a tile's LDS term buffer: a multiple of 4 (rows are read
// as float4), padded so that neighbouring rows start in different banks.
__host__ __device__ inline uint32_t term_stride(uint32_t units) { return ((units + 3) & ~3u) + 4; }

inline size_t align256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

// Plane sizes of a packed matrix.
inline void plane_bytes(uint32_t type, size_t rows, size_t cols, size_t out[3]) {
    const size_t blocks = rows * (cols / block_elems(type));
    out[0] = out[1] = out[2] = 0;
    switch (type) {
        case kQ4_0: out[0] = blocks * 16; out[1] = blocks * 2; break;
        case kQ4_1: out[0] = blocks * 16; out[1] = blocks * 2; out[2] = blocks * 2; break;
        case kQ5_0: out[0] = blocks * 16; out[1] = blocks * 2; out[2] = blocks * 4; break;
        case kQ8_0: out[0] = blocks * 32; out[1] = blocks * 2; break;
        case kQ4_K: out[0] = blocks * 128; out[1] = blocks * 16; out[2] = blocks * 16; break;
        case kQ5_K: out[0] = blocks * 128; out[1] = blocks * 16; out[2] = blocks * 48; break;
        case kQ6_K: out[0] = blocks * 128; out[1] = blocks * 64; out[2] = blocks * 20; break;
        case kTQ2_0: out[0] = blocks * 64; out[1] = blocks * 2; break;
        default: break;
    }
}

inline size_t packed_bytes(uint32_t type, size_t rows, size_t cols) {
    size_t p[3];
    plane_bytes(type, rows, cols, p);
    return align256(p[0]) + align256(p[1]) + align256(p[2]);
}

// GGUF bytes per block.
inline size_t gguf_block_bytes(uint32_t type) {
    switch (type) {
        case kQ4_0: return 18;
        case kQ4_1: return 20;
        case kQ5_0: return 22;
        case kQ8_0: return 34;
        case kQ4_K: return 144;
        case kQ5_K: return 176;
        case kQ6_K: return 210;
        case kTQ2_0: return 66;
        default: return 0;
    }
}

}  // namespace bh
