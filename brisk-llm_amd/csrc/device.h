// Device-side building blocks of the token loop: half conversion, activation
// quantisation into LDS, and the per-format integer block dots.
//
// Arithmetic contract (checked by the parity tests against the reference's
// scalar code): every integer block dot is exact, and the per-block float term
// is formed with the same operations in the same order as the reference's
// dot_* functions (src/quant.cpp:445-596, :789-802).  The whole library is
// compiled with -ffp-contract=off and IEEE-correct fp32 division/sqrt, so no
// product/sum pair is fused into an FMA the x86 reference does not have.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "layout.h"

namespace bh {

// Global-memory views of generic pointers: accesses through them are global
// (not flat) instructions, counted by the vector memory counter only.  A flat
// access also counts against lgkmcnt, so every wait for an LDS or scalar
// result would wait for it too (the weight loads issued ahead among them).
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gmem(const T* p) {
    return (const __attribute__((address_space(1))) T*)p;
}
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gmem(T* p) {
    return (__attribute__((address_space(1))) T*)p;
}
// Four floats at p (16-byte aligned, global memory).
__device__ __forceinline__ float4 gld4(const float* p) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    const v4f v = *gmem(reinterpret_cast<const v4f*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
// Element i of a T array at p (global memory).
template <class T>
__device__ __forceinline__ T gld(const void* p, size_t i) {
    return gmem(static_cast<const T*>(p))[i];
}

constexpr int kThreads = 256;        // every token-loop kernel runs 256-thread workgroups (4 waves of 64)
constexpr int kMaxCols = 8192;       // widest activation row a matvec takes (Llama-3.2-1B FFN)
constexpr int kTermCap = 8448;       // floats of LDS for the per-block terms of one tile

// ---------------------------------------------------------------- halves

// IEEE half -> float; exact (src/quant.cpp:61-85 is the same conversion).
__device__ __forceinline__ float h2f(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

// RN(q * h), h being the low (Hi = false) or high half of `w` as an f16, in one
// v_fma_mix_f32 (the half is widened inside the instruction): fma(q, h, -0) is
// the rounded product for every input, the sign of a zero product included,
// so it equals q * h2f(h) bit for bit (checked exhaustively over q by
// brisk_hip_div_selftest).  Saves the separate conversion.
template <bool Hi>
__device__ __forceinline__ float mul_h(float q, uint32_t w) {
    float r;
    if (Hi) asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(q), "v"(w), "v"(-0.0f));
    else asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(q), "v"(w), "v"(-0.0f));
    return r;
}

// float -> IEEE half, round to nearest even, with the reference's handling of
// overflow (infinity), underflow (signed zero) and NaN (quiet, payload
// dropped): src/quant.cpp:87-113, written out on the bits.  f2h below is the
// hardware conversion; brisk_hip_div_selftest checks the two agree on every
// float.
__device__ __forceinline__ uint16_t f2h_bits(float f) {
    const uint32_t bits = __float_as_uint(f);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const int32_t exponent = static_cast<int32_t>((bits >> 23) & 0xFF) - 127 + 15;
    uint32_t mantissa = bits & 0x7FFFFFu;
    if (((bits >> 23) & 0xFF) == 0xFF) return static_cast<uint16_t>(sign | 0x7C00u | (mantissa ? 0x200u : 0u));
    if (exponent >= 0x1F) return static_cast<uint16_t>(sign | 0x7C00u);
    if (exponent <= 0) {
        if (exponent < -10) return static_cast<uint16_t>(sign);
        mantissa |= 0x800000u;
        const uint32_t shift = static_cast<uint32_t>(14 - exponent);
        uint32_t half = mantissa >> shift;
        const uint32_t rem = mantissa & ((1u << shift) - 1), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half & 1))) ++half;
        return static_cast<uint16_t>(sign | half);
    }
    uint32_t half = (static_cast<uint32_t>(exponent) << 10) | (mantissa >> 13);
    const uint32_t rem = mantissa & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1))) ++half;
    return static_cast<uint16_t>(sign | half);
}

// The same conversion by v_cvt_f16_f32 (IEEE round to nearest even, half
// denormals kept), with NaN mapped to the reference's quiet NaN.
__device__ __forceinline__ uint16_t f2h(float f) {
    const uint16_t h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
    return f != f ? static_cast<uint16_t>(((__float_as_uint(f) >> 16) & 0x8000u) | 0x7E00u) : h;
}

// ---------------------------------------------------------------- exp

// expf as the reference's host libm computes it.  The reference calls std::exp
// on floats (softmax_f32, silu_mul_f32: src/kernels_f32.cpp:276-289), i.e.
// glibc's expf, whose x86-64 build picks its FMA variant at run time.  That
// routine (the table-driven design of ARM's optimized-routines, also in
// glibc's sysdeps/ieee754/flt-32/e_expf.c) works in double: k = round(x * 32 /
// ln 2), r = x * 32 / ln 2 - k (one fused multiply-add), 2^(k/32) from a
// 32-entry table of 2^(i/32) with the exponent bits of i folded out, times a
// degree-3 polynomial in r.  This restatement reproduces glibc's results on
// every one of the 2^32 float inputs (checked exhaustively on the host).
__constant__ const unsigned long long kExp2Table[32] = {  // bits(2^(i/32)) - (i << 52) / 32
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// The table in LDS: a kernel that calls ref_expf_s fills it first
// (exp_tab_fill, then a barrier before the first call), so the per-value
// lookup is an LDS read rather than a dependent global load.
__shared__ unsigned long long g_exp_tab[32];
__device__ __forceinline__ void exp_tab_fill() {
    if (threadIdx.x < 32) g_exp_tab[threadIdx.x] = kExp2Table[threadIdx.x];
}

template <bool kLds>
__device__ __forceinline__ float ref_expf_impl(float x) {
    const uint32_t ux = __float_as_uint(x);
    const uint32_t abstop = (ux >> 20) & 0x7FF;
    if (abstop >= 0x42Bu) {  // |x| >= 88 (top 12 bits of 88.0f), or inf / nan
        if (ux == 0xFF800000u) return 0.0f;
        if (abstop >= 0x7F8u) return x + x;
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7F800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = static_cast<double>(x);
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    const unsigned long long ki = static_cast<unsigned long long>(__double_as_longlong(kd));
    kd -= shift;
    const double r = __fma_rn(inv_ln2_n, xd, -kd);
    const unsigned long long t = (kLds ? g_exp_tab[ki % 32] : kExp2Table[ki % 32]) + (ki << 47);
    const double s = __longlong_as_double(static_cast<long long>(t));
    const double p = __fma_rn(c0, r, c1);
    const double r2 = r * r;
    double y = __fma_rn(c2, r, 1.0);
    y = __fma_rn(p, r2, y);
    y = y * s;
    return static_cast<float>(y);
}
__device__ inline float ref_expf(float x) { return ref_expf_impl<false>(x); }
__device__ __forceinline__ float ref_expf_s(float x) { return ref_expf_impl<true>(x); }

// ---------------------------------------------------------------- tanh

// tanhf and expm1f as the reference's host libm computes them (std::tanh on a
// float: gelu_mul_f32, src/kernels_f32.cpp:291-296, and the final softcap,
// src/model.cpp:1206-1209).  glibc 2.35 builds both from fdlibm's s_tanhf.c
// and s_expm1f.c (Sun Microsystems' freely distributable fdlibm 5.3; no FMA
// variant on x86-64): expm1 reduces x by k ln2 split in a hi and a lo part,
// takes a rational form in the reduced argument with five scaled
// coefficients, and puts k back into the exponent; tanh is 1 - 2 / (expm1(2|x|)
// + 2) for |x| >= 1 and -expm1(-2|x|) / (expm1(-2|x|) + 2) below.  This
// restatement gives glibc's result for every one of the 2^32 float inputs
// (checked exhaustively on the host).
//
// ref_expm1f and ref_tanhf restate fdlibm's s_expm1f.c and s_tanhf.c, whose
// notice follows:
//   Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//   Developed at SunPro, a Sun Microsystems, Inc. business.
//   Permission to use, copy, modify, and distribute this
//   software is freely granted, provided that this notice
//   is preserved.
//   (Conversion to float by Ian Lance Taylor, Cygnus Support, ian@cygnus.com.)
__device__ __forceinline__ float bits_to_f(uint32_t u) { return __uint_as_float(u); }

__device__ inline float ref_expm1f(float x) {
    const float one = 1.0f, huge = 1.0e+30f, tiny = 1.0e-30f, o_threshold = 8.8721679688e+01f;
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f, Q4 = 4.0082177293e-06f,
                Q5 = -2.0109921195e-07f;
    float y, hi, lo, c = 0.0f, t, e;
    int k;
    uint32_t hx = __float_as_uint(x);
    const uint32_t xsb = hx & 0x80000000u;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) {  // |x| >= 27 ln2
        if (hx >= 0x42b17218u) {
            if (hx > 0x7f800000u) return x + x;
            if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;
            if (x > o_threshold) return huge * huge;
        }
        if (xsb != 0) return tiny - one;
    }
    if (hx > 0x3eb17218u) {  // |x| > ln2 / 2
        if (hx < 0x3F851592u) {  // and < 3 ln2 / 2
            if (xsb == 0) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
            else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
        } else {
            k = static_cast<int>(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
            t = static_cast<float>(k);
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {  // |x| < 2^-25
        t = huge + x;
        return x - (t - (huge + x));
    } else {
        k = 0;
    }
    const float hfx = 0.5f * x, hxs = x * hfx;
    const float r1 = one + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    t = 3.0f - r1 * hfx;
    e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return one + 2.0f * (x - e);
    }
    if (k <= -2 || k > 56) {
        y = one - (e - x);
        return bits_to_f(__float_as_uint(y) + (static_cast<uint32_t>(k) << 23)) - one;
    }
    if (k < 23) {
        t = bits_to_f(0x3f800000u - (0x1000000u >> k));
        y = t - (e - x);
    } else {
        t = bits_to_f(static_cast<uint32_t>(0x7f - k) << 23);
        y = x - (e + t);
        y += one;
    }
    return bits_to_f(__float_as_uint(y) + (static_cast<uint32_t>(k) << 23));
}

__device__ inline float ref_tanhf(float x) {
    const float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
    const uint32_t jx = __float_as_uint(x), ix = jx & 0x7fffffffu;
    float z;
    if (ix >= 0x7f800000u) return (jx & 0x80000000u) == 0 ? one / x + one : one / x - one;
    if (ix < 0x41b00000u) {  // |x| < 22
        if (ix == 0) return x;
        if (ix < 0x24000000u) return x * (one + x);
        if (ix >= 0x3f800000u) {
            const float t = ref_expm1f(two * fabsf(x));
            z = one - two / (t + two);
        } else {
            const float t = ref_expm1f(-two * fabsf(x));
            z = -t / (t + two);
        }
    } else {
        z = one - tiny;
    }
    return (jx & 0x80000000u) == 0 ? z : -z;
}

// ---------------------------------------------------------------- log1p

// log1pf as the reference's host libm computes it (std::log1p on a float: the
// softplus of Qwen3.5's recurrence, src/model.cpp:827).  glibc 2.35 builds it
// from fdlibm's s_log1pf.c (no FMA variant on x86-64): 1 + x is split as
// 2^k (1 + f), with a correction term c for the rounding of 1 + x when k != 0;
// log(1 + f) = f - hfsq + s (hfsq + R(s^2)) with s = f / (2 + f), hfsq = f^2 / 2
// and R a degree-7 polynomial in s^2; k ln2 is added back in a hi and a lo part.
// This restatement gives glibc's result for every one of the 2^32 float inputs
// (checked exhaustively on the host).
__device__ inline float ref_log1pf(float x) {
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, two25 = 3.355443200e+07f;
    const float Lp1 = 6.6666668653e-01f, Lp2 = 4.0000000596e-01f, Lp3 = 2.8571429849e-01f, Lp4 = 2.2222198546e-01f,
                Lp5 = 1.8183572590e-01f, Lp6 = 1.5313838422e-01f, Lp7 = 1.4798198640e-01f;
    float f = 0.0f, c = 0.0f, u;
    const int32_t hx = static_cast<int32_t>(__float_as_uint(x)), ax = hx & 0x7fffffff;
    int32_t k = 1, hu = 0;
    if (hx < 0x3ed413d7) {  // x < 0.41422
        if (ax >= 0x3f800000) return x == -1.0f ? -two25 / 0.0f : (x - x) / (x - x);  // x <= -1
        if (ax < 0x31000000) return ax < 0x24800000 ? x : x - x * x * 0.5f;          // |x| < 2^-29
        if (hx > 0 || hx <= static_cast<int32_t>(0xbe95f61fu)) {  // -0.2929 < x < 0.41422
            k = 0;
            f = x;
            hu = 1;
        }
    } else if (hx >= 0x7f800000) {
        return x + x;
    }
    if (k != 0) {
        if (hx < 0x5a000000) {
            u = 1.0f + x;
            hu = static_cast<int32_t>(__float_as_uint(u));
            k = (hu >> 23) - 127;
            c = k > 0 ? 1.0f - (u - x) : x - (u - 1.0f);  // the rounding error of 1 + x
            c /= u;
        } else {
            u = x;
            hu = static_cast<int32_t>(__float_as_uint(u));
            k = (hu >> 23) - 127;
            c = 0.0f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = __uint_as_float(static_cast<uint32_t>(hu) | 0x3f800000u);
        } else {
            k += 1;
            u = __uint_as_float(static_cast<uint32_t>(hu) | 0x3f000000u);
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    const float hfsq = 0.5f * f * f;
    const float fk = static_cast<float>(k);
    if (hu == 0) {  // |f| < 2^-20
        if (f == 0.0f) return k == 0 ? 0.0f : fk * ln2_hi + (c + fk * ln2_lo);
        const float R = hfsq * (1.0f - 0.66666666666666666f * f);
        return k == 0 ? f - R : fk * ln2_hi - ((R - (fk * ln2_lo + c)) - f);
    }
    const float s = f / (2.0f + f), z = s * s;
    const float R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
    return k == 0 ? f - (hfsq - s * (hfsq + R)) : fk * ln2_hi - ((hfsq - (s * (hfsq + R) + (fk * ln2_lo + c))) - f);
}

// gelu_mul_f32's gate (src/kernels_f32.cpp:291-296): 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))),
// in its left-to-right order, times up.
__device__ __forceinline__ float gelu_mul(float x, float up) {
    return 0.5f * x * (1.0f + ref_tanhf(0.7978845608f * (x + 0.044715f * x * x * x))) * up;
}

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// ---------------------------------------------------------------- reductions

// Cross-lane exchange on DPP (a VALU operand modifier, no LDS round trip).
// Patterns: swap neighbours (xor 1), swap pairs (xor 2), mirror within 8 lanes,
// mirror within 16 lanes.  Applied in that order, each step pairs a lane with
// one holding the reduction of the other half of its group, so after k steps
// every lane of an aligned 2^k group holds the group's reduction (the same bits
// in every lane: each pairwise op is commutative).
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int Ctrl, class T>
__device__ __forceinline__ T dpp(T v) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), Ctrl, 0xF, 0xF, false));
    } else {
        static_assert(sizeof(T) == 8, "dpp: 4- or 8-byte values");
        const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
        const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_mov_dpp(static_cast<int>(u), Ctrl, 0xF, 0xF, false));
        const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_mov_dpp(static_cast<int>(u >> 32), Ctrl, 0xF, 0xF, false));
        return __builtin_bit_cast(T, (static_cast<unsigned long long>(hi) << 32) | lo);
    }
}

template <class T>
__device__ __forceinline__ T readlane(T v, int lane) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
    } else {
        const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
        const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(u), lane));
        const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), lane));
        return __builtin_bit_cast(T, (static_cast<unsigned long long>(hi) << 32) | lo);
    }
}

// Reduction over aligned groups of `Lanes` (2, 4, 8 or 16) lanes; every lane of a group gets the result.
template <int Lanes, class T, class Op>
__device__ __forceinline__ T group_reduce(T v, Op op) {
    static_assert(Lanes == 2 || Lanes == 4 || Lanes == 8 || Lanes == 16, "group_reduce: 2..16 lanes");
    v = op(v, dpp<kDppXor1>(v));
    if constexpr (Lanes >= 4) v = op(v, dpp<kDppXor2>(v));
    if constexpr (Lanes >= 8) v = op(v, dpp<kDppHalfMirror>(v));
    if constexpr (Lanes >= 16) v = op(v, dpp<kDppMirror>(v));
    return v;
}

// Reduction over the wave, uniform: the four 16-lane rows reduced, then
// combined as ((row0 op row1) op row2) op row3.
template <class T, class Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
    v = group_reduce<16>(v, op);
    return op(op(op(readlane(v, 0), readlane(v, 16)), readlane(v, 32)), readlane(v, 48));
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
    return wave_reduce(v, [](T a, T b) { return a + b; });
}
__device__ __forceinline__ float wave_max(float v) {
    return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
    return wave_reduce(v, [](unsigned long long a, unsigned long long b) { return a > b ? a : b; });
}

// The first index of the largest magnitude over a wave, with its signed value.
struct AbsMax {
    float amax;
    int idx;
    float sel;
};
__device__ __forceinline__ AbsMax absmax_op(const AbsMax& a, const AbsMax& b) {
    return (b.amax > a.amax || (b.amax == a.amax && b.idx < a.idx)) ? b : a;
}
template <int Ctrl>
__device__ __forceinline__ AbsMax dpp_absmax(const AbsMax& v) {
    return AbsMax{dpp<Ctrl>(v.amax), dpp<Ctrl>(v.idx), dpp<Ctrl>(v.sel)};
}
__device__ __forceinline__ AbsMax wave_absmax(AbsMax v) {
    v = absmax_op(v, dpp_absmax<kDppXor1>(v));
    v = absmax_op(v, dpp_absmax<kDppXor2>(v));
    v = absmax_op(v, dpp_absmax<kDppHalfMirror>(v));
    v = absmax_op(v, dpp_absmax<kDppMirror>(v));
    auto row = [&](int lane) { return AbsMax{readlane(v.amax, lane), readlane(v.idx, lane), readlane(v.sel, lane)}; };
    return absmax_op(absmax_op(absmax_op(row(0), row(16)), row(32)), row(48));
}

// The value of largest magnitude of a wave's 256-value block (lane l holding values 4 l .. 4 l + 3),
// the first one in index order on ties, as quantize_q8_k's `ax > amax` scan picks it (NaNs never
// picked), and that magnitude; 0 when every value is 0 or NaN.  The magnitude is a plain wave
// max; the value comes from the first lane holding it (a ballot) and, in that lane, its first
// such value.
__device__ __forceinline__ float block_first_absmax(const float v[4], float& amax) {
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = wave_max(am);
    amax = am > 0.0f ? am : 0.0f;
    if (!(am > 0.0f)) return 0.0f;
    float mine = 0.0f;
    bool has = false;
#pragma unroll
    for (int i = 3; i >= 0; --i)
        if (fabsf(v[i]) == am) {
            mine = v[i];
            has = true;
        }
    const unsigned long long hit = __builtin_amdgcn_ballot_w64(has);
    return readlane(mine, __builtin_ctzll(hit));
}

// Sum of float squares in double over a workgroup (the accumulator of rms_norm,
// src/model.cpp:89-90).  The double sum of float squares is exact unless the
// squares span more than ~29 binades, so the grouping rarely matters; every
// workgroup uses the same grouping, so all of them agree bit for bit.
__device__ __forceinline__ double block_sumsq(const float* x, int n, double* red /* LDS [4] */) {
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += kThreads) {
        const float v = x[i];
        s += static_cast<double>(v * v);
    }
    s = wave_sum(s);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = s;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

// ---------------------------------------------------------------- short exact divisions
//
// IEEE-correct division is a long dependent chain (scale, reciprocal, four
// FMAs, fix-up).  Two quotients the quantisation chain needs have shorter
// exact forms; brisk_hip_div_selftest compares both with IEEE division on
// every input they take.

// a / 127.0f, correctly rounded, for every finite a >= 0: a times RN(1/127),
// corrected once by the FMA residual.
__device__ __forceinline__ float div127(float a) {
    const float c = 0x1.020408p-7f;  // RN(1/127)
    const float q0 = a * c;
    return __builtin_fmaf(__builtin_fmaf(-q0, 127.0f, a), c, q0);
}

// 1.0f / d, correctly rounded: the hardware reciprocal corrected once by the
// FMA residual, exact for 2^-126 <= |d| < 2^126; other d take IEEE division.
__device__ __forceinline__ float rcp_rn(float d) {
    const float ad = fabsf(d);
    const bool slow = !(ad >= 0x1p-126f && ad < 0x1p126f);
    const float y0 = __builtin_amdgcn_rcpf(d);
    float y = __builtin_fmaf(__builtin_fmaf(-d, y0, 1.0f), y0, y0);
    // a wave-uniform branch, so the long division is not computed beside the short one
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(slow) != 0, 0)) {
        if (slow) y = 1.0f / d;
    }
    return y;
}

// max of two non-negative floats (|x| values): their bit patterns order the same way.
__device__ __forceinline__ float nnmax(float a, float b) {
    return __uint_as_float(max(__float_as_uint(a), __float_as_uint(b)));
}

// rms_norm's scale (src/model.cpp:91-92).  sum / n is a multiplication when n
// is a power of two (exact, so the same double).
__device__ __forceinline__ float rms_scale(double sum, int n, float eps) {
    const double m = (n & (n - 1)) == 0 ? sum * (1.0 / static_cast<double>(n)) : sum / static_cast<double>(n);
    const float mean = static_cast<float>(m);
    return rcp_rn(sqrtf(mean + eps));
}

// ---------------------------------------------------------------- memory policies

// How a phase reads and writes the small activation vectors it shares with
// other workgroups.  PlainIO: ordinary accesses, for the one-kernel-per-phase
// path (kernel boundaries make them visible).  CoherentIO: system-scope
// relaxed atomics, which go past the per-XCD L2 caches, so a persistent
// kernel can hand vectors between workgroups on different XCDs with a
// counter-based barrier and no cache writeback/invalidate.
struct PlainIO {
    static __device__ __forceinline__ float ld(const float* p) { return *p; }
    static __device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }  // generic: x may be in LDS
    static __device__ __forceinline__ void st(float* p, float v) { *p = v; }
};

struct CoherentIO {
    static __device__ __forceinline__ float ld(const float* p) {
        return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    static __device__ __forceinline__ float4 ld4(const float* p) { return make_float4(ld(p), ld(p + 1), ld(p + 2), ld(p + 3)); }
    static __device__ __forceinline__ void st(float* p, float v) {
        __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
};

// ---------------------------------------------------------------- activations in LDS

// One activation row, quantised, resident in LDS for the whole tile.
// Q8_0 family: xs = 32-value blocks, xd = half-rounded scale as float, xsum = sum of a block's values.
// Q8_K family: xs = 256-value blocks, xd = float scale, xsum = the 16 bsums of each block.
struct ActLds {
    int32_t xs[kMaxCols / 4];
    float xd[kMaxCols / 32];
    int32_t xsum[kMaxCols / 16];
};

// quantize_q8_0 (src/quant.cpp:115-142) of v = x (or rms_norm(x) * w when `w`
// is given) into LDS.  Each thread takes 4 consecutive values, so a 32-value
// block is 8 adjacent lanes.  Exact: IEEE division, round-half-even rint.
__device__ inline void act_q8_0(const float* x, const float* w, float scale, int cols, ActLds& a) {
    for (int base = threadIdx.x * 4; base < cols; base += kThreads * 4) {
        float v[4];
        const float4 xv = *reinterpret_cast<const float4*>(x + base);
        v[0] = xv.x; v[1] = xv.y; v[2] = xv.z; v[3] = xv.w;
        if (w != nullptr) {
            const float4 wv = *reinterpret_cast<const float4*>(w + base);
            v[0] = v[0] * scale * wv.x; v[1] = v[1] * scale * wv.y;
            v[2] = v[2] * scale * wv.z; v[3] = v[3] * scale * wv.w;
        }
        float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        amax = group_reduce<8>(amax, [](float a, float b) { return fmaxf(a, b); });
        const float d = div127(amax);
        const float inv = d != 0.0f ? rcp_rn(d) : 0.0f;
        int q[4], sum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q[i] = static_cast<int>(rintf(v[i] * inv));
            sum += q[i];
        }
        sum = group_reduce<8>(sum, [](int a, int b) { return a + b; });
        a.xs[base / 4] = (q[0] & 0xFF) | ((q[1] & 0xFF) << 8) | ((q[2] & 0xFF) << 16) | (q[3] << 24);
        if ((threadIdx.x & 7) == 0) {
            a.xd[base / 32] = h2f(f2h(d));
            a.xsum[base / 32] = sum;
        }
    }
}

// quantize_q8_k (src/quant.cpp:146-194) with `bits` 8 or 7, into LDS.  One
// wave per 256-value block (4 values a lane).  The scale comes from the first
// value of largest magnitude, signed, as the reference's scan picks it.
__device__ inline void act_q8_k(const float* x, const float* w, float scale, int cols, int bits, ActLds& a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int blk = wave; blk < cols / 256; blk += kThreads / 64) {
        const int base = blk * 256 + lane * 4;
        float v[4];
        const float4 xv = *reinterpret_cast<const float4*>(x + base);
        v[0] = xv.x; v[1] = xv.y; v[2] = xv.z; v[3] = xv.w;
        if (w != nullptr) {
            const float4 wv = *reinterpret_cast<const float4*>(w + base);
            v[0] = v[0] * scale * wv.x; v[1] = v[1] * scale * wv.y;
            v[2] = v[2] * scale * wv.z; v[3] = v[3] * scale * wv.w;
        }
        // the first value of the largest |v|
        float amax;
        const float sel = block_first_absmax(v, amax);
        int q[4];
        float d;
        if (amax == 0.0f) {
            d = 0.0f;
            q[0] = q[1] = q[2] = q[3] = 0;
        } else {
            const float extreme = bits == 7 ? 63.0f : 127.0f;
            const float inv = -extreme / sel;
            d = rcp_rn(inv);
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = static_cast<int>(fminf(127.0f, rintf(inv * v[i])));
        }
        int s = q[0] + q[1] + q[2] + q[3];
        s = group_reduce<4>(s, [](int a, int b) { return a + b; });
        a.xs[base / 4] = (q[0] & 0xFF) | ((q[1] & 0xFF) << 8) | ((q[2] & 0xFF) << 16) | (q[3] << 24);
        if ((lane & 3) == 0) a.xsum[blk * 16 + lane / 4] = static_cast<int16_t>(s);  // bsums are int16
        if (lane == 0) a.xd[blk] = d;
    }
}

// ---- the decode path's activation prologue, split in two so that its loads go
// out before the weight loads of the tile (a wave's loads complete in order) and
// its arithmetic overlaps the weight stream.  Element mapping: chunk c of a
// thread covers values c * 1024 + 4 * threadIdx.x .. + 3, so a Q8_0 block is 8
// adjacent lanes and a Q8_K block is one wave.

constexpr int kActRegChunks = 4;  // chunks held in registers (rows up to 4096 values); wider rows load late

struct ActRegs {
    float4 x[kActRegChunks];
    float4 w[kActRegChunks];
};

__device__ __forceinline__ float4 ld4(const float* p) { return gld4(p); }

// The norm weight's chunks alone (before the input is ready), then the input's.
__device__ __forceinline__ void act_issue_w(ActRegs& r, const float* w, int cols) {
#pragma unroll
    for (int c = 0; c < kActRegChunks; ++c) {
        const int base = (c * kThreads + static_cast<int>(threadIdx.x)) * 4;
        if (base < cols && w != nullptr) r.w[c] = ld4(w + base);
    }
}
template <class IO = PlainIO>
__device__ __forceinline__ void act_issue_x(ActRegs& r, const float* x, int cols) {
#pragma unroll
    for (int c = 0; c < kActRegChunks; ++c) {
        const int base = (c * kThreads + static_cast<int>(threadIdx.x)) * 4;
        if (base < cols) r.x[c] = IO::ld4(x + base);
    }
}

template <class IO = PlainIO>
__device__ __forceinline__ void act_issue(ActRegs& r, const float* x, const float* w, int cols) {
#pragma unroll
    for (int c = 0; c < kActRegChunks; ++c) {
        const int base = (c * kThreads + static_cast<int>(threadIdx.x)) * 4;
        if (base < cols) {
            r.x[c] = IO::ld4(x + base);
            if (w != nullptr) r.w[c] = ld4(w + base);
        }
    }
}

// quantize_q8_0 of one 4-value piece (src/quant.cpp:115-142): amax over the
// block's 8 lanes, d = amax / 127, q = rint(v / d), the half-rounded d and the
// block sum to LDS.
__device__ __forceinline__ void quant_piece_q8_0(const float v[4], int base, ActLds& a) {
    float amax = nnmax(nnmax(fabsf(v[0]), fabsf(v[1])), nnmax(fabsf(v[2]), fabsf(v[3])));
    amax = group_reduce<8>(amax, [](float a, float b) { return nnmax(a, b); });
    const float d = div127(amax);
    const float inv = d != 0.0f ? rcp_rn(d) : 0.0f;
    int q[4], sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        q[i] = static_cast<int>(rintf(v[i] * inv));
        sum += q[i];
    }
    sum = group_reduce<8>(sum, [](int a, int b) { return a + b; });
    a.xs[base / 4] = (q[0] & 0xFF) | ((q[1] & 0xFF) << 8) | ((q[2] & 0xFF) << 16) | (q[3] << 24);
    if ((threadIdx.x & 7) == 0) {
        a.xd[base / 32] = h2f(f2h(d));
        a.xsum[base / 32] = sum;
    }
}

// quant_piece_q8_0 of N pieces at once (their chains interleave).
template <int N>
__device__ __forceinline__ void quant_pieces_q8_0(const float (&v)[N][4], const int (&base)[N], int cols, ActLds& a) {
    float amax[N], d[N], inv[N];
    int q[N][4], sum[N];
#pragma unroll
    for (int k = 0; k < N; ++k) amax[k] = nnmax(nnmax(fabsf(v[k][0]), fabsf(v[k][1])), nnmax(fabsf(v[k][2]), fabsf(v[k][3])));
#pragma unroll
    for (int k = 0; k < N; ++k) amax[k] = nnmax(amax[k], dpp<kDppXor1>(amax[k]));
#pragma unroll
    for (int k = 0; k < N; ++k) amax[k] = nnmax(amax[k], dpp<kDppXor2>(amax[k]));
#pragma unroll
    for (int k = 0; k < N; ++k) amax[k] = nnmax(amax[k], dpp<kDppHalfMirror>(amax[k]));
#pragma unroll
    for (int k = 0; k < N; ++k) {
        d[k] = div127(amax[k]);
        inv[k] = d[k] != 0.0f ? rcp_rn(d[k]) : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < N; ++k) {
        sum[k] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q[k][i] = static_cast<int>(rintf(v[k][i] * inv[k]));
            sum[k] += q[k][i];
        }
    }
#pragma unroll
    for (int k = 0; k < N; ++k) sum[k] += dpp<kDppXor1>(sum[k]);
#pragma unroll
    for (int k = 0; k < N; ++k) sum[k] += dpp<kDppXor2>(sum[k]);
#pragma unroll
    for (int k = 0; k < N; ++k) sum[k] += dpp<kDppHalfMirror>(sum[k]);
#pragma unroll
    for (int k = 0; k < N; ++k) {
        if (base[k] < cols) {
            a.xs[base[k] / 4] = (q[k][0] & 0xFF) | ((q[k][1] & 0xFF) << 8) | ((q[k][2] & 0xFF) << 16) | (q[k][3] << 24);
            if ((threadIdx.x & 7) == 0) {
                a.xd[base[k] / 32] = h2f(f2h(d[k]));
                a.xsum[base[k] / 32] = sum[k];
            }
        }
    }
}

// quantize_q8_k (src/quant.cpp:146-194) of one 4-value piece: the wave is the
// 256-value block; the scale comes from the first value of largest magnitude.
__device__ __forceinline__ void quant_piece_q8_k(const float v[4], int base, int bits, ActLds& a) {
    const int lane = threadIdx.x & 63;
    float amax;
    const float sel = block_first_absmax(v, amax);
    int q[4];
    float d;
    if (amax == 0.0f) {
        d = 0.0f;
        q[0] = q[1] = q[2] = q[3] = 0;
    } else {
        const float extreme = bits == 7 ? 63.0f : 127.0f;
        const float inv = -extreme / sel;
        d = rcp_rn(inv);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = static_cast<int>(fminf(127.0f, rintf(inv * v[i])));
    }
    int s = q[0] + q[1] + q[2] + q[3];
    s = group_reduce<4>(s, [](int a, int b) { return a + b; });
    a.xs[base / 4] = (q[0] & 0xFF) | ((q[1] & 0xFF) << 8) | ((q[2] & 0xFF) << 16) | (q[3] << 24);
    if ((lane & 3) == 0) a.xsum[base / 16] = static_cast<int16_t>(s);
    if (lane == 0) a.xd[base / 256] = d;
}

// rms_norm (when w is given, src/model.cpp:87-97) and quantisation of the row
// whose first chunks act_issue loaded.  Ends with a barrier.
template <class IO = PlainIO>
__device__ inline void act_finish(const ActRegs& r, const float* x, const float* w, float eps, int cols, bool q8k, int bits,
                                  ActLds& a, double* red) {
    const int nch = (cols + 4 * kThreads - 1) / (4 * kThreads);
    float scale = 1.0f;
    if (w != nullptr) {
        double s = 0.0;
#pragma unroll
        for (int c = 0; c < kActRegChunks; ++c) {
            const int base = (c * kThreads + static_cast<int>(threadIdx.x)) * 4;
            if (c < nch && base < cols) {
                const float4 v = r.x[c];
                s += static_cast<double>(v.x * v.x); s += static_cast<double>(v.y * v.y);
                s += static_cast<double>(v.z * v.z); s += static_cast<double>(v.w * v.w);
            }
        }
        for (int c = kActRegChunks; c < nch; ++c) {
            const int base = (c * kThreads + static_cast<int>(threadIdx.x)) * 4;
            if (base < cols) {
                const float4 v = IO::ld4(x + base);
                s += static_cast<double>(v.x * v.x); s += static_cast<double>(v.y * v.y);
                s += static_cast<double>(v.z * v.z); s += static_cast<double>(v.w * v.w);
            }
        }
        s = wave_sum(s);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
        __syncthreads();
        scale = rms_scale(((red[0] + red[1]) + red[2]) + red[3], cols, eps);
    }
    if (!q8k && nch <= kActRegChunks) {  // Q8_0 from registers: all pieces together
        auto run = [&](auto n_tag) {
            constexpr int N = decltype(n_tag)::value;
            float v[N][4];
            int base[N];
#pragma unroll
            for (int k = 0; k < N; ++k) {
                base[k] = (k * kThreads + static_cast<int>(threadIdx.x)) * 4;
                const float4 xv = r.x[k];
                v[k][0] = xv.x; v[k][1] = xv.y; v[k][2] = xv.z; v[k][3] = xv.w;
                if (w != nullptr) {
                    const float4 wv = r.w[k];
                    v[k][0] = v[k][0] * scale * wv.x; v[k][1] = v[k][1] * scale * wv.y;
                    v[k][2] = v[k][2] * scale * wv.z; v[k][3] = v[k][3] * scale * wv.w;
                }
            }
            quant_pieces_q8_0<N>(v, base, cols, a);
        };
        switch (nch) {
            case 1: run(std::integral_constant<int, 1>{}); break;
            case 2: run(std::integral_constant<int, 2>{}); break;
            case 3: run(std::integral_constant<int, 3>{}); break;
            default: run(std::integral_constant<int, 4>{}); break;
        }
        __syncthreads();
        return;
    }
    auto piece = [&](float4 xv, float4 wv, int base) {
        float v[4] = {xv.x, xv.y, xv.z, xv.w};
        if (w != nullptr) {
            v[0] = v[0] * scale * wv.x; v[1] = v[1] * scale * wv.y;
            v[2] = v[2] * scale * wv.z; v[3] = v[3] * scale * wv.w;
        }
        if (q8k) quant_piece_q8_k(v, base, bits, a);
        else quant_piece_q8_0(v, base, a);
    };
#pragma unroll
    for (int c = 0; c < kActRegChunks; ++c) {
        const int base = (c * kThreads + static_cast<int>(threadIdx.x)) * 4;
        if (c < nch && base < cols) piece(r.x[c], r.w[c], base);
    }
    for (int c = kActRegChunks; c < nch; ++c) {
        const int base = (c * kThreads + static_cast<int>(threadIdx.x)) * 4;
        if (base < cols) piece(IO::ld4(x + base), w != nullptr ? ld4(w + base) : make_float4(0, 0, 0, 0), base);
    }
    __syncthreads();
}

// Same LDS image from already-quantised GGUF activation blocks (the KernelSet
// matvec contract: x is BlockQ8_0 / BlockQ8_K rows, src/kernels.h:19-21).
__device__ inline void act_from_q8_0(const uint8_t* xq, int cols, ActLds& a) {
    for (int b = threadIdx.x; b < cols / 32; b += kThreads) {
        const uint8_t* blk = xq + b * 34;
        a.xd[b] = h2f(static_cast<uint16_t>(blk[0] | (blk[1] << 8)));
        int s = 0;
        for (int j = 0; j < 8; ++j) {
            const int v = blk[2 + 4 * j] | (blk[3 + 4 * j] << 8) | (blk[4 + 4 * j] << 16) | (blk[5 + 4 * j] << 24);
            a.xs[b * 8 + j] = v;
            s = dot4(v, 0x01010101, s);
        }
        a.xsum[b] = s;
    }
}

__device__ inline void act_from_q8_k(const uint8_t* xq, int cols, ActLds& a) {
    for (int b = threadIdx.x; b < cols / 256; b += kThreads) {
        const uint8_t* blk = xq + b * 292;
        a.xd[b] = *reinterpret_cast<const float*>(blk);
        for (int j = 0; j < 64; ++j) a.xs[b * 64 + j] = *reinterpret_cast<const int32_t*>(blk + 4 + 4 * j);
        for (int j = 0; j < 16; ++j) a.xsum[b * 16 + j] = *reinterpret_cast<const int16_t*>(blk + 260 + 2 * j);
    }
}

// ---------------------------------------------------------------- block dots

// A weight unit is one GGUF block (Q4_0, Q8_0: 32 values; K-quants and TQ2_0:
// 256) of one row.  load() fetches its bytes into registers; term() forms the
// reference's per-block float term from them and the LDS activation.  Tiles
// issue every load of a thread before any term (and before the activation
// prologue), so the memory latency is paid once per tile, not once per block.

__device__ __forceinline__ uint4 ld16(const uint8_t* p) {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    const v4u v = *gmem(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

template <uint32_t T> struct Unit;

// dot_q4_0_q8_0 block term (src/quant.cpp:445-456): acc = sum((q - 8) x), exact;
// term = (float)acc * d_w * d_x.  Nibble bytes hold values 0..15, valid as
// signed int8, so sum(q x) runs on sdot4 and the -8 comes off via the block sum.
template <> struct Unit<kQ4_0> {
    static constexpr uint32_t kElems = 32;
    static constexpr int kMaxPerThread = 16;
    uint4 q;
    uint32_t d;
    __device__ __forceinline__ void load(const Packed& m, size_t blk) {
        q = ld16(m.p0 + blk * 16);
        d = gld<uint16_t>(m.p1, blk);
    }
    __device__ __forceinline__ float term(uint32_t b, const ActLds& a) const {
        const int32_t* x = a.xs + b * 8;
        int acc = 0;
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc = dot4(static_cast<int>(qw[j] & 0x0F0F0F0Fu), x[j], acc);
            acc = dot4(static_cast<int>((qw[j] >> 4) & 0x0F0F0F0Fu), x[4 + j], acc);
        }
        acc -= 8 * a.xsum[b];
        return static_cast<float>(acc) * h2f(static_cast<uint16_t>(d)) * a.xd[b];
    }
};

// dot_q4_1_q8_0 block term (src/quant.cpp:445-456 with the offset, :207-217):
// acc = sum(q x) over the unsigned nibbles, exact; term = (float)acc * d_w * d_x
// + m * (d_x * (float)sum(x)), the block sum coming with the activation.
template <> struct Unit<kQ4_1> {
    static constexpr uint32_t kElems = 32;
    static constexpr int kMaxPerThread = 16;
    uint4 q;
    uint32_t d, m;
    __device__ __forceinline__ void load(const Packed& mat, size_t blk) {
        q = ld16(mat.p0 + blk * 16);
        d = gld<uint16_t>(mat.p1, blk);
        m = gld<uint16_t>(mat.p2, blk);
    }
    __device__ __forceinline__ float term(uint32_t b, const ActLds& a) const {
        const int32_t* x = a.xs + b * 8;
        int acc = 0;
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc = dot4(static_cast<int>(qw[j] & 0x0F0F0F0Fu), x[j], acc);
            acc = dot4(static_cast<int>((qw[j] >> 4) & 0x0F0F0F0Fu), x[4 + j], acc);
        }
        const float dx = a.xd[b];
        return static_cast<float>(acc) * h2f(static_cast<uint16_t>(d)) * dx +
               h2f(static_cast<uint16_t>(m)) * (dx * static_cast<float>(a.xsum[b]));
    }
};

// Four bits of `v` (from bit `sh`) to bit 4 of four bytes: the product places
// bit k at bit 8k (the shifted copies 7k apart never overlap, so no carries).
__device__ __forceinline__ uint32_t spread4_hi(uint32_t v, int sh) {
    return (((v >> sh) & 0xFu) * 0x00204081u & 0x01010101u) << 4;
}

// dot_q5_0_q8_0 block term (src/quant.cpp:458-472): value e = (nibble | bit e of
// qh << 4) - 16; acc = sum(value x) = sum(q x) - 16 sum(x), exact; term =
// (float)acc * d_w * d_x.
template <> struct Unit<kQ5_0> {
    static constexpr uint32_t kElems = 32;
    static constexpr int kMaxPerThread = 16;
    uint4 q;
    uint32_t d, qh;
    __device__ __forceinline__ void load(const Packed& m, size_t blk) {
        q = ld16(m.p0 + blk * 16);
        d = gld<uint16_t>(m.p1, blk);
        qh = gld<uint32_t>(m.p2, blk);
    }
    __device__ __forceinline__ float term(uint32_t b, const ActLds& a) const {
        const int32_t* x = a.xs + b * 8;
        int acc = 0;
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc = dot4(static_cast<int>((qw[j] & 0x0F0F0F0Fu) | spread4_hi(qh, 4 * j)), x[j], acc);
            acc = dot4(static_cast<int>(((qw[j] >> 4) & 0x0F0F0F0Fu) | spread4_hi(qh, 16 + 4 * j)), x[4 + j], acc);
        }
        acc -= 16 * a.xsum[b];
        return static_cast<float>(acc) * h2f(static_cast<uint16_t>(d)) * a.xd[b];
    }
};

// dot_q8_0_q8_0 block term (src/quant.cpp:474-482).
template <> struct Unit<kQ8_0> {
    static constexpr uint32_t kElems = 32;
    static constexpr int kMaxPerThread = 8;
    uint4 q0, q1;
    uint32_t d;
    __device__ __forceinline__ void load(const Packed& m, size_t blk) {
        q0 = ld16(m.p0 + blk * 32);
        q1 = ld16(m.p0 + blk * 32 + 16);
        d = gld<uint16_t>(m.p1, blk);
    }
    __device__ __forceinline__ float term(uint32_t b, const ActLds& a) const {
        const int32_t* x = a.xs + b * 8;
        int acc = 0;
        acc = dot4(q0.x, x[0], acc); acc = dot4(q0.y, x[1], acc); acc = dot4(q0.z, x[2], acc); acc = dot4(q0.w, x[3], acc);
        acc = dot4(q1.x, x[4], acc); acc = dot4(q1.y, x[5], acc); acc = dot4(q1.z, x[6], acc); acc = dot4(q1.w, x[7], acc);
        return static_cast<float>(acc) * h2f(static_cast<uint16_t>(d)) * a.xd[b];
    }
};

// q4_k_scale_min (src/quant.h:256-264)
template <class P>
__device__ __forceinline__ void q4k_scale_min(P s, int j, int& scale, int& min) {
    if (j < 4) {
        scale = s[j] & 63;
        min = s[j + 4] & 63;
    } else {
        scale = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        min = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// dot_q4_k_q8_k super-block term (src/quant.cpp:500-521): weighted and offsets
// are exact int32; term = x.d * (d * weighted - dmin * offsets).
template <> struct Unit<kQ4_K> {
    static constexpr uint32_t kElems = 256;
    static constexpr int kMaxPerThread = 4;
    uint4 q[8];
    uint4 meta;  // d, dmin, scales[12]
    __device__ __forceinline__ void load(const Packed& m, size_t blk) {
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = ld16(m.p0 + blk * 128 + 16 * i);
        meta = ld16(m.p1 + blk * 16);
    }
    __device__ __forceinline__ float term(uint32_t b, const ActLds& a) const {
        const uint32_t mw[4] = {meta.x, meta.y, meta.z, meta.w};
        const uint8_t* mb = reinterpret_cast<const uint8_t*>(mw);
        const int32_t* x = a.xs + b * 64;
        int weighted = 0, offsets = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {  // chunk c: 32 bytes, low nibbles = sub-block 2c, high = 2c+1
            const uint32_t qw[8] = {q[2 * c].x, q[2 * c].y, q[2 * c].z, q[2 * c].w,
                                    q[2 * c + 1].x, q[2 * c + 1].y, q[2 * c + 1].z, q[2 * c + 1].w};
            int lo = 0, hi = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                lo = dot4(static_cast<int>(qw[j] & 0x0F0F0F0Fu), x[c * 16 + j], lo);
                hi = dot4(static_cast<int>((qw[j] >> 4) & 0x0F0F0F0Fu), x[c * 16 + 8 + j], hi);
            }
            int s0, m0, s1, m1;
            q4k_scale_min(mb + 4, 2 * c, s0, m0);
            q4k_scale_min(mb + 4, 2 * c + 1, s1, m1);
            weighted += s0 * lo + s1 * hi;
            const int* bs = a.xsum + b * 16 + 4 * c;
            offsets += m0 * (bs[0] + bs[1]) + m1 * (bs[2] + bs[3]);
        }
        const uint16_t d = static_cast<uint16_t>(meta.x & 0xFFFF), dmin = static_cast<uint16_t>(meta.x >> 16);
        return a.xd[b] * (h2f(d) * static_cast<float>(weighted) - h2f(dmin) * static_cast<float>(offsets));
    }
};

// dot_q5_k_q8_k super-block term (src/quant.cpp:523-547): Q4_K's with a fifth
// bit, bit s of qh[i] for value i of sub-block s (values 0..31, still valid
// signed bytes for sdot4); term = x.d * (d * weighted - dmin * offsets).
template <> struct Unit<kQ5_K> {
    static constexpr uint32_t kElems = 256;
    static constexpr int kMaxPerThread = 4;
    uint4 q[8];
    uint4 meta;   // d, dmin, scales[12]
    uint4 qh[2];  // qh[32]
    __device__ __forceinline__ void load(const Packed& m, size_t blk) {
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = ld16(m.p0 + blk * 128 + 16 * i);
        meta = ld16(m.p1 + blk * 16);
        qh[0] = ld16(m.p2 + blk * 48 + 16);
        qh[1] = ld16(m.p2 + blk * 48 + 32);
    }
    __device__ __forceinline__ float term(uint32_t b, const ActLds& a) const {
        const uint32_t mw[4] = {meta.x, meta.y, meta.z, meta.w};
        const uint8_t* mb = reinterpret_cast<const uint8_t*>(mw);
        const uint32_t hw[8] = {qh[0].x, qh[0].y, qh[0].z, qh[0].w, qh[1].x, qh[1].y, qh[1].z, qh[1].w};
        const int32_t* x = a.xs + b * 64;
        int weighted = 0, offsets = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {  // chunk c: 32 bytes, low nibbles = sub-block 2c, high = 2c+1
            const uint32_t qw[8] = {q[2 * c].x, q[2 * c].y, q[2 * c].z, q[2 * c].w,
                                    q[2 * c + 1].x, q[2 * c + 1].y, q[2 * c + 1].z, q[2 * c + 1].w};
            int lo = 0, hi = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t vl = (qw[j] & 0x0F0F0F0Fu) | (((hw[j] >> (2 * c)) & 0x01010101u) << 4);
                const uint32_t vh = ((qw[j] >> 4) & 0x0F0F0F0Fu) | (((hw[j] >> (2 * c + 1)) & 0x01010101u) << 4);
                lo = dot4(static_cast<int>(vl), x[c * 16 + j], lo);
                hi = dot4(static_cast<int>(vh), x[c * 16 + 8 + j], hi);
            }
            int s0, m0, s1, m1;
            q4k_scale_min(mb + 4, 2 * c, s0, m0);
            q4k_scale_min(mb + 4, 2 * c + 1, s1, m1);
            weighted += s0 * lo + s1 * hi;
            const int* bs = a.xsum + b * 16 + 4 * c;
            offsets += m0 * (bs[0] + bs[1]) + m1 * (bs[2] + bs[3]);
        }
        const uint16_t d = static_cast<uint16_t>(meta.x & 0xFFFF), dmin = static_cast<uint16_t>(meta.x >> 16);
        return a.xd[b] * (h2f(d) * static_cast<float>(weighted) - h2f(dmin) * static_cast<float>(offsets));
    }
};

// dot_q6_k_q8_k super-block term (src/quant.cpp:549-563, unpack_q6_k :285-297):
// per 16-value group g, dot = sum((v - 32) x) = sum(v x) - 32 bsum[g] with v in
// 0..63; weighted = sum scale_g dot_g, exact; term = x.d * d * weighted.
template <> struct Unit<kQ6_K> {
    static constexpr uint32_t kElems = 256;
    static constexpr int kMaxPerThread = 2;
    uint4 ql[8], qh[4];
    uint32_t meta[5];  // int8 scales[16], u16 d, pad
    __device__ __forceinline__ void load(const Packed& m, size_t blk) {
#pragma unroll
        for (int i = 0; i < 8; ++i) ql[i] = ld16(m.p0 + blk * 128 + 16 * i);
#pragma unroll
        for (int i = 0; i < 4; ++i) qh[i] = ld16(m.p1 + blk * 64 + 16 * i);
        const auto mp = gmem(reinterpret_cast<const uint32_t*>(m.p2 + blk * 20));
#pragma unroll
        for (int i = 0; i < 5; ++i) meta[i] = mp[i];
    }
    __device__ __forceinline__ float term(uint32_t b, const ActLds& a) const {
        const uint32_t* L = reinterpret_cast<const uint32_t*>(ql);
        const uint32_t* H = reinterpret_cast<const uint32_t*>(qh);
        const int8_t* sc = reinterpret_cast<const int8_t*>(meta);
        const int32_t* x = a.xs + b * 64;
        const int* bs = a.xsum + b * 16;
        int weighted = 0;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            int g4[4][2] = {{0, 0}, {0, 0}, {0, 0}, {0, 0}};
#pragma unroll
            for (int j = 0; j < 8; ++j) {  // values l = 4j..4j+3 of this half
                const uint32_t l0 = L[half * 16 + j], l1 = L[half * 16 + 8 + j], h = H[half * 8 + j];
                const int v0 = static_cast<int>((l0 & 0x0F0F0F0Fu) | (((h >> 0) & 0x03030303u) << 4));
                const int v1 = static_cast<int>((l1 & 0x0F0F0F0Fu) | (((h >> 2) & 0x03030303u) << 4));
                const int v2 = static_cast<int>(((l0 >> 4) & 0x0F0F0F0Fu) | (((h >> 4) & 0x03030303u) << 4));
                const int v3 = static_cast<int>(((l1 >> 4) & 0x0F0F0F0Fu) | (((h >> 6) & 0x03030303u) << 4));
                const int sg = j >> 2;
                g4[0][sg] = dot4(v0, x[half * 32 + 0 + j], g4[0][sg]);
                g4[1][sg] = dot4(v1, x[half * 32 + 8 + j], g4[1][sg]);
                g4[2][sg] = dot4(v2, x[half * 32 + 16 + j], g4[2][sg]);
                g4[3][sg] = dot4(v3, x[half * 32 + 24 + j], g4[3][sg]);
            }
#pragma unroll
            for (int qi = 0; qi < 4; ++qi) {
#pragma unroll
                for (int sg = 0; sg < 2; ++sg) {
                    const int g = half * 8 + qi * 2 + sg;
                    weighted += static_cast<int>(sc[g]) * (g4[qi][sg] - 32 * bs[g]);
                }
            }
        }
        const uint16_t d = static_cast<uint16_t>(meta[4] & 0xFFFF);
        return a.xd[b] * h2f(d) * static_cast<float>(weighted);
    }
};

// Ternary super-block term.  Element e of a TQ2_0 block sits in byte
// 32 (e / 128) + e % 32 at bit pair 2 ((e % 128) / 32) (src/quant.h:123-130), so
// bit pair l of bytes 32j..32j+31 is 32 consecutive values.  acc = sum((c - 1) x)
// is exact.  With lut16 the float order is the x86 load-time layout's,
// acc * d_w * x.d (dot_tq2_0x16_q8_k, src/quant.cpp:789-802); else the generic
// x.d * d_w * acc (dot_tq2_0_q8_k, :580-596).
template <> struct Unit<kTQ2_0> {
    static constexpr uint32_t kElems = 256;
    static constexpr int kMaxPerThread = 4;
    uint4 q[4];
    uint32_t d;
    bool lut16;
    __device__ __forceinline__ void load(const Packed& m, size_t blk) {
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = ld16(m.p0 + blk * 64 + 16 * i);
        d = gld<uint16_t>(m.p1, blk);
        lut16 = (m.flags & kFlagLut16) != 0;
    }
    __device__ __forceinline__ float term(uint32_t b, const ActLds& a) const {
        const int32_t* x = a.xs + b * 64;
        int acc = 0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t qw[8] = {q[2 * j].x, q[2 * j].y, q[2 * j].z, q[2 * j].w,
                                    q[2 * j + 1].x, q[2 * j + 1].y, q[2 * j + 1].z, q[2 * j + 1].w};
#pragma unroll
            for (int l = 0; l < 4; ++l) {
#pragma unroll
                for (int k = 0; k < 8; ++k) acc = dot4(static_cast<int>((qw[k] >> (2 * l)) & 0x03030303u), x[j * 32 + l * 8 + k], acc);
            }
        }
        int xsum = 0;
#pragma unroll
        for (int g = 0; g < 16; ++g) xsum += a.xsum[b * 16 + g];
        acc -= xsum;
        const float dw = h2f(static_cast<uint16_t>(d));
        return lut16 ? static_cast<float>(acc) * dw * a.xd[b] : a.xd[b] * dw * static_cast<float>(acc);
    }
};

// Row sums of `nrows` LDS term rows (stride floats apart, `units` terms each),
// one lane a row, in block order: read 32 terms at a time before the adds, so
// LDS latency is paid once per 32 terms.  out[r] for r < nrows.
__device__ __forceinline__ void row_sums(const float* terms, uint32_t stride, uint32_t units, int nrows, float* out) {
    if (threadIdx.x < static_cast<uint32_t>(nrows)) {
        const float* t = terms + threadIdx.x * stride;
        float s = 0.0f;
        uint32_t b = 0;
        for (; b + 32 <= units; b += 32) {
            float4 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = *reinterpret_cast<const float4*>(t + b + 4 * j);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                s += v[j].x; s += v[j].y; s += v[j].z; s += v[j].w;
            }
        }
        for (; b < units; ++b) s += t[b];
        out[threadIdx.x] = s;
    }
}

// A tile: rows [row0, row0 + R) of one matrix, all blocks.  Unit i of the tile
// (row i / units, block i % units) belongs to thread i % 256, slot i / 256.
template <uint32_t T, int M = Unit<T>::kMaxPerThread>
struct Tile {
    static constexpr int kMax = M;
    Unit<T> u[kMax];
    uint32_t row0;
    int R;

    // Issues the loads of every unit this thread owns.  Units past the tile or
    // the matrix re-read its last unit (never used) rather than skip the load:
    // with up to 4 units a thread (the persistent loop's tiles) every thread
    // issues all of them on every path, so the count of loads in flight is the
    // same everywhere and a later wait for this tile can leave the next tile's
    // loads in flight (vmcnt(n) rather than vmcnt(0)).  Larger tiles do the
    // same when the tile fills every unit of every thread (one straight run of
    // loads); a partial one skips the rounds wholly past it (uniform branches).
    __device__ __forceinline__ void load(const Packed& m, uint32_t first_row, int rows_in_tile) {
        row0 = first_row;
        R = rows_in_tile;
        const uint32_t units = m.cols / Unit<T>::kElems;
        const uint32_t total = static_cast<uint32_t>(R) * units;
        auto one = [&](int k) {
            const uint32_t i0 = threadIdx.x + k * kThreads, i = i0 < total ? i0 : total - 1;
            const uint32_t r = i / units, b = i - r * units;
            const uint32_t row = row0 + r < m.rows ? row0 + r : m.rows - 1;
            u[k].load(m, static_cast<size_t>(row) * units + b);
        };
        if (kMax <= 4 || total >= static_cast<uint32_t>(kMax * kThreads)) {
#pragma unroll
            for (int k = 0; k < kMax; ++k) one(k);
        } else {
#pragma unroll
            for (int k = 0; k < kMax; ++k)
                if (static_cast<uint32_t>(k * kThreads) < total) one(k);
        }
    }

    // Terms to LDS (R rows of term_stride(units) floats from `terms`); no barrier.
    __device__ __forceinline__ void terms(const Packed& m, const ActLds& a, float* terms) const {
        const uint32_t units = m.cols / Unit<T>::kElems;
        const uint32_t stride = term_stride(units);
        const uint32_t total = static_cast<uint32_t>(R) * units;
        if (kThreads % units == 0) {
            // every unit of this thread is the same block b of a different row, so the
            // activation block is read from LDS once for all of them: all terms are
            // formed in registers (no LDS store between the reads), then stored
            const uint32_t b = threadIdx.x % units, r0 = threadIdx.x / units, step = kThreads / units;
            float tv[kMax];
#pragma unroll
            for (int k = 0; k < kMax; ++k) tv[k] = u[k].term(b, a);
            if (total == static_cast<uint32_t>(kMax * kThreads) && row0 + static_cast<uint32_t>(R) <= m.rows) {
                // every unit of the tile is in the matrix (a uniform test): stores without
                // per-unit branches, so the units' independent chains interleave
#pragma unroll
                for (int k = 0; k < kMax; ++k) terms[(r0 + k * step) * stride + b] = tv[k];
            } else {
#pragma unroll
                for (int k = 0; k < kMax; ++k) {
                    const uint32_t r = r0 + k * step;
                    if (r < static_cast<uint32_t>(R) && row0 + r < m.rows) terms[r * stride + b] = tv[k];
                }
            }
            return;
        }
#pragma unroll
        for (int k = 0; k < kMax; ++k) {
            const uint32_t i = threadIdx.x + k * kThreads;
            if (i < total) {
                const uint32_t r = i / units, b = i - r * units;
                if (row0 + r < m.rows) terms[r * stride + b] = u[k].term(b, a);
            }
        }
    }

    // Terms, then one lane per row adds them in block order, as the reference's
    // sequential `sum +=` does: sums[r] is bit-identical to the reference's dot.
    // Ends with a barrier.
    __device__ __forceinline__ void sums(const Packed& m, const ActLds& a, float* terms_buf, float* out) const {
        terms(m, a, terms_buf);
        __syncthreads();
        row_sums(terms_buf, term_stride(m.cols / Unit<T>::kElems), m.cols / Unit<T>::kElems, R, out);
        __syncthreads();
    }
};

}  // namespace bh
