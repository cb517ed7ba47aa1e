/* TEST INFRASTRUCTURE ONLY — the CPU oracle (see oracle.h).
 *
 * Plain C restatement of roticv/brisk-llm's x86 CPU path.  Each function cites
 * the reference lines it follows.  Floating-point expressions keep the
 * reference's evaluation order and types (float products and sums, double
 * accumulators where it has them) so that, compiled like the reference
 * (gcc -O3, no -march: no FMA contraction on x86-64), results are bit-identical
 * to it.
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_err[256];
const char* or_last_error(void) { return g_err; }
static int fail(const char* msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    return -1;
}

/* ------------------------------------------------------------------ halves */

/* src/quant.cpp:61-85 */
float or_half_to_float(uint16_t half) {
    uint32_t h = half, sign = (h & 0x8000u) << 16, exponent = (h >> 10) & 0x1F, mantissa = h & 0x3FF, bits;
    if (exponent == 0x1F) {
        bits = sign | 0x7F800000u | (mantissa << 13);
    } else if (exponent != 0) {
        bits = sign | ((exponent + 112) << 23) | (mantissa << 13);
    } else if (mantissa != 0) {
        exponent = 113;
        while ((mantissa & 0x400) == 0) {
            mantissa <<= 1;
            --exponent;
        }
        bits = sign | (exponent << 23) | ((mantissa & 0x3FF) << 13);
    } else {
        bits = sign;
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* src/quant.cpp:87-113: round to nearest, ties to even. */
uint16_t or_float_to_half(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const int32_t exponent = (int32_t)((bits >> 23) & 0xFF) - 127 + 15;
    uint32_t mantissa = bits & 0x7FFFFF;
    if (((bits >> 23) & 0xFF) == 0xFF) return (uint16_t)(sign | 0x7C00u | (mantissa ? 0x200u : 0u));
    if (exponent >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (exponent <= 0) {
        if (exponent < -10) return (uint16_t)sign;
        mantissa |= 0x800000u;
        const uint32_t shift = (uint32_t)(14 - exponent);
        uint32_t half = mantissa >> shift;
        const uint32_t rem = mantissa & ((1u << shift) - 1), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half & 1))) ++half;
        return (uint16_t)(sign | half);
    }
    uint32_t half = ((uint32_t)exponent << 10) | (mantissa >> 13);
    const uint32_t rem = mantissa & 0x1FFF;
    if (rem > 0x1000 || (rem == 0x1000 && (half & 1))) ++half;
    return (uint16_t)(sign | half);
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ------------------------------------------------------------------ activation quantisation */

/* src/quant.cpp:115-142 (portable branch).  Block = {u16 d, i8 qs[32]} (34 bytes). */
void or_quantize_q8_0(const float* x, void* out_, size_t count) {
    uint8_t* out = (uint8_t*)out_;
    for (size_t b = 0; b < count / 32; ++b) {
        const float* block = x + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(block[i]));
        const float d = amax / 127.0f;
        const float inverse = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = or_float_to_half(d);
        uint8_t* o = out + b * 34;
        o[0] = (uint8_t)dh;
        o[1] = (uint8_t)(dh >> 8);
        for (int i = 0; i < 32; ++i) o[2 + i] = (uint8_t)(int8_t)nearbyintf(block[i] * inverse);
    }
}

/* src/quant.cpp:146-194 (portable branch).  Block = {f32 d, i8 qs[256], i16 bsums[16]} (292 bytes). */
void or_quantize_q8_k(const float* x, void* out_, size_t count, int bits) {
    uint8_t* out = (uint8_t*)out_;
    for (size_t b = 0; b < count / 256; ++b) {
        const float* block = x + b * 256;
        uint8_t* y = out + b * 292;
        float max = 0.0f, amax = 0.0f;
        for (int i = 0; i < 256; ++i) {
            const float ax = fabsf(block[i]);
            if (ax > amax) {
                amax = ax;
                max = block[i];
            }
        }
        if (amax == 0.0f) {
            memset(y, 0, 292);
            continue;
        }
        const float extreme = bits == 7 ? 63.0f : 127.0f;
        const float inverse = -extreme / max;
        const float d = 1.0f / inverse;
        memcpy(y, &d, 4);
        int8_t* qs = (int8_t*)(y + 4);
        for (int i = 0; i < 256; ++i) qs[i] = (int8_t)fminf(127.0f, nearbyintf(inverse * block[i]));
        for (int g = 0; g < 16; ++g) {
            int sum = 0;
            for (int i = 0; i < 16; ++i) sum += qs[g * 16 + i];
            const int16_t s16 = (int16_t)sum;
            memcpy(y + 260 + 2 * g, &s16, 2);
        }
    }
}

/* ------------------------------------------------------------------ dots */

/* src/quant.cpp:445-456.  Q4_0 = {u16 d, u8 qs[16]}: low nibbles elements 0-15, high 16-31. */
static float dot_q4_0(const uint8_t* w, const uint8_t* x, size_t blocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t* wb = w + b * 18;
        const uint8_t* xb = x + b * 34;
        const int8_t* xq = (const int8_t*)(xb + 2);
        int32_t acc = 0;
        for (int i = 0; i < 16; ++i) {
            acc += ((wb[2 + i] & 0x0F) - 8) * xq[i];
            acc += ((wb[2 + i] >> 4) - 8) * xq[i + 16];
        }
        sum += (float)acc * or_half_to_float(rd16(wb)) * or_half_to_float(rd16(xb));
    }
    return sum;
}

/* src/quant.cpp:474-482 */
static float dot_q8_0(const uint8_t* w, const uint8_t* x, size_t blocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t* wb = w + b * 34;
        const uint8_t* xb = x + b * 34;
        const int8_t* wq = (const int8_t*)(wb + 2);
        const int8_t* xq = (const int8_t*)(xb + 2);
        int32_t acc = 0;
        for (int i = 0; i < 32; ++i) acc += wq[i] * xq[i];
        sum += (float)acc * or_half_to_float(rd16(wb)) * or_half_to_float(rd16(xb));
    }
    return sum;
}

/* src/quant.cpp:484-498.  Q4_1 = {u16 d, u16 m, u8 qs[16]}: weight = q d + m; the x block sum
 * enters as m (dx xsum). */
static float dot_q4_1(const uint8_t* w, const uint8_t* x, size_t blocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t* wb = w + b * 20;
        const uint8_t* xb = x + b * 34;
        const int8_t* xq = (const int8_t*)(xb + 2);
        int32_t acc = 0, xsum = 0;
        for (int i = 0; i < 16; ++i) {
            acc += (wb[4 + i] & 0x0F) * xq[i];
            acc += (wb[4 + i] >> 4) * xq[i + 16];
            xsum += xq[i] + xq[i + 16];
        }
        const float dx = or_half_to_float(rd16(xb));
        sum += (float)acc * or_half_to_float(rd16(wb)) * dx + or_half_to_float(rd16(wb + 2)) * (dx * (float)xsum);
    }
    return sum;
}

/* src/quant.cpp:458-472.  Q5_0 = {u16 d, u8 qh[4], u8 qs[16]}: the fifth bit of element e is
 * bit e of qh (little-endian word); weight = (q - 16) d. */
static float dot_q5_0(const uint8_t* w, const uint8_t* x, size_t blocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t* wb = w + b * 22;
        const uint8_t* xb = x + b * 34;
        const int8_t* xq = (const int8_t*)(xb + 2);
        uint32_t qh;
        memcpy(&qh, wb + 2, 4);
        int32_t acc = 0;
        for (int i = 0; i < 16; ++i) {
            const int lo = ((wb[6 + i] & 0x0F) | (int)(((qh >> i) & 1) << 4)) - 16;
            const int hi = ((wb[6 + i] >> 4) | (int)(((qh >> (i + 16)) & 1) << 4)) - 16;
            acc += lo * xq[i] + hi * xq[i + 16];
        }
        sum += (float)acc * or_half_to_float(rd16(wb)) * or_half_to_float(rd16(xb));
    }
    return sum;
}

/* src/quant.h:256-264 */
static void q4_k_scale_min(const uint8_t* scales, int j, uint8_t* scale, uint8_t* min) {
    if (j < 4) {
        *scale = scales[j] & 63;
        *min = scales[j + 4] & 63;
    } else {
        *scale = (uint8_t)((scales[j + 4] & 0xF) | ((scales[j - 4] >> 6) << 4));
        *min = (uint8_t)((scales[j + 4] >> 4) | ((scales[j] >> 6) << 4));
    }
}

static inline float q8k_d(const uint8_t* xb) {
    float d;
    memcpy(&d, xb, 4);
    return d;
}
static inline int16_t q8k_bsum(const uint8_t* xb, int g) {
    int16_t s;
    memcpy(&s, xb + 260 + 2 * g, 2);
    return s;
}

/* src/quant.cpp:500-521.  Q4_K = {u16 d, u16 dmin, u8 scales[12], u8 qs[128]}. */
static float dot_q4_k(const uint8_t* w, const uint8_t* x, size_t blocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t* wb = w + b * 144;
        const uint8_t* xb = x + b * 292;
        const int8_t* xqs = (const int8_t*)(xb + 4);
        int32_t weighted = 0, offsets = 0;
        for (int sb = 0; sb < 8; ++sb) {
            uint8_t scale, min;
            q4_k_scale_min(wb + 4, sb, &scale, &min);
            const uint8_t* q = wb + 16 + (sb / 2) * 32;
            const int8_t* xq = xqs + sb * 32;
            int32_t dot = 0;
            for (int i = 0; i < 32; ++i) dot += ((sb % 2 == 0) ? (q[i] & 0xF) : (q[i] >> 4)) * xq[i];
            weighted += scale * dot;
            offsets += min * (q8k_bsum(xb, 2 * sb) + q8k_bsum(xb, 2 * sb + 1));
        }
        sum += q8k_d(xb) * (or_half_to_float(rd16(wb)) * (float)weighted - or_half_to_float(rd16(wb + 2)) * (float)offsets);
    }
    return sum;
}

/* src/quant.cpp:523-547.  Q5_K = {u16 d, u16 dmin, u8 scales[12], u8 qh[32], u8 qs[128]}: Q4_K
 * with a fifth bit, bit sb of qh[i] for element i of sub-block sb. */
static float dot_q5_k(const uint8_t* w, const uint8_t* x, size_t blocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t* wb = w + b * 176;
        const uint8_t* xb = x + b * 292;
        const int8_t* xqs = (const int8_t*)(xb + 4);
        const uint8_t* qh = wb + 16;
        int32_t weighted = 0, offsets = 0;
        for (int sb = 0; sb < 8; ++sb) {
            uint8_t scale, min;
            q4_k_scale_min(wb + 4, sb, &scale, &min);
            const uint8_t* q = wb + 48 + (sb / 2) * 32;
            const uint8_t bit = (uint8_t)(1u << sb);
            const int8_t* xq = xqs + sb * 32;
            int32_t dot = 0;
            for (int i = 0; i < 32; ++i) {
                const int v = ((sb % 2 == 0) ? (q[i] & 0xF) : (q[i] >> 4)) | ((qh[i] & bit) ? 16 : 0);
                dot += v * xq[i];
            }
            weighted += scale * dot;
            offsets += min * (q8k_bsum(xb, 2 * sb) + q8k_bsum(xb, 2 * sb + 1));
        }
        sum += q8k_d(xb) * (or_half_to_float(rd16(wb)) * (float)weighted - or_half_to_float(rd16(wb + 2)) * (float)offsets);
    }
    return sum;
}

/* src/quant.cpp:285-297.  Q6_K = {u8 ql[128], u8 qh[64], i8 scales[16], u16 d}. */
static void unpack_q6_k(const uint8_t* block, int8_t* q) {
    for (int half = 0; half < 2; ++half) {
        const uint8_t* ql = block + half * 64;
        const uint8_t* qh = block + 128 + half * 32;
        int8_t* y = q + half * 128;
        for (int l = 0; l < 32; ++l) {
            y[l] = (int8_t)(((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32);
            y[l + 32] = (int8_t)(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
            y[l + 64] = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
            y[l + 96] = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
        }
    }
}

/* src/quant.cpp:549-563 */
static float dot_q6_k(const uint8_t* w, const uint8_t* x, size_t blocks) {
    int8_t q[256];
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t* wb = w + b * 210;
        const uint8_t* xb = x + b * 292;
        const int8_t* xq = (const int8_t*)(xb + 4);
        const int8_t* scales = (const int8_t*)(wb + 192);
        unpack_q6_k(wb, q);
        int32_t weighted = 0;
        for (int g = 0; g < 16; ++g) {
            int32_t dot = 0;
            for (int i = 0; i < 16; ++i) dot += q[g * 16 + i] * xq[g * 16 + i];
            weighted += scales[g] * dot;
        }
        sum += q8k_d(xb) * or_half_to_float(rd16(wb + 208)) * (float)weighted;
    }
    return sum;
}

/* Element e of a TQ2_0 block {u8 qs[64], u16 d}: byte j + m (j in {0, 32}) holds elements
 * 128 (j/32) + 32 l + m at bit pair 2l (src/quant.h:123-130, src/quant.cpp:566-578). */
static inline int tq2_code(const uint8_t* wb, int e) {
    const int j = (e / 128) * 32, l = (e % 128) / 32, m = e % 32;
    return (wb[j + m] >> (2 * l)) & 3;
}

/* src/quant.cpp:580-596: the generic TQ2_0 dot (8-bit activations). */
static float dot_tq2_0(const uint8_t* w, const uint8_t* x, size_t blocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t* wb = w + b * 66;
        const uint8_t* xb = x + b * 292;
        const int8_t* xq = (const int8_t*)(xb + 4);
        int32_t acc = 0;
        for (int e = 0; e < 256; ++e) acc += tq2_code(wb, e) * xq[e];
        int32_t xsum = 0;
        for (int g = 0; g < 16; ++g) xsum += q8k_bsum(xb, g);
        sum += q8k_d(xb) * or_half_to_float(rd16(wb + 64)) * (float)(acc - xsum);
    }
    return sum;
}

/* src/quant.cpp:789-802 on the TQ2_0x16 layout, restated on the GGUF block: the pair
 * index idx = c0 * 3 + c1 gives weights idx/3 - 1 and idx%3 - 1, i.e. the two codes
 * minus one, so acc is the same integer; the float order is acc * d_w * d_x. */
static float dot_tq2_0x16(const uint8_t* w, const uint8_t* x, size_t blocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t* wb = w + b * 66;
        const uint8_t* xb = x + b * 292;
        const int8_t* xq = (const int8_t*)(xb + 4);
        int32_t acc = 0;
        for (int e = 0; e < 256; ++e) acc += (tq2_code(wb, e) - 1) * xq[e];
        sum += (float)acc * or_half_to_float(rd16(wb + 64)) * q8k_d(xb);
    }
    return sum;
}

float or_dot(int type, int lut16, const void* w, const void* x, size_t blocks) {
    switch (type) {
        case OR_Q4_0: return dot_q4_0((const uint8_t*)w, (const uint8_t*)x, blocks);
        case OR_Q8_0: return dot_q8_0((const uint8_t*)w, (const uint8_t*)x, blocks);
        case OR_Q4_1: return dot_q4_1((const uint8_t*)w, (const uint8_t*)x, blocks);
        case OR_Q5_0: return dot_q5_0((const uint8_t*)w, (const uint8_t*)x, blocks);
        case OR_Q4_K: return dot_q4_k((const uint8_t*)w, (const uint8_t*)x, blocks);
        case OR_Q5_K: return dot_q5_k((const uint8_t*)w, (const uint8_t*)x, blocks);
        case OR_Q6_K: return dot_q6_k((const uint8_t*)w, (const uint8_t*)x, blocks);
        case OR_TQ2_0: return lut16 ? dot_tq2_0x16((const uint8_t*)w, (const uint8_t*)x, blocks)
                                    : dot_tq2_0((const uint8_t*)w, (const uint8_t*)x, blocks);
    }
    return NAN;
}

static size_t block_elems(int type) {
    return (type == OR_Q4_0 || type == OR_Q8_0 || type == OR_Q4_1 || type == OR_Q5_0) ? 32 : 256;
}
static size_t block_bytes(int type) {
    switch (type) {
        case OR_Q4_0: return 18;
        case OR_Q4_1: return 20;
        case OR_Q5_0: return 22;
        case OR_Q8_0: return 34;
        case OR_Q4_K: return 144;
        case OR_Q5_K: return 176;
        case OR_Q6_K: return 210;
        case OR_TQ2_0: return 66;
    }
    return 0;
}

/* src/model.cpp:496-503 + src/quant.cpp:144: on x86, TQ2_0 matrices with rows % 16 == 0 are
 * repacked to TQ2_0x16, whose kernels take 7-bit activations. */
int or_activation_bits(int type, size_t rows) { return (type == OR_TQ2_0 && rows % 16 == 0) ? 7 : 8; }
static int takes_q8_k(int type) { return type == OR_Q4_K || type == OR_Q5_K || type == OR_Q6_K || type == OR_TQ2_0; }

/* matvec_generic (src/kernels.cpp:13-19) */
void or_matvec(int type, const void* w, size_t rows, size_t cols, const void* x, float* out) {
    const size_t blocks = cols / block_elems(type), rb = blocks * block_bytes(type);
    const int lut16 = type == OR_TQ2_0 && rows % 16 == 0;
    for (size_t r = 0; r < rows; ++r) out[r] = or_dot(type, lut16, (const uint8_t*)w + r * rb, x, blocks);
}

/* src/quant.cpp:196-239, :299-307, :566-578 */
void or_dequantize(int type, const void* blocks_, float* out, size_t count) {
    const uint8_t* blocks = (const uint8_t*)blocks_;
    const size_t nb = count / block_elems(type);
    for (size_t b = 0; b < nb; ++b) {
        float* y = out + b * block_elems(type);
        const uint8_t* wb = blocks + b * block_bytes(type);
        switch (type) {
            case OR_Q4_0: {
                const float d = or_half_to_float(rd16(wb));
                for (int i = 0; i < 16; ++i) {
                    y[i] = (float)((wb[2 + i] & 0x0F) - 8) * d;
                    y[i + 16] = (float)((wb[2 + i] >> 4) - 8) * d;
                }
                break;
            }
            case OR_Q8_0: {
                const float d = or_half_to_float(rd16(wb));
                for (int i = 0; i < 32; ++i) y[i] = (float)((const int8_t*)(wb + 2))[i] * d;
                break;
            }
            case OR_Q4_1: {  /* src/quant.cpp:207-217 */
                const float d = or_half_to_float(rd16(wb)), m = or_half_to_float(rd16(wb + 2));
                for (int i = 0; i < 16; ++i) {
                    y[i] = (float)(wb[4 + i] & 0x0F) * d + m;
                    y[i + 16] = (float)(wb[4 + i] >> 4) * d + m;
                }
                break;
            }
            case OR_Q5_0: {  /* src/quant.cpp:219-232 */
                const float d = or_half_to_float(rd16(wb));
                uint32_t qh;
                memcpy(&qh, wb + 2, 4);
                for (int i = 0; i < 16; ++i) {
                    const int lo = (wb[6 + i] & 0x0F) | (int)(((qh >> i) & 1) << 4);
                    const int hi = (wb[6 + i] >> 4) | (int)(((qh >> (i + 16)) & 1) << 4);
                    y[i] = (float)(lo - 16) * d;
                    y[i + 16] = (float)(hi - 16) * d;
                }
                break;
            }
            case OR_Q5_K: {  /* src/quant.cpp:263-283 */
                const float d = or_half_to_float(rd16(wb)), dmin = or_half_to_float(rd16(wb + 2));
                const uint8_t* qh = wb + 16;
                for (int chunk = 0; chunk < 4; ++chunk) {
                    uint8_t scale, min;
                    q4_k_scale_min(wb + 4, 2 * chunk, &scale, &min);
                    const float d1 = d * scale, m1 = dmin * min;
                    q4_k_scale_min(wb + 4, 2 * chunk + 1, &scale, &min);
                    const float d2 = d * scale, m2 = dmin * min;
                    const uint8_t* q = wb + 48 + chunk * 32;
                    const uint8_t lo_bit = (uint8_t)(1u << (2 * chunk)), hi_bit = (uint8_t)(lo_bit << 1);
                    for (int i = 0; i < 32; ++i) {
                        y[chunk * 64 + i] = d1 * (float)((q[i] & 0xF) | ((qh[i] & lo_bit) ? 16 : 0)) - m1;
                        y[chunk * 64 + 32 + i] = d2 * (float)((q[i] >> 4) | ((qh[i] & hi_bit) ? 16 : 0)) - m2;
                    }
                }
                break;
            }
            case OR_Q4_K: {
                const float d = or_half_to_float(rd16(wb)), dmin = or_half_to_float(rd16(wb + 2));
                for (int chunk = 0; chunk < 4; ++chunk) {
                    uint8_t scale, min;
                    q4_k_scale_min(wb + 4, 2 * chunk, &scale, &min);
                    const float d1 = d * scale, m1 = dmin * min;
                    q4_k_scale_min(wb + 4, 2 * chunk + 1, &scale, &min);
                    const float d2 = d * scale, m2 = dmin * min;
                    const uint8_t* q = wb + 16 + chunk * 32;
                    for (int i = 0; i < 32; ++i) {
                        y[chunk * 64 + i] = d1 * (float)(q[i] & 0xF) - m1;
                        y[chunk * 64 + 32 + i] = d2 * (float)(q[i] >> 4) - m2;
                    }
                }
                break;
            }
            case OR_Q6_K: {
                int8_t q[256];
                const float d = or_half_to_float(rd16(wb + 208));
                const int8_t* scales = (const int8_t*)(wb + 192);
                unpack_q6_k(wb, q);
                for (int i = 0; i < 256; ++i) y[i] = d * scales[i / 16] * q[i];
                break;
            }
            case OR_TQ2_0: {
                const float d = or_half_to_float(rd16(wb + 64));
                for (int e = 0; e < 256; ++e) y[e] = (float)(tq2_code(wb, e) - 1) * d;
                break;
            }
        }
    }
}

/* tq2_0_pair_indices + repack_tq2_0x16_scalar (src/quant.cpp:636-672): 16 rows per group,
 * byte (p/2)*16 + r holds row r's pair indices 2k (low nibble) and 2k+1 (high), then d[16]. */
void or_repack_tq2_0x16(const void* in_, size_t rows, size_t blocks, void* out_) {
    const uint8_t* in = (const uint8_t*)in_;
    uint8_t* out = (uint8_t*)out_;
    for (size_t g = 0; g < rows / 16; ++g) {
        for (size_t b = 0; b < blocks; ++b) {
            uint8_t* packed = out + (g * blocks + b) * 1056;
            memset(packed, 0, 1024);
            for (size_t r = 0; r < 16; ++r) {
                const uint8_t* block = in + ((g * 16 + r) * blocks + b) * 66;
                memcpy(packed + 1024 + 2 * r, block + 64, 2);
                for (int p = 0; p < 128; p += 2) {
                    const int i0 = tq2_code(block, 2 * p) * 3 + tq2_code(block, 2 * p + 1);
                    const int i1 = tq2_code(block, 2 * p + 2) * 3 + tq2_code(block, 2 * p + 3);
                    packed[(p / 2) * 16 + r] = (uint8_t)(i0 | (i1 << 4));
                }
            }
        }
    }
}

/* ------------------------------------------------------------------ float kernels */

/* dot_f32, portable branch (src/kernels_f32.cpp:231-243): 16 lane partials, tail, then lanes in order. */
float or_dot_f32(const float* a, const float* b, size_t n) {
    float lanes[16] = {0};
    size_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int j = 0; j < 16; ++j) lanes[j] += a[i + j] * b[i + j];
    float sum = 0.0f;
    for (; i < n; ++i) sum += a[i] * b[i];
    for (int j = 0; j < 16; ++j) sum += lanes[j];
    return sum;
}

/* softmax_f32 (src/kernels_f32.cpp:276-284) */
void or_softmax(float* x, size_t n) {
    float max = x[0];
    for (size_t i = 1; i < n; ++i)
        if (x[i] > max) max = x[i];
    double sum = 0.0;
    for (size_t i = 0; i < n; ++i) {
        x[i] = expf(x[i] - max);
        sum += x[i];
    }
    const float scale = (float)(1.0 / sum);
    for (size_t i = 0; i < n; ++i) x[i] *= scale;
}

/* rms_norm (src/model.cpp:87-97): squares in float, summed in double. x and out may alias. */
void or_rms_norm(const float* x, const float* w, float eps, float* out, size_t n) {
    double sum = 0.0;
    for (size_t i = 0; i < n; ++i) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    if (!w) { /* no weight: plain normalisation (Gemma 4's V) */
        for (size_t i = 0; i < n; ++i) out[i] = x[i] * scale;
        return;
    }
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * scale * w[i];
}

/* apply_rope (src/model.cpp:104-115) */
static void apply_rope(float* head, const float* rope, size_t dim, int neox) {
    const size_t half = dim / 2;
    for (size_t i = 0; i < half; ++i) {
        const float c = rope[2 * i], s = rope[2 * i + 1];
        float* a = &head[neox ? i : 2 * i];
        float* b = &head[neox ? i + half : 2 * i + 1];
        const float x0 = *a, x1 = *b;
        *a = x0 * c - x1 * s;
        *b = x0 * s + x1 * c;
    }
}

/* ------------------------------------------------------------------ expf */

/* glibc's expf, as the reference calls it (std::exp on float). */
void or_expf_batch(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = expf(x[i]);
}

/* The restatement of glibc's expf that the HIP token loop runs (its table-driven
 * double-precision algorithm, with the x86-64 FMA variant's fused reduction
 * r = x * 32/ln2 - k).  or_expf_check compares it with the host's expf on every
 * `stride`-th 32-bit pattern and returns the number of differing results. */
static uint64_t g_exp_tab[32];
static float expf_restated(float x) {
    uint32_t ux;
    memcpy(&ux, &x, 4);
    const uint32_t abstop = (ux >> 20) & 0x7FF;
    if (abstop >= 0x42Bu) {
        if (ux == 0xFF800000u) return 0.0f;
        if (abstop >= 0x7F8u) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0, c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x, z = inv_ln2_n * xd;
    double kd = z + shift;
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    const uint64_t t = g_exp_tab[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    const double p = fma(c0, r, c1), r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(p, r2, y);
    return (float)(y * s);
}

uint64_t or_expf_check(uint32_t stride, uint64_t* checked) {
    for (int i = 0; i < 32; ++i) {
        const double d = exp2((double)i / 32.0);
        memcpy(&g_exp_tab[i], &d, 8);
        g_exp_tab[i] -= ((uint64_t)i << 52) / 32;
    }
    uint64_t bad = 0, n = 0;
    for (uint64_t b = 0; b <= 0xFFFFFFFFull; b += stride) {
        const uint32_t bits = (uint32_t)b;
        float x;
        memcpy(&x, &bits, 4);
        if (isnan(x)) continue;
        const float a = expf(x), e = expf_restated(x);
        uint32_t ua, ue;
        memcpy(&ua, &a, 4);
        memcpy(&ue, &e, 4);
        bad += ua != ue;
        ++n;
    }
    if (checked) *checked = n;
    return bad;
}

/* glibc's tanhf, as the reference calls it (std::tanh on float: gelu_mul_f32 and the
 * final softcap, src/kernels_f32.cpp:291-296, src/model.cpp:1206-1209). */
void or_tanhf_batch(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = tanhf(x[i]);
}

/* The restatement of glibc 2.35's tanhf that the HIP Gemma epilogues run: fdlibm's
 * s_tanhf.c over its s_expm1f.c (argument reduction by k ln2 in a hi and a lo part,
 * a rational form with five scaled coefficients, k put back into the exponent).
 * or_tanhf_check compares it with the host's tanhf on every `stride`-th 32-bit
 * pattern and returns the number of differing results. */
static inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float ffrom(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static float expm1f_restated(float x) {
    const float one = 1.0f, huge = 1.0e+30f, tiny = 1.0e-30f, o_threshold = 8.8721679688e+01f;
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f, Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
    float y, hi, lo, c = 0, t, e, hxs, hfx, r1;
    int32_t k;
    uint32_t hx = fbits(x);
    const uint32_t xsb = hx & 0x80000000u;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) {
        if (hx >= 0x42b17218u) {
            if (hx > 0x7f800000u) return x + x;
            if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;
            if (x > o_threshold) return huge * huge;
        }
        if (xsb != 0) return tiny - one;
    }
    if (hx > 0x3eb17218u) {
        if (hx < 0x3F851592u) {
            if (xsb == 0) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
            else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
        } else {
            k = (int32_t)(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
            t = (float)k;
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {
        t = huge + x;
        return x - (t - (huge + x));
    } else k = 0;
    hfx = 0.5f * x;
    hxs = x * hfx;
    r1 = one + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
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
        return ffrom(fbits(y) + ((uint32_t)k << 23)) - one;
    }
    if (k < 23) {
        t = ffrom(0x3f800000u - (0x1000000u >> k));
        y = t - (e - x);
        y = ffrom(fbits(y) + ((uint32_t)k << 23));
    } else {
        t = ffrom((uint32_t)(0x7f - k) << 23);
        y = x - (e + t);
        y += one;
        y = ffrom(fbits(y) + ((uint32_t)k << 23));
    }
    return y;
}
static float tanhf_restated(float x) {
    const float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
    float t, z;
    const uint32_t jx = fbits(x), ix = jx & 0x7fffffffu;
    if (ix >= 0x7f800000u) return (jx & 0x80000000u) == 0 ? one / x + one : one / x - one;
    if (ix < 0x41b00000u) {
        if (ix == 0) return x;
        if (ix < 0x24000000u) return x * (one + x);
        if (ix >= 0x3f800000u) {
            t = expm1f_restated(two * fabsf(x));
            z = one - two / (t + two);
        } else {
            t = expm1f_restated(-two * fabsf(x));
            z = -t / (t + two);
        }
    } else z = one - tiny;
    return (jx & 0x80000000u) == 0 ? z : -z;
}

uint64_t or_tanhf_check(uint32_t stride, uint64_t* checked) {
    uint64_t bad = 0, n = 0;
    for (uint64_t b = 0; b <= 0xFFFFFFFFull; b += stride) {
        const float x = ffrom((uint32_t)b);
        if (isnan(x)) continue;
        const float a = tanhf(x), e = tanhf_restated(x);
        bad += fbits(a) != fbits(e);
        ++n;
    }
    if (checked) *checked = n;
    return bad;
}

/* glibc's log1pf, as the reference calls it (std::log1p on float: the softplus of Qwen3.5's
 * recurrence, src/model.cpp:827). */
void or_log1pf_batch(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = log1pf(x[i]);
}

/* The restatement of glibc 2.35's log1pf that the HIP recurrence runs: fdlibm's s_log1pf.c
 * (1 + x split as 2^k (1 + f) with a correction term c for the rounding of 1 + x, then
 * log(1 + f) = f - hfsq + s (hfsq + R(s^2)), s = f / (2 + f), R a degree-7 polynomial in
 * s^2, plus k ln2 in a hi and a lo part).  or_log1pf_check compares it with the host's
 * log1pf on every `stride`-th 32-bit pattern and returns the number of differing results. */
static float log1pf_restated(float x) {
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, two25 = 3.355443200e+07f;
    const float Lp1 = 6.6666668653e-01f, Lp2 = 4.0000000596e-01f, Lp3 = 2.8571429849e-01f, Lp4 = 2.2222198546e-01f,
                Lp5 = 1.8183572590e-01f, Lp6 = 1.5313838422e-01f, Lp7 = 1.4798198640e-01f;
    float hfsq, f = 0.0f, c = 0.0f, s, z, R, u;
    const int32_t hx = (int32_t)fbits(x), ax = hx & 0x7fffffff;
    int32_t k = 1, hu = 0;
    if (hx < 0x3ed413d7) { /* x < 0.41422 */
        if (ax >= 0x3f800000) { /* x <= -1 */
            if (x == -1.0f) return -two25 / 0.0f;
            return (x - x) / (x - x);
        }
        if (ax < 0x31000000) { /* |x| < 2^-29 */
            if (ax < 0x24800000) return x;
            return x - x * x * 0.5f;
        }
        if (hx > 0 || hx <= (int32_t)0xbe95f61f) { /* -0.2929 < x < 0.41422 */
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
            hu = (int32_t)fbits(u);
            k = (hu >> 23) - 127;
            c = k > 0 ? 1.0f - (u - x) : x - (u - 1.0f); /* the rounding error of 1 + x */
            c /= u;
        } else {
            u = x;
            hu = (int32_t)fbits(u);
            k = (hu >> 23) - 127;
            c = 0.0f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = ffrom((uint32_t)hu | 0x3f800000u);
        } else {
            k += 1;
            u = ffrom((uint32_t)hu | 0x3f000000u);
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    hfsq = 0.5f * f * f;
    if (hu == 0) { /* |f| < 2^-20 */
        if (f == 0.0f) {
            if (k == 0) return 0.0f;
            c += k * ln2_lo;
            return k * ln2_hi + c;
        }
        R = hfsq * (1.0f - 0.66666666666666666f * f);
        if (k == 0) return f - R;
        return k * ln2_hi - ((R - (k * ln2_lo + c)) - f);
    }
    s = f / (2.0f + f);
    z = s * s;
    R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + R));
    return k * ln2_hi - ((hfsq - (s * (hfsq + R) + (k * ln2_lo + c))) - f);
}

uint64_t or_log1pf_check(uint32_t stride, uint64_t* checked) {
    uint64_t bad = 0, n = 0;
    for (uint64_t b = 0; b <= 0xFFFFFFFFull; b += stride) {
        const float x = ffrom((uint32_t)b);
        if (isnan(x)) continue;
        const float a = log1pf(x), e = log1pf_restated(x);
        bad += fbits(a) != fbits(e) && !(isnan(a) && isnan(e));
        ++n;
    }
    if (checked) *checked = n;
    return bad;
}

/* ------------------------------------------------------------------ session */

typedef struct {
    int type;
    size_t rows, cols;
    const uint8_t* data;
} matrix;

typedef struct {
    const float *attn_norm, *q_norm, *k_norm, *attn_sub_norm, *ffn_norm, *ffn_sub_norm;
    const float *q_bias, *k_bias, *v_bias; /* all or none (src/model.cpp:411-416) */
    const float *attn_post_norm, *ffn_post_norm; /* Gemma (src/model.cpp:399-402) */
    matrix q, k, v, o, gate, up, down;
    matrix conv_in, conv_out;  /* LFM2 short convolution (src/model.cpp:360-364) */
    const float* conv_w;       /* [embd][taps]; non-NULL marks a convolution layer */
    uint16_t* conv_cache;      /* bx per position, fp16 [max_context][embd] */
    /* Qwen3.5 Gated DeltaNet layer (src/model.cpp:343-358); ssm_a non-NULL marks it */
    matrix ssm_qkv, ssm_gate, ssm_alpha, ssm_beta, ssm_out;
    const float *ssm_a, *ssm_dt, *ssm_conv_w, *ssm_norm;
    float *state, *ring;           /* S[head][j][i] (value j, key i); the conv's last ssm_conv - 1 inputs */
    float *snap_state, *snap_ring; /* both as they were before the last evaluated token */
    /* Gemma 4: the per-layer embedding's gate and projection and its norm; the output scale */
    matrix ple_gate, ple_proj;
    const float* ple_post_norm;
    float out_scale;
} layer_t;

struct oracle_session {
    oracle_config c;
    matrix embd, out;
    const float* out_norm;
    layer_t* layers;
    uint16_t **kcache, **vcache;
    size_t position;
    /* scratch */
    float *h, *normed, *q, *k, *v, *att, *proj, *gate, *up, *scores, *rope, *rope_local, *conv;
    const float* rope_factors; /* rope_freqs, or Phi-3's short / long factors; NULL: none */
    uint8_t* xq;
    /* Qwen3.5: the query|gate rows, the gates, the recurrence's projections and conv outputs */
    float *qg, *agate, *sqkv, *sconv, *sz, *sab;
    int snap_valid;
    size_t snap_pos;
    /* Gemma 4's per-layer embeddings (src/model.cpp:319-324): table, projection, its norm; the
     * token's inputs [layers][ple_dim], its table row and the gate */
    matrix ple_tok, ple_model_proj;
    const float* ple_proj_norm;
    float *ple, *ple_row, *ple_g;
};

/* ModelConfig's per-layer accessors (src/model.h:87-118). */
static int layer_slides(const oracle_config* c, int l) {
    if (c->sliding_pattern) return c->sliding_pattern[l] != 0;
    return c->sliding_window != 0 && l % 6 != 5;
}
static size_t head_dim_of(const oracle_config* c, int l) {
    return c->head_dim_local != 0 && layer_slides(c, l) ? (size_t)c->head_dim_local : (size_t)c->head_dim;
}
static size_t kv_heads_of(const oracle_config* c, int l) { return c->kv_head_counts ? (size_t)c->kv_head_counts[l] : (size_t)c->kv_heads; }
static size_t ff_of(const oracle_config* c, int l) { return c->ff_dims ? (size_t)c->ff_dims[l] : (size_t)c->ff; }
static int kv_layer_of(const oracle_config* c, int l) {
    if (c->kv_from_start == 0 || l < c->kv_from_start) return l;
    return c->kv_from_start - (layer_slides(c, l) ? 2 : 1);
}

static const oracle_tensor* find(const oracle_tensor* t, size_t n, const char* name) {
    for (size_t i = 0; i < n; ++i)
        if (strcmp(t[i].name, name) == 0) return &t[i];
    return NULL;
}

oracle_session* or_session_create(const oracle_config* cfg, const oracle_tensor* t, size_t n) {
    oracle_session* s = (oracle_session*)calloc(1, sizeof *s);
    s->c = *cfg;
    const oracle_config* c = cfg;
    char name[128];
#define GETM(dst, nm)                                                                    \
    do {                                                                                 \
        const oracle_tensor* x_ = find(t, n, nm);                                        \
        if (!x_) { snprintf(g_err, sizeof g_err, "missing tensor '%s'", nm); goto bad; } \
        (dst).type = x_->type; (dst).rows = x_->rows; (dst).cols = x_->cols;              \
        (dst).data = (const uint8_t*)x_->data;                                           \
    } while (0)
#define GETV(dst, nm)                                                                    \
    do {                                                                                 \
        const oracle_tensor* x_ = find(t, n, nm);                                        \
        if (!x_) { snprintf(g_err, sizeof g_err, "missing tensor '%s'", nm); goto bad; } \
        (dst) = (const float*)x_->data;                                                  \
    } while (0)
    GETM(s->embd, "token_embd.weight");
    if (find(t, n, "output.weight")) GETM(s->out, "output.weight");
    else s->out = s->embd;  /* src/model.cpp:328-330 */
    GETV(s->out_norm, c->arch == OR_LFM2 ? "token_embd_norm.weight" : "output_norm.weight"); /* src/model.cpp:331 */
    if (c->ple_dim != 0) { /* src/model.cpp:319-324 */
        GETM(s->ple_tok, "per_layer_token_embd.weight");
        GETM(s->ple_model_proj, "per_layer_model_proj.weight");
        GETV(s->ple_proj_norm, "per_layer_proj_norm.weight");
    }
    /* per-frequency factors (src/model.cpp:312-318) and LongRoPE's choice (:691-694) */
    {
        const oracle_tensor* f = find(t, n, "rope_freqs.weight");
        if (c->arch == OR_PHI3 && find(t, n, "rope_factors_short.weight"))
            f = find(t, n, c->rope_original_context != 0 && c->max_context > c->rope_original_context ? "rope_factors_long.weight"
                                                                                                       : "rope_factors_short.weight");
        s->rope_factors = f ? (const float*)f->data : NULL;
    }
    s->layers = (layer_t*)calloc((size_t)c->layers, sizeof(layer_t));
    for (int l = 0; l < c->layers; ++l) {
        layer_t* L = &s->layers[l];
#define LN(sfx) (snprintf(name, sizeof name, "blk.%d.%s", l, sfx), name)
        GETV(L->attn_norm, LN("attn_norm.weight"));
        L->out_scale = 1.0f;
        if (c->arch == OR_QWEN35 && find(t, n, LN("ssm_a"))) { /* src/model.cpp:343-358 */
            const size_t qkv = 2 * (size_t)c->ssm_k_heads * c->ssm_state + (size_t)c->ssm_inner;
            GETM(L->ssm_qkv, LN("attn_qkv.weight"));
            GETM(L->ssm_gate, LN("attn_gate.weight"));
            GETM(L->ssm_alpha, LN("ssm_alpha.weight"));
            GETM(L->ssm_beta, LN("ssm_beta.weight"));
            GETV(L->ssm_a, LN("ssm_a"));
            GETV(L->ssm_dt, LN("ssm_dt.bias"));
            GETV(L->ssm_conv_w, LN("ssm_conv1d.weight"));
            GETV(L->ssm_norm, LN("ssm_norm.weight"));
            GETM(L->ssm_out, LN("ssm_out.weight"));
            GETV(L->ffn_norm, LN("post_attention_norm.weight"));
            GETM(L->gate, LN("ffn_gate.weight"));
            GETM(L->up, LN("ffn_up.weight"));
            GETM(L->down, LN("ffn_down.weight"));
            const size_t st = (size_t)c->ssm_v_heads * c->ssm_state * c->ssm_state, rg = (size_t)(c->ssm_conv - 1) * qkv;
            L->state = (float*)calloc(st, 4);
            L->snap_state = (float*)calloc(st, 4);
            L->ring = (float*)calloc(rg, 4);
            L->snap_ring = (float*)calloc(rg, 4);
            continue;
        }
        if (c->arch == OR_LFM2 && find(t, n, LN("shortconv.in_proj.weight"))) {
            GETM(L->conv_in, LN("shortconv.in_proj.weight"));
            GETM(L->conv_out, LN("shortconv.out_proj.weight"));
            GETV(L->conv_w, LN("shortconv.conv.weight"));
            GETV(L->ffn_norm, LN("ffn_norm.weight"));
            GETM(L->gate, LN("ffn_gate.weight"));
            GETM(L->up, LN("ffn_up.weight"));
            GETM(L->down, LN("ffn_down.weight"));
            L->conv_cache = (uint16_t*)calloc((size_t)c->max_context * (size_t)c->embd, 2);
            continue;
        }
        if (c->arch == OR_PHI3) { /* rows of the fused tensors (load_matrix_rows, src/model.cpp:370-380) */
            const size_t qd = (size_t)c->heads * c->head_dim, kvd = (size_t)c->kv_heads * c->head_dim;
            GETM(L->q, LN("attn_qkv.weight"));
            L->k = L->q;
            L->v = L->q;
            const size_t rb = block_bytes(L->q.type) * (L->q.cols / block_elems(L->q.type));
            L->q.rows = qd;
            L->k.rows = kvd; L->k.data += qd * rb;
            L->v.rows = kvd; L->v.data += (qd + kvd) * rb;
            GETM(L->gate, LN("ffn_up.weight"));
            L->up = L->gate;
            L->gate.rows = (size_t)c->ff;
            L->up.rows = (size_t)c->ff; L->up.data += (size_t)c->ff * rb;
        } else {
            GETM(L->q, LN("attn_q.weight"));
            if (kv_layer_of(c, l) == l) {
                GETM(L->k, LN("attn_k.weight"));
                /* Gemma 4 global layers may have no V projection: K serves as V (src/model.cpp:386-388) */
                if (find(t, n, LN("attn_v.weight"))) GETM(L->v, LN("attn_v.weight"));
                else L->v = L->k;
            }
            GETM(L->gate, LN("ffn_gate.weight"));
            GETM(L->up, LN("ffn_up.weight"));
        }
        GETM(L->o, LN("attn_output.weight"));
        GETV(L->ffn_norm, LN(c->arch == OR_QWEN35 ? "post_attention_norm.weight" : "ffn_norm.weight")); /* src/model.cpp:418 */
        GETM(L->down, LN("ffn_down.weight"));
        if (c->arch == OR_GEMMA3 || c->arch == OR_GEMMA4) {
            GETV(L->attn_post_norm, LN("post_attention_norm.weight"));
            GETV(L->ffn_post_norm, LN("post_ffw_norm.weight"));
        }
        if (c->arch == OR_QWEN3 || c->arch == OR_GEMMA3 || c->arch == OR_LFM2 || c->arch == OR_QWEN35 || c->arch == OR_GEMMA4) { /* src/model.cpp:394-398 */
            GETV(L->q_norm, LN("attn_q_norm.weight"));
            if (kv_layer_of(c, l) == l) GETV(L->k_norm, LN("attn_k_norm.weight"));
        }
        if (c->ple_dim != 0) { /* src/model.cpp:403-407 */
            GETM(L->ple_gate, LN("inp_gate.weight"));
            GETM(L->ple_proj, LN("proj.weight"));
            GETV(L->ple_post_norm, LN("post_norm.weight"));
        }
        if (find(t, n, LN("layer_output_scale.weight"))) { /* src/model.cpp:408-410 */
            const float* os;
            GETV(os, LN("layer_output_scale.weight"));
            L->out_scale = os[0];
        }
        if (c->arch == OR_BITNET) {
            GETV(L->attn_sub_norm, LN("attn_sub_norm.weight"));
            GETV(L->ffn_sub_norm, LN("ffn_sub_norm.weight"));
        }
        if (find(t, n, LN("attn_q.bias"))) {
            GETV(L->q_bias, LN("attn_q.bias"));
            GETV(L->k_bias, LN("attn_k.bias"));
            GETV(L->v_bias, LN("attn_v.bias"));
        }
    }
    {
        s->kcache = (uint16_t**)calloc((size_t)c->layers, sizeof(uint16_t*));
        s->vcache = (uint16_t**)calloc((size_t)c->layers, sizeof(uint16_t*));
        for (int l = 0; l < c->layers; ++l) {
            if (kv_layer_of(c, l) != l) continue;
            const size_t kvsz = kv_heads_of(c, l) * c->max_context * head_dim_of(c, l);
            s->kcache[l] = (uint16_t*)calloc(kvsz, 2);
            s->vcache[l] = (uint16_t*)calloc(kvsz, 2);
        }
        if (c->ple_dim != 0) {
            const size_t pall = (size_t)c->ple_dim * c->layers;
            s->ple = (float*)calloc(pall, 4);
            s->ple_row = (float*)calloc(pall, 4);
            s->ple_g = (float*)calloc((size_t)c->ple_dim, 4);
        }
        const size_t qd = (size_t)c->heads * c->head_dim, kvd = (size_t)c->kv_heads * c->head_dim;
        const size_t wide = (size_t)(c->embd > c->ff ? c->embd : c->ff) + qd;
        s->h = (float*)calloc(c->embd, 4);
        s->normed = (float*)calloc(c->embd, 4);
        s->q = (float*)calloc(qd, 4);
        s->k = (float*)calloc(kvd, 4);
        s->v = (float*)calloc(kvd, 4);
        s->att = (float*)calloc(qd > (size_t)c->ssm_inner ? qd : (size_t)c->ssm_inner, 4);
        if (c->arch == OR_QWEN35) {
            const size_t qkv = 2 * (size_t)c->ssm_k_heads * c->ssm_state + (size_t)c->ssm_inner;
            s->qg = (float*)calloc(2 * qd, 4);
            s->agate = (float*)calloc(qd, 4);
            s->sqkv = (float*)calloc(qkv, 4);
            s->sconv = (float*)calloc(qkv, 4);
            s->sz = (float*)calloc((size_t)c->ssm_inner, 4);
            s->sab = (float*)calloc(2 * (size_t)c->ssm_v_heads, 4);
        }
        s->proj = (float*)calloc(c->embd, 4);
        s->gate = (float*)calloc(c->ff, 4);
        s->up = (float*)calloc(c->ff, 4);
        s->scores = (float*)calloc((size_t)c->max_context, 4);
        s->rope = (float*)calloc(c->head_dim, 4);
        s->rope_local = (float*)calloc(c->head_dim, 4);
        s->conv = (float*)calloc(3 * (size_t)c->embd, 4);
        s->xq = (uint8_t*)calloc(wide / 32 * 34 + wide / 256 * 292 + 1024, 1);
    }
    return s;
bad:
    or_session_destroy(s);
    return NULL;
#undef GETM
#undef GETV
#undef LN
}

void or_session_destroy(oracle_session* s) {
    if (!s) return;
    if (s->kcache)
        for (int l = 0; l < s->c.layers; ++l) free(s->kcache[l]);  /* shared layers hold NULL */
    if (s->vcache)
        for (int l = 0; l < s->c.layers; ++l) free(s->vcache[l]);
    free(s->ple); free(s->ple_row); free(s->ple_g);
    free(s->kcache);
    free(s->vcache);
    for (int l = 0; s->layers && l < s->c.layers; ++l) {
        layer_t* L = &s->layers[l];
        free(L->conv_cache); free(L->state); free(L->ring); free(L->snap_state); free(L->snap_ring);
    }
    free(s->qg); free(s->agate); free(s->sqkv); free(s->sconv); free(s->sz); free(s->sab);
    free(s->layers);
    free(s->h); free(s->normed); free(s->q); free(s->k); free(s->v); free(s->att);
    free(s->proj); free(s->gate); free(s->up); free(s->scores); free(s->rope); free(s->rope_local); free(s->conv); free(s->xq);
    free(s);
}

size_t or_session_position(const oracle_session* s) { return s->position; }
void or_session_set_position(oracle_session* s, size_t p) { s->position = p; }
uint16_t* or_session_kv(oracle_session* s, int layer, int value) { return value ? s->vcache[layer] : s->kcache[layer]; }

/* Qwen3.5's recurrent layers back to zero (Session::reset_recurrent, src/model.cpp:729-733). */
static void reset_recurrent(oracle_session* s) {
    const oracle_config* c = &s->c;
    const size_t qkv = 2 * (size_t)c->ssm_k_heads * c->ssm_state + (size_t)c->ssm_inner;
    for (int l = 0; l < c->layers; ++l) {
        layer_t* L = &s->layers[l];
        if (!L->ssm_a) continue;
        memset(L->state, 0, (size_t)c->ssm_v_heads * c->ssm_state * c->ssm_state * 4);
        memset(L->ring, 0, (size_t)(c->ssm_conv - 1) * qkv * 4);
    }
    s->snap_valid = 0;
}

/* Session::rollback (src/model.cpp:735-752): the caches keep their rows; Qwen3.5's recurrent
 * states step back only to the snapshot before the last evaluated token, any other earlier
 * position restarts them at position 0. */
int or_session_rollback(oracle_session* s, size_t position) {
    if (position > s->position) return fail("model: cannot roll forward"); /* src/model.cpp:736 */
    if (s->c.arch == OR_QWEN35 && position != s->position) {
        const oracle_config* c = &s->c;
        const size_t qkv = 2 * (size_t)c->ssm_k_heads * c->ssm_state + (size_t)c->ssm_inner;
        if (s->snap_valid && s->snap_pos == position) {
            for (int l = 0; l < c->layers; ++l) {
                layer_t* L = &s->layers[l];
                if (!L->ssm_a) continue;
                memcpy(L->state, L->snap_state, (size_t)c->ssm_v_heads * c->ssm_state * c->ssm_state * 4);
                memcpy(L->ring, L->snap_ring, (size_t)(c->ssm_conv - 1) * qkv * 4);
            }
            s->snap_valid = 0;
        } else {
            reset_recurrent(s);
            position = 0;
        }
    }
    s->position = position;
    return 0;
}

/* Session::multiply (src/model.cpp:546-653) for one token: quantise x to the matrix's
 * activation format, then the generic matvec. */
static void multiply(oracle_session* s, const matrix* m, const float* x, float* out) {
    if (takes_q8_k(m->type)) or_quantize_q8_k(x, s->xq, m->cols, or_activation_bits(m->type, m->rows));
    else or_quantize_q8_0(x, s->xq, m->cols);
    or_matvec(m->type, m->data, m->rows, m->cols, s->xq, out);
}

/* embedding_row (src/model.cpp:27-70) */
static void embedding_row(const matrix* m, size_t r, float* out) {
    const size_t rb = m->cols / block_elems(m->type) * block_bytes(m->type);
    or_dequantize(m->type, m->data + r * rb, out, m->cols);
}

/* One token of Session::eval_batch (src/model.cpp:867-1212) at position s->position.  Every
 * computation of eval_batch is per token (matmul_generic runs the matvec dot per token,
 * attention rows only see their own visible range), so a batch equals its tokens in order. */
static void forward_token(oracle_session* s, int32_t token, float* logits) {
    const oracle_config* c = &s->c;
    const size_t embd = c->embd, hd = c->head_dim, pos = s->position, ctx = (size_t)c->max_context;
    const int neox = c->arch != OR_LLAMA && c->arch != OR_SMOLLM3; /* src/model.cpp:167 */
    const int gemma = c->arch == OR_GEMMA3 || c->arch == OR_GEMMA4;
    const size_t hd_local = c->head_dim_local != 0 ? (size_t)c->head_dim_local : hd;
    /* build_rope (src/model.cpp:880-894), attn factor 1, no factors; Gemma 3: the global
     * table at scale 1 / rope.scaling.factor, the sliding layers' at their own base, scale 1 */
    {
        const float scale = gemma && c->rope_scale != 0.0f ? c->rope_scale : 1.0f;
        const float af = c->rope_attn_factor != 0.0f ? c->rope_attn_factor : 1.0f;
        const size_t rd = c->rope_dim ? (size_t)c->rope_dim : hd;
        const float theta_scale = powf(c->rope_base, -2.0f / (float)rd);
        float theta = (float)pos * scale;
        for (size_t i = 0; i < rd / 2; ++i) {
            const float angle = s->rope_factors ? theta / s->rope_factors[i] : theta;
            s->rope[2 * i] = cosf(angle) * af;
            s->rope[2 * i + 1] = sinf(angle) * af;
            theta *= theta_scale;
        }
        if (gemma && c->sliding_window != 0) { /* the sliding layers' head size (src/model.cpp:875, :894) */
            const float ts = powf(c->rope_base_local, -2.0f / (float)hd_local);
            float th = (float)pos * 1.0f;
            for (size_t i = 0; i < hd_local / 2; ++i) {
                s->rope_local[2 * i] = cosf(th) * 1.0f;
                s->rope_local[2 * i + 1] = sinf(th) * 1.0f;
                th *= ts;
            }
        }
    }
    embedding_row(&s->embd, (size_t)token, s->h);
    if (gemma) { /* src/model.cpp:286, :899-901 */
        const float es = sqrtf((float)embd);
        for (size_t i = 0; i < embd; ++i) s->h[i] *= es;
    }
    if (c->ple_dim != 0) { /* Gemma 4's per-layer embedding inputs (src/model.cpp:905-925) */
        const size_t pd = (size_t)c->ple_dim;
        multiply(s, &s->ple_model_proj, s->h, s->ple);
        const float proj_scale = 1.0f / sqrtf((float)embd);
        const float table_scale = sqrtf((float)pd);
        embedding_row(&s->ple_tok, (size_t)token, s->ple_row);
        for (int l = 0; l < c->layers; ++l) {
            float* slice = s->ple + (size_t)l * pd;
            for (size_t i = 0; i < pd; ++i) slice[i] *= proj_scale;
            or_rms_norm(slice, s->ple_proj_norm, c->eps, slice, pd);
            for (size_t i = 0; i < pd; ++i) slice[i] = (slice[i] + s->ple_row[(size_t)l * pd + i] * table_scale) * 0.70710678f;
        }
    }

    for (int l = 0; l < c->layers; ++l) {
        const layer_t* L = &s->layers[l];
        or_rms_norm(s->h, L->attn_norm, c->eps, s->normed, embd);
        if (L->ssm_a) { /* Qwen3.5 Gated DeltaNet, Session::forward_recurrent (src/model.cpp:754-865) for one token */
            const size_t heads = (size_t)c->ssm_v_heads, dim = (size_t)c->ssm_state, taps = (size_t)c->ssm_conv;
            const size_t k_off = (size_t)c->ssm_k_heads * dim, v_off = 2 * k_off, qkv = 2 * k_off + (size_t)c->ssm_inner;
            multiply(s, &L->ssm_qkv, s->normed, s->sqkv);
            multiply(s, &L->ssm_gate, s->normed, s->sz);
            multiply(s, &L->ssm_alpha, s->normed, s->sab);
            multiply(s, &L->ssm_beta, s->normed, s->sab + heads);
            /* the causal conv over the ring's taps - 1 inputs (oldest first) and this one, then SiLU */
            for (size_t ch = 0; ch < qkv; ++ch) s->sconv[ch] = 0.0f;
            for (size_t i = 0; i < taps; ++i) {
                const float* in = i + 1 < taps ? L->ring + i * qkv : s->sqkv;
                for (size_t ch = 0; ch < qkv; ++ch) s->sconv[ch] += L->ssm_conv_w[ch * taps + i] * in[ch];
            }
            for (size_t ch = 0; ch < qkv; ++ch) s->sconv[ch] = s->sconv[ch] / (1.0f + expf(-s->sconv[ch]));
            const float q_scale = 1.0f / sqrtf((float)dim);
            for (size_t hh = 0; hh < heads; ++hh) {
                float q[256], k[256], d[256];
                const float* row = s->sconv;
                for (int which = 0; which < 2; ++which) { /* L2 norms of q (times 1/sqrt(dim)) and k */
                    const float* src = row + (which ? k_off : 0) + hh * dim;
                    float* dst = which ? k : q;
                    float sum = 0.0f;
                    for (size_t i = 0; i < dim; ++i) sum += src[i] * src[i];
                    const float inv = (which ? 1.0f : q_scale) / sqrtf(sum + c->eps);
                    for (size_t i = 0; i < dim; ++i) dst[i] = src[i] * inv;
                }
                const float* v = row + v_off + hh * dim;
                const float alpha = s->sab[hh] + L->ssm_dt[hh];
                const float softplus = alpha > 20.0f ? alpha : log1pf(expf(alpha));
                const float decay = expf(softplus * L->ssm_a[hh]);
                const float beta = 1.0f / (1.0f + expf(-s->sab[heads + hh]));
                float* S = L->state + hh * dim * dim;
                for (size_t j = 0; j < dim; ++j) {
                    float* Sj = S + j * dim;
                    float sk = 0.0f;
                    for (size_t i = 0; i < dim; ++i) {
                        Sj[i] *= decay;
                        sk += Sj[i] * k[i];
                    }
                    d[j] = (v[j] - sk) * beta;
                }
                float* o = s->att + hh * dim;
                for (size_t j = 0; j < dim; ++j) {
                    float* Sj = S + j * dim;
                    float oj = 0.0f;
                    for (size_t i = 0; i < dim; ++i) {
                        Sj[i] += k[i] * d[j];
                        oj += Sj[i] * q[i];
                    }
                    o[j] = oj;
                }
                or_rms_norm(o, L->ssm_norm, c->eps, o, dim); /* the gated norm */
                const float* z = s->sz + hh * dim;
                for (size_t j = 0; j < dim; ++j) o[j] *= z[j] / (1.0f + expf(-z[j]));
            }
            /* the ring: the last taps - 1 inputs */
            for (size_t i = 0; i + 2 < taps; ++i) memcpy(L->ring + i * qkv, L->ring + (i + 1) * qkv, qkv * 4);
            memcpy(L->ring + (taps - 2) * qkv, s->sqkv, qkv * 4);
            multiply(s, &L->ssm_out, s->att, s->proj);
            for (size_t i = 0; i < embd; ++i) s->h[i] += s->proj[i];
            goto ffn;
        }
        if (L->conv_w) { /* LFM2 short convolution (src/model.cpp:935-969) */
            const size_t taps = (size_t)c->conv_taps;
            float* bcx = s->conv;
            multiply(s, &L->conv_in, s->normed, bcx);
            for (size_t d = 0; d < embd; ++d) {
                bcx[2 * embd + d] *= bcx[d];
                L->conv_cache[pos * embd + d] = or_float_to_half(bcx[2 * embd + d]);
            }
            for (size_t d = 0; d < embd; ++d) s->att[d] = 0.0f;
            for (size_t k = 0; k < taps; ++k) {
                if (pos + k + 1 < taps) continue;
                const uint16_t* row = L->conv_cache + (pos + k + 1 - taps) * embd;
                for (size_t d = 0; d < embd; ++d) s->att[d] += L->conv_w[d * taps + k] * or_half_to_float(row[d]);
            }
            for (size_t d = 0; d < embd; ++d) s->att[d] *= bcx[embd + d];
            multiply(s, &L->conv_out, s->att, s->proj);
            for (size_t i = 0; i < embd; ++i) s->h[i] += s->proj[i];
            goto ffn;
        }
        /* the layer's head size, key/value heads and cache (Gemma 4: sliding layers' smaller heads,
         * per-layer key/value heads, later layers reading an earlier layer's cache; src/model.h:111-117) */
        const size_t hdl = head_dim_of(c, l), qdl = (size_t)c->heads * hdl, kvh = kv_heads_of(c, l), kvdl = kvh * hdl;
        const size_t hpkl = (size_t)c->heads / kvh;
        const int src = kv_layer_of(c, l), own_kv = src == l;
        const float attention_scale = c->attention_scale != 0.0f ? c->attention_scale : 1.0f / sqrtf((float)hdl);
        if (c->arch == OR_QWEN35) { /* each head's query followed by its gate (src/model.cpp:1002-1012) */
            multiply(s, &L->q, s->normed, s->qg);
            for (int h = 0; h < c->heads; ++h) {
                memcpy(s->q + h * hdl, s->qg + 2 * h * hdl, hdl * 4);
                memcpy(s->agate + h * hdl, s->qg + 2 * h * hdl + hdl, hdl * 4);
            }
        } else {
            multiply(s, &L->q, s->normed, s->q);
        }
        if (own_kv) {
            multiply(s, &L->k, s->normed, s->k);
            multiply(s, &L->v, s->normed, s->v);
        }
        /* SmolLM3: every fourth layer has no RoPE (layer_has_rope, src/model.h:110; step 4, src/model.cpp:168) */
        /* Gemma: the sliding layers (layer_slides, src/model.h:87-90) */
        const int slides = gemma && layer_slides(c, l);
        /* the rotated width (src/model.cpp:1024): none, the head, or the partial rotary dimension */
        const size_t rd_g = c->rope_dim ? (size_t)c->rope_dim : hd;
        const size_t rope_dim = (c->arch == OR_SMOLLM3 && (l + 1) % 4 == 0) ? 0 : slides ? hdl : (rd_g < hdl ? rd_g : hdl);
        const float* rope = slides ? s->rope_local : s->rope;
        if (L->q_bias) { /* add_bias (src/model.cpp:117-119, :1026-1030) */
            for (size_t i = 0; i < qdl; ++i) s->q[i] += L->q_bias[i];
            for (size_t i = 0; i < kvdl; ++i) s->k[i] += L->k_bias[i];
            for (size_t i = 0; i < kvdl; ++i) s->v[i] += L->v_bias[i];
        }
        for (int h = 0; h < c->heads; ++h) {
            float* q = s->q + h * hdl;
            if (L->q_norm) or_rms_norm(q, L->q_norm, c->eps, q, hdl);
            apply_rope(q, rope, rope_dim, neox);
        }
        if (own_kv)
            for (size_t h = 0; h < kvh; ++h) {
                float* k = s->k + h * hdl;
                float* v = s->v + h * hdl;
                if (L->k_norm) or_rms_norm(k, L->k_norm, c->eps, k, hdl);
                if (c->value_norm) or_rms_norm(v, NULL, c->eps, v, hdl); /* Gemma 4: V normalised, no weight (:1041) */
                apply_rope(k, rope, rope_dim, neox);
                uint16_t* kr = s->kcache[l] + (h * ctx + pos) * hdl;
                uint16_t* vr = s->vcache[l] + (h * ctx + pos) * hdl;
                for (size_t i = 0; i < hdl; ++i) {
                    kr[i] = or_float_to_half(k[i]);
                    vr[i] = or_float_to_half(v[i]);
                }
            }
        /* attention (src/model.cpp:1050-1093, src/kernels_f32.cpp:256-284) over the cache of layer src */
        {
            const size_t visible = pos + 1;
            /* a sliding layer sees the last sliding_window positions (src/model.cpp:1084-1085) */
            const size_t start = slides && visible > (size_t)c->sliding_window ? visible - (size_t)c->sliding_window : 0;
            const uint16_t* kc = s->kcache[src];
            const uint16_t* vc = s->vcache[src];
            float* key = s->proj; /* free until the output projection */
            for (int h = 0; h < c->heads; ++h) {
                const size_t kv = (size_t)h / hpkl;
                const float* q = s->q + h * hdl;
                for (size_t p = start; p < visible; ++p) {
                    const uint16_t* kr = kc + (kv * ctx + p) * hdl;
                    for (size_t i = 0; i < hdl; ++i) key[i] = or_half_to_float(kr[i]);
                    s->scores[p] = or_dot_f32(q, key, hdl) * attention_scale;
                }
                or_softmax(s->scores + start, visible - start);
                float* out = s->att + h * hdl;
                for (size_t i = 0; i < hdl; ++i) out[i] = 0.0f;
                for (size_t p = start; p < visible; ++p) {
                    const uint16_t* vr = vc + (kv * ctx + p) * hdl;
                    const float w = s->scores[p];
                    for (size_t i = 0; i < hdl; ++i) out[i] += w * or_half_to_float(vr[i]);
                }
            }
        }
        if (L->attn_sub_norm) or_rms_norm(s->att, L->attn_sub_norm, c->eps, s->att, qdl);
        if (c->arch == OR_QWEN35) /* the sigmoid gate (src/model.cpp:1102-1108) */
            for (size_t i = 0; i < qdl; ++i) s->att[i] *= 1.0f / (1.0f + expf(-s->agate[i]));
        multiply(s, &L->o, s->att, s->proj);
        if (L->attn_post_norm) or_rms_norm(s->proj, L->attn_post_norm, c->eps, s->proj, embd); /* :1116-1119 */
        for (size_t i = 0; i < embd; ++i) s->h[i] += s->proj[i];
    ffn:
        or_rms_norm(s->h, L->ffn_norm, c->eps, s->normed, embd);
        multiply(s, &L->gate, s->normed, s->gate);
        multiply(s, &L->up, s->normed, s->up);
        const size_t ffl = ff_of(c, l); /* Gemma 4: the layer's width (ff_dim_of, src/model.h:118) */
        for (size_t i = 0; i < ffl; ++i) { /* src/model.cpp:1128-1143, src/kernels_f32.cpp:287-289 */
            const float g = s->gate[i];
            if (c->arch == OR_BITNET) {
                const float r = g > 0.0f ? g : 0.0f;
                s->gate[i] = r * r * s->up[i];
            } else if (gemma) { /* gelu_mul_f32, src/kernels_f32.cpp:291-296 */
                s->gate[i] = 0.5f * g * (1.0f + tanhf(0.7978845608f * (g + 0.044715f * g * g * g))) * s->up[i];
            } else {
                s->gate[i] = g / (1.0f + expf(-g)) * s->up[i];
            }
        }
        if (L->ffn_sub_norm) or_rms_norm(s->gate, L->ffn_sub_norm, c->eps, s->gate, ffl);
        multiply(s, &L->down, s->gate, s->proj);
        if (L->ffn_post_norm) or_rms_norm(s->proj, L->ffn_post_norm, c->eps, s->proj, embd); /* :1156-1159 */
        for (size_t i = 0; i < embd; ++i) s->h[i] += s->proj[i];
        if (c->ple_dim != 0) { /* h = (h + norm(proj(gelu(gate h) * ple_input[l]))) * scale (src/model.cpp:1163-1177) */
            const size_t pd = (size_t)c->ple_dim;
            multiply(s, &L->ple_gate, s->h, s->ple_g);
            const float* in = s->ple + (size_t)l * pd;
            for (size_t i = 0; i < pd; ++i) {
                const float g = s->ple_g[i];
                s->ple_g[i] = 0.5f * g * (1.0f + tanhf(0.7978845608f * (g + 0.044715f * g * g * g))) * in[i];
            }
            multiply(s, &L->ple_proj, s->ple_g, s->proj);
            or_rms_norm(s->proj, L->ple_post_norm, c->eps, s->proj, embd);
            for (size_t i = 0; i < embd; ++i) s->h[i] = (s->h[i] + s->proj[i]) * L->out_scale;
        } else if (L->out_scale != 1.0f) {
            for (size_t i = 0; i < embd; ++i) s->h[i] *= L->out_scale;
        }

        if (getenv("BRISK_CPU_DEBUG") != NULL) { /* the reference's per-layer line, src/model.cpp:1183-1192 */
            double sum = 0.0;
            float peak = 0.0f;
            for (size_t i = 0; i < embd; ++i) {
                sum += fabs(s->h[i]);
                if (fabsf(s->h[i]) > peak) peak = fabsf(s->h[i]);
            }
            fprintf(stderr, "layer %d pos %zu: max|h| %.4f mean|h| %.6f  h[0..3] %.5f %.5f %.5f %.5f\n", l, pos, peak,
                    sum / (double)embd, s->h[0], s->h[1], s->h[2], s->h[3]);
        }
    }
    if (logits) {
        or_rms_norm(s->h, s->out_norm, c->eps, s->normed, embd);
        multiply(s, &s->out, s->normed, logits);
        if (gemma && c->final_softcap != 0.0f) { /* src/model.cpp:1206-1209 */
            const float cap = c->final_softcap;
            for (int i = 0; i < c->vocab; ++i) logits[i] = cap * tanhf(logits[i] / cap);
        }
    }
    s->position += 1;
}

int or_session_eval(oracle_session* s, const int32_t* tokens, size_t n, int all_logits, float* out) {
    if (n == 0) return fail("model: no tokens to evaluate");
    for (size_t i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= s->c.vocab) return fail("model: token id out of range");
    if (n > (size_t)s->c.max_context - s->position) return fail("model: context length exceeded");
    const oracle_config* c = &s->c;
    const size_t qkv = 2 * (size_t)c->ssm_k_heads * c->ssm_state + (size_t)c->ssm_inner;
    for (size_t i = 0; i < n; ++i) {
        float* row = all_logits ? out + i * (size_t)s->c.vocab : (i + 1 == n ? out : NULL);
        if (c->arch == OR_QWEN35 && i + 1 == n) { /* the snapshot before the last token (src/model.cpp:798-812) */
            for (int l = 0; l < c->layers; ++l) {
                layer_t* L = &s->layers[l];
                if (!L->ssm_a) continue;
                memcpy(L->snap_state, L->state, (size_t)c->ssm_v_heads * c->ssm_state * c->ssm_state * 4);
                memcpy(L->snap_ring, L->ring, (size_t)(c->ssm_conv - 1) * qkv * 4);
            }
            s->snap_pos = s->position;
            s->snap_valid = 1;
        }
        forward_token(s, tokens[i], row);
    }
    return 0;
}
