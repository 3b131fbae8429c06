/*
 * q4_0_ref.c -- fp16 conversion and Q4_0 block quantization, restated.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Compiled with -ffp-contract=off so
 * that every multiply and add below rounds on its own, as the C source of
 * ggml's reference quantizer is written.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

/* IEEE-754 binary32 -> binary16, round to nearest, ties to even, with
 * gradual underflow.  This is what GGML_FP32_TO_FP16 computes on an F16C
 * host (_cvtss_sh(x, 0)) and what the reference's eager KV write uses
 * (src/bmo_compute.cpp:885-886). */
uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t bexp = (x >> 23) & 0xFFu;
    uint32_t mant = x & 0x7FFFFFu;

    if (bexp == 0xFFu) {
        if (mant == 0) return (uint16_t)(sign | 0x7C00u);        /* +-inf */
        return (uint16_t)(sign | 0x7E00u | (mant >> 13));         /* quiet NaN */
    }
    if (bexp == 0) {
        /* fp32 zero or subnormal: magnitude < 2^-126, far below half of the
         * smallest fp16 subnormal (2^-25), so it rounds to a signed zero. */
        return (uint16_t) sign;
    }
    const int32_t e = (int32_t) bexp - 127 + 15; /* biased fp16 exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);               /* overflow */
    if (e <= 0) {
        /* fp16 subnormal: value = M * 2^(E+1) in units of 2^-24, with
         * M = 1.mant as a 24-bit integer and E = e - 15, so the code is
         * M >> (14 - e) rounded to nearest even. */
        const int shift = 14 - e;
        if (shift > 24) return (uint16_t) sign; /* below 2^-25: rounds to 0 */
        const uint32_t m = mant | 0x800000u;
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) r += 1u;
        return (uint16_t)(sign | r); /* r == 0x400 is the smallest normal */
    }
    uint32_t h = ((uint32_t) e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* may carry to inf */
    return (uint16_t)(sign | h);
}

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t) h & 0x8000u) << 16;
    const uint32_t bexp = ((uint32_t) h >> 10) & 0x1Fu;
    const uint32_t mant = (uint32_t) h & 0x3FFu;
    uint32_t x;
    if (bexp == 0x1Fu) {
        x = sign | 0x7F800000u | (mant << 13);
    } else if (bexp == 0) {
        if (mant == 0) {
            x = sign;
        } else {
            /* subnormal: mant * 2^-24, exactly representable in fp32 */
            float v = (float) mant * 5.9604644775390625e-08f; /* 2^-24 */
            memcpy(&x, &v, sizeof x);
            x |= sign;
        }
    } else {
        x = sign | ((bexp - 15u + 127u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &x, sizeof f);
    return f;
}

/* ggml quantize_row_q4_0_ref, restated step by step per 32-element block:
 *   (a) signed value of largest magnitude, first occurrence on ties
 *       (strict "<" against a running |max| that starts at +0.0f);
 *   (b) d = max / -8, id = d != 0 ? 1/d : 0 (fp32, correctly rounded);
 *   (c) the stored scale is fp16(d), round to nearest even;
 *   (d) code = min(15, (int8_t)(x*id + 8.5f)) with the product and the sum
 *       rounded separately and truncation toward zero;
 *   (e) qs[j] = code[j] | code[j+16] << 4.
 * The codes use the fp32 id, not the fp16-rounded scale.  Inputs must be
 * finite (ggml's cast is undefined for NaN). */
void orc_quantize_row_q4_0(const float *x, orc_block_q4_0 *y, int64_t k) {
    const int64_t nb = k / ORC_QK4_0;
    for (int64_t i = 0; i < nb; ++i) {
        const float *xb = x + i * ORC_QK4_0;
        float amax = 0.0f;
        float vmax = 0.0f;
        for (int j = 0; j < ORC_QK4_0; ++j) {
            const float a = fabsf(xb[j]);
            if (amax < a) {
                amax = a;
                vmax = xb[j];
            }
        }
        const float d = vmax / -8.0f;
        const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
        y[i].d = orc_fp32_to_fp16(d);
        for (int j = 0; j < ORC_QK4_0 / 2; ++j) {
            const float p0 = xb[j] * id;
            const float p1 = xb[j + ORC_QK4_0 / 2] * id;
            const float s0 = p0 + 8.5f;
            const float s1 = p1 + 8.5f;
            int c0 = (int) (int8_t) s0;
            int c1 = (int) (int8_t) s1;
            if (c0 > 15) c0 = 15;
            if (c1 > 15) c1 = 15;
            y[i].qs[j] = (uint8_t)((unsigned) c0 | ((unsigned) c1 << 4));
        }
    }
}

/* Element j of a block is (code_j - 8) * fp32(d). */
void orc_dequantize_row_q4_0(const orc_block_q4_0 *x, float *y, int64_t k) {
    const int64_t nb = k / ORC_QK4_0;
    for (int64_t i = 0; i < nb; ++i) {
        const float d = orc_fp16_to_fp32(x[i].d);
        for (int j = 0; j < ORC_QK4_0 / 2; ++j) {
            const int c0 = (int) (x[i].qs[j] & 0x0F) - 8;
            const int c1 = (int) (x[i].qs[j] >> 4) - 8;
            y[i * ORC_QK4_0 + j] = (float) c0 * d;
            y[i * ORC_QK4_0 + j + ORC_QK4_0 / 2] = (float) c1 * d;
        }
    }
}

float orc_round_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, sizeof u);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) {
        u |= 0x00400000u;
        u &= 0xFFFF0000u;
    } else {
        const uint32_t lsb = (u >> 16) & 1u;
        u += 0x7FFFu + lsb;
        u &= 0xFFFF0000u;
    }
    float r;
    memcpy(&r, &u, sizeof r);
    return r;
}
