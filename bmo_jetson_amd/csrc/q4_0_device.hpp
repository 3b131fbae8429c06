// q4_0_device.hpp -- device-side Q4_0 block quantization, bit-exact with
// ggml quantize_row_q4_0_ref as compiled for x86-64.
//
// Exactness rests on properties of this build (checked in the ISA and by the
// parity tests): fp32 division is correctly rounded (hipcc emits the
// div_scale/div_fmas/div_fixup sequence), fp32 and fp16 denormals are kept
// (float_denorm_mode 3), the fp32->fp16 conversion rounds to nearest even,
// and no multiply-add below is contracted into an FMA (the library is built
// with -ffp-contract=off; kernels ask for FMAs explicitly with fmaf).  The
// scale d is also pinned in a register before its fp16 conversion: otherwise
// the backend folds fp16(m * -0.125) into a mixed-precision FMA with a +0
// addend, which turns the -0.0 scale of an all-zero block into +0.0.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ring_layout.hpp"

namespace bmo {

__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
    const _Float16 h = (_Float16) x;
    return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    return (float) __builtin_bit_cast(_Float16, (uint16_t) bits);
}

// (int8_t)s as an x86-64 compiler evaluates it: a truncating 32-bit
// conversion that yields 0x80000000 for NaN or out-of-range values, whose low
// byte is then kept.  Only scales whose reciprocal overflows
// (|max| < ~2^-125) reach the out-of-range branch.
__device__ __forceinline__ int x86_trunc_to_i8(float s) {
    const int i = (__builtin_fabsf(s) < 2147483648.0f) ? (int) s : (int) 0x80000000;
    return (int) (int8_t) (i & 0xFF);
}

// Quantizes one 32-element block (ggml quantize_row_q4_0_ref steps):
//   signed value of largest magnitude, first occurrence, running |max| from
//   +0.0f; d = max / -8; id = d ? 1/d : 0; scale stored as fp16(d);
//   code = min(15, (int8_t)(x*id + 8.5f)) with separately rounded multiply
//   and add.  d16 receives the fp16 scale bits and qs[c] bytes 4c..4c+3 of
//   the block (byte j = code j | code j+16 << 4).  This is the literal form,
//   exact for every input (NaN, infinities, scales whose reciprocal
//   overflows).
__device__ __forceinline__ void quantize_block_q4_0_literal(const float (&x)[kQK], uint16_t &d16,
                                                            uint32_t (&qs)[4]) {
#pragma clang fp contract(off)
    float amax = 0.0f;
    float vmax = 0.0f;
#pragma unroll
    for (int j = 0; j < kQK; ++j) {
        const float a = __builtin_fabsf(x[j]);
        if (amax < a) {
            amax = a;
            vmax = x[j];
        }
    }
    float d = vmax / -8.0f;
    asm volatile("" : "+v"(d));  // materialize d in fp32 (see the header note)
    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    d16 = f32_to_f16_bits(d);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = 4 * c + i;
            const float p0 = x[j] * id;
            const float p1 = x[j + 16] * id;
            int c0 = x86_trunc_to_i8(p0 + 8.5f);
            int c1 = x86_trunc_to_i8(p1 + 8.5f);
            c0 = c0 > 15 ? 15 : c0;
            c1 = c1 > 15 ? 15 : c1;
            const uint32_t byte = ((uint32_t) c0 | ((uint32_t) c1 << 4)) & 0xFFu;
            w |= byte << (8 * i);
        }
        qs[c] = w;
    }
}

// The same function, with a short path for the common block: the largest
// magnitude comes from NaN-propagating max/min trees (v_maximum3/v_minimum3),
// and the sign of the first value of that magnitude is the sign of whichever
// extreme reaches it (a scan settles blocks holding both +max and -max).
// With no NaN, no infinity and |max| >= 2^-124 (so 1/d is finite and
// |x*id| <= 8 up to rounding) or |max| == 0, x*id + 8.5f lies in [0, 17):
// the truncation is the plain conversion and only the clamp to 15 remains.
// Other blocks take the literal form.
__device__ __forceinline__ void quantize_block_q4_0(const float (&x)[kQK], uint16_t &d16,
                                                    uint32_t (&qs)[4]) {
#pragma clang fp contract(off)
    float hi = x[0], lo = x[0];
#pragma unroll
    for (int j = 1; j < kQK; ++j) {
        hi = __builtin_elementwise_maximum(hi, x[j]);
        lo = __builtin_elementwise_minimum(lo, x[j]);
    }
    const float amax = __builtin_elementwise_maximum(hi, -lo);  // NaN if any x is NaN
    if (!(amax <= 3.40282347e38f && (amax >= 0x1p-124f || amax == 0.0f))) {
        quantize_block_q4_0_literal(x, d16, qs);
        return;
    }
    float vmax;
    if (hi == amax && lo == -amax && amax != 0.0f) {
        // both signs reach |max|: the first occurrence decides
        vmax = 0.0f;
#pragma unroll
        for (int j = kQK - 1; j >= 0; --j) vmax = __builtin_fabsf(x[j]) == amax ? x[j] : vmax;
    } else {
        vmax = hi == amax ? amax : -amax;
    }
    vmax = amax == 0.0f ? 0.0f : vmax;  // an all-zero block keeps the initial +0
    float d = vmax / -8.0f;
    asm volatile("" : "+v"(d));  // materialize d in fp32 (see the header note)
    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    d16 = f32_to_f16_bits(d);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = 4 * c + i;
            int c0 = (int) (x[j] * id + 8.5f);
            int c1 = (int) (x[j + 16] * id + 8.5f);
            c0 = c0 > 15 ? 15 : c0;
            c1 = c1 > 15 ? 15 : c1;
            w |= ((uint32_t) c0 | ((uint32_t) c1 << 4)) << (8 * i);
        }
        qs[c] = w;
    }
}

// Loads one block's 32 fp32 elements (16-byte aligned source).
__device__ __forceinline__ void load_block_f32(const float *__restrict__ src, float (&x)[kQK]) {
    const float4 *s4 = reinterpret_cast<const float4 *>(src);
#pragma unroll
    for (int c = 0; c < kQK / 4; ++c) {
        const float4 t = s4[c];
        x[4 * c + 0] = t.x;
        x[4 * c + 1] = t.y;
        x[4 * c + 2] = t.z;
        x[4 * c + 3] = t.w;
    }
}

// Stores a quantized block of K (which == 0) or V (which == 1) at slot
// `slot`, block `blk` of a ring stripe (layout in ring_layout.hpp: K codes
// are stored as code ^ 8, the scale goes to its half of the slot's scale
// dword).
__device__ __forceinline__ void store_block(uint8_t *__restrict__ stripe, const RingGeom &g,
                                            int slot, int blk, int which, uint16_t d16,
                                            const uint32_t (&qs)[4]) {
    const uint32_t flip = which == 0 ? 0x88888888u : 0u;
    uint4 *codes = reinterpret_cast<uint4 *>(
        stripe + (which == 0 ? g.kcode_offset(slot, blk) : g.vcode_offset(slot, blk)));
    *codes = make_uint4(qs[0] ^ flip, qs[1] ^ flip, qs[2] ^ flip, qs[3] ^ flip);
    uint16_t *sc = reinterpret_cast<uint16_t *>(stripe + g.scale_offset(slot, blk)) + which;
    *sc = d16;
}

}  // namespace bmo
