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

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t) __builtin_amdgcn_mov_dpp((int) v, CTRL, 0xF, 0xF, true);
}

// Reductions over an aligned group of BL = 8 or 16 lanes of one 16-lane row:
// lane ^ 1 and lane ^ 2 (quad_perm), then the mirrored quad of the half-row
// (row_half_mirror) and, for 16, the mirrored half-row (row_mirror).  Every
// lane of the group must be active.
template <int BL>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0xB1>(v));
    v = max(v, dpp_u32<0x4E>(v));
    v = max(v, dpp_u32<0x141>(v));
    if constexpr (BL == 16) v = max(v, dpp_u32<0x140>(v));
    return v;
}
template <int BL>
__device__ __forceinline__ uint32_t group_min_u32(uint32_t v) {
    v = min(v, dpp_u32<0xB1>(v));
    v = min(v, dpp_u32<0x4E>(v));
    v = min(v, dpp_u32<0x141>(v));
    if constexpr (BL == 16) v = min(v, dpp_u32<0x140>(v));
    return v;
}

// Lane-parallel quantization of one block spread over BL = 8 or 16
// consecutive lanes (the group starts at a multiple of BL): lane i of the
// group holds E = 32 / BL elements, x[t] = element i*E/2 + t and
// x[E/2 + t] = element i*E/2 + t + 16 (t < E/2), so its codes fill E/2 whole
// bytes of the block.  Bit-identical to quantize_block_q4_0_literal for every
// input:
//   M = the largest |x_j| over non-NaN elements, 0 if there is none (from the
//   fp32 bit patterns, which order non-negative values as unsigned integers);
//   vmax = the first x_j with |x_j| == M, +0 when M == 0: the literal form's
//   scan "if (amax < |x_j|)" from amax = +0 keeps exactly that element (a NaN
//   never compares greater, a tie never replaces an earlier element), and
//   its sign comes from a group minimum over keys 2 j + sign;
//   d, id and each code as the literal form computes them.
// Returns code dword i*E/8 of the block (bytes 4c..4c+3), assembled in every
// lane that contributes to it, and the fp16 scale bits in d16.
template <int BL>
__device__ __forceinline__ uint32_t quantize_block_q4_0_lanes(const float (&x)[32 / BL], int i,
                                                              uint16_t &d16) {
#pragma clang fp contract(off)
    constexpr int E = 32 / BL, HE = E / 2;
    uint32_t a[E];
    uint32_t m = 0;
#pragma unroll
    for (int t = 0; t < E; ++t) {
        const uint32_t ab = __builtin_bit_cast(uint32_t, x[t]) & 0x7FFFFFFFu;
        a[t] = ab > 0x7F800000u ? 0u : ab;  // a NaN counts as 0
        m = max(m, a[t]);
    }
    const uint32_t M = group_max_u32<BL>(m);
    uint32_t key = 0xFFFFFFFFu;
#pragma unroll
    for (int t = 0; t < E; ++t) {
        const uint32_t j = (uint32_t) (i * HE + (t < HE ? t : t - HE + 16));
        const uint32_t k = (j << 1) | (__builtin_bit_cast(uint32_t, x[t]) >> 31);
        key = a[t] == M ? min(key, k) : key;
    }
    const uint32_t K = group_min_u32<BL>(key);
    const float vmax = M == 0u ? 0.0f : __builtin_bit_cast(float, M | (K << 31));
    float d = vmax / -8.0f;
    asm volatile("" : "+v"(d));  // materialize d in fp32 (see the header note)
    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    d16 = f32_to_f16_bits(d);
    uint32_t w = 0;
#pragma unroll
    for (int t = 0; t < HE; ++t) {
        int c0 = x86_trunc_to_i8(x[t] * id + 8.5f);
        int c1 = x86_trunc_to_i8(x[t + HE] * id + 8.5f);
        c0 = c0 > 15 ? 15 : c0;
        c1 = c1 > 15 ? 15 : c1;
        const uint32_t byte = ((uint32_t) c0 | ((uint32_t) c1 << 4)) & 0xFFu;
        w |= byte << (8 * ((i * HE + t) & 3));
    }
    // the 4 / HE lanes of one dword are adjacent
    w |= dpp_u32<0xB1>(w);
    if constexpr (HE == 1) w |= dpp_u32<0x4E>(w);
    return w;
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
