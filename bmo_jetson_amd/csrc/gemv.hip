// gemv.hip -- Q4_0 weight matrix times an fp32 activation row, the reference's
// launch_gemv_q4_0_q8_1 (src/bmo_cuda_kernels.cu:529-711), reading ggml's
// 18-byte AoS block_q4_0 rows in place.
//
// Semantics (kept from the reference): the activation row is quantized to
// Q8_1 per 32 elements (d = amax/127, q = clamp(roundf(x/d)), s = fp16 of the
// sequential fp32 sum of the x values); every weight block contributes
// d4 * (sumi * d8 - 8 * s8) with sumi the exact integer dot product of its
// unsigned codes with q.
//
// One kernel, no scratch: every workgroup quantizes the activation row into
// LDS itself (bit-exact with the reference's quantizer: four lanes per block
// share the max through DPP, codes are elementwise, and one lane forms the
// sequential sum), while the first weight loads of its rows are in flight.
// A wave owns R consecutive rows; lane l reads block pairs (2p, 2p+1),
// p = l, l+64, ..., as 36 contiguous dword-aligned bytes (an even number of
// blocks per row keeps every pair dword-aligned), and forms each block's
// integer dot product with 8 v_dot4_i32_i8 against the LDS copy of q.
#include <math.h>
#include <stdlib.h>

#include <algorithm>

#include "kernels.hpp"

namespace bmo {

namespace {

template <int CTRL>
__device__ __forceinline__ float gdpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF,
                                                               0xF, true));
}

// Sum over the 64 lanes, result in every lane.
__device__ __forceinline__ float wave_sum(float v) {
    v += gdpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += gdpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += gdpp<0x124>(v);  // row_ror:4
    v += gdpp<0x128>(v);  // row_ror:8
    const int iv = __builtin_bit_cast(int, v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
}

// C roundf: nearest integer, halves away from zero (|p| < 2^23).
__device__ __forceinline__ int round_half_away(float p) {
    const float t = __builtin_truncf(p);
    const float r = __builtin_fabsf(p - t) >= 0.5f ? t + __builtin_copysignf(1.0f, p) : t;
    return (int) r;
}

__device__ __forceinline__ float f16_to_f32(uint32_t bits) {
    return (float) __builtin_bit_cast(_Float16, (uint16_t) bits);
}

__device__ __forceinline__ uint32_t f32_to_f16(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16) x);
}

}  // namespace

template <int R, int PFD, bool PAD>
__global__ __launch_bounds__(512) void gemv_kernel(GemvParams p) {
    constexpr int NT = 512;
    constexpr int NB = PFD + 1;  // weight buffers: PFD iterations in flight
    extern __shared__ __align__(16) uint8_t smem[];
    const int nblk = p.cols / 32;
    const int npairs = nblk / 2;
    int8_t *sq = reinterpret_cast<int8_t *>(smem);                  // [cols] codes of x
    float *sd = reinterpret_cast<float *>(smem + p.cols);           // [nblk] d8
    float *ss = sd + nblk;                                          // [nblk] s8

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t row_bytes = (int64_t) nblk * 18;
    // Work of a wave: chunks of R consecutive rows, c = wave id, + stride,
    // ..., each in n_it pair-iterations, n_pos (chunk, iteration) positions
    // in all; the loads of the next PFD positions are in flight while the
    // current one is multiplied.
    const int n_it = (npairs + 63) / 64;
    const int n_chunks = (p.rows + R - 1) / R;
    const int stride = gridDim.x * (NT / 64);
    const int c0 = blockIdx.x * (NT / 64) + wave;
    const int n_pos = (c0 < n_chunks ? (n_chunks - 1 - c0) / stride + 1 : 0) * n_it;

    // This lane's block pair of iteration it of chunk c (clamped to the
    // matrix: loads past the end read its last pair and are never used).
    auto load_pairs = [&](int c, int it, uint32_t (&w)[R][9]) {
        const int pr = min(it * 64 + lane, npairs - 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(c * R + r, p.rows - 1);
            const uint32_t *src = reinterpret_cast<const uint32_t *>(p.w + row * row_bytes + pr * 36);
            const uint4 a = *reinterpret_cast<const uint4 *>(src);
            const uint4 b = *reinterpret_cast<const uint4 *>(src + 4);
            w[r][0] = a.x; w[r][1] = a.y; w[r][2] = a.z; w[r][3] = a.w;
            w[r][4] = b.x; w[r][5] = b.y; w[r][6] = b.z; w[r][7] = b.w;
            w[r][8] = src[8];
        }
    };
    // load head: the next position to fetch.  Past the wave's end it
    // re-reads the wave's own last position (every position issues the same
    // loads, so the waits stay exact, and the extra reads hit lines this
    // wave has just read rather than one line all waves would share).
    const int c_last = n_pos > 0 ? c0 + (n_pos / n_it - 1) * stride : n_chunks - 1;
    int lc = c0, lit = 0;
    auto load_next = [&](uint32_t (&w)[R][9]) {
        const bool past = lc > c_last;
        load_pairs(past ? c_last : lc, past ? n_it - 1 : lit, w);
        if (++lit == n_it) {
            lit = 0;
            lc += stride;
        }
    };
    uint32_t wb[NB][R][9];

    // Activation row -> Q8_1 in LDS.  Thread t: block t/4 (+128 k), elements
    // 8 (t%4) .. 8 (t%4) + 7.  The first pass's x loads go out before the
    // weight loads: loads return in order, so the quantization then overlaps
    // the weights' flight instead of waiting for it.
    for (int base = 0; base < nblk; base += NT / 4) {
        const int blk = base + (int) (threadIdx.x >> 2);
        const int part = threadIdx.x & 3;
        const int b = min(blk, nblk - 1);
        const float *xb = p.x + b * 32;
        const float4 u = *reinterpret_cast<const float4 *>(xb + 8 * part);
        const float4 v = *reinterpret_cast<const float4 *>(xb + 8 * part + 4);
        if (base == 0) {
#pragma unroll
            for (int j = 0; j < PFD; ++j) load_next(wb[j]);
        }
        const float x8[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, __builtin_fabsf(x8[j]));
        amax = fmaxf(amax, gdpp<0xB1>(amax));
        amax = fmaxf(amax, gdpp<0x4E>(amax));
        const float d = amax / 127.0f;
        const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
        uint32_t qw[2] = {0u, 0u};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int q = min(max(round_half_away(x8[j] * id), -128), 127);
            qw[j >> 2] |= ((uint32_t) q & 0xFFu) << (8 * (j & 3));
        }
        // the reference's sequential fp32 sum of the block's 32 values, in
        // lane part 0, which reads its quad-mates' values through DPP
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) sum += x8[j];
#pragma unroll
        for (int j = 0; j < 8; ++j) sum += gdpp<0x55>(x8[j]);  // quad_perm [1,1,1,1]
#pragma unroll
        for (int j = 0; j < 8; ++j) sum += gdpp<0xAA>(x8[j]);  // quad_perm [2,2,2,2]
#pragma unroll
        for (int j = 0; j < 8; ++j) sum += gdpp<0xFF>(x8[j]);  // quad_perm [3,3,3,3]
        if (blk < nblk) {
            *reinterpret_cast<uint2 *>(sq + blk * 32 + 8 * part) = make_uint2(qw[0], qw[1]);
            const uint32_t d16 = f32_to_f16(d), s16 = f32_to_f16(sum);
            if (part == 0) {
                sd[blk] = f16_to_f32(d16);
                ss[blk] = f16_to_f32(s16);
            }
            if (p.q8_out && blockIdx.x == 0) {
                // the reference's scratch: block_q8_1 {half2 ds; int8 qs[32]}
                uint32_t *dst = reinterpret_cast<uint32_t *>(p.q8_out + (int64_t) blk * 36);
                if (part == 0) dst[0] = d16 | (s16 << 16);
                dst[1 + 2 * part] = qw[0];
                dst[2 + 2 * part] = qw[1];
            }
        }
    }
    __syncthreads();

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    // compute tail: position k is (chunk c, iteration it)
    int c = c0, it = 0;
    auto multiply = [&](const uint32_t (&wcur)[R][9]) {
        const int pr = it * 64 + lane;
        if (pr < npairs) {
            const int b0 = 2 * pr;
            const uint4 *q0 = reinterpret_cast<const uint4 *>(sq + b0 * 32);
            const uint4 qa = q0[0], qb = q0[1], qc = q0[2], qd = q0[3];
            const int qv0[8] = {(int) qa.x, (int) qa.y, (int) qa.z, (int) qa.w,
                                (int) qb.x, (int) qb.y, (int) qb.z, (int) qb.w};
            const int qv1[8] = {(int) qc.x, (int) qc.y, (int) qc.z, (int) qc.w,
                                (int) qd.x, (int) qd.y, (int) qd.z, (int) qd.w};
            const float d8a = sd[b0], s8a = ss[b0], d8b = sd[b0 + 1], s8b = ss[b0 + 1];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t *w = wcur[r];
                // even block: scale in bytes 0-1, codes in bytes 2-17
                const uint32_t ca[4] = {__builtin_amdgcn_alignbyte(w[1], w[0], 2),
                                        __builtin_amdgcn_alignbyte(w[2], w[1], 2),
                                        __builtin_amdgcn_alignbyte(w[3], w[2], 2),
                                        __builtin_amdgcn_alignbyte(w[4], w[3], 2)};
                // odd block: scale in bytes 18-19, codes in bytes 20-35
                const uint32_t cb[4] = {w[5], w[6], w[7], w[8]};
                int sa = 0, sb = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    sa = __builtin_amdgcn_sdot4((int) (ca[k] & 0x0F0F0F0Fu), qv0[k], sa, false);
                    sa = __builtin_amdgcn_sdot4((int) ((ca[k] >> 4) & 0x0F0F0F0Fu), qv0[4 + k], sa, false);
                    sb = __builtin_amdgcn_sdot4((int) (cb[k] & 0x0F0F0F0Fu), qv1[k], sb, false);
                    sb = __builtin_amdgcn_sdot4((int) ((cb[k] >> 4) & 0x0F0F0F0Fu), qv1[4 + k], sb, false);
                }
                const float d4a = f16_to_f32(w[0] & 0xFFFFu);
                const float d4b = f16_to_f32(w[4] >> 16);
                acc[r] += d4a * ((float) sa * d8a - 8.0f * s8a);
                acc[r] += d4b * ((float) sb * d8b - 8.0f * s8b);
            }
        }
        if (it == n_it - 1) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float y = wave_sum(acc[r]);
                if (lane == 0 && c * R + r < p.rows) p.y[c * R + r] = y;
                acc[r] = 0.0f;
            }
        }
        if (++it == n_it) {
            it = 0;
            c += stride;
        }
    };
    // Buffer of position k: k % NB.  Each step refills the buffer freed by
    // the step before with position k + PFD, then multiplies position k.
    // Steady state: unconditional loads, so each multiply waits for its own
    // position's loads only.  The last 2 NB - 2 positions: with PAD, loads
    // stay unconditional (past the wave's last position they re-read it);
    // without, they go out only while positions remain, so the wave issues
    // no loads past its last position (they would hold it until they
    // return), at the price of a conservative wait: a multiply that follows
    // a conditional load waits for that load as well.  Measured: rows of one
    // 64-pair iteration (cols <= 4096) without, longer rows with.
    int k = 0;
    for (; k + 2 * NB - 2 < n_pos; k += NB) {
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            load_next(wb[(u + PFD) % NB]);
            multiply(wb[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < 2 * NB - 2; ++u) {
        const int kk = k + u;
        if constexpr (PAD) {
            load_next(wb[(u + PFD) % NB]);
            if (kk < n_pos) multiply(wb[u % NB]);
        } else if (kk < n_pos) {
            if (kk + PFD < n_pos) load_next(wb[(u + PFD) % NB]);
            multiply(wb[u % NB]);
        }
    }
}

size_t gemv_lds_bytes(int cols) { return (size_t) cols + (size_t) (cols / 32) * 8; }

namespace {

// At most one workgroup per CU (256 CUs, measured best for 4096..12288
// rows); each wave then walks several row chunks, so the activation's
// quantization is paid once per workgroup.  BMO_GEMV_WGS overrides the cap.
template <int R>
void launch_rows(const GemvParams &p, hipStream_t stream) {
    const int rows_per_wg = 8 * R;
    int wgs = (p.rows + rows_per_wg - 1) / rows_per_wg;
    int cap = 256;
    if (const char *e = std::getenv("BMO_GEMV_WGS")) cap = std::max(1, std::atoi(e));
    wgs = std::min(wgs, cap);
    // One position in flight beside the one being multiplied: 2, 3 and 4
    // were measured slower at every shape (QKV 8.06 / 9.57 / 9.85 us against
    // 7.62; out-proj 5.29 / 6.43 / 7.23 against 4.50).
    if (p.cols > 4096)
        hipLaunchKernelGGL((gemv_kernel<R, 1, true>), dim3((unsigned) wgs), dim3(512), gemv_lds_bytes(p.cols),
                           stream, p);
    else
        hipLaunchKernelGGL((gemv_kernel<R, 1, false>), dim3((unsigned) wgs), dim3(512), gemv_lds_bytes(p.cols),
                           stream, p);
}

}  // namespace

bool launch_gemv(const GemvParams &p, hipStream_t stream) {
    // Rows per wave chunk (2 measured best on MI355X for 4096..12288 rows);
    // BMO_GEMV_ROWS = 1 | 2 | 4 overrides (tuning).
    int r = 2;
    if (const char *e = std::getenv("BMO_GEMV_ROWS")) r = std::atoi(e);
    if (r == 4)
        launch_rows<4>(p, stream);
    else if (r == 2)
        launch_rows<2>(p, stream);
    else
        launch_rows<1>(p, stream);
    return true;
}

}  // namespace bmo
