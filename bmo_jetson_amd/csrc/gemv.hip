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

// The activation's Q8_1 blocks in LDS: codes sq[cols], d8 sd[nblk], s8
// ss[nblk] (the fp16 values widened).  Thread t of a 512-thread workgroup
// quantizes elements 8 (t % 4) .. + 7 of block base + t / 4.
struct XPart {
    float4 u, v;
};

__device__ __forceinline__ XPart load_x_part(const GemvParams &p, int base, int nblk) {
    const int b = min(base + (int) (threadIdx.x >> 2), nblk - 1);
    const float *xb = p.x + b * 32 + 8 * (threadIdx.x & 3);
    return XPart{*reinterpret_cast<const float4 *>(xb), *reinterpret_cast<const float4 *>(xb + 4)};
}

__device__ __forceinline__ void quantize_x_part(const GemvParams &p, int base, int nblk, const XPart &xp,
                                                int8_t *sq, float *sd, float *ss) {
    const int blk = base + (int) (threadIdx.x >> 2);
    const int part = threadIdx.x & 3;
    const float x8[8] = {xp.u.x, xp.u.y, xp.u.z, xp.u.w, xp.v.x, xp.v.y, xp.v.z, xp.v.w};
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

// The activation's block pair (2 pr, 2 pr + 1): codes as dwords, d8, s8.
struct XPair {
    int q0[8], q1[8];
    float d8a, s8a, d8b, s8b;
};

__device__ __forceinline__ XPair load_x_pair(const int8_t *sq, const float *sd, const float *ss, int pr) {
    const int b0 = 2 * pr;
    const uint4 *q = reinterpret_cast<const uint4 *>(sq + b0 * 32);
    const uint4 qa = q[0], qb = q[1], qc = q[2], qd = q[3];
    return XPair{{(int) qa.x, (int) qa.y, (int) qa.z, (int) qa.w, (int) qb.x, (int) qb.y, (int) qb.z, (int) qb.w},
                 {(int) qc.x, (int) qc.y, (int) qc.z, (int) qc.w, (int) qd.x, (int) qd.y, (int) qd.z, (int) qd.w},
                 sd[b0], ss[b0], sd[b0 + 1], ss[b0 + 1]};
}

// Adds one weight block pair (36 bytes as 9 dwords: even block's fp16 scale in
// bytes 0-1 and codes in bytes 2-17, odd block's scale in bytes 18-19 and
// codes in bytes 20-35) times the activation pair: each block contributes
// d4 * (sumi * d8 - 8 * s8), sumi from 8 v_dot4_i32_i8 on the exact codes.
__device__ __forceinline__ void pair_acc(float &acc, const uint32_t (&w)[9], const XPair &x) {
    const uint32_t ca[4] = {__builtin_amdgcn_alignbyte(w[1], w[0], 2), __builtin_amdgcn_alignbyte(w[2], w[1], 2),
                            __builtin_amdgcn_alignbyte(w[3], w[2], 2), __builtin_amdgcn_alignbyte(w[4], w[3], 2)};
    int sa = 0, sb = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        sa = __builtin_amdgcn_sdot4((int) (ca[k] & 0x0F0F0F0Fu), x.q0[k], sa, false);
        sa = __builtin_amdgcn_sdot4((int) ((ca[k] >> 4) & 0x0F0F0F0Fu), x.q0[4 + k], sa, false);
        sb = __builtin_amdgcn_sdot4((int) (w[5 + k] & 0x0F0F0F0Fu), x.q1[k], sb, false);
        sb = __builtin_amdgcn_sdot4((int) ((w[5 + k] >> 4) & 0x0F0F0F0Fu), x.q1[4 + k], sb, false);
    }
    const float d4a = f16_to_f32(w[0] & 0xFFFFu);
    const float d4b = f16_to_f32(w[4] >> 16);
    acc += d4a * ((float) sa * x.d8a - 8.0f * x.s8a);
    acc += d4b * ((float) sb * x.d8b - 8.0f * x.s8b);
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
        const XPart xp = load_x_part(p, base, nblk);
        if (base == 0) {
#pragma unroll
            for (int j = 0; j < PFD; ++j) load_next(wb[j]);
        }
        quantize_x_part(p, base, nblk, xp, sq, sd, ss);
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
            const XPair xq = load_x_pair(sq, sd, ss, pr);
#pragma unroll
            for (int r = 0; r < R; ++r) pair_acc(acc[r], wcur[r], xq);
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

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Streaming variant for rows whose byte length is a multiple of 16 (cols a
// multiple of 256, at most 6144).  A wave owns up to NPOS chunks of two
// consecutive rows (c0, c0 + stride, ...), at most NPC KiB of contiguous
// bytes each (4608 bytes at 4096 columns).  Lane l loads the chunk's 16-byte
// pieces j * 1024 + 16 l with nontemporal loads (every byte is loaded once,
// by one lane), the wave copies the chunk into its own LDS area and each
// lane reads its block pair from there.  One chunk is in flight at a time:
// the next chunk's loads go out as soon as the current chunk has arrived,
// before it is multiplied, and the outputs are stored after the last chunk,
// so that no store enters a wait.  (Against gemv_kernel at cols = 4096:
// more bytes in flight per wave, two chunks or all of them, were measured
// slower, as were smaller chunks or more workgroups.)
constexpr int kStreamMaxPos = 4;  // chunks per wave

__host__ __device__ constexpr size_t gemv_stream_stage_offset(int cols) {
    return ((size_t) cols + (size_t) (cols / 32) * 8 + 15) / 16 * 16;
}

// NPC: 1024-byte pieces of a two-row chunk; NIT: block pairs per lane and
// row (64 * NIT >= the row's pairs).
template <int NPOS, int NPC, int NIT>
__global__ __launch_bounds__(512) void gemv_stream_kernel(GemvParams p) {
    constexpr int NT = 512;
    constexpr int R = 2;
    extern __shared__ __align__(16) uint8_t smem[];
    const int nblk = p.cols / 32;
    const int npairs = nblk / 2;
    int8_t *sq = reinterpret_cast<int8_t *>(smem);
    float *sd = reinterpret_cast<float *>(smem + p.cols);
    float *ss = sd + nblk;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    uint8_t *stage = smem + gemv_stream_stage_offset(p.cols) + wave * (NPC * 1024);
    const int row_bytes = nblk * 18;
    const int chunk_bytes = R * row_bytes;
    const int64_t mat_bytes = (int64_t) p.rows * row_bytes;
    const int n_chunks = (p.rows + R - 1) / R;
    const int stride = gridDim.x * (NT / 64);
    const int c0 = blockIdx.x * (NT / 64) + wave;
    const int n_mine = c0 < n_chunks ? min(NPOS, (n_chunks - 1 - c0) / stride + 1) : 0;

    // chunk k's pieces, unconditionally (so that the waits before the
    // quantization count loads exactly): pieces past the chunk (or the
    // matrix) re-read its last 16 bytes and land in the stage past the bytes
    // that are read (rows are a multiple of 16 bytes), and a wave without
    // chunks reads the last chunk
    auto issue = [&](int k, u32x4_t (&w)[NPC]) {
        const int64_t cbase = (int64_t) min(c0 + k * stride, n_chunks - 1) * chunk_bytes;
        const int64_t last = min(cbase + chunk_bytes, mat_bytes) - 16;
#pragma unroll
        for (int j = 0; j < NPC; ++j)
            w[j] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4_t *>(p.w + min(cbase + j * 1024 + 16 * lane, last)));
    };
    // the activation's loads go out first (loads return in order; one pass
    // of NT / 4 blocks per pair a lane holds), then the first chunk's, and
    // the quantization runs while the chunk is in flight
    XPart xp[NIT];
#pragma unroll
    for (int i = 0; i < NIT; ++i) xp[i] = load_x_part(p, i * (NT / 4), nblk);
    __builtin_amdgcn_sched_barrier(0);
    u32x4_t wr[2][NPC];
    issue(0, wr[0]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NIT; ++i)
        if (i * (NT / 4) < nblk) quantize_x_part(p, i * (NT / 4), nblk, xp[i], sq, sd, ss);
    __syncthreads();
    if (n_mine == 0) return;

    // this lane's activation pairs, the same for every chunk
    XPair xq[NIT];
#pragma unroll
    for (int i = 0; i < NIT; ++i) xq[i] = load_x_pair(sq, sd, ss, min(lane + 64 * i, npairs - 1));
    float yv[NPOS][R];
#pragma unroll
    for (int k = 0; k < NPOS; ++k) {
        if (k < n_mine) {  // (wave-uniform)
            // chunk k is the only one in flight: once it has arrived, the
            // next goes out (the wait precedes the branch, so that no path
            // leaves chunk k's registers pending)
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            __builtin_amdgcn_sched_barrier(0);
            if (k + 1 < n_mine) issue(k + 1, wr[(k + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < NPC; ++j)
                *reinterpret_cast<u32x4_t *>(stage + j * 1024 + 16 * lane) = wr[k & 1][j];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float acc = 0.0f;
#pragma unroll
                for (int i = 0; i < NIT; ++i) {
                    const int pr = lane + 64 * i;
                    if (pr < npairs) {
                        const uint32_t *src = reinterpret_cast<const uint32_t *>(stage + r * row_bytes + 36 * pr);
                        uint32_t w[9];
#pragma unroll
                        for (int e = 0; e < 9; ++e) w[e] = src[e];
                        pair_acc(acc, w, xq[i]);
                    }
                }
                yv[k][r] = wave_sum(acc);
            }
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < NPOS; ++k) {
            const int c = c0 + k * stride;
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (k < n_mine && c * R + r < p.rows) p.y[c * R + r] = yv[k][r];
        }
    }
}

template <int NPC, int NIT>
void launch_stream(const GemvParams &p, int npos, int n_chunks, hipStream_t stream) {
    const int wgs = (n_chunks + 8 * npos - 1) / (8 * npos);
    const size_t lds = gemv_stream_stage_offset(p.cols) + (size_t) 8 * NPC * 1024;
    const dim3 grid((unsigned) wgs), block(512);
    if (npos == 1)
        hipLaunchKernelGGL((gemv_stream_kernel<1, NPC, NIT>), grid, block, lds, stream, p);
    else if (npos == 2)
        hipLaunchKernelGGL((gemv_stream_kernel<2, NPC, NIT>), grid, block, lds, stream, p);
    else if (npos == 3)
        hipLaunchKernelGGL((gemv_stream_kernel<3, NPC, NIT>), grid, block, lds, stream, p);
    else
        hipLaunchKernelGGL((gemv_stream_kernel<4, NPC, NIT>), grid, block, lds, stream, p);
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
    // Rows of at most 6144 columns whose byte length is a multiple of 16
    // (cols a multiple of 256, so that every piece inside a chunk is loaded
    // at its own offset), a 16-byte aligned matrix, and up to kStreamMaxPos
    // two-row chunks per wave of 256 workgroups: the streaming kernel
    // (BMO_GEMV_STREAM=0 turns it off, for comparison).  Chunks of up to
    // 4608 bytes take 5 pieces, up to 6912 bytes 7 (56 KB of stages).
    const int n_chunks = (p.rows + 1) / 2;
    const int npos = (n_chunks + 256 * 8 - 1) / (256 * 8);
    const char *se = std::getenv("BMO_GEMV_STREAM");
    if (p.cols <= 6144 && p.cols % 256 == 0 && (reinterpret_cast<uintptr_t>(p.w) & 15) == 0 &&
        npos <= kStreamMaxPos && !(se && se[0] == '0')) {
        if (p.cols <= 4096)
            launch_stream<5, 1>(p, npos, n_chunks, stream);
        else
            launch_stream<7, 2>(p, npos, n_chunks, stream);
        return true;
    }
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
