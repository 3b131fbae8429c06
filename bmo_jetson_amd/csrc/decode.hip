// decode.hip -- sliding-window decode attention over the Q4_0 ring.
//
// Semantics follow the reference kernel bmo_decode_attention_kernel
// (src/bmo_cuda_kernels.cu:713-848) and its CPU twin
// (src/bmo_compute.cpp:927-970): for query head h at absolute position p the
// keys are the min(p+1, n_ctx) most recent positions of kv head
// h / (n_heads / n_kv_heads); scores are (q . k) * scale, softmax with max
// subtraction, output sum_i p_i v_i.  The window's slots are always slots
// [0, window) of the ring (while the ring fills the window starts at
// position 0, afterwards it is the whole ring), and softmax does not depend on
// key order, so keys are visited in slot order.
//
// Work decomposition (gfx950, wave64): one workgroup of NW waves per (batch
// entry, query head).  Lane (kk, blk) of a wave owns block blk of key kk of
// an iteration: LPK = head_dim/32 lanes per key, KPI = 64/LPK keys per wave
// iteration.  One 128-bit load per lane fetches a whole block's 16 code bytes,
// so each wave load instruction reads KPI consecutive key rows (1 KiB) of the
// nibble plane; scales come from the fp16 scale plane as one coalesced 2-byte
// load per lane.  Waves take iterations round-robin, TIT iterations per tile;
// the loads of the next PF tiles are in flight while a tile is computed.  Loads
// are unconditional (slots clamped into the ring); keys outside the window
// (and, fused, the slot being written) get score -inf and weight 0 by select,
// so stale bytes never reach the sums.
//
// K side (q . k), two forms:
//   KDOT8: the lane's 32 query values are turned once into 20-bit fixed point,
//     U_e = round(q_e / sq) + 2^19, held as five nibble planes laid out like
//     the code dwords; v_dot8_u32_u4 then multiplies 8 codes by 8 query
//     nibbles per instruction:  sum_e c_e U_e = sum_i 16^i sum_e c_e u_ei,
//     and sum_e (c_e - 8) q_e = sq (sum_e c_e U_e - 2^19 sum_e c_e - 8 sum_e Q_e).
//     Quantizing q costs at most sq/2 = max|q| / (2^20 - 2) per element.
//   fma-mix: masking a code dword with 0x000F000F (0x00F000F0) leaves two
//     fp16 subnormals equal to c * 2^-24 (c * 2^-20); v_fma_mix_f32 reads them
//     next to the fp32 query pre-scaled by 2^24 (2^20):
//     sum_e (c_e - 8) d q_e = d (sum_e c_e q_e - 8 sum_e q_e).
// V side: the same fma-mix form accumulates sum_i (p_i d_i) c_ie, and
// 8 sum_i p_i d_i is subtracted at the end.  q is pre-multiplied by
// scale * log2(e) so the softmax uses exp2.
//
// Each lane keeps a running (max, sum, acc[32]) over its keys (online softmax,
// rescaled only when some lane's max rose); at the end every lane is brought
// to the wave max, the lanes of each 16-lane row that share a block are summed
// by DPP rotations, the row sums go to LDS, and the first head_dim threads
// merge waves and rows.
//
// Fused append (the reference's write-then-attend,
// src/bmo_cuda_kernels.cu:749-754): the current token's K/V rows are quantized
// in registers with the bit-exact quantizer, wave 0 attends to that key from
// registers, and the first query head of each kv group stores the blocks to
// slot pos % n_ctx.  Every workgroup masks that slot out of its ring reads.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <type_traits>

#include "kernels.hpp"
#include "q4_0_device.hpp"

namespace bmo {

namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr float kTwo24 = 16777216.0f;
constexpr float kTwo20 = 1048576.0f;
constexpr int kQFix = 524287;  // 2^19 - 1: largest |Q| of the fixed-point query

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF,
                                                               0xF, true));
}

// Sum over the LPK lanes of one key (lanes 4k..4k+3, or 2k..2k+1).
template <int LPK>
__device__ __forceinline__ float key_sum(float v) {
    v += dpp<0xB1>(v);                          // quad_perm [1,0,3,2]: lane ^ 1
    if constexpr (LPK == 4) v += dpp<0x4E>(v);  // quad_perm [2,3,0,1]: lane ^ 2
    return v;
}

// Sum over the lanes of a 16-lane row that own the same block (lane % LPK).
template <int LPK>
__device__ __forceinline__ float row_block_sum(float v) {
    if constexpr (LPK == 2) v += dpp<0x122>(v);  // row_ror:2
    v += dpp<0x124>(v);                          // row_ror:4
    v += dpp<0x128>(v);                          // row_ror:8
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Element of the block held by nibble k (0..7, from bit 0) of code dword c:
// dword c holds code bytes 4c..4c+3, byte j has element j in its low and
// element j+16 in its high nibble.
__host__ __device__ constexpr int nibble_element(int c, int k) { return 4 * c + (k >> 1) + 16 * (k & 1); }

// Element read by operand slot s (0..7) of code dword c in the fma-mix
// operand order (A.x, A.y, B.x, B.y, C.x, C.y, D.x, D.y) with
// A = w & 0x000F000F, B = w & 0x00F000F0, C = (w >> 8) & 0x000F000F,
// D = (w >> 8) & 0x00F000F0.
__host__ __device__ constexpr int mix_slot_element(int c, int s) {
    return 4 * c + ((s >> 2) & 1) + 2 * (s & 1) + 16 * ((s >> 1) & 1);
}

// K-side scorer over fp32 queries: sum_e (c_e - 8) q_e of one block, before
// the block scale.
struct MixScorer {
    float qm[32];  // query in fma-mix operand order, scaled by 2^24 / 2^20
    float qsum;

    __device__ __forceinline__ void init(const float (&qe)[32]) {
        qsum = 0.0f;
#pragma unroll
        for (int e = 0; e < 32; ++e) qsum += qe[e];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const int e = mix_slot_element(c, s);
                qm[8 * c + s] = qe[e] * ((e >= 16) ? kTwo20 : kTwo24);
            }
    }
    __device__ __forceinline__ float operator()(const uint4 &w4) const {
        const uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t w8 = w[c] >> 8;
            const half2_t A = __builtin_bit_cast(half2_t, w[c] & 0x000F000Fu);
            const half2_t B = __builtin_bit_cast(half2_t, w[c] & 0x00F000F0u);
            const half2_t C = __builtin_bit_cast(half2_t, w8 & 0x000F000Fu);
            const half2_t D = __builtin_bit_cast(half2_t, w8 & 0x00F000F0u);
            a0 = __builtin_fmaf((float) A.x, qm[8 * c + 0], a0);
            a1 = __builtin_fmaf((float) A.y, qm[8 * c + 1], a1);
            a0 = __builtin_fmaf((float) B.x, qm[8 * c + 2], a0);
            a1 = __builtin_fmaf((float) B.y, qm[8 * c + 3], a1);
            a0 = __builtin_fmaf((float) C.x, qm[8 * c + 4], a0);
            a1 = __builtin_fmaf((float) C.y, qm[8 * c + 5], a1);
            a0 = __builtin_fmaf((float) D.x, qm[8 * c + 6], a0);
            a1 = __builtin_fmaf((float) D.y, qm[8 * c + 7], a1);
        }
        return (a0 + a1) - 8.0f * qsum;
    }
};

// K-side scorer over the 20-bit fixed-point query (v_dot8_u32_u4).
struct Dot8Scorer {
    uint32_t dig[5][4];  // nibble plane i of U, laid out like code dword c
    int bias;            // 8 * sum_e Q_e
    float sq;            // fixed-point step of the query

    __device__ __forceinline__ void init(const float (&qe)[32]) {
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 32; ++e) amax = fmaxf(amax, __builtin_fabsf(qe[e]));
        const float inv = amax > 0.0f ? (float) kQFix / amax : 0.0f;
        sq = amax * (1.0f / (float) kQFix);
        int qs = 0;
        uint32_t u[32];
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            int Q = (int) __builtin_rintf(qe[e] * inv);
            Q = min(max(Q, -kQFix), kQFix);
            qs += Q;
            u[e] = (uint32_t) (Q + kQFix + 1);
        }
        bias = 8 * qs;
#pragma unroll
        for (int i = 0; i < 5; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                uint32_t d = 0;
#pragma unroll
                for (int k = 0; k < 8; ++k) d |= ((u[nibble_element(c, k)] >> (4 * i)) & 15u) << (4 * k);
                dig[i][c] = d;
            }
    }
    __device__ __forceinline__ float operator()(const uint4 &w4) const {
        const uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
        uint32_t S[5];
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            uint32_t a = __builtin_amdgcn_udot8(w[0], dig[i][0], 0u, false);
            a = __builtin_amdgcn_udot8(w[1], dig[i][1], a, false);
            a = __builtin_amdgcn_udot8(w[2], dig[i][2], a, false);
            S[i] = __builtin_amdgcn_udot8(w[3], dig[i][3], a, false);
        }
        uint32_t n = __builtin_amdgcn_udot8(w[0], 0x11111111u, 0u, false);
        n = __builtin_amdgcn_udot8(w[1], 0x11111111u, n, false);
        n = __builtin_amdgcn_udot8(w[2], 0x11111111u, n, false);
        n = __builtin_amdgcn_udot8(w[3], 0x11111111u, n, false);
        // sum_e c_e U_e - 2^19 sum_e c_e - 8 sum_e Q_e, exact in 32-bit integers
        const uint32_t t = S[0] + (S[1] << 4) + (S[2] << 8) + (S[3] << 12) + (S[4] << 16);
        const int T = (int) (t - (n << 19)) - bias;
        return (float) T * sq;
    }
};

// acc[e] += pd * c_e for the 32 elements of one block (acc in element order).
__device__ __forceinline__ void block_axpy(const uint4 &w4, float pd, float (&acc)[32]) {
    const uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
    const float pl = pd * kTwo24;
    const float ph = pd * kTwo20;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t w8 = w[c] >> 8;
        const half2_t A = __builtin_bit_cast(half2_t, w[c] & 0x000F000Fu);
        const half2_t B = __builtin_bit_cast(half2_t, w[c] & 0x00F000F0u);
        const half2_t C = __builtin_bit_cast(half2_t, w8 & 0x000F000Fu);
        const half2_t D = __builtin_bit_cast(half2_t, w8 & 0x00F000F0u);
        acc[4 * c + 0] = __builtin_fmaf((float) A.x, pl, acc[4 * c + 0]);
        acc[4 * c + 2] = __builtin_fmaf((float) A.y, pl, acc[4 * c + 2]);
        acc[4 * c + 16] = __builtin_fmaf((float) B.x, ph, acc[4 * c + 16]);
        acc[4 * c + 18] = __builtin_fmaf((float) B.y, ph, acc[4 * c + 18]);
        acc[4 * c + 1] = __builtin_fmaf((float) C.x, pl, acc[4 * c + 1]);
        acc[4 * c + 3] = __builtin_fmaf((float) C.y, pl, acc[4 * c + 3]);
        acc[4 * c + 17] = __builtin_fmaf((float) D.x, ph, acc[4 * c + 17]);
        acc[4 * c + 19] = __builtin_fmaf((float) D.y, ph, acc[4 * c + 19]);
    }
}

}  // namespace

template <int D, int NW, int TIT, int PF, bool KDOT8, bool FUSED>
__global__ __launch_bounds__(64 * NW) void decode_kernel(DecodeParams p) {
    constexpr int LPK = D / kQK;   // lanes (blocks) per key row
    constexpr int KPI = 64 / LPK;  // keys per wave iteration
    constexpr int ROWS = 4;        // 16-lane rows per wave
    using Scorer = typename std::conditional<KDOT8, Dot8Scorer, MixScorer>::type;

    __shared__ float s_acc[NW * ROWS * D];
    __shared__ float s_m[NW];
    __shared__ float s_l[NW];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int kk = lane / LPK;
    const int blk = lane % LPK;

    const int unit = blockIdx.x;
    const int b = unit / p.n_heads;
    const int h = unit - b * p.n_heads;

    const RingGeom &g = p.g;
    const int sid = p.session_ids ? p.session_ids[b] : b;
    const int pos = p.pos ? p.pos[b] : p.pos_scalar;
    float *out_row = p.out + (int64_t) unit * D;
    if (sid < 0 || sid >= g.n_sessions || pos < 0) {
        for (int i = threadIdx.x; i < D; i += blockDim.x) out_row[i] = 0.0f;
        return;
    }
    const int q_per_kv = p.n_heads / p.n_kv;
    const int kvh = h / q_per_kv;
    const int n_ctx = g.n_ctx;
    const int window = (int) min((int64_t) pos + 1, (int64_t) n_ctx);
    const int cur = pos % n_ctx;

    const int64_t soff = g.stripe_offset(p.layer, sid, kvh);
    const uint8_t *knib = p.k_base + soff;
    const uint8_t *vnib = p.v_base + soff;
    const uint8_t *kscl = knib + g.nib_bytes;
    const uint8_t *vscl = vnib + g.nib_bytes;

    // Tiles: wave w visits the global iterations (t*TIT + i)*NW + w,
    // t = 0, 1, ...; a tile is TIT such iterations.  NB tiles are resident: the
    // loads of the next NB-1 tiles are in flight while one is computed.  The
    // first tiles' loads are issued before the query preparation so that it
    // overlaps their latency.
    constexpr int NB = PF + 1;
    const int n_iter = (window + KPI - 1) / KPI;
    const int n_tiles = (n_iter - wave + NW * TIT - 1) / (NW * TIT);
    const int last_slot = n_ctx - 1;
    struct Tile {
        uint4 kq[TIT], vq[TIT];
        uint32_t ksc[TIT], vsc[TIT];
    };
    auto slot_of = [&](int t, int i) { return ((t * TIT + i) * NW + wave) * KPI + kk; };
    auto slot_ok = [&](int slot) {
        bool ok = slot < window;
        if constexpr (FUSED) ok = ok && slot != cur;
        return ok;
    };
    auto load_tile = [&](int t, Tile &T) {
#pragma unroll
        for (int i = 0; i < TIT; ++i) {
            const uint32_t slot = (uint32_t) min(slot_of(t, i), last_slot);
            const uint32_t on = slot * (uint32_t) (D / 2) + (uint32_t) blk * 16u;
            const uint32_t os = (slot * (uint32_t) LPK + (uint32_t) blk) * 2u;
            T.kq[i] = *reinterpret_cast<const uint4 *>(knib + on);
            T.vq[i] = *reinterpret_cast<const uint4 *>(vnib + on);
            T.ksc[i] = *reinterpret_cast<const uint16_t *>(kscl + os);
            T.vsc[i] = *reinterpret_cast<const uint16_t *>(vscl + os);
        }
    };
    Tile buf[NB];
#pragma unroll
    for (int j = 0; j < NB - 1; ++j)
        if (j < n_tiles) load_tile(j, buf[j]);

    Scorer score;
    {
        const float4 *q4 = reinterpret_cast<const float4 *>(p.q + (int64_t) unit * D + blk * kQK);
        float qe[32];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float4 t = q4[c];
            qe[4 * c + 0] = t.x * p.qscale;
            qe[4 * c + 1] = t.y * p.qscale;
            qe[4 * c + 2] = t.z * p.qscale;
            qe[4 * c + 3] = t.w * p.qscale;
        }
        score.init(qe);
    }

    float m = -INFINITY;  // running max of this lane's keys (log2 domain)
    float l = 0.0f;       // running sum of this lane's keys (each key counted LPK times)
    float csum = 0.0f;    // sum of p*d over this lane's keys
    float acc[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) acc[e] = 0.0f;

    if constexpr (FUSED) {
        if (wave == 0) {
            // The current token's K and V blocks: lanes 0..LPK-1 (kk == 0) own
            // block blk of the kv head's new rows.
            float s_new = 0.0f;
            uint4 vq_new = make_uint4(0, 0, 0, 0);
            float vd_new = 0.0f;
            if (kk == 0) {
                const int64_t row = ((int64_t) b * p.n_kv + kvh) * D + blk * kQK;
                float x[kQK];
                uint16_t kd16, vd16;
                uint32_t kqs[4], vqs[4];
                load_block_f32(p.k_new + row, x);
                quantize_block_q4_0(x, kd16, kqs);
                load_block_f32(p.v_new + row, x);
                quantize_block_q4_0(x, vd16, vqs);
                vq_new = make_uint4(vqs[0], vqs[1], vqs[2], vqs[3]);
                s_new = f16_bits_to_f32(kd16) * score(make_uint4(kqs[0], kqs[1], kqs[2], kqs[3]));
                vd_new = f16_bits_to_f32(vd16);
                if (h % q_per_kv == 0) {
                    store_block(p.k_wbase + soff, g, cur, blk, kd16, kqs);
                    store_block(p.v_wbase + soff, g, cur, blk, vd16, vqs);
                }
            }
            s_new = key_sum<LPK>(s_new);
            if (kk == 0) {
                m = s_new;
                l = 1.0f;  // exp2(s_new - m)
                csum = vd_new;
                block_axpy(vq_new, vd_new, acc);
            }
        }
    }

    auto compute_tile = [&](int t, const Tile &T) {
        float s[TIT];
        float tmax = m;
#pragma unroll
        for (int i = 0; i < TIT; ++i) {
            const float sk = key_sum<LPK>(f16_bits_to_f32(T.ksc[i]) * score(T.kq[i]));
            s[i] = slot_ok(slot_of(t, i)) ? sk : -INFINITY;
            tmax = fmaxf(tmax, s[i]);
        }
        if (__any(tmax > m)) {
            float alpha = 1.0f;
            if (tmax > m) alpha = (m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - tmax);
            m = tmax;
            l *= alpha;
            csum *= alpha;
#pragma unroll
            for (int e = 0; e < 32; ++e) acc[e] *= alpha;
        }
#pragma unroll
        for (int i = 0; i < TIT; ++i) {
            const bool ok = s[i] != -INFINITY;
            const float pk = ok ? __builtin_amdgcn_exp2f(s[i] - m) : 0.0f;
            l += pk;
            const float pd = ok ? pk * f16_bits_to_f32(T.vsc[i]) : 0.0f;
            csum += pd;
            block_axpy(T.vq[i], pd, acc);
        }
    };
    for (int t = 0; t < n_tiles; t += NB) {
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int tt = t + u;
            if (tt < n_tiles) {
                if (tt + NB - 1 < n_tiles) load_tile(tt + NB - 1, buf[(u + NB - 1) % NB]);
                compute_tile(tt, buf[u]);
            }
        }
    }

    // Bring every lane to the wave max, fold the -8 code offset, sum the lanes
    // of each row that share a block, and publish the row sums.
    const float m_wave = wave_max(m);
    {
        const float f = (m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - m_wave);
        l *= f;
        csum *= f;
#pragma unroll
        for (int e = 0; e < 32; ++e) acc[e] *= f;
    }
    const float l_wave = wave_sum(l) * (1.0f / LPK);
#pragma unroll
    for (int e = 0; e < 32; ++e) acc[e] = row_block_sum<LPK>(__builtin_fmaf(-8.0f, csum, acc[e]));
    const int row = lane >> 4;
    if ((lane & 15) < LPK) {
        float4 *dst = reinterpret_cast<float4 *>(s_acc + (wave * ROWS + row) * D + blk * kQK);
#pragma unroll
        for (int c = 0; c < 8; ++c)
            dst[c] = make_float4(acc[4 * c], acc[4 * c + 1], acc[4 * c + 2], acc[4 * c + 3]);
    }
    if (lane == 0) {
        s_m[wave] = m_wave;
        s_l[wave] = l_wave;
    }
    __syncthreads();

    // Merge waves and rows; a workgroup may have fewer threads than head_dim.
    float M = s_m[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, s_m[w]);
    float fw[NW];
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        fw[w] = (s_m[w] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(s_m[w] - M);
        L = __builtin_fmaf(fw[w], s_l[w], L);
    }
    const float inv_l = (L > 0.0f) ? 1.0f / L : 0.0f;
    for (int o = threadIdx.x; o < D; o += 64 * NW) {
        float acc_o = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            float r = 0.0f;
#pragma unroll
            for (int rr = 0; rr < ROWS; ++rr) r += s_acc[(w * ROWS + rr) * D + o];
            acc_o = __builtin_fmaf(fw[w], r, acc_o);
        }
        out_row[o] = acc_o * inv_l;
    }
}

namespace {

template <int D, int NW, int TIT, int PF, bool KDOT8>
void launch_variant(const DecodeParams &p, bool fused, hipStream_t stream) {
    const dim3 grid((unsigned) ((int64_t) p.n_batch * p.n_heads)), block(64 * NW);
    if (fused)
        hipLaunchKernelGGL((decode_kernel<D, NW, TIT, PF, KDOT8, true>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((decode_kernel<D, NW, TIT, PF, KDOT8, false>), grid, block, 0, stream, p);
}

struct Shape {
    int nw, tit, pf, kdot8;
};

// Workgroup shape per call.  Few (entry, head) units: 4 waves per unit so the
// window streams with enough loads in flight, fp32 queries (no per-wave query
// preparation on the latency path).  Many units: one wave per unit walking the
// whole window with double-buffered tiles and the fixed-point K scorer, whose
// one-time preparation is spread over the window.  BMO_ATTN_SHAPE =
// "nw,tit,pf,kdot8" overrides the choice (tuning; unknown shapes fall back).
Shape pick_shape(int64_t units) {
    Shape s = units < 512 ? Shape{4, 4, 0, 0} : Shape{1, 4, 1, 1};
    if (const char *e = std::getenv("BMO_ATTN_SHAPE")) {
        Shape o{0, 0, 0, 0};
        if (std::sscanf(e, "%d,%d,%d,%d", &o.nw, &o.tit, &o.pf, &o.kdot8) == 4) s = o;
    }
    return s;
}

template <int D>
bool launch_shape(const DecodeParams &p, bool fused, hipStream_t stream, const Shape &s) {
#define BMO_SHAPE(NW_, TIT_, PF_, K8_)                                   \
    if (s.nw == NW_ && s.tit == TIT_ && s.pf == PF_ && s.kdot8 == K8_) { \
        launch_variant<D, NW_, TIT_, PF_, K8_>(p, fused, stream);        \
        return true;                                                     \
    }
    BMO_SHAPE(4, 4, 0, 0)
    BMO_SHAPE(4, 2, 1, 0)
    BMO_SHAPE(4, 4, 1, 0)
    BMO_SHAPE(1, 4, 1, 1)
    BMO_SHAPE(1, 4, 2, 1)
    BMO_SHAPE(1, 2, 2, 1)
    BMO_SHAPE(1, 2, 3, 1)
    BMO_SHAPE(1, 8, 1, 1)
    BMO_SHAPE(2, 4, 1, 1)
    BMO_SHAPE(2, 2, 2, 1)
#undef BMO_SHAPE
    return false;
}

}  // namespace

bool launch_decode(const DecodeParams &p, bool fused, hipStream_t stream) {
    const int64_t units = (int64_t) p.n_batch * p.n_heads;
    if (units <= 0) return true;
    const Shape s = pick_shape(units);
    if (p.g.head_dim == 128) {
        if (!launch_shape<128>(p, fused, stream, s))
            launch_variant<128, 4, 4, 0, false>(p, fused, stream);
    } else if (p.g.head_dim == 64) {
        if (!launch_shape<64>(p, fused, stream, s)) launch_variant<64, 4, 4, 0, false>(p, fused, stream);
    } else {
        return false;
    }
    return true;
}

}  // namespace bmo
