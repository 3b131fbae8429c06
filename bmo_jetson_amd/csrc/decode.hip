// decode.hip -- sliding-window decode attention over the Q4_0 ring.
//
// Semantics follow the reference kernel bmo_decode_attention_kernel
// (src/bmo_cuda_kernels.cu:713-848) and its CPU twin
// (src/bmo_compute.cpp:927-970): for query head h at absolute position p the
// keys are the min(p+1, n_ctx) most recent positions of kv head
// h / (n_heads / n_kv_heads); scores are (q . k) * scale, softmax with max
// subtraction, output sum_i p_i v_i.  The window's slots are always slots
// [0, window) of the ring (when the ring is not yet full the window starts at
// position 0, otherwise it is the whole ring), and softmax is invariant to
// key order, so keys are visited in slot order.
//
// Work decomposition (gfx950, wave64):
//   workgroup = 4 waves = one (batch entry, query head, window split);
//   lane (kk, blk) of a wave owns block blk of key kk of the current
//   iteration, LPK = head_dim/32 lanes per key, KPI = 64/LPK keys per wave
//   iteration; one 128-bit load per lane fetches a whole block's 16 code
//   bytes, so each wave load instruction reads KPI consecutive key rows
//   (1 KiB) of the nibble plane; scales come from the fp16 scale plane as
//   one coalesced 2-byte load per lane.
// The dequantized dot product is folded:  sum_j (c_j - 8) d q_j
//   = d * (sum_j c_j q_j - 8 sum_j q_j), with q pre-multiplied by
// scale*log2(e) so the softmax uses exp2.  P.V accumulates
// sum_i (p_i d_i) c_ij and subtracts 8 sum_i p_i d_i at the end.
//
// Each wave keeps a running (max, sum, acc[32]) over its keys (online
// softmax across tiles), the four waves merge through LDS, and when the
// window is split over several workgroups the partial (max, sum, acc[D]) go
// to a workspace and the last workgroup of the unit (atomic counter) merges
// them and resets the counter.
//
// Fused append (the reference's write-then-attend, :749-754): split 0 of the
// unit quantizes the current token's K/V rows in registers with the
// bit-exact quantizer, wave 0 attends to that key from registers, the first
// query head of each kv group stores the blocks to slot pos % n_ctx, and
// every workgroup skips that slot when reading the ring, so no workgroup
// reads a slot another one is writing.
#include <math.h>

#include "kernels.hpp"
#include "q4_0_device.hpp"

namespace bmo {

namespace {

constexpr int kWaves = 4;

__device__ __forceinline__ float dpp_swap1(float v) {  // lane ^ 1 within a quad
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF,
                                                               0xF, true));
}
__device__ __forceinline__ float dpp_swap2(float v) {  // lane ^ 2 within a quad
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF,
                                                               0xF, true));
}

template <int LPK>
__device__ __forceinline__ float key_sum(float v) {
    v += dpp_swap1(v);
    if constexpr (LPK == 4) v += dpp_swap2(v);
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

// sum_j c_j q_j over one block held as four code dwords; ql/qh are the
// query values of the low / high nibble elements (elements 4c+i / 16+4c+i).
__device__ __forceinline__ float block_dot(const uint4 &w4, const float (&ql)[16],
                                           const float (&qh)[16]) {
    const uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t lo = w[c] & 0x0F0F0F0Fu;
        const uint32_t hi = (w[c] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc = fmaf((float) ((lo >> (8 * i)) & 0xFFu), ql[4 * c + i], acc);
            acc = fmaf((float) ((hi >> (8 * i)) & 0xFFu), qh[4 * c + i], acc);
        }
    }
    return acc;
}

// acc[e] += pd * c_e for the 32 elements of one block (acc in element order).
__device__ __forceinline__ void block_axpy(const uint4 &w4, float pd, float (&acc)[32]) {
    const uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t lo = w[c] & 0x0F0F0F0Fu;
        const uint32_t hi = (w[c] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[4 * c + i] = fmaf(pd, (float) ((lo >> (8 * i)) & 0xFFu), acc[4 * c + i]);
            acc[16 + 4 * c + i] = fmaf(pd, (float) ((hi >> (8 * i)) & 0xFFu), acc[16 + 4 * c + i]);
        }
    }
}

}  // namespace

template <int D, bool FUSED>
__global__ __launch_bounds__(64 * kWaves) void decode_kernel(DecodeParams p) {
    constexpr int LPK = D / kQK;     // lanes (blocks) per key row
    constexpr int KPI = 64 / LPK;    // keys per wave iteration
    constexpr int TIT = 8;           // iterations per tile (per wave)
    constexpr int LSTRIDE = 36;      // LDS floats per lane chunk (32 + pad)

    __shared__ float s_acc[kWaves * 64 * LSTRIDE];
    __shared__ float s_m[kWaves];
    __shared__ float s_l[kWaves];
    __shared__ float s_part[256];
    __shared__ int s_last;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int kk = lane / LPK;
    const int blk = lane % LPK;

    // Workgroup i is dispatched to XCD i % 8; give consecutive logical ids
    // (the splits of one unit) the same XCD so a split merge stays in one L2.
    int lid = blockIdx.x;
    const int G = gridDim.x;
    if ((G & 7) == 0) lid = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
    const int unit = lid / p.n_split;
    const int split = lid - unit * p.n_split;
    const int b = unit / p.n_heads;
    const int h = unit - b * p.n_heads;

    const RingGeom &g = p.g;
    const int sid = p.session_ids ? p.session_ids[b] : b;
    const int pos = p.pos ? p.pos[b] : p.pos_scalar;
    float *out_row = p.out + (int64_t) unit * D;
    if (sid < 0 || sid >= g.n_sessions || pos < 0) {
        if (split == 0)
            for (int i = threadIdx.x; i < D; i += blockDim.x) out_row[i] = 0.0f;
        return;
    }
    const int q_per_kv = p.n_heads / p.n_kv;
    const int kvh = h / q_per_kv;
    const int n_ctx = g.n_ctx;
    const int window = (int) min((int64_t) pos + 1, (int64_t) n_ctx);
    const int cur = pos % n_ctx;

    // This workgroup's slot range [lo, hi).
    int chunk = (window + p.n_split - 1) / p.n_split;
    chunk = (chunk + KPI - 1) / KPI * KPI;
    const int lo = min(split * chunk, window);
    const int hi = min(lo + chunk, window);

    const int64_t soff = g.stripe_offset(p.layer, sid, kvh);
    const uint8_t *knib = p.k_base + soff;
    const uint8_t *vnib = p.v_base + soff;
    const uint16_t *kscl = reinterpret_cast<const uint16_t *>(knib + g.nib_bytes);
    const uint16_t *vscl = reinterpret_cast<const uint16_t *>(vnib + g.nib_bytes);

    // Query values of this lane's block, scaled for exp2.
    float ql[16], qh[16];
    float qsum = 0.0f;
    {
        const float4 *q4 = reinterpret_cast<const float4 *>(p.q + (int64_t) unit * D + blk * kQK);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float4 a = q4[c];
            const float4 bq = q4[4 + c];
            ql[4 * c + 0] = a.x * p.qscale;
            ql[4 * c + 1] = a.y * p.qscale;
            ql[4 * c + 2] = a.z * p.qscale;
            ql[4 * c + 3] = a.w * p.qscale;
            qh[4 * c + 0] = bq.x * p.qscale;
            qh[4 * c + 1] = bq.y * p.qscale;
            qh[4 * c + 2] = bq.z * p.qscale;
            qh[4 * c + 3] = bq.w * p.qscale;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) qsum += ql[j] + qh[j];
    }

    float m = -INFINITY;  // wave-uniform running max (log2 domain)
    float l = 0.0f;       // lane-local running sum (each key counted LPK times)
    float csum = 0.0f;    // sum of p*d over this lane's keys
    float acc[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) acc[j] = 0.0f;

    if constexpr (FUSED) {
        if (split == 0 && wave == 0) {
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
                const uint4 kq4 = make_uint4(kqs[0], kqs[1], kqs[2], kqs[3]);
                vq_new = make_uint4(vqs[0], vqs[1], vqs[2], vqs[3]);
                s_new = f16_bits_to_f32(kd16) * (block_dot(kq4, ql, qh) - 8.0f * qsum);
                vd_new = f16_bits_to_f32(vd16);
                if (h % q_per_kv == 0) {
                    uint8_t *kw = p.k_wbase + soff;
                    uint8_t *vw = p.v_wbase + soff;
                    store_block(kw, g, cur, blk, kd16, kqs);
                    store_block(vw, g, cur, blk, vd16, vqs);
                }
            }
            s_new = key_sum<LPK>(s_new);
            s_new = __shfl(s_new, 0);
            m = s_new;
            if (kk == 0) {
                l = 1.0f;  // exp2(s_new - m)
                csum = vd_new;
                block_axpy(vq_new, vd_new, acc);
            }
        }
    }

    // Main loop: wave w visits global iterations (t*TIT + i)*kWaves + w.
    const int n_iter = (hi - lo + KPI - 1) / KPI;
    for (int t0 = 0; t0 * kWaves < n_iter; t0 += TIT) {
        uint4 kq[TIT], vq[TIT];
        uint32_t ksc[TIT], vsc[TIT];
        bool valid[TIT];
#pragma unroll
        for (int i = 0; i < TIT; ++i) {
            const int it = (t0 + i) * kWaves + wave;
            const int slot = lo + it * KPI + kk;
            bool ok = slot < hi;
            if constexpr (FUSED) ok = ok && slot != cur;
            valid[i] = ok;
            if (ok) {
                kq[i] = *reinterpret_cast<const uint4 *>(knib + (int64_t) slot * (D / 2) + blk * 16);
                vq[i] = *reinterpret_cast<const uint4 *>(vnib + (int64_t) slot * (D / 2) + blk * 16);
                ksc[i] = kscl[(int64_t) slot * LPK + blk];
                vsc[i] = vscl[(int64_t) slot * LPK + blk];
            } else {
                kq[i] = make_uint4(0, 0, 0, 0);
                vq[i] = make_uint4(0, 0, 0, 0);
                ksc[i] = 0;
                vsc[i] = 0;
            }
        }
        float s[TIT];
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < TIT; ++i) {
            const float part = f16_bits_to_f32(ksc[i]) * (block_dot(kq[i], ql, qh) - 8.0f * qsum);
            const float sk = key_sum<LPK>(part);
            s[i] = valid[i] ? sk : -INFINITY;
            tmax = fmaxf(tmax, s[i]);
        }
        tmax = wave_max(tmax);
        const float m_new = fmaxf(m, tmax);
        if (m_new == -INFINITY) continue;  // no valid key yet in this wave
        if (m != m_new && m != -INFINITY) {
            const float alpha = exp2f(m - m_new);
            l *= alpha;
            csum *= alpha;
#pragma unroll
            for (int j = 0; j < 32; ++j) acc[j] *= alpha;
        }
        m = m_new;
#pragma unroll
        for (int i = 0; i < TIT; ++i) {
            const float pk = valid[i] ? exp2f(s[i] - m) : 0.0f;
            l += pk;
            const float pd = pk * f16_bits_to_f32(vsc[i]);
            csum += pd;
            block_axpy(vq[i], pd, acc);
        }
    }

    // Fold the -8 code offset and publish this wave's partials.
#pragma unroll
    for (int j = 0; j < 32; ++j) acc[j] = fmaf(-8.0f, csum, acc[j]);
    const float l_wave = wave_sum(l) * (1.0f / LPK);
    {
        float4 *dst = reinterpret_cast<float4 *>(s_acc + (wave * 64 + lane) * LSTRIDE);
#pragma unroll
        for (int c = 0; c < 8; ++c)
            dst[c] = make_float4(acc[4 * c], acc[4 * c + 1], acc[4 * c + 2], acc[4 * c + 3]);
    }
    if (lane == 0) {
        s_m[wave] = m;
        s_l[wave] = l_wave;
    }
    __syncthreads();

    // Merge the waves: output element o = blk*32 + e of key-lane kk of wave w
    // sits at s_acc[(w*64 + kk*LPK + blk)*LSTRIDE + e].
    float M = s_m[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w]);
    float fw[kWaves];
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        fw[w] = (s_m[w] == -INFINITY) ? 0.0f : exp2f(s_m[w] - M);
        L += fw[w] * s_l[w];
    }
    constexpr int PARTS = 256 / D;  // threads per output element
    {
        const int o = threadIdx.x % D;
        const int part = threadIdx.x / D;
        const int ob = o / kQK;
        const int oe = o % kQK;
        float sum = 0.0f;
        // waves and key-lanes are spread over the PARTS threads of element o
        for (int idx = part; idx < kWaves * KPI; idx += PARTS) {
            const int w = idx / KPI;
            const int k2 = idx % KPI;
            sum += fw[w] * s_acc[(w * 64 + k2 * LPK + ob) * LSTRIDE + oe];
        }
        s_part[threadIdx.x] = sum;
    }
    __syncthreads();
    float o_val = 0.0f;
    if (threadIdx.x < D) {
#pragma unroll
        for (int part = 0; part < PARTS; ++part) o_val += s_part[part * D + threadIdx.x];
    }

    if (p.n_split == 1) {
        if (threadIdx.x < D) out_row[threadIdx.x] = (L > 0.0f) ? o_val / L : 0.0f;
        return;
    }

    // Cross-workgroup merge of the window splits.
    float *mine = p.partial + ((int64_t) unit * p.n_split + split) * (D + 2);
    if (threadIdx.x < D) mine[threadIdx.x] = o_val;
    if (threadIdx.x == 0) {
        mine[D] = M;
        mine[D + 1] = L;
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = atomicAdd(&p.counters[unit], 1u);
        s_last = (prev == (unsigned) (p.n_split - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    if (threadIdx.x < D) {
        const float *base = p.partial + (int64_t) unit * p.n_split * (D + 2);
        float Mx = -INFINITY;
        for (int s2 = 0; s2 < p.n_split; ++s2) Mx = fmaxf(Mx, base[s2 * (D + 2) + D]);
        float num = 0.0f, den = 0.0f;
        for (int s2 = 0; s2 < p.n_split; ++s2) {
            const float ms = base[s2 * (D + 2) + D];
            if (ms == -INFINITY) continue;
            const float f = exp2f(ms - Mx);
            num += f * base[s2 * (D + 2) + threadIdx.x];
            den += f * base[s2 * (D + 2) + D + 1];
        }
        out_row[threadIdx.x] = (den > 0.0f) ? num / den : 0.0f;
    }
    if (threadIdx.x == 0) p.counters[unit] = 0u;
}

bool launch_decode(const DecodeParams &p, bool fused, hipStream_t stream) {
    const int64_t units = (int64_t) p.n_batch * p.n_heads;
    const int64_t grid = units * p.n_split;
    if (grid <= 0) return true;
    const dim3 gdim((unsigned) grid), bdim(64 * kWaves);
    if (p.g.head_dim == 128) {
        if (fused)
            hipLaunchKernelGGL((decode_kernel<128, true>), gdim, bdim, 0, stream, p);
        else
            hipLaunchKernelGGL((decode_kernel<128, false>), gdim, bdim, 0, stream, p);
    } else if (p.g.head_dim == 64) {
        if (fused)
            hipLaunchKernelGGL((decode_kernel<64, true>), gdim, bdim, 0, stream, p);
        else
            hipLaunchKernelGGL((decode_kernel<64, false>), gdim, bdim, 0, stream, p);
    } else {
        return false;
    }
    return true;
}

}  // namespace bmo
