// prefill.hip -- chunked prefill into the Q4_0 ring with MFMA attention.
//
// A chunk of n_tok tokens at positions pos0 .. pos0+n_tok-1 of one session
// attends causally within the chunk and to the ring's window before it:
// query i (position p = pos0 + i) sees positions max(0, p - n_ctx + 1) .. p,
// those before pos0 from the ring as it stands, chunk positions from the
// chunk's own K/V quantized to Q4_0 exactly as an append quantizes them.
// Afterwards the chunk occupies ring slots (pos0 + i) % n_ctx.  The
// reference's multi-token path (src/bmo_compute.cpp:2376-2418) writes the
// chunk linearly at n_past and attends without a mask; this is the ring
// (src/bmo_cuda_kernels.cu:739-747) extended to a causal chunk.
//
// The chunk overwrites slots that its own early queries still read (query 0
// needs positions back to pos0 - n_ctx + 1), so one call runs three kernels
// in stream order:
//   stage_kernel   quantizes the chunk's bf16 K/V into a staging stripe with
//                  the ring's group layout (slot i = chunk token i);
//   prefill_kernel attention over the ring and the staged chunk;
//   commit_kernel  copies the staged blocks into their ring slots.
//
// prefill_kernel: a workgroup of QW waves serves 16*QW queries of one
// (entry, head); wave w owns 16 of them.  Keys stream through LDS in tiles of
// 32 positions: all threads dequantize the tile (K row-major, V transposed)
// to fp16 value (code - 8) * d, then each wave computes S^T = K Q^T with
// v_mfma_f32_16x16x32_f16 (the D layout of S^T puts 8 keys of one query in a
// lane, exactly the A layout the P.V product needs), runs an online softmax
// in the log2 domain and accumulates O += P V with the same instruction.
// Operands: q (bf16 inputs, scaled by scale*log2 e) and the dequantized K, V
// and the weights P in fp16, accumulation in fp32.  K and V values fit fp16
// as the reference's F16 cache requires.
#include <math.h>

#include "kernels.hpp"
#include "q4_0_device.hpp"

namespace bmo {

namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kTK = 32;          // keys per tile
constexpr float kRescale = 8.0f; // lazy rescale threshold, log2 units

__device__ __forceinline__ float bf16_to_f32(uint32_t bits) {
    return __builtin_bit_cast(float, bits << 16);
}

// Order of the 8 fp16 values dequantized from code dword c of a block
// (element 4c + kPerm[r]): the pairs the nibble masks produce.
__host__ __device__ constexpr int perm_elem(int r) {
    return (r & 4 ? 16 : 0) + (r & 1 ? 2 : 0) + ((r >> 1) & 1);
}

// Dequantizes code dword w (plain codes, bytes 4c..4c+3 of a block) with
// fp16 scale bits d16 into 8 fp16 values in perm_elem order:
// (code - 8) * d, the subtraction exact, the product rounded to nearest.
__device__ __forceinline__ half8_t dequant_dword(uint32_t w, uint32_t d16) {
    const half2_t off = {(_Float16) -1032.0f, (_Float16) -1032.0f};
    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t) d16);
    const half2_t dd = {d, d};
    half2_t r[4];
    const uint32_t src[4] = {w & 0x000F000Fu, (w >> 8) & 0x000F000Fu, (w >> 4) & 0x000F000Fu,
                             (w >> 12) & 0x000F000Fu};
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r[i] = (__builtin_bit_cast(half2_t, src[i] | 0x64006400u) + off) * dd;
    // r[0] = (e0, e2), r[1] = (e1, e3), r[2] = (e16, e18), r[3] = (e17, e19)
    half8_t o;
    o[0] = r[0].x;
    o[1] = r[0].y;
    o[2] = r[1].x;
    o[3] = r[1].y;
    o[4] = r[2].x;
    o[5] = r[2].y;
    o[6] = r[3].x;
    o[7] = r[3].y;
    return o;
}

}  // namespace

// One thread per (row, K/V, kv head, block) of the chunk: bf16 -> fp32 ->
// Q4_0 (the bit-exact quantizer) -> staging slot i of stripe (entry, head).
__global__ __launch_bounds__(256) void stage_kernel(PrefillParams p) {
    const int nblk = p.g.head_dim / kQK;
    const int64_t per_row = (int64_t) p.n_kv * nblk * 2;
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= per_row * p.n_batch * p.n_tok) return;
    const int64_t r = t / per_row;  // b * n_tok + i
    int rem = (int) (t % per_row);
    const int which = rem / (p.n_kv * nblk);
    rem %= p.n_kv * nblk;
    const int h = rem / nblk;
    const int blk = rem % nblk;
    const int b = (int) (r / p.n_tok);
    const int i = (int) (r % p.n_tok);
    const uint16_t *src = (which == 0 ? p.k : p.v) + (r * p.n_kv + h) * p.g.head_dim + blk * kQK;
    float x[kQK];
    const uint4 *s4 = reinterpret_cast<const uint4 *>(src);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint4 u = s4[c];
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[8 * c + 2 * j] = bf16_to_f32(w[j] & 0xFFFFu);
            x[8 * c + 2 * j + 1] = bf16_to_f32(w[j] >> 16);
        }
    }
    uint16_t d16;
    uint32_t qs[4];
    quantize_block_q4_0(x, d16, qs);
    store_block(p.stage + p.sg.stripe_offset(0, b, h), p.sg, i, blk, which, d16, qs);
}

// One thread per (entry, chunk token, kv head, block): staged K/V blocks to
// ring slot (pos0 + i) % n_ctx.  Skipped entries write nothing.
__global__ __launch_bounds__(256) void commit_kernel(PrefillParams p) {
    const int nblk = p.g.head_dim / kQK;
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t) p.n_batch * p.n_tok * p.n_kv * nblk) return;
    const int blk = (int) (t % nblk);
    const int h = (int) ((t / nblk) % p.n_kv);
    const int i = (int) ((t / ((int64_t) nblk * p.n_kv)) % p.n_tok);
    const int b = (int) (t / ((int64_t) nblk * p.n_kv * p.n_tok));
    const int sid = p.session_ids ? p.session_ids[b] : b;
    const int pos0 = p.pos0[b];
    if (sid < 0 || sid >= p.g.n_sessions || pos0 < 0) return;
    const int slot = (int) (((int64_t) pos0 + i) % p.g.n_ctx);
    const uint8_t *src = p.stage + p.sg.stripe_offset(0, b, h);
    uint8_t *dst = p.base + p.g.stripe_offset(p.layer, sid, h);
    *reinterpret_cast<uint4 *>(dst + p.g.kcode_offset(slot, blk)) =
        *reinterpret_cast<const uint4 *>(src + p.sg.kcode_offset(i, blk));
    *reinterpret_cast<uint4 *>(dst + p.g.vcode_offset(slot, blk)) =
        *reinterpret_cast<const uint4 *>(src + p.sg.vcode_offset(i, blk));
    *reinterpret_cast<uint32_t *>(dst + p.g.scale_offset(slot, blk)) =
        *reinterpret_cast<const uint32_t *>(src + p.sg.scale_offset(i, blk));
}

template <int D, int QW>
__global__ __launch_bounds__(64 * QW) void prefill_kernel(PrefillParams p) {
    constexpr int NBLK = D / kQK;
    constexpr int KROW = D + 8;    // fp16 per K row in LDS (padded)
    constexpr int VROW = kTK + 8;  // fp16 per V^T row in LDS (padded)
    constexpr int QT = 16 * QW;    // queries per workgroup
    constexpr int NT = D / 16;     // output column tiles per wave

    __shared__ __align__(16) _Float16 sK[kTK * KROW];
    __shared__ __align__(16) _Float16 sV[D * VROW];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n_qt = (p.n_tok + QT - 1) / QT;
    const int qt = blockIdx.x % n_qt;
    const int unit = blockIdx.x / n_qt;
    const int b = unit / p.n_heads;
    const int h = unit - b * p.n_heads;
    const int i0 = qt * QT;
    const int q_per_kv = p.n_heads / p.n_kv;
    const int kvh = h / q_per_kv;

    const int sid = p.session_ids ? p.session_ids[b] : b;
    const int pos0 = p.pos0[b];
    const int nq = min(QT, p.n_tok - i0);  // valid queries of this workgroup
    if (sid < 0 || sid >= p.g.n_sessions || pos0 < 0) {
        for (int e = threadIdx.x; e < nq * D; e += blockDim.x) {
            const int qi = e / D;
            p.out[(((int64_t) b * p.n_tok + i0 + qi) * p.n_heads + h) * D + e % D] = 0.0f;
        }
        return;
    }
    const int n_ctx = p.g.n_ctx;
    const int64_t p_first = (int64_t) pos0 + i0;
    const int64_t p_last = (int64_t) pos0 + i0 + nq - 1;
    const int64_t k_lo = max((int64_t) 0, p_first - n_ctx + 1);
    const int n_tiles = (int) ((p_last - k_lo) / kTK) + 1;
    const uint8_t *ring = p.base + p.g.stripe_offset(p.layer, sid, kvh);
    const uint8_t *stage = p.stage + p.sg.stripe_offset(0, b, kvh);

    // Query operand (B of S^T = K Q^T): lane l holds query n = l % 16 of this
    // wave, block b's values at elements 4c + perm_elem(r), c = l / 16.
    const int n = lane & 15;
    const int c = lane >> 4;
    const int qi = i0 + wave * 16 + n;
    const bool q_ok = qi < p.n_tok;
    half8_t qop[NBLK];
    {
        const uint16_t *qrow = p.q + (((int64_t) b * p.n_tok + qi) * p.n_heads + h) * D;
#pragma unroll
        for (int bb = 0; bb < NBLK; ++bb) {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const float x = q_ok ? bf16_to_f32(qrow[bb * kQK + 4 * c + perm_elem(r)]) : 0.0f;
                qop[bb][r] = (_Float16) (x * p.qscale);
            }
        }
    }
    const int64_t pq = (int64_t) pos0 + qi;  // this lane's query position (S^T layout)

    float m = -INFINITY;  // running max of query n (log2 domain)
    float l = 0.0f;       // this lane's part of query n's weight sum
    float4_t acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // Dequantization items: (K/V, key, block, code dword).
    constexpr int ITEMS = 2 * kTK * NBLK * 4;
    for (int tile = 0; tile < n_tiles; ++tile) {
        const int64_t t0 = k_lo + (int64_t) tile * kTK;
        __syncthreads();  // the previous tile's readers are done
        for (int it = threadIdx.x; it < ITEMS; it += blockDim.x) {
            const int cd = it & 3;
            const int bb = (it >> 2) % NBLK;
            const int key = (it >> 2) / NBLK % kTK;
            const int which = it / (kTK * NBLK * 4);
            const int64_t t = t0 + key;
            half8_t vals;
            if (t <= p_last) {
                const uint8_t *src;
                int slot;
                const RingGeom *gg;
                if (t < pos0) {
                    src = ring;
                    slot = (int) (t % n_ctx);
                    gg = &p.g;
                } else {
                    src = stage;
                    slot = (int) (t - pos0);
                    gg = &p.sg;
                }
                uint32_t w = *reinterpret_cast<const uint32_t *>(
                    src + (which == 0 ? gg->kcode_offset(slot, bb) : gg->vcode_offset(slot, bb)) +
                    4 * cd);
                if (which == 0) w ^= 0x88888888u;  // K codes are stored as code ^ 8
                const uint32_t d16 =
                    *reinterpret_cast<const uint16_t *>(src + gg->scale_offset(slot, bb) + 2 * which);
                vals = dequant_dword(w, d16);
            } else {
#pragma unroll
                for (int r = 0; r < 8; ++r) vals[r] = (_Float16) 0.0f;
            }
            if (which == 0) {
                // K row-major, the 8 values of dword cd at slots 8cd..8cd+7 of
                // the block (the order the query operand uses)
                *reinterpret_cast<half8_t *>(&sK[key * KROW + bb * kQK + 8 * cd]) = vals;
            } else {
#pragma unroll
                for (int r = 0; r < 8; ++r) sV[(bb * kQK + 4 * cd + perm_elem(r)) * VROW + key] = vals[r];
            }
        }
        __syncthreads();

        // S^T for keys 0..15 and 16..31 of the tile: lane l gets keys
        // 4c + v (and 16 + 4c + v) of query n.
        float4_t s[2];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            float4_t a = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int bb = 0; bb < NBLK; ++bb) {
                const half8_t kop =
                    *reinterpret_cast<const half8_t *>(&sK[(sub * 16 + n) * KROW + bb * kQK + 8 * c]);
                a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qop[bb], a, 0, 0, 0);
            }
            s[sub] = a;
        }
        // mask (causal + window) and tile max of query n
        float tmax = -INFINITY;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t t = t0 + sub * 16 + 4 * c + v;
                const bool ok = q_ok && t <= pq && t > pq - n_ctx;
                s[sub][v] = ok ? s[sub][v] : -INFINITY;
                tmax = fmaxf(tmax, s[sub][v]);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const bool need = tmax > m + kRescale;
        if (__any(need)) {
            const float alpha = need ? ((m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - tmax)) : 1.0f;
            m = need ? tmax : m;
            l *= alpha;
            // acc rows are queries 4c + v: fetch their alphas from lanes 4c + v
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float av = __shfl(alpha, 4 * c + v);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t][v] *= av;
            }
        }
        half8_t pop;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float pv = (s[sub][v] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(s[sub][v] - m);
                l += pv;
                pop[sub * 4 + v] = (_Float16) pv;
            }
        // O += P V: B operand lane l = element n of the column tile, keys
        // 4c..4c+3 and 16+4c..16+4c+3 (the key order of pop)
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const _Float16 *vrow = &sV[(t * 16 + n) * VROW];
            const uint2 lo = *reinterpret_cast<const uint2 *>(vrow + 4 * c);
            const uint2 hi = *reinterpret_cast<const uint2 *>(vrow + 16 + 4 * c);
            const uint4 vv = make_uint4(lo.x, lo.y, hi.x, hi.y);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pop, __builtin_bit_cast(half8_t, vv), acc[t],
                                                            0, 0, 0);
        }
    }

    // Row sums of query n, then every acc row (query 4c + v) divides by its own.
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const float lv = __shfl(l, 4 * c + v);
        const int qv = i0 + wave * 16 + 4 * c + v;
        if (qv < p.n_tok) {
            float *orow = p.out + (((int64_t) b * p.n_tok + qv) * p.n_heads + h) * D;
            const float inv = lv > 0.0f ? 1.0f / lv : 0.0f;
#pragma unroll
            for (int t = 0; t < NT; ++t) orow[t * 16 + n] = acc[t][v] * inv;
        }
    }
}

bool launch_prefill(const PrefillParams &p, hipStream_t stream) {
    const int nblk = p.g.head_dim / kQK;
    const int64_t stage_threads = (int64_t) p.n_batch * p.n_tok * p.n_kv * nblk * 2;
    hipLaunchKernelGGL(stage_kernel, dim3((unsigned) ((stage_threads + 255) / 256)), dim3(256), 0,
                       stream, p);
    constexpr int QW = 4;
    const int n_qt = (p.n_tok + 16 * QW - 1) / (16 * QW);
    const dim3 grid((unsigned) ((int64_t) p.n_batch * p.n_heads * n_qt));
    if (p.g.head_dim == 128)
        hipLaunchKernelGGL((prefill_kernel<128, QW>), grid, dim3(64 * QW), 0, stream, p);
    else if (p.g.head_dim == 64)
        hipLaunchKernelGGL((prefill_kernel<64, QW>), grid, dim3(64 * QW), 0, stream, p);
    else
        return false;
    const int64_t commit_threads = (int64_t) p.n_batch * p.n_tok * p.n_kv * nblk;
    hipLaunchKernelGGL(commit_kernel, dim3((unsigned) ((commit_threads + 255) / 256)), dim3(256), 0,
                       stream, p);
    return true;
}

}  // namespace bmo
