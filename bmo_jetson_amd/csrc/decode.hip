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
// Work decomposition (gfx950, wave64).  A workgroup of NW waves serves one
// (batch entry, query head) unit; its waves take contiguous pieces of the
// window.  Batches with many units use one wave per unit; small batches (B=1
// decode) use 2 to 8 waves per unit (16 on request) so that enough waves run,
// merging in LDS (a split across workgroups would have to merge through
// device-scope atomics, which serialize across the XCDs).  The ring stores
// slots in groups of G = 64 / LPK keys
// (ring_layout.hpp), LPK = head_dim / 32 blocks per key, so one group is one
// wave iteration: lane l owns block l % LPK of key l / LPK and fetches its 16
// K code bytes, 16 V code bytes and its (K, V) scale dword with three
// coalesced loads from the group's 2304 contiguous bytes.  The loads are
// nontemporal: every ring byte is read once per step and the working set is
// far larger than the caches.  Each wave walks a contiguous run of groups,
// keeping the loads of the next PF groups in flight while one group is
// computed.  Keys past the window (and, fused, the slot being written) get
// weight 0 by select.
//
// K side: q (times scale * log2 e) is turned once per wave into 31-bit fixed
// point per 32-element block with a power-of-two step: with the block's
// largest magnitude amax = m * 2^ex (m in [0.5, 1)), sq = 2^(ex-30) and
// Q_e = rint(q_e / sq), |Q_e| <= 2^30.  Dividing by a power of two is exact,
// so Q_e sq equals q_e exactly whenever |q_e| >= amax / 64 (an fp32 value of
// magnitude >= 2^23 is an integer) and is within sq / 2 <= amax * 2^-30 of it
// otherwise: at least as close as fp32 arithmetic on q itself.  Q_e is
// written as eight planes of signed base-16 digits, Q_e = sum_i 16^i s_ie
// with s_ie in [-8, 7], laid out like the code dwords.  The ring keeps K codes
// as signed nibbles c_e - 8, so v_dot8_i32_i4 gives
//   sum_e (c_e - 8) Q_e = 2^16 sum_{i>=4} 16^(i-4) P_i + sum_{i<4} 16^i P_i,
//   P_i = sum_e (c_e - 8) s_ie,
// in 32 instructions per block, exactly, with no correction terms; the two
// partial sums stay below 2^24 in magnitude, so each converts to fp32
// exactly, and the block score is one fma of them with 2^16 sq and sq,
// rounded once, times the block scale.  A block holding a NaN or an infinity
// gets sq = NaN, so that head's output is NaN, as fp32 scoring would make it.
//
// V side: masking a code dword with 0x000F000F (0x00F000F0) leaves two fp16
// subnormals equal to c * 2^-24 (c * 2^-20); v_fma_mix_f32 reads them next to
// the fp32 weight 2^24 * p * d and accumulates sum_i p_i d_i c_ie in fp32
// (16 times that for the high nibbles, rescaled at the end); 8 sum_i p_i d_i
// is subtracted at the end.
//
// Softmax is online per lane (running max m, sum l, acc[32]).  A lane
// rescales only when a score exceeds its running max by more than 8 (log2
// units), so weights stay below 2^8 and rescaling is rare after the first
// keys; the result does not depend on the threshold.  Weights are carried
// times 2^24 (the stored max is m - 24), which is the scale the subnormal
// V codes need, so one multiply by the V scale makes a key's weight.  At the end every lane
// is brought to the wave max, the four 16-lane rows are summed by permlane
// swaps and the lanes sharing a block by DPP rotations; a one-wave unit
// stores its output from registers, several waves merge through LDS.
//
// Fused append (the reference's write-then-attend,
// src/bmo_cuda_kernels.cu:749-754): wave 0 quantizes the current token's K/V
// rows in registers with the bit-exact quantizer, spread over all 64 lanes
// (32 / LPK lanes per block, reductions by DPP), attends to that key from
// registers, and the first query head of each kv group stores the blocks to
// slot pos % n_ctx.  Every workgroup masks that slot out of its ring reads.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include "kernels.hpp"
#include "q4_0_device.hpp"

namespace bmo {

namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// Q + kQBias = sum_i 16^i u_i with u_i in [0, 15] and s_i = u_i - 8; any
// |Q| <= 2^30 lies in the representable [-kQBias, 0x77777777].
constexpr uint32_t kQBias = 0x88888888u;  // 8 * sum_{i<8} 16^i
constexpr int kQBits = 30;                // |Q| <= 2^kQBits
constexpr int kPlanes = 8;                // base-16 digit planes per element
constexpr float kRescale = 8.0f;  // lazy rescale threshold, log2 units
// Weights are kept scaled by 2^24 (the running max is stored minus 24), so
// the fp16-subnormal codes c * 2^-24 multiply them without a per-key scaling.
constexpr float kWScale = 24.0f;
// Running-max floor: finite, so a masked score (-inf) gives exp2(-inf - m) = 0
// with no select.
constexpr float kMaxFloor = -1.0e30f;

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

// Wave-wide max / sum without LDS: DPP within each 16-lane row, then the
// four row results through readlane.
__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));   // lane ^ 1
    v = fmaxf(v, dpp<0x4E>(v));   // lane ^ 2
    v = fmaxf(v, dpp<0x124>(v));  // row_ror:4
    return fmaxf(v, dpp<0x128>(v));  // row_ror:8
}
__device__ __forceinline__ float row_sum(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x124>(v);
    return v + dpp<0x128>(v);
}
// v_permlane32_swap / v_permlane16_swap (gfx950) as inline asm: the
// compiler's builtins for them hand back one register for both halves of the
// returned pair.  The instruction exchanges lanes 32-63 of a with lanes 0-31
// of b (permlane32: a = {a rows 0-1, b rows 0-1}, b = {a rows 2-3, b rows
// 2-3}) or the odd rows of a with the even rows of b (permlane16: a = {a r0,
// b r0, a r2, b r2}, b = {a r1, b r1, a r3, b r3}).  The compiler's hazard
// pass does not look inside inline asm, so the s_nop provides the wait
// states itself: 4, which covers a VALU write of the operands (2 needed) and
// a VALU write of EXEC (v_cmpx) right before the swap as well.
__device__ __forceinline__ float swap_sum32(float a, float b) {
    asm("s_nop 3\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return a + b;
}
__device__ __forceinline__ float swap_sum16(float a, float b) {
    asm("s_nop 3\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return a + b;
}
__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ float wave_max(float v) {
    v = row_max(v);
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}
__device__ __forceinline__ float wave_sum(float v) {
    v = row_sum(v);
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

// K-side scorer: sum_e (c_e - 8) q_e of one block, before the block scale.
struct Scorer {
    uint32_t dig[kPlanes][4];  // signed digit plane i, laid out like code dword c
    float sq;                  // fixed-point step of this lane's block (a power of two)
    float sqh;                 // 2^16 * sq

    // w4: the block's 16 K code bytes as stored (signed nibbles c - 8).
    // Each partial sum is at most 32 * 8 * 8 * 0x1111 < 2^24 in magnitude.
    __device__ __forceinline__ float operator()(const uint4 &w4) const {
        const int w[4] = {(int) w4.x, (int) w4.y, (int) w4.z, (int) w4.w};
        int lo = 0, hi = 0;
#pragma unroll
        for (int i = 3; i >= 0; --i) {
            if (i != 3) {
                lo <<= 4;
                hi <<= 4;
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                lo = __builtin_amdgcn_sdot8(w[c], (int) dig[i][c], lo, false);
                hi = __builtin_amdgcn_sdot8(w[c], (int) dig[i + 4][c], hi, false);
            }
        }
        return __builtin_fmaf((float) hi, sqh, (float) lo * sq);
    }
};

// Interleaved RoPE (src/bmo_cuda_kernels.cu:317-354): pair (x[2i], x[2i+1])
// of a head turns by pos * theta^(-2i/head_dim).  Lane i < D/2 of a wave
// writes cos and sin (fp32) of pair i to tab: the frequency r^i by binary
// powers of r = theta^(-2/D) and the angle, cosine and sine in double, so
// the table is the exact rotation rounded once (the reference evaluates it
// with fp32 fast intrinsics).
template <int D>
__device__ __forceinline__ void rope_table(int pos, double r, int lane, float2 *tab) {
    if (lane < D / 2) {
        double f = 1.0, b = r;
        for (int i = lane; i; i >>= 1) {
            if (i & 1) f *= b;
            b *= b;
        }
        double sn, cs;
        sincos((double) pos * f, &sn, &cs);
        tab[lane] = make_float2((float) cs, (float) sn);
    }
}

// (a, b) rotated by (c, s) = tab entry, every product and sum rounded.
__device__ __forceinline__ void rope_pair(float &a, float &b, float2 cs) {
    const float ac = a * cs.x, bs = b * cs.y, as = a * cs.y, bc = b * cs.x;
    a = ac - bs;
    b = as + bc;
}

// One wave turns the query row of its unit into the Scorer digit planes of
// every block: lane l makes dword c = l % 4 of planes i = (l / 4) % 4 and
// i + 4 of block (l / 16) % LPK, which hold the digits of elements 4c..4c+3
// (low nibbles) and 4c+16..4c+19 (high nibbles).  Results go to this wave's
// LDS slice: plane i of block b at dwords b * 32 + i * 4 .. +3, and the
// block's step at s_sq[b].
// The query elements lane l works on: 4c..4c+3 and 4c+16..4c+19 of block
// (l / 16) % LPK, c = l % 4 (loaded early, ahead of the table and quantizer
// work of the prologue).
template <int D>
__device__ __forceinline__ void prep_load(const float *__restrict__ qrow, int lane, float4 &lo,
                                          float4 &hi) {
    constexpr int LPK = D / kQK;
    const int blk = (lane >> 4) % LPK;
    const int c = lane & 3;
    lo = *reinterpret_cast<const float4 *>(qrow + blk * kQK + 4 * c);
    hi = *reinterpret_cast<const float4 *>(qrow + blk * kQK + 4 * c + 16);
}

template <int D>
__device__ __forceinline__ void prep_digits(float4 lo, float4 hi, float qscale, int lane,
                                            uint32_t *s_dig, float *s_sq, const float2 *rope) {
    constexpr int LPK = D / kQK;
    const int blk = (lane >> 4) % LPK;
    const int i = (lane >> 2) & 3;
    const int c = lane & 3;
    if (rope) {
        // elements 4c..4c+3 and 4c+16..4c+19 of the block are pairs
        // blk*16 + 2c, +1 and blk*16 + 2c + 8, +9
        const int j = blk * 16 + 2 * c;
        rope_pair(lo.x, lo.y, rope[j]);
        rope_pair(lo.z, lo.w, rope[j + 1]);
        rope_pair(hi.x, hi.y, rope[j + 8]);
        rope_pair(hi.z, hi.w, rope[j + 9]);
    }
    const float x[8] = {lo.x * qscale, lo.y * qscale, lo.z * qscale, lo.w * qscale,
                        hi.x * qscale, hi.y * qscale, hi.z * qscale, hi.w * qscale};
    float amax = 0.0f;
    float finite = 0.0f;  // 0 when every element is finite, else NaN
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        amax = fmaxf(amax, __builtin_fabsf(x[j]));
        finite += x[j] * 0.0f;
    }
    amax = fmaxf(amax, dpp<0xB1>(amax));  // the four lanes c = 0..3 of this block
    amax = fmaxf(amax, dpp<0x4E>(amax));
    finite += dpp<0xB1>(finite);
    finite += dpp<0x4E>(finite);
    // amax = m * 2^ex with m in [0.5, 1): x * 2^(30 - ex) is exact and below
    // 2^30 in magnitude (0 for amax = 0, whose exponent reads as 0)
    const int ex = __builtin_amdgcn_frexp_expf(amax);
    uint32_t dw_lo = 0, dw_hi = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int Q = (int) __builtin_rintf(__builtin_amdgcn_ldexpf(x[j], kQBits - ex));
        const uint32_t u = (uint32_t) Q + kQBias;  // in [kQBias - 2^30, kQBias + 2^30]
        const int nib = (j < 4) ? 2 * j : 2 * (j - 4) + 1;
        dw_lo |= (((u >> (4 * i)) & 15u) ^ 8u) << (4 * nib);
        dw_hi |= (((u >> (4 * i + 16)) & 15u) ^ 8u) << (4 * nib);
    }
    if (lane < 16 * LPK) {
        s_dig[blk * 32 + i * 4 + c] = dw_lo;
        s_dig[blk * 32 + (i + 4) * 4 + c] = dw_hi;
        if ((lane & 15) == 0)
            s_sq[blk] = finite == 0.0f ? __builtin_amdgcn_ldexpf(1.0f, ex - kQBits) : __builtin_nanf("");
    }
}

// acc[e] += w * c_e * 2^-24 for elements 0..15 and w * c_e * 2^-20 for
// elements 16..31 of one block (acc in element order; w4 holds plain codes
// 0..15): a masked code dword is a pair of fp16 subnormals c * 2^-24 (low
// nibble of a byte) or c * 2^-20 (high nibble), which v_fma_mix_f32 reads
// directly.  The caller scales elements 16..31 by 1/16 at the end.
__device__ __forceinline__ void block_axpy(const uint4 &w4, float w, float (&acc)[32]) {
    const uint32_t wd[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t w8 = wd[c] >> 8;
        const half2_t A = __builtin_bit_cast(half2_t, wd[c] & 0x000F000Fu);
        const half2_t B = __builtin_bit_cast(half2_t, wd[c] & 0x00F000F0u);
        const half2_t C = __builtin_bit_cast(half2_t, w8 & 0x000F000Fu);
        const half2_t E = __builtin_bit_cast(half2_t, w8 & 0x00F000F0u);
        acc[4 * c + 0] = __builtin_fmaf((float) A.x, w, acc[4 * c + 0]);
        acc[4 * c + 2] = __builtin_fmaf((float) A.y, w, acc[4 * c + 2]);
        acc[4 * c + 16] = __builtin_fmaf((float) B.x, w, acc[4 * c + 16]);
        acc[4 * c + 18] = __builtin_fmaf((float) B.y, w, acc[4 * c + 18]);
        acc[4 * c + 1] = __builtin_fmaf((float) C.x, w, acc[4 * c + 1]);
        acc[4 * c + 3] = __builtin_fmaf((float) C.y, w, acc[4 * c + 3]);
        acc[4 * c + 17] = __builtin_fmaf((float) E.x, w, acc[4 * c + 17]);
        acc[4 * c + 19] = __builtin_fmaf((float) E.y, w, acc[4 * c + 19]);
    }
}

// fp32 value of the fp16 in the low (HI = false) or high half of a dword.
template <bool HI>
__device__ __forceinline__ float half_of(uint32_t v) {
    const half2_t h = __builtin_bit_cast(half2_t, v);
    return HI ? (float) h.y : (float) h.x;
}

}  // namespace

template <int D, int NW, int PF, bool FUSED>
__global__ __launch_bounds__(64 * NW) void decode_kernel(DecodeParams p) {
    constexpr int LPK = D / kQK;   // lanes (blocks) per key
    constexpr int G = 64 / LPK;    // keys per group = per wave iteration
    constexpr int NB = PF + 1;     // resident groups per wave

    __shared__ __align__(16) float s_acc[NW * D];
    __shared__ __align__(16) uint32_t s_dig[NW][kPlanes * 4 * LPK];
    __shared__ float s_m[NW];
    __shared__ float s_l[NW];
    __shared__ float s_sq[NW][4];
    __shared__ float2 s_rope[NW][D / 2];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int kk = lane / LPK;
    const int blk = lane % LPK;

    const int unit = blockIdx.x;
    const int b = (int) p.div_heads.div((uint32_t) unit);
    const int h = unit - b * p.n_heads;

    const RingGeom &g = p.g;
    const int sid_in = p.session_ids ? p.session_ids[b] : b;
    const bool sid_ok = sid_in >= 0 && sid_in < g.n_sessions;
    const int sid = sid_ok ? sid_in : 0;  // an in-bounds stripe for loads issued before the check
    const int q_per_kv = p.q_per_kv;
    const int kvh = (int) p.div_qkv.div((uint32_t) h);
    uint8_t *stripe = p.base + g.stripe_offset(p.layer, sid, kvh);
    float *out_row = p.out + (int64_t) unit * D;

    // Contiguous group run of this wave.  Fused with several waves per
    // unit, wave 0 quantizes and attends to the current token and the other
    // waves split the window, so the new token's work is off the window's
    // critical path.
    constexpr bool kSplitNew = FUSED && NW > 1;
    constexpr int NWW = kSplitNew ? NW - 1 : NW;  // waves that stream the window
    const int ww = kSplitNew ? wave - 1 : wave;
    int g0 = 0, n_it = 0;

    struct Grp {
        uint4 k, v;
        uint32_t sc;
    };
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    auto load = [&](int it, Grp &T) {
        const uint8_t *gp = stripe + (int64_t) (g0 + it) * g.group_stride;
        const u32x4 kc = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(gp + lane * 16));
        const u32x4 vc =
            __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(gp + kVCodeOff + lane * 16));
        T.k = make_uint4(kc.x, kc.y, kc.z, kc.w);
        T.v = make_uint4(vc.x, vc.y, vc.z, vc.w);
        T.sc = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(gp + kScaleOff + lane * 4));
    };
    // Prologue loads are unconditional (a group index past this wave's run
    // is clamped to the stripe's last group, a harmless in-bounds read), so
    // the outstanding-load count at the steady-state loop below is the same
    // on every path and the compiler's wait counts stay exact.
    auto load_clamped = [&](int it, Grp &T) { load(min(it, g.n_groups - 1 - g0), T); };
    Grp buf[NB];
    float4 q_lo, q_hi;
    // The query does not depend on the position, so it is requested before
    // the position is read (the scalar read's latency then overlaps its
    // own); with one wave per unit the run starts at group 0 whatever the
    // position, so the first groups go out ahead of it as well.
    if constexpr (NW == 1) {
#pragma unroll
        for (int j = 0; j < NB - 1; ++j) load_clamped(j, buf[j]);
    }
    prep_load<D>(p.q + (int64_t) unit * D, lane, q_lo, q_hi);
    // Fused: wave 0 holds the current token's K and V rows spread over its
    // lanes for the lane-parallel quantizer, BL lanes per block: lane l
    // takes block nb = l / BL (K block nb for nb < LPK, else V block
    // nb - LPK), elements gi*NE/2 + t and gi*NE/2 + t + 16 of it (t < NE/2),
    // gi = l % BL.  Requested before the position, which they do not need.
    constexpr int BL = 32 / LPK;
    constexpr int NE = LPK;
    const int nb = lane / BL;
    const int gi = lane % BL;
    float xnew[NE];
    if constexpr (FUSED) {
        if (wave == 0) {
            const float *src = (nb < LPK ? p.k_new : p.v_new) + ((int64_t) b * p.n_kv + kvh) * D +
                               (nb % LPK) * kQK + gi * (NE / 2);
#pragma unroll
            for (int t = 0; t < NE / 2; ++t) {
                xnew[t] = src[t];
                xnew[NE / 2 + t] = src[16 + t];
            }
        }
    }
    const int pos = p.pos ? p.pos[b] : p.pos_scalar;
    if (!sid_ok || pos < 0) {
        for (int i = threadIdx.x; i < D; i += blockDim.x) out_row[i] = 0.0f;
        return;
    }
    const int window = (int) min((int64_t) pos + 1, (int64_t) g.n_ctx);
    const int cur = pos - (int) p.div_ctx.div((uint32_t) pos) * g.n_ctx;  // pos % n_ctx
    const int n_grp = (window + G - 1) / G;
    g0 = ww < 0 ? 0 : ww * n_grp / NWW;
    n_it = ww < 0 ? 0 : (ww + 1) * n_grp / NWW - g0;
    if constexpr (NW > 1) {
#pragma unroll
        for (int j = 0; j < NB - 1; ++j) load_clamped(j, buf[j]);
    }
    if (p.rope) rope_table<D>(pos, p.rope_r, lane, s_rope[wave]);  // wave-private LDS
    prep_digits<D>(q_lo, q_hi, p.qscale, lane, s_dig[wave], s_sq[wave], p.rope ? s_rope[wave] : nullptr);
    __syncthreads();
    Scorer score;
#pragma unroll
    for (int i = 0; i < kPlanes; ++i) {
        const uint4 d4 = *reinterpret_cast<const uint4 *>(&s_dig[wave][blk * 32 + i * 4]);
        score.dig[i][0] = d4.x;
        score.dig[i][1] = d4.y;
        score.dig[i][2] = d4.z;
        score.dig[i][3] = d4.w;
    }
    score.sq = s_sq[wave][blk];
    score.sqh = score.sq * 65536.0f;

    // Softmax state of this lane's keys (log2 domain): mm = running max - 24,
    // mt = running max + 8 (the lazy rescale threshold), l = sum of weights
    // times 2^24 (each key counted LPK times), csum = sum of weight * V scale
    // times 2^24.
    float mm = kMaxFloor;
    float mt = kMaxFloor;
    float l = 0.0f;
    float csum = 0.0f;
    float acc[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) acc[e] = 0.0f;

    if constexpr (FUSED) {
        if (wave == 0) {
            // The current token's blocks, quantized by the whole wave (BL
            // lanes per block); the K and V codes and scales of block blk
            // then move to lane blk (kk == 0), which attends to the new key.
            constexpr int HE = NE / 2;
            constexpr int LPD = 4 / HE;  // lanes per code dword
            if (p.rope) {
                // K pairs (2m, 2m+1) of the head turn by table entry m
                const float2 *tab = s_rope[0] + (nb % LPK) * 16;
                if constexpr (HE == 2) {
                    float a0 = xnew[0], b0 = xnew[1], a1 = xnew[2], b1 = xnew[3];
                    rope_pair(a0, b0, tab[gi]);
                    rope_pair(a1, b1, tab[gi + 8]);
                    if (nb < LPK) {
                        xnew[0] = a0;
                        xnew[1] = b0;
                        xnew[2] = a1;
                        xnew[3] = b1;
                    }
                } else {
                    // elements gi and gi + 16: each pair spans lanes gi, gi ^ 1
                    const bool odd = gi & 1;
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const float x = xnew[t];
                        const float y = dpp<0xB1>(x);  // the other element of the pair
                        const float2 cs = tab[gi / 2 + 8 * t];
                        // (a, b) -> (a c - b s, a s + b c), products rounded apart
                        const float r = odd ? y * cs.y + x * cs.x : x * cs.x - y * cs.y;
                        if (nb < LPK) xnew[t] = r;
                    }
                }
            }
            uint16_t d16;
            const uint32_t dw = quantize_block_q4_0_lanes<BL>(xnew, gi, d16);
            if (h == kvh * q_per_kv) {  // the first query head of the kv group
                // the first lane of each code dword stores it, lane 0 of the
                // block the scale (ring_layout.hpp: K codes as code ^ 8)
                // (the offsets of RingGeom::kcode_offset / vcode_offset /
                // scale_offset, with this kernel's compile-time G)
                const int which = nb < LPK ? 0 : 1;
                const int bb = nb % LPK;
                uint8_t *grp = stripe + (int64_t) ((unsigned) cur / G) * g.group_stride;
                const int key = (int) ((unsigned) cur % G);
                if (gi % LPD == 0)
                    *reinterpret_cast<uint32_t *>(grp + which * kVCodeOff + key * (D / 2) + bb * 16 +
                                                  4 * (gi / LPD)) = which == 0 ? dw ^ 0x88888888u : dw;
                if (gi == 0)
                    reinterpret_cast<uint16_t *>(grp + kScaleOff + (key * LPK + bb) * 4)[which] = d16;
            }
            // lane blk gathers K block blk (lanes blk*BL + c*LPD) and V block
            // blk (lanes (LPK + blk)*BL + c*LPD)
            uint32_t kq[4], vq[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                kq[c] = (uint32_t) __shfl((int) dw, blk * BL + c * LPD);
                vq[c] = (uint32_t) __shfl((int) dw, (LPK + blk) * BL + c * LPD);
            }
            const uint32_t kd16 = (uint32_t) __shfl((int) d16, blk * BL);
            const uint32_t vd16 = (uint32_t) __shfl((int) d16, (LPK + blk) * BL);
            float s_new = 0.0f;
            if (kk == 0) {
                const uint4 kflip = make_uint4(kq[0] ^ 0x88888888u, kq[1] ^ 0x88888888u,
                                               kq[2] ^ 0x88888888u, kq[3] ^ 0x88888888u);
                s_new = f16_bits_to_f32(kd16) * score(kflip);
            }
            s_new = key_sum<LPK>(s_new);
            if (kk == 0) {
                const float w_new = 16777216.0f * f16_bits_to_f32(vd16);  // 2^24 * exp2(0) * d
                mm = s_new - kWScale;
                mt = s_new + kRescale;
                l = 16777216.0f;
                csum = w_new;
                block_axpy(make_uint4(vq[0], vq[1], vq[2], vq[3]), w_new, acc);
            }
        }
    }

    auto compute = [&](int it, const Grp &T) {
        const int slot = (g0 + it) * G + kk;
        bool ok = slot < window;
        if constexpr (FUSED) ok = ok && slot != cur;
        const float sk = key_sum<LPK>(score(T.k) * half_of<false>(T.sc));
        const float s = ok ? sk : -INFINITY;
        const bool need = s > mt;
        if (__any(need)) {
            const float mm_new = need ? s - kWScale : mm;
            const float alpha = __builtin_amdgcn_exp2f(mm - mm_new);
            mm = mm_new;
            mt = need ? s + kRescale : mt;
            l *= alpha;
            csum *= alpha;
#pragma unroll
            for (int e = 0; e < 32; ++e) acc[e] *= alpha;
        }
        const float pk = __builtin_amdgcn_exp2f(s - mm);  // 2^24 * weight; 0 if masked
        l += pk;
        // a masked key adds exactly nothing, whatever its slot holds (a
        // non-finite V scale outside the window must not reach the output)
        const float w = ok ? pk * half_of<true>(T.sc) : 0.0f;
        csum += w;
        block_axpy(T.v, w, acc);
    };
    // Steady state: every load is unconditional, so the wait before a group's
    // compute is for that group's loads only (a conditional prefetch would
    // make the compiler wait for the prefetch as well).  buf[u] holds group
    // t + u at the top of each pass.
    int t = 0;
    for (; t + 2 * NB - 2 < n_it; t += NB) {
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            load(t + u + NB - 1, buf[(u + NB - 1) % NB]);
            compute(t + u, buf[u]);
        }
    }
    // Tail: at most 2 * NB - 2 groups, loads only while groups remain.
#pragma unroll
    for (int u = 0; u < 2 * NB - 2; ++u) {
        const int tt = t + u;
        if (tt < n_it) {
            if (tt + NB - 1 < n_it) load(tt + NB - 1, buf[(u + NB - 1) % NB]);
            compute(tt, buf[u % NB]);
        }
    }

    // Bring every lane to the wave max (the factor is folded into one fma
    // per element), undo the 2^-20 scale of elements 16..31 and fold the -8
    // code offset.
    const float m_wave = wave_max(mm);
    const float f = __builtin_amdgcn_exp2f(mm - m_wave);
    const float l_wave = wave_sum(l * f) * (1.0f / LPK);
    const float c8 = (-8.0f / 16777216.0f) * (csum * f);  // -8 * sum of p * d, in acc units
    const float f_hi = f * 0.0625f;
#pragma unroll
    for (int e = 0; e < 32; ++e) acc[e] = __builtin_fmaf(acc[e], e < 16 ? f : f_hi, c8);
    // Sum the four 16-lane rows without LDS: v_permlane32_swap on element
    // pairs (2i, 2i+1) leaves rows 0-1 with element 2i and rows 2-3 with
    // 2i+1, each summed over rows {r, r+2}; v_permlane16_swap on the pairs of
    // those leaves row r with element 4j + {0, 2, 1, 3}[r] summed over all
    // four rows.  Then the lanes of a row that own the same block are summed.
    float z[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        z[i] = swap_sum32(acc[2 * i], acc[2 * i + 1]);
    }
    float ws[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        ws[j] = row_block_sum<LPK>(swap_sum16(z[2 * j], z[2 * j + 1]));
    }
    // Lane l (row r = l / 16) now holds elements blk * 32 + 4 j + mr, j < 8,
    // mr = {0, 2, 1, 3}[r], replicated over the REP = 16 / LPK lanes of its
    // row that own block blk; replica ri keeps j = jj * REP + ri, jj < 8 / REP,
    // so each of the 8 / REP stores below has all 64 lanes writing distinct
    // elements and together they cover the D outputs.
    constexpr int REP = 16 / LPK;
    constexpr int NJ = 8 / REP;
    static_assert(REP <= 8 && NJ * REP == 8, "head_dim 64 or 128");
    const int row = lane >> 4;
    const int mr = (row & 1) * 2 + (row >> 1);
    const int ri = (lane & 15) / LPK;
    float o[NJ];
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
        float v = ws[jj * REP];
#pragma unroll
        for (int r = 1; r < REP; ++r) v = (ri == r) ? ws[jj * REP + r] : v;
        o[jj] = v;
    }
    const int obase = blk * kQK + 4 * ri + mr;  // element of o[jj] is obase + 4 REP jj
    float L = l_wave;  // 2^24 times the weight sum of the whole window
    if constexpr (NW == 1) {
        const float inv_l = (L > 0.0f) ? 16777216.0f / L : 0.0f;
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj) out_row[obase + 4 * REP * jj] = o[jj] * inv_l;
    } else {
        // Merge the waves: each writes its row of sums and its (max, sum).
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj) s_acc[wave * D + obase + 4 * REP * jj] = o[jj];
        if (lane == 0) {
            s_m[wave] = m_wave;
            s_l[wave] = l_wave;
        }
        __syncthreads();
        float M = s_m[0];
#pragma unroll
        for (int w = 1; w < NW; ++w) M = fmaxf(M, s_m[w]);
        float fw[NW];
        L = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            fw[w] = __builtin_amdgcn_exp2f(s_m[w] - M);
            L = __builtin_fmaf(fw[w], s_l[w], L);
        }
        const float inv_l = (L > 0.0f) ? 16777216.0f / L : 0.0f;
        if (threadIdx.x < D) {
            float a = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w) a = __builtin_fmaf(fw[w], s_acc[w * D + threadIdx.x], a);
            out_row[threadIdx.x] = a * inv_l;
        }
    }
}

namespace {

template <int D, int NW, int PF>
void launch_variant(const DecodeParams &p, bool fused, hipStream_t stream) {
    const dim3 grid((unsigned) ((int64_t) p.n_batch * p.n_heads)), block(64 * NW);
    if (fused)
        hipLaunchKernelGGL((decode_kernel<D, NW, PF, true>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((decode_kernel<D, NW, PF, false>), grid, block, 0, stream, p);
}

struct Shape {
    int nw, pf;
};

// The shapes launch_shape instantiates.
constexpr Shape kShapes[] = {{1, 1}, {1, 2}, {1, 3}, {2, 1}, {4, 1}, {8, 1}, {8, 2}, {16, 1}};

constexpr bool shape_instantiated(Shape s) {
    for (const Shape &k : kShapes)
        if (k.nw == s.nw && k.pf == s.pf) return true;
    return false;
}

// Workgroup shape per call: one wave per (entry, head) unit with two groups
// of loads in flight when there are enough units to fill the chip (measured
// best over sustained runs of BASELINE config 3), else enough waves per unit
// for about 512 waves in all.  Below 128 units, 8 waves per unit (B=1, 32
// units, over a 32-layer model step whose windows come from HBM: 6.86 us
// plain and 7.03 us fused per layer, against 7.44 and 8.16 us with 4 waves;
// fused, wave 0 takes the new token), with two groups in flight per wave
// when plain (5.62 against 5.74 us per layer with one) and one when fused
// (5.87 against 5.89 us with two).  A window of fewer groups than waves
// halves the waves, with one group in flight below 8 waves.
constexpr Shape default_shape(int64_t units, int n_groups, bool fused) {
    Shape s{1, 2};
    if (units < 128) s = Shape{8, fused ? 1 : 2};
    else if (units < 256) s = Shape{4, 1};
    else if (units < 512) s = Shape{2, 1};
    while (s.nw > 1 && s.nw > n_groups) {  // no more waves than groups
        s.nw /= 2;
        s.pf = 1;
    }
    return s;
}

constexpr bool default_shapes_instantiated() {
    for (int64_t units : {1, 32, 127, 128, 255, 256, 511, 512, 1 << 20})
        for (int n_groups = 1; n_groups <= 64; ++n_groups)
            for (bool fused : {false, true})
                if (!shape_instantiated(default_shape(units, n_groups, fused))) return false;
    return true;
}
static_assert(default_shapes_instantiated(), "every default decode shape has a kernel");

// BMO_ATTN_SHAPE = "nw,pf" overrides the default (tuning); a shape without a
// kernel falls back to one wave with one group in flight.
Shape pick_shape(int64_t units, int n_groups, bool fused) {
    Shape s = default_shape(units, n_groups, fused);
    if (const char *e = std::getenv("BMO_ATTN_SHAPE")) {
        Shape o{0, 0};
        if (std::sscanf(e, "%d,%d", &o.nw, &o.pf) == 2) s = o;
    }
    return s;
}

template <int D>
bool launch_shape(const DecodeParams &p, bool fused, hipStream_t stream, const Shape &s) {
#define BMO_SHAPE(NW_, PF_)                                \
    static_assert(shape_instantiated(Shape{NW_, PF_}));    \
    if (s.nw == NW_ && s.pf == PF_) {                      \
        launch_variant<D, NW_, PF_>(p, fused, stream);     \
        return true;                                       \
    }
    BMO_SHAPE(1, 1)
    BMO_SHAPE(1, 2)
    BMO_SHAPE(1, 3)
    BMO_SHAPE(2, 1)
    BMO_SHAPE(4, 1)
    BMO_SHAPE(8, 1)
    BMO_SHAPE(8, 2)
    BMO_SHAPE(16, 1)
#undef BMO_SHAPE
    static_assert(sizeof(kShapes) / sizeof(kShapes[0]) == 8, "kShapes lists the shapes dispatched above");
    return false;
}

}  // namespace

bool launch_decode(const DecodeParams &params, bool fused, hipStream_t stream) {
    const int64_t units = (int64_t) params.n_batch * params.n_heads;
    if (units <= 0) return true;
    DecodeParams p = params;
    p.q_per_kv = p.n_heads / p.n_kv;
    p.div_heads = make_fastdiv((uint32_t) p.n_heads);
    p.div_qkv = make_fastdiv((uint32_t) p.q_per_kv);
    p.div_ctx = make_fastdiv((uint32_t) p.g.n_ctx);
    const Shape s = pick_shape(units, p.g.n_groups, fused);
    if (p.g.head_dim == 128) {
        if (!launch_shape<128>(p, fused, stream, s)) launch_variant<128, 1, 1>(p, fused, stream);
    } else if (p.g.head_dim == 64) {
        if (!launch_shape<64>(p, fused, stream, s)) launch_variant<64, 1, 1>(p, fused, stream);
    } else {
        return false;
    }
    return true;
}

}  // namespace bmo
