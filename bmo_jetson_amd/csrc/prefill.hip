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
// needs positions back to pos0 - n_ctx + 1).  With one query head per kv
// head and at most 256 tokens, one workgroup reads each ring stripe: it
// quantizes the chunk into LDS, attends, and writes each chunk block into
// the ring once the ring tile holding the slot's old position has been
// dequantized (one kernel).  Otherwise one call runs three
// kernels in stream order:
//   stage_kernel   quantizes the chunk's bf16 K/V into a staging stripe with
//                  the ring's group layout (slot i = chunk token i);
//   prefill_kernel attention over the ring and the staged chunk;
//   commit_kernel  copies the staged blocks into their ring slots.
//
// prefill_kernel: a workgroup of QW waves serves 16*QB*QW queries of one
// (entry, head); each wave owns QB blocks of 16, so every K and V operand it
// reads from LDS feeds QB matrix instructions.  Keys stream through four LDS
// buffers in tiles of 32 positions: each thread of the loading waves holds
// its share of the Q4_0 bytes of the next tiles in registers and
// dequantizes the oldest two into free buffers (K and V row-major); one
// barrier publishes each pair of tiles.  A wave skips tiles that hold no key
// its queries may see, and the tiles are paired so that, where the causal
// and window masks allow, the two tiles of a pair are seen by different
// waves.  Each wave computes S^T = K Q^T with v_mfma_f32_16x16x32_f16 (the D
// layout of S^T puts 8 keys of one query in a lane, exactly the A layout the
// P.V product needs), runs an online softmax in the log2 domain and
// accumulates O += P V with the same instruction, its V operand read from
// the row-major tile with ds_read_b64_tr_b16.
// Precision.  The scores are as close as fp32 arithmetic on the bf16 q and
// the dequantized K: K enters the matrix cores as its codes (c - 8), exact
// in fp16, one product per 32-element block, and each block's fp16 scale d
// multiplies that product in fp32; q enters as q * 2^e, exact in fp16, with
// e chosen per query row, and scale * log2(e) * 2^-e multiplies the fp32
// score.  V enters as the fp16 value (c - 8) * d and the weights P as fp16,
// accumulation in fp32.  V values fit fp16 as the reference's F16 cache
// requires.
#include <limits.h>
#include <math.h>

#include "kernels.hpp"
#include "q4_0_device.hpp"

namespace bmo {

namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// Reads an int at a wave-uniform index through the scalar cache.  For
// arrays that no kernel writes while the reading kernel runs (session ids,
// positions), so the constant address space is exact.
__device__ __forceinline__ int load_scalar_i32(const int *ptr, int i) {
    return ((const __attribute__((address_space(4))) int *) ptr)[i];
}

template <bool B>
struct BoolC {
    static constexpr bool value = B;
};

constexpr int kTK = 32;          // keys per tile
constexpr float kRescale = 8.0f; // lazy rescale threshold, log2 units
// Running-max floor: far below any real score, so a query's first finite
// score always triggers a rescale, and finite, so a masked score (-inf)
// never does (and its weight exp2(-inf) is 0 with no select).
constexpr float kMaxFloor = -1.0e30f;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits) {
    return __builtin_bit_cast(float, bits << 16);
}

// ds_read_b64_tr_b16: within each 16-lane group, lanes 4j..4j+3 address 16
// consecutive halves of some row j (4 each); lane i receives element i of
// rows 0..3.
__device__ __forceinline__ half4_t lds_read_tr16(const _Float16 *p) {
    typedef __fp16 fp16x4 __attribute__((vector_size(8)));
    typedef __attribute__((address_space(3))) fp16x4 lds_fp16x4;
    return __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4 *) p));
}

// The value of v in lane (l & ~3) + (CTRL >> 2(l & 3)) & 3 (DPP quad_perm).
template <int CTRL>
__device__ __forceinline__ float quad_perm(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Maximum without operand canonicalization (v_maximum3_f32): scores are
// never NaN, and fmaxf's quieting of signalling NaNs costs an instruction per
// operand.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Workgroup barrier for LDS hand-off only: waits for this wave's LDS
// operations, not for its global loads (__syncthreads' fence would also wait
// for the loads of the tiles being prefetched).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Order of the 8 fp16 values dequantized from code dword c of a block
// (element 4c + kPerm[r]): the pairs the nibble masks produce.
__host__ __device__ constexpr int perm_elem(int r) {
    return (r & 4 ? 16 : 0) + (r & 1 ? 2 : 0) + ((r >> 1) & 1);
}

// Logical element of LDS column s of a dequantized row: slot 8c + r of a
// block holds element 4c + perm_elem(r).
__host__ __device__ constexpr int col_elem(int s) {
    return (s & ~31) + 4 * ((s & 31) >> 3) + perm_elem(s & 7);
}

// Place of key k's block scale within a block's 32 entries: keys 4c + v and
// 16 + 4c + v (v = 0..3) at 8c + v and 8c + 4 + v, the order in which lane
// group c holds the scores of its keys in the two S^T products of a tile.
__host__ __device__ constexpr int kd_slot(int k) { return 8 * ((k >> 2) & 3) + 4 * (k >> 4) + (k & 3); }

// The output store's float4 layout: lane 4qd + j of a 16-lane group holds
// column slot 16t + 4qd + j, element base(qd, t) + {0, 2, 1, 3}[j].
__host__ __device__ constexpr bool store_layout_matches() {
    for (int t = 0; t < 8; ++t)
        for (int n = 0; n < 16; ++n) {
            const int qd = n >> 2, j = n & 3;
            const int base = 32 * (t >> 1) + 8 * (t & 1) + 4 * (qd >> 1) + 16 * (qd & 1);
            if (col_elem(16 * t + n) != base + (j == 1 ? 2 : j == 2 ? 1 : j)) return false;
        }
    return true;
}
static_assert(store_layout_matches(), "output float4 layout");

// xor constants of dequant_dword: stored K nibbles are code ^ 8, V nibbles
// plain codes.
constexpr uint32_t kXorLoK = 0x64086408u, kXorHiK = 0x54805480u;
constexpr uint32_t kXorLoV = 0x64006400u, kXorHiV = 0x54005400u;

// Dequantizes code dword w (bytes 4c..4c+3 of a block) with fp16 scale bits
// d16 (low half) into 8 fp16 values in perm_elem order: (code - 8) * d, the
// subtraction exact, the product rounded to nearest.  A low nibble n under
// the fp16 pattern 0x6400 reads 1024 + n; a high nibble, left in place
// (n << 4) under 0x5400, reads 64 + n, so no shift per nibble is needed.
// xlo/xhi are those patterns, K's with the stored bit 3 flipped back (the xor
// touches only nibble bits and the pattern's own, disjoint bits).
// SCALED false: the codes alone, (code - 8) exactly (d16 unused).
template <bool SCALED = true>
__device__ __forceinline__ half8_t dequant_dword(uint32_t w, uint32_t d16, uint32_t xlo, uint32_t xhi) {
    const half2_t off_lo = {(_Float16) -1032.0f, (_Float16) -1032.0f};
    const half2_t off_hi = {(_Float16) -72.0f, (_Float16) -72.0f};
    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t) d16);
    const half2_t dd = {d, d};
    const uint32_t y = w >> 8;
    half2_t r[4];
    r[0] = __builtin_bit_cast(half2_t, (w & 0x000F000Fu) ^ xlo) + off_lo;
    r[1] = __builtin_bit_cast(half2_t, (y & 0x000F000Fu) ^ xlo) + off_lo;
    r[2] = __builtin_bit_cast(half2_t, (w & 0x00F000F0u) ^ xhi) + off_hi;
    r[3] = __builtin_bit_cast(half2_t, (y & 0x00F000F0u) ^ xhi) + off_hi;
    if constexpr (SCALED) {
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] *= dd;
    }
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
// Thread indices fit 32 bits (the API bounds the chunk's block count).
__global__ __launch_bounds__(256) void stage_kernel(PrefillParams p) {
    const int nblk = p.g.head_dim / kQK;
    const int per_row = p.n_kv * nblk * 2;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= per_row * p.n_batch * p.n_tok) return;
    const int r = t / per_row;  // b * n_tok + i
    int rem = t - r * per_row;
    const int which = rem / (p.n_kv * nblk);
    rem -= which * (p.n_kv * nblk);
    const int h = rem / nblk;
    const int blk = rem - h * nblk;
    const int b = r / p.n_tok;
    const int i = r - b * p.n_tok;
    const uint16_t *src = (which == 0 ? p.k : p.v) + ((int64_t) r * p.n_kv + h) * p.g.head_dim + blk * kQK;
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
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= p.n_batch * p.n_tok * p.n_kv * nblk) return;
    const int blk = t % nblk;
    const int h = (t / nblk) % p.n_kv;
    const int i = (t / (nblk * p.n_kv)) % p.n_tok;
    const int b = t / (nblk * p.n_kv * p.n_tok);
    const int sid = p.session_ids ? p.session_ids[b] : b;
    const int pos0 = p.pos0[b];
    if (sid < 0 || sid >= p.g.n_sessions || pos0 < 0 || pos0 > INT_MAX - p.n_tok) return;
    const int slot = (pos0 + i) % p.g.n_ctx;
    const uint8_t *src = p.stage + p.sg.stripe_offset(0, b, h);
    uint8_t *dst = p.base + p.g.stripe_offset(p.layer, sid, h);
    *reinterpret_cast<uint4 *>(dst + p.g.kcode_offset(slot, blk)) =
        *reinterpret_cast<const uint4 *>(src + p.sg.kcode_offset(i, blk));
    *reinterpret_cast<uint4 *>(dst + p.g.vcode_offset(slot, blk)) =
        *reinterpret_cast<const uint4 *>(src + p.sg.vcode_offset(i, blk));
    *reinterpret_cast<uint32_t *>(dst + p.g.scale_offset(slot, blk)) =
        *reinterpret_cast<const uint32_t *>(src + p.sg.scale_offset(i, blk));
}

// Launch bounds: 64 * QW threads, one workgroup per CU (QW = 16: four waves
// per SIMD, at most 128 VGPRs each, which holds the accumulators, the query
// operands and the fetched tile bytes without spilling).
//
// DIRECT: every (entry, kv head) stripe is read by this one workgroup (one
// query head per kv head, the whole chunk in one workgroup).  The workgroup
// then quantizes its chunk's K/V itself into LDS (the staging stripe's role),
// reads the chunk's keys from there, and writes the chunk's blocks into the
// ring during the tile loop, each once no wave reads its slot's old contents
// from memory any more; no stage or commit kernel runs.
// Phase timestamps, in a diagnostic build only (BMO_PREFILL_PHASES=1,
// libbmo_attn_phases.so, which bench.py --prefill-phases reads): lane 0 of
// every wave of the first 512 workgroups records s_memtime at its phase
// boundaries, plus s_memrealtime at its start and end, into a device array:
// record [0] real-time start, [1] start, [2] query rows converted, [3] chunk
// quantized and published (DIRECT), [4] loop start, [5] loop end, [6] end,
// [7] real-time end, [8] the number of loop stamps; loop stamps from [16]
// on, four per barrier period: the iteration's start, arrival at the
// barrier, departure, and the end of the ring writes (DIRECT waves without
// items).  Scheduling barriers keep the compiler from moving work across a
// stamp.  The normal build compiles none of it.
#ifndef BMO_PREFILL_PHASES
#define BMO_PREFILL_PHASES 0
#endif
#if BMO_PREFILL_PHASES
constexpr int kPhaseUnits = 512;
constexpr int kPhaseRec = 128;
__device__ uint64_t g_prefill_phases[kPhaseUnits * 16 * kPhaseRec];
#define BMO_PHASE(i)                                                           \
    do {                                                                       \
        __builtin_amdgcn_sched_barrier(0);                                     \
        const uint64_t t_ = __builtin_amdgcn_s_memtime();                      \
        __builtin_amdgcn_sched_barrier(0);                                     \
        if (lane == 0) phase_rec[i] = t_;                                      \
    } while (0)
#define BMO_PHASE_LOOP()                                                       \
    do {                                                                       \
        __builtin_amdgcn_sched_barrier(0);                                     \
        const uint64_t t_ = __builtin_amdgcn_s_memtime();                      \
        __builtin_amdgcn_sched_barrier(0);                                     \
        if (lane == 0 && phase_n < kPhaseRec - 16) phase_rec[16 + phase_n] = t_; \
        ++phase_n;                                                             \
    } while (0)
#else
#define BMO_PHASE(i) \
    do {             \
    } while (0)
#define BMO_PHASE_LOOP() \
    do {                 \
    } while (0)
#endif

template <int D, int QW, int QB, bool DIRECT, bool ALIGNED>
__global__ __launch_bounds__(64 * QW, QW / 4) void prefill_kernel(PrefillParams p) {
    static_assert(!DIRECT || ALIGNED, "the direct path serves rings of a multiple of 32 slots");
    constexpr int NBLK = D / kQK;
    // LDS rows (fp16) of D + 16 halves, K and V alike: with that stride the
    // K operand reads (ds_read_b128: lane l reads a 16-byte chunk of key
    // l % 16) and the V operand reads (ds_read_b64_tr_b16) are free of bank
    // conflicts on gfx950, as SQ_LDS_BANK_CONFLICT shows for both head dims.
    // Rows of D + 8 cost every K read 0.8 extra LDS cycles on average (3.2
    // instead of 2.4), on the reads every wave issues right after a barrier.
    constexpr int KROW = D + 16;
    constexpr int VROW = D + 16;
    constexpr int QWV = 16 * QB;   // queries per wave
    constexpr int QT = QWV * QW;   // queries per workgroup
    constexpr int NT = D / 16;     // output column tiles
    constexpr int NTHR = 64 * QW;
    // dequantization items per tile: (K/V, key, block, 8-byte half)
    constexpr int ITEMS = 2 * kTK * NBLK * 2;
    constexpr int IPT = (ITEMS + NTHR - 1) / NTHR;
    constexpr int G = keys_per_group(D);
    static_assert((G & (G - 1)) == 0, "slot groups are a power of two");

    // Tiles per barrier: TPB tiles are dequantized, published by one barrier
    // and then multiplied, through 2 * TPB LDS buffers, so the waves of a
    // workgroup synchronize once per TPB tiles.
    constexpr int TPB = 2;
    constexpr int NBUF = 2 * TPB;
    // Blocks whose S^T products are issued together (operands and scales
    // read first): all of them on the direct path; two on the staged path,
    // whose fetch holds more registers (four spill there).
    constexpr int SB = DIRECT ? NBLK : (NBLK < 2 ? NBLK : 2);
    static_assert(NBLK % SB == 0, "whole groups of blocks");

    // K rows hold the codes (c - 8), exact in fp16, and sKd the blocks'
    // fp16 scales d: element (key k, block bb) at bb * 32 + kd_slot(k), so
    // that lane group c reads the scales of its keys 4c..4c+3 and
    // 16+4c..16+4c+3 of a block as one 16-byte piece.  The scores then take
    // (c - 8) . q per block from the matrix cores and the factor d in fp32:
    // an fp16 (c - 8) * d would be rounded to 11 bits, an error that large
    // query elements amplify past the tolerance.
    __shared__ __align__(16) _Float16 sK[NBUF][kTK * KROW];
    __shared__ __align__(16) _Float16 sKd[NBUF][kTK * NBLK];
    __shared__ __align__(16) _Float16 sV[NBUF][kTK * VROW];
    __shared__ __align__(16) _Float16 sOnes[8];  // B operand of the row-sum product
    if (threadIdx.x < 8) sOnes[threadIdx.x] = (_Float16) 1.0f;  // (published by the loop's first barrier)
    // DIRECT: the chunk's blocks in ring format: codes [K/V][token][block]
    // (K as code ^ 8), scale dwords [token][block] (K low half, V high)
    __shared__ __align__(16) uint4 sCc[DIRECT ? 2 * QT * NBLK : 1];
    __shared__ __align__(16) uint32_t sCs[DIRECT ? QT * NBLK : 1];

    const int lane = threadIdx.x & 63;
    // wave-uniform (readfirstlane), so that everything derived from it --
    // the tile skip, the whole-tile test -- is a scalar branch
    const int wave = __builtin_amdgcn_readfirstlane((int) threadIdx.x >> 6);
#if BMO_PREFILL_PHASES
    uint64_t *const phase_rec = g_prefill_phases + ((size_t) (blockIdx.x % kPhaseUnits) * QW + wave) * kPhaseRec;
    int phase_n = 0;
    if (lane == 0) phase_rec[0] = __builtin_amdgcn_s_memrealtime();
    BMO_PHASE(1);
#endif
    // (scalars: the divisions run on the vector unit, readfirstlane keeps
    // their results, and the addresses derived from them, in SGPRs)
    const int n_qt = (p.n_tok + QT - 1) / QT;
    const int unit = __builtin_amdgcn_readfirstlane((int) blockIdx.x / n_qt);
    const int qt = (int) blockIdx.x - unit * n_qt;
    const int b = __builtin_amdgcn_readfirstlane(unit / p.n_heads);
    const int h = unit - b * p.n_heads;
    const int i0 = qt * QT;
    const int q_per_kv = p.n_heads / p.n_kv;
    const int kvh = __builtin_amdgcn_readfirstlane(h / q_per_kv);

    // Scalar loads: as vector loads they returned only after the loads that
    // the workgroup's other waves had issued before them (up to 5 us for the
    // last wave at cfg5, measured), and that wave's own loads waited for
    // them.  (The call's time at cfg5 is the same either way: there the
    // prologue's loads are bandwidth-bound.)
    const int sid = p.session_ids ? load_scalar_i32(p.session_ids, b) : b;
    const int pos0 = load_scalar_i32(p.pos0, b);
    const int nq = min(QT, p.n_tok - i0);  // valid queries of this workgroup
    if (sid < 0 || sid >= p.g.n_sessions || pos0 < 0 || pos0 > INT_MAX - p.n_tok) {
        for (int e = threadIdx.x; e < nq * D; e += blockDim.x) {
            const int qi = e / D;
            p.out[(((int64_t) b * p.n_tok + i0 + qi) * p.n_heads + h) * D + e % D] = 0.0f;
        }
        return;
    }
    const int n_ctx = p.g.n_ctx;
    const int p_first = pos0 + i0;
    const int p_last = pos0 + i0 + nq - 1;
    const int k_lo = max(0, p_first - n_ctx + 1);
    // Tiles: the ring's keys k_lo .. pos0 - 1 in tiles aligned to 32
    // positions (tiles 0 .. n_rt - 1), then the chunk's keys in tiles
    // aligned to pos0, so that no tile mixes ring and chunk keys.  A key of a
    // tile outside its source's live range (ring [k_lo, pos0), chunk
    // [pos0, p_last]) is dequantized with scale 0 and masked.
    const int r_start = k_lo & ~(kTK - 1);
    const int n_rt = k_lo < pos0 ? (pos0 - 1 - r_start) / kTK + 1 : 0;
    const int c_start = pos0 + ((max(k_lo, pos0) - pos0) & ~(kTK - 1));
    const int n_tiles = n_rt + (p_last - c_start) / kTK + 1;
    // (helpers capture by value: a select between captured references can
    // keep the closures in scratch memory, as noted at src_diff below)
    auto tile_t0 = [=](int T) { return T < n_rt ? r_start + T * kTK : c_start + (T - n_rt) * kTK; };
    // Processing order.  A query at position P sees ring tile r only while
    // P <= (last key of r) + n_ctx - 1, and chunk tile c only from P >=
    // (first key of c) on: ring tiles are seen by the early waves, chunk
    // tiles by the late ones.  gam puts the first key of chunk tile r + gam
    // past the last query that sees ring tile r.  That key is a multiple of
    // 32 positions after p_first, and each wave's first query is a multiple
    // of its 16 or 32 queries after p_first, so a wave that sees the chunk
    // tile starts at or after it and cannot see the ring tile: processing
    // them as the two tiles of one barrier period lets each wave multiply
    // one of them instead of some wave multiplying both.  The first
    // 2 n_pair tiles alternate ring r / chunk r + gam, the rest follow in
    // index order.  (Any order gives the same result up to rounding: the
    // softmax is online.)
    const int gam = (r_start + kTK - 2 - p_first + n_ctx) / kTK + 1 + (p_first - c_start) / kTK;
    const int n_pair = max(0, min(n_rt, n_tiles - n_rt - gam));
    // (selects, not branches: the callers' blocks stay whole)
    auto tile_of = [=](int i) {
        const int paired = (i & 1) ? n_rt + (i >> 1) + gam : (i >> 1);
        const int j = i - 2 * n_pair;             // position among the unpaired tiles
        const int jc = j - (n_rt - n_pair);       // ... among the unpaired chunk tiles
        const int rest = j < n_rt - n_pair ? n_pair + j : n_rt + (jc < gam ? jc : jc + n_pair);
        return i < 2 * n_pair ? paired : rest;    // padding positions map to themselves
    };
    const uint8_t *ring = p.base + p.g.stripe_offset(p.layer, sid, kvh);
    const uint8_t *stage = p.stage + p.sg.stripe_offset(0, b, kvh);
    const uint32_t ring_gs = (uint32_t) p.g.group_stride;
    const uint32_t stage_gs = (uint32_t) p.sg.group_stride;
    // Staging minus ring: the fetch selects between the two sources as ring
    // + (staged ? difference : 0).  (A select between two captured values
    // becomes, once hipcc simplifies the lambda, a select between two
    // addresses in its closure, which keeps the closure and everything it
    // refers to in scratch memory.)
    const int64_t src_diff = stage - ring;
    const int32_t gs_diff = (int32_t) (stage_gs - ring_gs);
    const int rg_last = p.g.n_groups - 1;                    // last group of a ring stripe
    const int glast_diff = p.sg.n_groups - p.g.n_groups;    // ... staging minus ring

    // This thread's items: item j is (K/V, key, block, 8-byte half) =
    // (which, key, bb, hf) of every tile.  A wave's 64 items share `which`
    // and the key's slot group key / G (static_asserts below), so those are
    // scalars and a tile's loads use a scalar group address plus these
    // per-item offsets inside the group.
    static_assert((2 * kTK * NBLK) % 64 == 0, "a wave's items share K/V");
    static_assert(G % (32 / NBLK) == 0, "a wave's items share a slot group");
    int it_key[IPT], it_grp[IPT];
    bool it_v[IPT];
    uint32_t it_code[IPT], it_scale[IPT], it_lds[IPT], it_slds[IPT];
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
        const int it = min((int) threadIdx.x + j * NTHR, ITEMS - 1);
        const int hf = it & 1;
        const int bb = (it >> 1) % NBLK;
        const int key = (it >> 1) / NBLK % kTK;
        const int which = __builtin_amdgcn_readfirstlane(it / (2 * kTK * NBLK));
        it_key[j] = key;
        it_grp[j] = __builtin_amdgcn_readfirstlane(key / G);
        it_v[j] = which != 0;
        it_code[j] = (uint32_t) ((key % G) * (D / 2) + bb * 16 + which * kVCodeOff + 8 * hf);
        it_scale[j] = (uint32_t) (kScaleOff + ((key % G) * NBLK + bb) * 4);
        it_lds[j] = (uint32_t) (((which * QT + key) * NBLK + bb) * 16 + 8 * hf);
        it_slds[j] = (uint32_t) ((key * NBLK + bb) * 4);
    }

    // Raw tile bytes, fetched PF tiles ahead: this thread's items.  Every
    // fetch issues its loads (tiles whose keys come from elsewhere -- DIRECT
    // chunk tiles, padding tiles past the end -- read the ring stripe's first
    // slots, which stay cached), so the number of loads in flight is the same
    // on every path and the compiler's waits stay exact.  Depth: 3 tiles
    // with 16 waves (4 per SIMD hide the rest; at cfg5 depth 7 measured
    // 85.7 vs 84.0 us in one earlier build and 78.4 vs 74.2 us in a later
    // one, where it spilled 3 VGPRs; depth 3 spills in no instantiation), 7
    // with fewer.
    constexpr int PF = QW >= 16 ? 3 : 7;
    static_assert((PF + 1) % NBUF == 0, "the unrolled slot must determine the LDS buffer");
    uint2 raw[PF + 1][IPT];
    uint32_t rawd[PF + 1][IPT];
    int f_next = 0;                        // next position in processing order to fetch
    const int r_slot = r_start % n_ctx;    // ring slot of ring tile 0
    auto fetch = [&](uint2 (&rw)[IPT], uint32_t (&rd)[IPT]) {
        const int T = tile_of(f_next++);
        const bool ring_t = T < n_rt;
        // a ring tile's first slot (r_start + 32 T) % n_ctx; 32 T <= n_ctx
        // + 29, so one subtraction suffices when n_ctx is a multiple of 32
        int slot0 = r_slot + T * kTK;
        if (slot0 >= n_ctx) slot0 -= n_ctx;
        if (!ALIGNED && slot0 >= n_ctx) slot0 %= n_ctx;
        const bool staged_t = !DIRECT && !ring_t && T < n_tiles;
        // Scalar: the slot group of the tile's first key (ALIGNED: a ring
        // tile's slots t0 % n_ctx .. +31 never wrap) and the last group the
        // tile may address; keys past the staged chunk clamp to its last
        // group, and a tile with no keys to load reads group 0 only, so
        // every address stays inside the stripe.
        const int g_first = staged_t ? (tile_t0(T) - pos0) / G : ring_t ? slot0 / G : 0;
        const int g_last = (ring_t || staged_t) ? rg_last + (staged_t ? glast_diff : 0) : 0;
        const uint8_t *gsrc = ring + (staged_t ? src_diff : 0);
        const uint32_t gs = ring_gs + (uint32_t) (staged_t ? gs_diff : 0);
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            const uint8_t *gp = gsrc + (uint64_t) (uint32_t) min(g_first + it_grp[j], g_last) * gs;
            uint32_t co = it_code[j], so = it_scale[j];
            if constexpr (!ALIGNED) {
                // the ring's slots wrap inside a tile: per-key slot
                if (ring_t) {
                    const uint32_t slot = (uint32_t) (slot0 + it_key[j]) % (uint32_t) n_ctx;
                    const uint32_t row = slot % G;
                    const uint32_t in_row = it_code[j] - (uint32_t) (it_key[j] % G) * (D / 2);
                    gp = ring + (uint64_t) (slot / G) * ring_gs;
                    co = row * (D / 2) + in_row;
                    so = it_scale[j] + (row - (uint32_t) (it_key[j] % G)) * (NBLK * 4);
                }
            }
            rw[j] = *reinterpret_cast<const uint2 *>(gp + co);
            // the whole scale dword: a 16-bit load would be zero-extended
            // into a copy that hipcc places at the loop's back edge, waiting
            // for the load there
            rd[j] = *reinterpret_cast<const uint32_t *>(gp + so);
        }
    };
    // Dequantizes fetched items of tile T into LDS buffer `buf`: K and V
    // row-major, the values of code dword cd at slots 8cd..8cd+7 of the block
    // (the order the query operand uses; col_elem maps a column back to its
    // element).
    auto deposit = [&](int buf, int T, const uint2 (&rw)[IPT], const uint32_t (&rd)[IPT]) {
        const bool ring_t = T < n_rt;
        const int t0 = tile_t0(T);
        const int lo = ring_t ? k_lo : pos0;
        const uint32_t span = (uint32_t) ((ring_t ? pos0 - 1 : p_last) - lo);
        // DIRECT chunk tiles: the chunk's blocks in LDS (clamped for padding
        // tiles, whose keys are all dead)
        const uint32_t coff = (uint32_t) min(max(t0 - pos0, 0), QT - kTK) * (NBLK * 16);
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            const int it = threadIdx.x + j * NTHR;
            if (it < ITEMS) {
                const int key = it_key[j];
                const bool live = (uint32_t) (t0 + key - lo) <= span;
                uint2 w = rw[j];
                uint32_t sd = rd[j];
                if constexpr (DIRECT) {
                    const uint8_t *cp = reinterpret_cast<const uint8_t *>(sCc) + it_lds[j] + coff;
                    const uint2 cw = *reinterpret_cast<const uint2 *>(cp);
                    const uint32_t cs = *reinterpret_cast<const uint32_t *>(
                        reinterpret_cast<const uint8_t *>(sCs) + it_slds[j] + coff / 4);
                    w = ring_t ? w : cw;
                    sd = ring_t ? sd : cs;
                }
                const uint32_t dw = it_v[j] ? sd >> 16 : sd;
                const uint32_t d16 = live ? dw : 0u;
                const int bb = (it >> 1) % NBLK;
                const int hf = it & 1;
                half8_t v0, v1;
                _Float16 *dst;
                if (it_v[j]) {  // (wave-uniform)
                    v0 = dequant_dword(w.x, d16, kXorLoV, kXorHiV);
                    v1 = dequant_dword(w.y, d16, kXorLoV, kXorHiV);
                    dst = &sV[buf][key * VROW + bb * kQK + 16 * hf];
                } else {
                    v0 = dequant_dword<false>(w.x, 0u, kXorLoK, kXorHiK);
                    v1 = dequant_dword<false>(w.y, 0u, kXorLoK, kXorHiK);
                    dst = &sK[buf][key * KROW + bb * kQK + 16 * hf];
                    // a dead key's scale is 0, so its (finite) block dot
                    // products add nothing before the mask replaces them
                    if (hf == 0) sKd[buf][bb * kTK + kd_slot(key)] = __builtin_bit_cast(_Float16, (uint16_t) d16);
                }
                *reinterpret_cast<half8_t *>(dst) = v0;
                *reinterpret_cast<half8_t *>(dst + 8) = v1;
            }
        }
    };


    // Loads, in the order they are waited for (loads return in order): the
    // query rows, the first PF tiles, then (DIRECT) the chunk's bf16 K/V; the
    // query conversion runs while the later ones are in flight.
    // Query operands (B of S^T = K Q^T): for query block qb lane l holds
    // query n = l % 16 of that block, block b's values at elements
    // 4c + perm_elem(r), c = l / 16.  Rows past the chunk read row 0 and are
    // zeroed.
    const int n = lane & 15;
    const int c = lane >> 4;
    const int wq0 = i0 + wave * QWV;  // first query of this wave
    uint2 qlo[QB][NBLK], qhi[QB][NBLK];
    int mrel[QB];  // this lane's query position minus 4c (mask arithmetic)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const int qi = wq0 + qb * 16 + n;
        mrel[qb] = pos0 + qi - 4 * c;
        const uint16_t *qrow = p.q + (((int64_t) b * p.n_tok + (qi < p.n_tok ? qi : 0)) * p.n_heads + h) * D;
#pragma unroll
        for (int bb = 0; bb < NBLK; ++bb) {
            qlo[qb][bb] = *reinterpret_cast<const uint2 *>(qrow + bb * kQK + 4 * c);
            qhi[qb][bb] = *reinterpret_cast<const uint2 *>(qrow + bb * kQK + 4 * c + 16);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // The trip count is padded to a multiple of PF + 1 tiles (an empty tile
    // past the chunk is zeros and skipped by every wave), so the unrolled
    // body has no per-tile condition around its loads.  The scheduling
    // barriers keep hipcc from hoisting later loads above earlier ones, so
    // that each wait covers the oldest loads only.
    // Waves with dequantization items (the first ITEMS / 64: 8 of 16 at
    // head_dim 128, 4 at head_dim 64) fetch and deposit; the others only
    // multiply.  Wave-uniform.
    const bool has_items = (IPT - 1) * NTHR + wave * 64 < ITEMS;
    if (has_items) {
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            fetch(raw[j], rawd[j]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // DIRECT: this thread's blocks of the chunk's K and V (bf16), all in
    // flight at once
    constexpr int NQ = DIRECT ? (2 * QT * NBLK + NTHR - 1) / NTHR : 1;
    uint4 braw[NQ][4];
    if constexpr (DIRECT) {
        const int nblocks = 2 * p.n_tok * NBLK;
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            const int e = min((int) threadIdx.x + k * NTHR, nblocks - 1);
            const int bb = e % NBLK;
            const int i = (e / NBLK) % p.n_tok;
            const int which = e / (NBLK * p.n_tok);
            const uint4 *src = reinterpret_cast<const uint4 *>(
                (which == 0 ? p.k : p.v) + (((int64_t) b * p.n_tok + i) * p.n_kv + kvh) * D + bb * kQK);
#pragma unroll
            for (int cq = 0; cq < 4; ++cq) braw[k][cq] = src[cq];
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // Query operands: each row is scaled by the power of two 2^eq that puts
    // its largest magnitude in [2^14, 2^15), so every bf16 element (8
    // significant bits) is exact in fp16 down to 2^-31 of the row's maximum
    // and no row overflows, whatever its range.  fq = scale * log2(e) *
    // 2^-eq, applied to the fp32 scores, carries the rest of the factor.
    // (A NaN or an infinity in a row makes that query's output NaN.)
    half8_t qop[QB][NBLK];
    float fq[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const bool q_ok = wq0 + qb * 16 + n < p.n_tok;
        float xq[NBLK][8];
        float amax = 0.0f;
#pragma unroll
        for (int bb = 0; bb < NBLK; ++bb) {
            // elements 4c + {0,1,2,3} in lo, 4c + 16 + {0,1,2,3} in hi; the
            // operand order is perm_elem: 0, 2, 1, 3, 16, 18, 17, 19
            const uint2 lo = qlo[qb][bb], hi = qhi[qb][bb];
            const uint32_t e[8] = {lo.x & 0xFFFFu, lo.y & 0xFFFFu, lo.x >> 16, lo.y >> 16,
                                   hi.x & 0xFFFFu, hi.y & 0xFFFFu, hi.x >> 16, hi.y >> 16};
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                xq[bb][r] = q_ok ? bf16_to_f32(e[r]) : 0.0f;
                amax = fmaxf(amax, fabsf(xq[bb][r]));
            }
        }
        // the row's other elements are in lanes n + 16, n + 32, n + 48
        amax = fmaxf(amax, __shfl_xor(amax, 16));
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        const int eq = 15 - __builtin_amdgcn_frexp_expf(amax);  // amax = m 2^ex, m in [0.5, 1)
        fq[qb] = __builtin_amdgcn_ldexpf(p.qscale, -eq);
#pragma unroll
        for (int bb = 0; bb < NBLK; ++bb)
#pragma unroll
            for (int r = 0; r < 8; ++r) qop[qb][bb][r] = (_Float16) __builtin_amdgcn_ldexpf(xq[bb][r], eq);
    }
    BMO_PHASE(2);
    // this wave's query positions and the keys they may see (wave-uniform)
    const int wq1 = min(wq0 + QWV - 1, p.n_tok - 1);
    const int w_hi = pos0 + wq1;
    const int w_lo = pos0 + wq0 - n_ctx + 1;

    // Accumulators: acc[qb][t] = O columns 16t..16t+15, and accl[qb] = P
    // times a ones operand, whose every column is the weight sum of a query
    // row; both use the D layout (lane l: column l % 16, queries 4c + v), so
    // the final division needs no cross-lane exchange.
    // Softmax state per query block (log2 domain).  A lane's scores are
    // fq * (sum over blocks of d * (c - 8) . q') - off, one fma from the
    // blocks' sum, with off a per-query offset; dl = running max - off.  off
    // is 0 until a query's first rescale, which sets off to the running max
    // (dl = 0) and is exact then because the scores were taken from 0.  A
    // rescale happens whenever a score exceeds the running max by kRescale,
    // so after the test below every query with a finite score has dl = 0
    // and its weights are exp2 of the scores themselves; a query still at
    // the floor has only -inf scores, whose weights are 0 either way.
    float dl[QB];
    float cneg[QB];  // -off
    float4_t acc[QB][NT];
    float4_t accl[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        dl[qb] = kMaxFloor;
        cneg[qb] = 0.0f;
        accl[qb] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[qb][t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }

    auto compute = [&](int buf, int T) {
        const bool ring_t = T < n_rt;
        const int t0 = tile_t0(T);
        if (wq0 >= p.n_tok || t0 > w_hi || t0 + kTK - 1 < w_lo) return;  // nothing to see
        // S^T for keys 0..15 and 16..31 of the tile: lane l gets keys
        // 4c + v (and 16 + 4c + v) of query n of each query block.  One
        // product per block over its 32 codes (exact integers times exact
        // fp16 q'), scaled by the block's d in fp32.
        const float4_t zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
        float4_t s[QB][2];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
            for (int b0 = 0; b0 < NBLK; b0 += SB) {
                // SB blocks' operands and scales first, then their independent
                // products, then the scaling: the products issue back to back
                // instead of one LDS round trip each
                half8_t kop[SB];
                half4_t dv[SB];  // d of keys sub * 16 + 4c + v
#pragma unroll
                for (int j = 0; j < SB; ++j) {
                    const int bb = b0 + j;
                    kop[j] = *reinterpret_cast<const half8_t *>(&sK[buf][(sub * 16 + n) * KROW + bb * kQK + 8 * c]);
                    dv[j] = *reinterpret_cast<const half4_t *>(&sKd[buf][bb * kTK + 8 * c + 4 * sub]);
                }
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    float4_t t[SB];
#pragma unroll
                    for (int j = 0; j < SB; ++j)
                        t[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[j], qop[qb][b0 + j], zero4, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        float a = b0 == 0 ? 0.0f : s[qb][sub][v];
#pragma unroll
                        for (int j = 0; j < SB; ++j) a = fmaf(t[j][v], (float) dv[j][v], a);
                        s[qb][sub][v] = a;
                    }
                }
            }
        }
        // Mask (causal + window) unless every key of the tile is visible to
        // every query of the wave.  Query rows past the chunk are left
        // unmasked: their scores are finite and their outputs never stored.
        // A ring tile's keys must also precede pos0 (its last tile may reach
        // into the chunk's positions, which the chunk tiles supply).
        const bool whole = t0 + kTK - 1 <= (ring_t ? pos0 - 1 : pos0 + wq0) && t0 > w_hi - n_ctx;
        // the lane's 8 scores as scalars: masking and the rescale shift then
        // update them in place on both paths
        float sv[QB][8];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int k = 0; k < 8; ++k) sv[qb][k] = fmaf(s[qb][k >> 2][k & 3], fq[qb], cneg[qb]);
        if (!whole) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                // key t0 + 16 sub + 4c + v is visible to query position P iff
                // P - n_ctx < t <= P (and t < pos0 in a ring tile; every
                // P >= pos0), i.e. 16 sub + v in (rel - n_ctx, rel_hi]
                const int rel = mrel[qb] - t0;
                const int rel_hi = ring_t ? pos0 - 1 - 4 * c - t0 : rel;
#pragma unroll
                for (int sub = 0; sub < 2; ++sub)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int kk = sub * 16 + v;
                        const bool ok = kk <= rel_hi && kk > rel - n_ctx;
                        sv[qb][sub * 4 + v] = ok ? sv[qb][sub * 4 + v] : -INFINITY;
                    }
            }
        }
        half8_t pop[QB];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            // This lane's 8 scores (relative to off) against the running
            // max; the exact per-query maximum (a cross-lane reduction) is
            // only needed when some score exceeds the running max by
            // kRescale.
            float tmax = vmax(vmax(vmax(sv[qb][0], sv[qb][1]), sv[qb][2]),
                              vmax(vmax(vmax(sv[qb][3], sv[qb][4]), sv[qb][5]), vmax(sv[qb][6], sv[qb][7])));
            if (__any(tmax > dl[qb] + kRescale)) {
                tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
                tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
                const bool need = tmax > dl[qb] + kRescale;
                const float alpha = need ? __builtin_amdgcn_exp2f(dl[qb] - tmax) : 1.0f;
                // the new running max becomes off: shift it, and this tile's
                // products, by tmax
                const float shift = need ? tmax : 0.0f;
                dl[qb] = need ? 0.0f : dl[qb];
                cneg[qb] -= shift;
#pragma unroll
                for (int k = 0; k < 8; ++k) sv[qb][k] -= shift;
                // acc rows are queries 4c + v: fetch their alphas from lanes 4c + v
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float av = __shfl(alpha, 4 * c + v);
                    accl[qb][v] *= av;
#pragma unroll
                    for (int t = 0; t < NT; ++t) acc[qb][t][v] *= av;
                }
            }
#pragma unroll
            for (int sub = 0; sub < 2; ++sub)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    pop[qb][sub * 4 + v] = (_Float16) __builtin_amdgcn_exp2f(sv[qb][sub * 4 + v]);
            // the all-ones operand from LDS for each product (a volatile LDS
            // read, so that it holds no registers between tiles; through a
            // generic pointer it would become a flat load that waits for
            // every load in flight)
            const half8_t ones = *(const volatile __attribute__((address_space(3))) half8_t *) sOnes;
            accl[qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pop[qb], ones, accl[qb], 0, 0, 0);
        }
        // O += P V: B operand lane l = column t*16 + n of the tile, keys
        // 4c..4c+3 and 16+4c..16+4c+3 (the key order of pop), read with two
        // transposing loads (lane 4j + mm of the group addresses chunk mm of
        // key row 4c + j, resp. 16 + 4c + j), shared by the query blocks
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const _Float16 *vb = &sV[buf][(4 * c + (n >> 2)) * VROW + t * 16 + 4 * (n & 3)];
            const half4_t lo = lds_read_tr16(vb);
            const half4_t hi = lds_read_tr16(vb + 16 * VROW);
            const half8_t vop = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
                acc[qb][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pop[qb], vop, acc[qb][t], 0, 0, 0);
        }
    };

    // DIRECT: the chunk's K and V blocks (bf16 -> Q4_0, the append
    // quantizer) into LDS in ring format; the barrier publishes them
    auto quantize_chunk = [&]() {
        const int nblocks = 2 * p.n_tok * NBLK;
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            const int e = min((int) threadIdx.x + k * NTHR, nblocks - 1);
            const int bb = e % NBLK;
            const int i = (e / NBLK) % p.n_tok;
            const int which = e / (NBLK * p.n_tok);
            float x[kQK];
#pragma unroll
            for (int cq = 0; cq < 4; ++cq) {
                const uint4 u = braw[k][cq];
                const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    x[8 * cq + 2 * jj] = bf16_to_f32(wv[jj] & 0xFFFFu);
                    x[8 * cq + 2 * jj + 1] = bf16_to_f32(wv[jj] >> 16);
                }
            }
            uint16_t d16;
            uint32_t qs[4];
            quantize_block_q4_0(x, d16, qs);
            if ((int) threadIdx.x + k * NTHR < nblocks) {
                const uint32_t flip = which == 0 ? 0x88888888u : 0u;
                sCc[(which * QT + i) * NBLK + bb] = make_uint4(qs[0] ^ flip, qs[1] ^ flip, qs[2] ^ flip, qs[3] ^ flip);
                reinterpret_cast<uint16_t *>(&sCs[i * NBLK + bb])[which] = d16;
            }
        }
        lds_barrier();
    };
    // The tile at position i of the processing order lives in raw slot
    // i % (PF + 1) and LDS buffer i % NBUF; its loads are issued PF positions
    // ahead, into the slot of position i - 1.  Buffer safety: the barrier of
    // a tile pair follows every wave's multiplication of the pair before, so
    // writing a buffer NBUF positions later is safe.
    if constexpr (DIRECT) quantize_chunk();
    BMO_PHASE(3);
    // DIRECT: the chunk's blocks go into their ring slots (pos0 + i) % n_ctx
    // while the tiles are multiplied.  Chunk key i replaces old position
    // pos0 + i - n_ctx, which only its ring tile carries (a 17th ring tile,
    // sharing slots with the first, is live only at slots of positions below
    // pos0 - n_ctx), and every wave reads that tile from LDS once it is
    // deposited; the processing order visits the ring tiles in increasing
    // order.  So once the ring tiles below r_done are published, keys whose
    // old position precedes r_start + 32 r_done can be written.  The waves
    // without dequantization items write them right after each barrier:
    // they issue no global loads in the loop, so the stores delay no wait.
    // No other workgroup reads this stripe.  (Loads of padding tiles read
    // group 0 and may see new blocks; their values are never used.)
    static_assert(!DIRECT || IPT == 1, "non-loading threads are those past the items");
    static_assert(!DIRECT || NTHR > ITEMS, "the direct path needs threads without items to commit the chunk");
    constexpr int NL_FIRST = DIRECT ? ITEMS : 0;  // first thread without items
    uint8_t *const wring = p.base + p.g.stripe_offset(p.layer, sid, kvh);
    int i_done = 0;  // chunk keys written (wave-uniform, non-loading waves)
    auto commit_until = [&](int lim) {
        for (int e = (int) threadIdx.x - NL_FIRST + i_done * NBLK; e < lim * NBLK; e += NTHR - NL_FIRST) {
            const int bb = e % NBLK;
            const int i = e / NBLK;
            const int slot = (pos0 + i) % n_ctx;
            *reinterpret_cast<uint4 *>(wring + p.g.kcode_offset(slot, bb)) = sCc[i * NBLK + bb];
            *reinterpret_cast<uint4 *>(wring + p.g.vcode_offset(slot, bb)) = sCc[(QT + i) * NBLK + bb];
            *reinterpret_cast<uint32_t *>(wring + p.g.scale_offset(slot, bb)) = sCs[i * NBLK + bb];
        }
        i_done = max(i_done, lim);
    };
    // keys writable once the positions below P are published: ring tiles
    // among them (the paired part's even positions, then the rest's first
    // n_rt - n_pair), and keys whose old position precedes their end
    auto commit_limit = [&](int P) {
        const int r_done = P <= 2 * n_pair ? (P + 1) / 2 : n_pair + min(P - 2 * n_pair, n_rt - n_pair);
        return min(p.n_tok, max(0, (r_start - pos0) + kTK * r_done + n_ctx));
    };
    // DIRECT: 8 tiles before the loop's end (4 barrier periods) the waves
    // without items read one dword of every 128-byte line of the query rows
    // of workgroup blockIdx.x + n_resident, the one the dispatcher is likely
    // to start when a workgroup of this XCD finishes (workgroups go to the
    // XCDs in turn, and this one's XCD is that one's).  Its query loads then
    // hit this XCD's L2 (64 KB a workgroup, 2 MB an XCD at cfg5; the output's
    // nontemporal stores leave the L2 to them).  A round's whole input does
    // not fit the L2, and touching the chunk's K rows too was slower (75.9
    // vs 72.7 us).  At cfg5, in the build before the exact block scales,
    // against the same kernel without the touch and with plain output
    // stores: 70.5 vs 73.2-74.2 us full history, 46.1 vs 47.0 us empty;
    // halfway through the loop instead, 71.3-71.7 / 46.7-47.7.
    const int succ = (int) blockIdx.x + p.n_resident;
    const bool touch_on = DIRECT && p.n_resident > 0 && succ < (int) gridDim.x;
    constexpr int LPR = D * 2 / 128;  // 128-byte lines of a query row
    const int touch_at = max(0, (n_tiles + PF) / (PF + 1) * (PF + 1) - 8) & ~(TPB - 1);
    uint32_t touched = 0;
    auto touch_successor = [&]() {
        const int su = succ / n_qt;
        const int sb = su / p.n_heads;
        const int sh = su - sb * p.n_heads;
        const int t = (int) threadIdx.x - NL_FIRST;
        const int row = min(t / LPR, p.n_tok - 1);
        const uint16_t *line = p.q + (((int64_t) sb * p.n_tok + row) * p.n_heads + sh) * D + (t % LPR) * 64;
        touched = *reinterpret_cast<const uint32_t *>(line);
    };
    // The loop in two copies, so that the loading copy has its loads on
    // every path and the compiler's waits count exactly (loads behind a
    // branch turn every wait into a wait for all loads).
    auto tile_loop = [&](auto loads) {
        constexpr bool LOADS = decltype(loads)::value;
        for (int base = 0; base < n_tiles; base += PF + 1) {
#pragma unroll
            for (int u = 0; u <= PF; u += TPB) {
                BMO_PHASE_LOOP();
                if constexpr (LOADS) {
#pragma unroll
                    for (int k = 0; k < TPB; ++k)
                        deposit((u + k) % NBUF, tile_of(base + u + k), raw[u + k], rawd[u + k]);
                    // the next tiles' loads refill the registers just
                    // dequantized; issued before the barrier, they are in
                    // flight while the waves wait (the barrier waits for LDS
                    // operations only)
#pragma unroll
                    for (int k = 0; k < TPB; ++k) {
                        const int nxt = (u + k + PF) % (PF + 1);
                        fetch(raw[nxt], rawd[nxt]);
                    }
                }
                BMO_PHASE_LOOP();
                lds_barrier();  // these TPB buffers are complete
                BMO_PHASE_LOOP();
                if constexpr (DIRECT && !LOADS) {
                    const int lim = commit_limit(base + u + TPB);
                    if (lim > i_done) commit_until(lim);
                    if (touch_on && base + u == touch_at) touch_successor();
                }
                BMO_PHASE_LOOP();
#pragma unroll
                for (int k = 0; k < TPB; ++k) compute((u + k) % NBUF, tile_of(base + u + k));
            }
        }
    };
    BMO_PHASE(4);
    if (has_items)
        tile_loop(BoolC<true>{});
    else
        tile_loop(BoolC<false>{});
    BMO_PHASE(5);
#if BMO_PREFILL_PHASES
    if (lane == 0) phase_rec[8] = (uint64_t) phase_n;
#endif
    // (the touched value is needed by nothing; the read must not be dropped)
    asm volatile("" ::"v"(touched));
    // The loop has written every key: its last barrier publishes every ring
    // tile, after which commit_limit is n_tok, and with no ring tile at all
    // (pos0 = 0) the limit is n_ctx >= n_tok from the first barrier on.
    // Only a ring of fewer than 32 slots could leave keys for this call
    // (n_ctx = 1 at a pos0 off the 32-slot grid keeps the limit at 0), and
    // such rings take the staged path; it stays as a guard.
    if constexpr (DIRECT)
        if (!has_items) commit_until(p.n_tok);

    // Every acc row (query 4c + v) divides by its weight sum.  Lane 4qd + j
    // (of the 16 sharing c) holds, for column tile t, element
    // 32(t / 2) + 8(t % 2) + 4(qd / 2) + 16(qd % 2) + {0, 2, 1, 3}[j] of the
    // row (col_elem), i.e. the 4 lanes of a quad hold one float4 of the row
    // per t.  A 4x4 transpose inside the quad (DPP lane ^ 1, lane ^ 2) over
    // t = 4g .. 4g + 3 gives lane j the whole float4 of t = 4g + j, so each
    // lane stores 16-byte pieces and a store instruction covers 256
    // contiguous bytes of each of 4 rows.
    const int jq = lane & 3;
    const int qd = (lane >> 2) & 3;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float lv = accl[qb][v];
            const int qv = wq0 + qb * 16 + 4 * c + v;
            const float inv = lv > 0.0f ? __builtin_amdgcn_rcpf(lv) : 0.0f;  // within 1 ulp
            float *orow = p.out + (((int64_t) b * p.n_tok + min(qv, p.n_tok - 1)) * p.n_heads + h) * D;
#pragma unroll
            for (int g = 0; g < NT / 4; ++g) {
                const float a0 = acc[qb][4 * g][v] * inv, a1 = acc[qb][4 * g + 1][v] * inv;
                const float a2 = acc[qb][4 * g + 2][v] * inv, a3 = acc[qb][4 * g + 3][v] * inv;
                // every lane reads its partner before the selects: a DPP
                // read from a lane the branch disabled returns nothing
                const bool odd = jq & 1, up = jq & 2;
                const float x0 = quad_perm<0xB1>(a0), x1 = quad_perm<0xB1>(a1);
                const float x2 = quad_perm<0xB1>(a2), x3 = quad_perm<0xB1>(a3);
                const float b0 = odd ? x1 : a0, b1 = odd ? a1 : x0;
                const float b2 = odd ? x3 : a2, b3 = odd ? a3 : x2;
                const float y0 = quad_perm<0x4E>(b0), y1 = quad_perm<0x4E>(b1);
                const float y2 = quad_perm<0x4E>(b2), y3 = quad_perm<0x4E>(b3);
                const float c0 = up ? y2 : b0, c1 = up ? y3 : b1;
                const float c2 = up ? b2 : y0, c3 = up ? b3 : y1;
                // c_k is element base + {0, 2, 1, 3}[k] of tile t = 4g + jq
                const int t = 4 * g + jq;
                const int base = 32 * (t >> 1) + 8 * (t & 1) + 4 * (qd >> 1) + 16 * (qd & 1);
                // nontemporal: nothing here reads the output again, and it
                // would displace the L2 lines the next workgroups load
                if (qv < p.n_tok)
                    __builtin_nontemporal_store(float4_t{c0, c2, c1, c3}, reinterpret_cast<float4_t *>(orow + base));
            }
        }
    }
    BMO_PHASE(6);
#if BMO_PREFILL_PHASES
    if (lane == 0) phase_rec[7] = __builtin_amdgcn_s_memrealtime();
#endif
}

namespace {

// One workgroup per 256 queries of a head: 16 waves x 16 queries (QB = 1),
// 4 waves on each SIMD (at most 128 VGPRs each), so one wave's LDS and
// matrix latencies overlap another's work.  Against 8 waves x 32 queries
// (QB = 2, each K/V operand read feeding two matrix instructions, half the
// LDS reads per query), both on the staged path at cfg5: 92.7-93.0 vs
// 106.5-106.6 us (ring history full), 60.7 vs 69.1 us (empty); in an
// earlier build also GQA 4:1, 256 tokens: 84-85 vs 91-94 us; 512-token
// chunks: 91-93 vs 99-100 us; head_dim 64 GQA 4:1 on an 8-slot ring: 13.9
// vs 16.7 us.
// Smaller workgroups for short chunks (4 waves below 129 tokens) were
// measured slower whenever the ring holds history: the window's tiles
// dominate, and all waves share their dequantization.
constexpr int kQW = 16;
constexpr int kQB = 1;
constexpr int kQT = 16 * kQB * kQW;  // queries per workgroup

template <int D>
void launch_attention(const PrefillParams &p, bool direct, dim3 grid, hipStream_t stream) {
    // ring tiles 32 slots wide never wrap when n_ctx is a multiple of 32
    // (the direct path requires it)
    if (direct)
        hipLaunchKernelGGL((prefill_kernel<D, kQW, kQB, true, true>), grid, dim3(64 * kQW), 0, stream, p);
    else if (p.g.n_ctx % kTK == 0)
        hipLaunchKernelGGL((prefill_kernel<D, kQW, kQB, false, true>), grid, dim3(64 * kQW), 0, stream, p);
    else
        hipLaunchKernelGGL((prefill_kernel<D, kQW, kQB, false, false>), grid, dim3(64 * kQW), 0, stream, p);
}

}  // namespace

// Workgroups of prefill_kernel that the current device runs at once: its
// CU count (one workgroup fills a CU).  Looked up once per device.
static int resident_workgroups() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (cached[dev] <= 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
        cached[dev] = n > 0 ? n : -1;
    }
    return cached[dev] > 0 ? cached[dev] : 0;
}

// The direct path: one query head per kv head, the chunk in one workgroup,
// and ring tiles that never wrap (the per-key slots of other ring sizes do
// not fit its register budget beside the exact block scales; those rings
// take the staged path).
#if BMO_PREFILL_PHASES
// The diagnostic build's phase records (kPhaseUnits workgroups x 16 waves x
// kPhaseRec stamps), copied to host memory after a synchronization.
extern "C" __attribute__((visibility("default"))) int bmo_prefill_phase_stamps(void *dst, size_t bytes) {
    if (!dst || bytes > sizeof(g_prefill_phases)) return 2;
    if (hipDeviceSynchronize() != hipSuccess) return 8;
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_prefill_phases), bytes, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : 8;
}
#endif

bool prefill_is_direct(const PrefillParams &p) {
    return p.n_heads == p.n_kv && p.n_tok <= kQT && p.g.n_ctx % kTK == 0;
}

bool launch_prefill(const PrefillParams &p, hipStream_t stream) {
    if (p.g.head_dim != 128 && p.g.head_dim != 64) return false;
    const int nblk = p.g.head_dim / kQK;
    const bool direct = prefill_is_direct(p);
    if (!direct) {
        const int stage_threads = p.n_batch * p.n_tok * p.n_kv * nblk * 2;
        hipLaunchKernelGGL(stage_kernel, dim3((unsigned) ((stage_threads + 255) / 256)), dim3(256), 0,
                           stream, p);
    }
    const int qt = kQT;
    const dim3 grid((unsigned) ((int64_t) p.n_batch * p.n_heads * ((p.n_tok + qt - 1) / qt)));
    PrefillParams pa = p;
    pa.n_resident = resident_workgroups();
    if (p.g.head_dim == 128)
        launch_attention<128>(pa, direct, grid, stream);
    else
        launch_attention<64>(pa, direct, grid, stream);
    if (!direct) {
        const int commit_threads = p.n_batch * p.n_tok * p.n_kv * nblk;
        hipLaunchKernelGGL(commit_kernel, dim3((unsigned) ((commit_threads + 255) / 256)), dim3(256), 0,
                           stream, p);
    }
    return true;
}

}  // namespace bmo
