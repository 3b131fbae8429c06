// kernels.hpp -- parameter blocks and launchers of the ring kernels (internal
// to libbmo_attn.so; the public surface is include/bmo_attn.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ring_layout.hpp"

namespace bmo {

// Rows of fp32 K/V to quantize into ring slots.  Row r of the input goes to
//   batched mode (session_ids/pos set): session session_ids[r] (or r),
//                                       slot pos[r] % n_ctx;
//   run mode (pos == nullptr):          session `session`,
//                                       slot (pos0 + r) % n_ctx.
struct AppendParams {
    uint8_t *base;  // ring allocation (layout in ring_layout.hpp)
    RingGeom g;
    int layer;
    int n_rows;
    const int *session_ids;  // device, nullable (batched mode)
    const int *pos;          // device (batched mode) or nullptr (run mode)
    int session;             // run mode
    int64_t pos0;            // run mode
    const float *k;          // [n_rows][n_kv_heads][head_dim]
    const float *v;
};

// Division by a run-time constant d in [1, 2^31) of numerators n in
// [0, 2^31) without the integer-division sequence (Granlund and Montgomery,
// "Division by invariant integers using multiplication", 1994, section 4:
// with s = ceil(log2 d) and m = floor(2^32 (2^s - d) / d) + 1, n / d equals
// (mulhi(n, m) + n) >> s; mulhi(n, m) < n keeps the sum below 2^32).
struct FastDiv {
    uint32_t m;
    uint32_t s;
    __host__ __device__ uint32_t div(uint32_t n) const {
        return ((uint32_t) (((uint64_t) n * m) >> 32) + n) >> s;
    }
};

inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t s = 0;
    while ((uint64_t(1) << s) < d) ++s;
    const uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1;
    return FastDiv{(uint32_t) m, s};
}

struct DecodeParams {
    uint8_t *base;  // ring allocation; the fused path writes the current slot
    RingGeom g;
    int layer;
    int n_batch;
    int n_heads;
    int n_kv;                // logical kv heads: GQA map and k_new/v_new row stride
                             // (g.n_kv_heads is the allocated head count per stripe set)
    const int *session_ids;  // device, nullable
    const int *pos;          // device [n_batch], or nullptr -> pos_scalar
    int pos_scalar;
    const float *q;      // [n_batch][n_heads][head_dim]
    const float *k_new;  // [n_batch][n_kv][head_dim] (fused only)
    const float *v_new;
    float *out;          // [n_batch][n_heads][head_dim]
    float qscale;        // softmax scale * log2(e)
    int rope;            // nonzero: rotate q (and the fused k_new) by interleaved RoPE at pos
    double rope_r;       // theta^(-2/head_dim): pair i turns by pos * rope_r^i
    // set by launch_decode: n_heads / n_kv and dividers by n_heads, by
    // n_heads / n_kv and by g.n_ctx
    int q_per_kv;
    FastDiv div_heads, div_qkv, div_ctx;
};

// Chunked prefill of n_tok tokens per batch entry (prefill.hip).
struct PrefillParams {
    uint8_t *base;  // ring allocation
    RingGeom g;
    uint8_t *stage;  // staging stripes [n_batch][n_kv] of n_tok slots
    RingGeom sg;     // staging geometry (1 layer, n_batch "sessions", n_kv, head_dim, n_tok)
    int layer;
    int n_batch;
    int n_heads;
    int n_kv;
    const int *session_ids;  // device, nullable
    const int *pos0;         // device [n_batch]: position of each entry's first chunk token
    int n_tok;
    const uint16_t *q;  // bf16 [n_batch][n_tok][n_heads][head_dim]
    const uint16_t *k;  // bf16 [n_batch][n_tok][n_kv][head_dim]
    const uint16_t *v;
    float *out;    // [n_batch][n_tok][n_heads][head_dim]
    float qscale;  // softmax scale * log2(e)
    int n_resident;  // set by launch_prefill: workgroups the device runs at once (0: unknown)
};

// Launchers enqueue only; they leave launch errors for the caller's
// hipGetLastError().  launch_decode returns false for an unsupported head_dim.
void launch_append(const AppendParams &p, hipStream_t stream);
void launch_advance(int *pos, int n, int delta, hipStream_t stream);
void launch_set_pos(int *pos, int value, hipStream_t stream);
bool launch_decode(const DecodeParams &p, bool fused, hipStream_t stream);
// stage, attend, commit (three kernels in stream order); false for an
// unsupported head_dim.
bool launch_prefill(const PrefillParams &p, hipStream_t stream);

struct GemvParams {
    const uint8_t *w;  // ggml block_q4_0 rows [rows][cols/32] (18 bytes each)
    const float *x;    // [cols]
    float *y;          // [rows]
    int rows;
    int cols;          // a multiple of 64
    uint8_t *q8_out;   // nullable: the activation's Q8_1 blocks (36 bytes each)
};
// LDS bytes gemv_kernel needs for cols columns.
size_t gemv_lds_bytes(int cols);
bool launch_gemv(const GemvParams &p, hipStream_t stream);
// True when launch_prefill runs one attention kernel that quantizes and
// commits the chunk itself (no staging stripes are read or written).
bool prefill_is_direct(const PrefillParams &p);
// Message of the last ring call that failed on the calling thread (empty if
// none): unlike the ring's own message, no other thread's call can replace it.
const char *ring_thread_last_error();
// Writes the zero state (ring_layout.hpp) into n_ranges ranges of
// range_bytes bytes (a multiple of the group size) spaced range_stride apart.
void launch_clear(uint8_t *base, int64_t range_bytes, int64_t range_stride, int n_ranges,
                  hipStream_t stream);

}  // namespace bmo
