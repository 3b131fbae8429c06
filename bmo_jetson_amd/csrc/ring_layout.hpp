// ring_layout.hpp -- where each Q4_0 block of the ring lives in HBM.
//
// The reference keeps K and V as two fp16 ggml tensors ne = [head_dim, n_ctx,
// n_heads, n_layers] (src/bmo.cpp:1401-1402).  Here each region (K, V) is
// [n_layers][n_sessions][n_kv_heads] stripes; one stripe is the nibble plane
// [n_ctx][head_dim/2] bytes followed by the fp16 scale plane
// [n_ctx][head_dim/32].  Splitting the 18-byte ggml block into a 16-byte
// nibble part and a 2-byte scale part keeps every nibble row 16-byte aligned,
// so one lane fetches one whole block's codes with a single 128-bit load and
// a 64-lane wave reads 1 KiB of contiguous codes per load instruction.
#pragma once

#include <stdint.h>

namespace bmo {

constexpr int kQK = 32;  // elements per Q4_0 block

struct RingGeom {
    int n_layers;
    int n_sessions;
    int n_kv_heads;
    int head_dim;
    int n_ctx;
    int64_t stripe_bytes;  // bytes per (layer, session, kv head) stripe
    int64_t nib_bytes;     // offset of the scale plane inside a stripe

    __host__ __device__ int64_t stripe_offset(int layer, int session, int head) const {
        return ((int64_t) layer * n_sessions * n_kv_heads + (int64_t) session * n_kv_heads + head) *
               stripe_bytes;
    }
    __host__ __device__ int64_t region_bytes() const {
        return (int64_t) n_layers * n_sessions * n_kv_heads * stripe_bytes;
    }
};

__host__ __device__ inline int64_t stripe_bytes_for(int head_dim, int n_ctx) {
    const int64_t raw = (int64_t) n_ctx * head_dim / 2 + (int64_t) n_ctx * (head_dim / kQK) * 2;
    return (raw + 255) / 256 * 256;
}

__host__ __device__ inline RingGeom make_geom(int n_layers, int n_sessions, int n_kv_heads,
                                              int head_dim, int n_ctx) {
    RingGeom g;
    g.n_layers = n_layers;
    g.n_sessions = n_sessions;
    g.n_kv_heads = n_kv_heads;
    g.head_dim = head_dim;
    g.n_ctx = n_ctx;
    g.stripe_bytes = stripe_bytes_for(head_dim, n_ctx);
    g.nib_bytes = (int64_t) n_ctx * head_dim / 2;
    return g;
}

}  // namespace bmo
