// ring_layout.hpp -- where each Q4_0 block of the ring lives in HBM.
//
// The reference keeps K and V as two fp16 ggml tensors ne = [head_dim, n_ctx,
// n_heads, n_layers] (src/bmo.cpp:1401-1402).  Here the n_ctx slots of one
// (layer, session, kv head) -- a stripe -- are cut into groups of
// G = 2048 / head_dim consecutive slots (16 at head_dim 128, 32 at head_dim
// 64), and one allocation holds the groups as [n_layers][n_groups]
// [n_sessions][n_kv_heads]: group g of every (session, head) of a layer sits
// side by side, so the waves of a decode launch, which walk their windows in
// step, read one contiguous region at a time (measured 4% faster on MI355X
// than stripes stored whole).  One group is 2304 contiguous bytes:
//
//   [0, 1024)     K codes: G rows of head_dim/2 bytes, 16 bytes per 32-element
//                 block, ggml nibble order (byte j: element j low nibble,
//                 element j+16 high nibble), each nibble stored as the 4-bit
//                 two's complement of (code - 8), i.e. code ^ 8;
//   [1024, 2048)  V codes: same shape, plain ggml codes 0..15;
//   [2048, 2304)  scales: per (slot, block) one dword, K scale (fp16) in the
//                 low half and V scale in the high half.
//
// A 64-lane wave that gives lane l block (l % (head_dim/32)) of key
// (l / (head_dim/32)) reads one group with three fully coalesced loads: 16
// bytes of K codes at l*16, 16 bytes of V codes at 1024 + l*16 and the scale
// dword at 2048 + l*4.  Consecutive groups of a stripe are group_stride bytes
// apart.  Slots of the last group past n_ctx are padding that no read uses.
// The zero state of a slot (the reference's zeroed fp16 cache) is the ggml
// block with d = 0 and all codes 0: K code bytes 0x88, everything else 0.
#pragma once

#include <stdint.h>

namespace bmo {

constexpr int kQK = 32;            // elements per Q4_0 block
constexpr int kGroupBytes = 2304;  // bytes per slot group (any supported head_dim)
constexpr int kVCodeOff = 1024;    // offset of the V codes inside a group
constexpr int kScaleOff = 2048;    // offset of the scale dwords inside a group
constexpr uint8_t kKCodeZero = 0x88;  // stored K byte of two zero-offset codes

__host__ __device__ constexpr int keys_per_group(int head_dim) { return 2048 / head_dim; }

struct RingGeom {
    int n_layers;
    int n_sessions;
    int n_kv_heads;
    int head_dim;
    int n_ctx;
    int n_groups;          // groups per stripe
    int64_t stripe_bytes;  // bytes of one stripe (n_groups groups, not contiguous)
    int64_t group_stride;  // bytes between consecutive groups of a stripe

    // Offset of group 0 of the (layer, session, head) stripe.
    __host__ __device__ int64_t stripe_offset(int layer, int session, int head) const {
        return (int64_t) layer * n_groups * group_stride +
               ((int64_t) session * n_kv_heads + head) * kGroupBytes;
    }
    __host__ __device__ int64_t total_bytes() const {
        return (int64_t) n_layers * n_groups * group_stride;
    }
    // Byte offsets, from the stripe's group 0, of block blk of slot `slot`.
    __host__ __device__ int64_t kcode_offset(int slot, int blk) const {
        const int G = keys_per_group(head_dim);
        return (int64_t) (slot / G) * group_stride + (slot % G) * (head_dim / 2) + blk * 16;
    }
    __host__ __device__ int64_t vcode_offset(int slot, int blk) const {
        return kcode_offset(slot, blk) + kVCodeOff;
    }
    __host__ __device__ int64_t scale_offset(int slot, int blk) const {
        const int G = keys_per_group(head_dim);
        return (int64_t) (slot / G) * group_stride + kScaleOff +
               ((slot % G) * (head_dim / kQK) + blk) * 4;
    }
};

__host__ __device__ inline int64_t stripe_bytes_for(int head_dim, int n_ctx) {
    const int G = keys_per_group(head_dim);
    return (int64_t) ((n_ctx + G - 1) / G) * kGroupBytes;
}

__host__ __device__ inline RingGeom make_geom(int n_layers, int n_sessions, int n_kv_heads,
                                              int head_dim, int n_ctx) {
    RingGeom g;
    g.n_layers = n_layers;
    g.n_sessions = n_sessions;
    g.n_kv_heads = n_kv_heads;
    g.head_dim = head_dim;
    g.n_ctx = n_ctx;
    const int G = keys_per_group(head_dim);
    g.n_groups = (n_ctx + G - 1) / G;
    g.stripe_bytes = (int64_t) g.n_groups * kGroupBytes;
    g.group_stride = (int64_t) n_sessions * n_kv_heads * kGroupBytes;
    return g;
}

// A stripe's groups packed back to back (group_stride = kGroupBytes): the
// layout of a host copy of one stripe's groups.
__host__ __device__ inline RingGeom packed_stripe_geom(const RingGeom &g) {
    RingGeom p = g;
    p.n_layers = 1;
    p.n_sessions = 1;
    p.n_kv_heads = 1;
    p.group_stride = kGroupBytes;
    return p;
}

}  // namespace bmo
