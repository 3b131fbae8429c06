// ring_layout.hpp -- where each Q4_0 block of the ring lives in HBM.
//
// The reference keeps K and V as two fp16 ggml tensors ne = [head_dim, n_ctx,
// n_heads, n_layers] (src/bmo.cpp:1401-1402).  Here one allocation holds
// [n_layers][n_sessions][n_kv_heads] stripes; a stripe holds the n_ctx slots
// of one kv head in groups of G = 2048 / head_dim consecutive slots (16 at
// head_dim 128, 32 at head_dim 64).  One group is 2304 contiguous bytes:
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
// dword at 2048 + l*4.  Consecutive groups are adjacent, so a wave walking a
// window streams one contiguous range.  Slots of the last group past n_ctx are
// padding that no read uses.  The zero state of a slot (the reference's
// zeroed fp16 cache) is the ggml block with d = 0 and all codes 0: K code
// bytes 0x88, everything else 0.
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
    int64_t stripe_bytes;  // bytes per (layer, session, kv head) stripe

    __host__ __device__ int64_t stripe_offset(int layer, int session, int head) const {
        return ((int64_t) layer * n_sessions * n_kv_heads + (int64_t) session * n_kv_heads + head) *
               stripe_bytes;
    }
    __host__ __device__ int64_t total_bytes() const {
        return (int64_t) n_layers * n_sessions * n_kv_heads * stripe_bytes;
    }
    // Byte offsets inside a stripe of block blk of slot `slot`.
    __host__ __device__ int64_t kcode_offset(int slot, int blk) const {
        const int G = keys_per_group(head_dim);
        return (int64_t) (slot / G) * kGroupBytes + (slot % G) * (head_dim / 2) + blk * 16;
    }
    __host__ __device__ int64_t vcode_offset(int slot, int blk) const {
        return kcode_offset(slot, blk) + kVCodeOff;
    }
    __host__ __device__ int64_t scale_offset(int slot, int blk) const {
        const int G = keys_per_group(head_dim);
        return (int64_t) (slot / G) * kGroupBytes + kScaleOff +
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
    return g;
}

}  // namespace bmo
