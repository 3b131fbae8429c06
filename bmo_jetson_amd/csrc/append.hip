// append.hip -- quantize fp32 K/V rows into Q4_0 ring slots.
//
// The reference writes the current token's K and V as fp16 into slot
// pos % n_ctx (src/bmo_cuda_kernels.cu:749-754) and, on its multi-token path,
// copies a chunk into consecutive slots (src/bmo_compute.cpp:2390-2401).  Here
// the write quantizes to Q4_0, bit-exactly as ggml quantize_row_q4_0_ref.
//
// One thread owns one 32-element block: it loads the block's 128 contiguous
// bytes with eight 128-bit loads, runs the sequential first-occurrence max
// scan of the reference algorithm in registers, and stores 16 code bytes and
// a 2-byte scale.  The traffic is 2 * n_kv_heads * head_dim * 4 bytes in per
// row, so this kernel is small next to the attention read; it is written for
// exactness, with coalescing left to the cache.
#include <algorithm>

#include "kernels.hpp"
#include "q4_0_device.hpp"

namespace bmo {

__global__ __launch_bounds__(256) void append_kernel(AppendParams p) {
    const int nblk = p.g.head_dim / kQK;
    const int64_t per_row = (int64_t) p.g.n_kv_heads * nblk * 2;  // blocks of K and V
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= per_row * p.n_rows) return;
    const int r = (int) (t / per_row);
    int rem = (int) (t % per_row);
    const int which = rem / (p.g.n_kv_heads * nblk);  // 0 = K, 1 = V
    rem %= p.g.n_kv_heads * nblk;
    const int h = rem / nblk;
    const int blk = rem % nblk;

    int session;
    int64_t pos;
    if (p.pos != nullptr) {
        session = p.session_ids ? p.session_ids[r] : r;
        pos = p.pos[r];
    } else {
        session = p.session;
        pos = p.pos0 + r;
    }
    if (session < 0 || session >= p.g.n_sessions || pos < 0) return;
    const int slot = (int) (pos % p.g.n_ctx);

    const float *src = (which == 0 ? p.k : p.v) +
                       ((int64_t) r * p.g.n_kv_heads + h) * p.g.head_dim + blk * kQK;
    float x[kQK];
    load_block_f32(src, x);
    uint16_t d16;
    uint32_t qs[4];
    quantize_block_q4_0(x, d16, qs);
    store_block(p.base + p.g.stripe_offset(p.layer, session, h), p.g, slot, blk, which, d16, qs);
}

// Zero state of the ring (ring_layout.hpp): K code bytes 0x88, the rest 0.
// Ranges are whole groups; blockIdx.y strides over the ranges.
__global__ __launch_bounds__(256) void clear_kernel(uint8_t *base, int64_t range_bytes,
                                                    int64_t range_stride, int n_ranges) {
    const int64_t n = range_bytes / 16;
    constexpr int per_group = kGroupBytes / 16;
    constexpr int k_codes = kVCodeOff / 16;
    const uint32_t kz = 0x01010101u * kKCodeZero;
    for (int r = blockIdx.y; r < n_ranges; r += gridDim.y) {
        uint4 *dst = reinterpret_cast<uint4 *>(base + (int64_t) r * range_stride);
        for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n;
             i += (int64_t) gridDim.x * blockDim.x) {
            const uint32_t w = (int) (i % per_group) < k_codes ? kz : 0u;
            dst[i] = make_uint4(w, w, w, w);
        }
    }
}

void launch_clear(uint8_t *base, int64_t range_bytes, int64_t range_stride, int n_ranges,
                  hipStream_t stream) {
    if (range_bytes <= 0 || n_ranges <= 0) return;
    const int64_t vecs = range_bytes / 16;
    const unsigned gx = (unsigned) std::min<int64_t>((vecs + 255) / 256, 8192);
    const unsigned gy = (unsigned) std::min(n_ranges, 65535);
    hipLaunchKernelGGL(clear_kernel, dim3(gx, gy), dim3(256), 0, stream, base, range_bytes,
                       range_stride, n_ranges);
}

// pos[i] += delta for i < n (positions that live in device memory, so that a
// captured decode step advances them on every replay).
__global__ __launch_bounds__(256) void advance_kernel(int *pos, int n, int delta) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) pos[i] += delta;
}

// pos[0] = value (a session handle's device position; a kernel rather than a
// copy, so that no host buffer has to outlive the call).
__global__ __launch_bounds__(64) void set_pos_kernel(int *pos, int value) {
    if (threadIdx.x == 0) pos[0] = value;
}

void launch_set_pos(int *pos, int value, hipStream_t stream) {
    hipLaunchKernelGGL(set_pos_kernel, dim3(1), dim3(64), 0, stream, pos, value);
}

void launch_advance(int *pos, int n, int delta, hipStream_t stream) {
    hipLaunchKernelGGL(advance_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, stream, pos, n,
                       delta);
}

void launch_append(const AppendParams &p, hipStream_t stream) {
    const int nblk = p.g.head_dim / kQK;
    const int64_t threads = (int64_t) p.n_rows * p.g.n_kv_heads * nblk * 2;
    if (threads <= 0) return;
    const int64_t grid = (threads + 255) / 256;
    hipLaunchKernelGGL(append_kernel, dim3((unsigned) grid), dim3(256), 0, stream, p);
}

}  // namespace bmo
