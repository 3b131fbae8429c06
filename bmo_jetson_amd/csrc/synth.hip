// synth.hip -- the device side of include/bmo_synth.h: the seeded synthetic
// inputs of the benchmark configurations, bit for bit the stream the CPU
// restates, and the benchmark's read probe.  Every floating-point step is an IEEE double add,
// subtract, multiply, divide or square root (correctly rounded on gfx950 as
// on the host), the build contracts none of them (-ffp-contract=off), and
// the integer steps are exact, so each element is a pure function of
// (seed, index) on either side.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../../include/bmo_synth.h"

namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// ln x, x in [2^-54, 1]: x = m 2^e, m folded into [sqrt(1/2), sqrt(2)],
// e ln 2 + 2 atanh((m - 1)/(m + 1)), the series in s^2 by Horner to s^21.
__device__ double stream_ln(double x) {
    const uint64_t bits = __builtin_bit_cast(uint64_t, x);
    int e = (int) ((bits >> 52) & 0x7FF) - 1023;
    double m = __builtin_bit_cast(double, (bits & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull);
    if (m > 0x1.6a09e667f3bcdp+0) {
        m = m * 0.5;
        e = e + 1;
    }
    const double s = (m - 1.0) / (m + 1.0);
    const double s2 = s * s;
    constexpr double kInvOdd[10] = {0x1.8618618618618p-5, 0x1.af286bca1af28p-5, 0x1.e1e1e1e1e1e1ep-5,
                                    0x1.1111111111111p-4, 0x1.3b13b13b13b14p-4, 0x1.745d1745d1746p-4,
                                    0x1.c71c71c71c71cp-4, 0x1.2492492492492p-3, 0x1.999999999999ap-3,
                                    0x1.5555555555555p-2};  // 1/21, 1/19, ..., 1/3
    double p = kInvOdd[0];
#pragma unroll
    for (int i = 1; i < 10; ++i) p = p * s2 + kInvOdd[i];
    p = p * s2 + 1.0;
    return (double) e * 0x1.62e42fefa39efp-1 + 2.0 * (s * p);
}

// cos(2 pi t), t in [0, 1): quadrant n of 4t and the fraction g (exact);
// cos, -sin, -cos, sin of y = pi/2 g for n = 0..3, g > 1/2 folded to 1 - g
// with sine and cosine swapped, Taylor series in y^2 by Horner.
__device__ double stream_cos2pi(double t) {
    const double t4 = t * 4.0;
    const int n = (int) t4;
    double g = t4 - (double) n;
    bool use_sin = (n & 1) != 0;
    const bool neg = n == 1 || n == 2;
    if (g > 0.5) {
        g = 1.0 - g;
        use_sin = !use_sin;
    }
    const double y = g * 0x1.921fb54442d18p+0;
    const double y2 = y * y;
    double r;
    if (use_sin) {
        constexpr double kSin[8] = {0x1.ae7f3e733b81fp-41, 0x1.6124613a86d09p-33, 0x1.ae64567f544e4p-26,
                                    0x1.71de3a556c734p-19, 0x1.a01a01a01a01ap-13, 0x1.1111111111111p-7,
                                    0x1.5555555555555p-3, 1.0};  // 1/15!, ..., 1/3!, 1
        double p = 0x1.952c77030ad4ap-49;                       // 1/17!
#pragma unroll
        for (int i = 0; i < 8; ++i) p = kSin[i] - y2 * p;
        r = y * p;
    } else {
        constexpr double kCos[8] = {0x1.93974a8c07c9dp-37, 0x1.1eed8eff8d898p-29, 0x1.27e4fb7789f5cp-22,
                                    0x1.a01a01a01a01ap-16, 0x1.6c16c16c16c17p-10, 0x1.5555555555555p-5,
                                    0.5, 1.0};  // 1/14!, ..., 1/2!, 1
        double p = 0x1.ae7f3e733b81fp-45;      // 1/16!
#pragma unroll
        for (int i = 0; i < 8; ++i) p = kCos[i] - y2 * p;
        r = p;
    }
    return neg ? -r : r;
}

__device__ float stream_normal(uint64_t seed, uint64_t c) {
    const uint64_t a = mix64(seed ^ mix64(2 * c));
    const uint64_t b = mix64(seed ^ mix64(2 * c + 1));
    const double u1 = ((double) (a >> 11) + 0.5) * 0x1p-53;
    const double u2 = (double) (b >> 11) * 0x1p-53;
    return (float) (__builtin_sqrt(-2.0 * stream_ln(u1)) * stream_cos2pi(u2));
}

__global__ __launch_bounds__(256) void fill_kernel(float *out, int64_t n, uint64_t seed, uint64_t offset,
                                                   int outliers) {
    const int64_t step = (int64_t) gridDim.x * blockDim.x;
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
        const uint64_t c = offset + (uint64_t) i;
        float z = stream_normal(seed, c);
        if (outliers && (mix64((seed ^ 0xD1B54A32D192ED03ull) ^ mix64(c)) >> 32) < 42949673u) z = z * 8.0f;
        out[i] = z;
    }
}

}  // namespace

extern "C" int bmo_synth_fill_normal(float *out, int64_t n, uint64_t seed, uint64_t offset, int outliers,
                                     void *stream) {
    if (n < 0 || (n > 0 && !out)) return 2;
    if (n == 0) return 0;
    const int64_t blocks = (n + 255) / 256;
    const unsigned grid = (unsigned) (blocks < 65536 ? blocks : 65536);
    hipLaunchKernelGGL(fill_kernel, dim3(grid), dim3(256), 0, (hipStream_t) stream, out, n, seed, offset,
                       outliers);
    return hipGetLastError() == hipSuccess ? 0 : 8;
}

namespace {

typedef unsigned int probe_u32x4 __attribute__((ext_vector_type(4)));

// One 16-byte nontemporal load per thread: piece i of the buffer is read by
// thread i once, and a workgroup retires as soon as its loads return.  The
// xor test keeps the loads (its store fires only for one value in 2^32).
__global__ __launch_bounds__(256) void read_probe_kernel(const probe_u32x4 *src, int64_t n16, uint32_t *sink) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= n16) return;
    const probe_u32x4 v = __builtin_nontemporal_load(src + i);
    if ((v.x ^ v.y ^ v.z ^ v.w) == 0x9E3779B9u) sink[threadIdx.x] = 1u;
}

}  // namespace

extern "C" int bmo_synth_read_probe(const void *buf, int64_t bytes, uint32_t *sink, void *stream) {
    if (bytes < 0 || bytes % 16 != 0 || (bytes > 0 && (!buf || !sink)) ||
        (reinterpret_cast<uintptr_t>(buf) & 15) != 0)
        return 2;
    if (bytes == 0) return 0;
    const int64_t n16 = bytes / 16;
    const int64_t blocks = (n16 + 255) / 256;
    if (blocks > 0x7FFFFFFF) return 2;
    hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned) blocks), dim3(256), 0, (hipStream_t) stream,
                       reinterpret_cast<const probe_u32x4 *>(buf), n16, sink);
    return hipGetLastError() == hipSuccess ? 0 : 8;
}
