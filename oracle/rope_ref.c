/*
 * rope_ref.c -- oracle restatement of the reference's interleaved RoPE
 * (TEST INFRASTRUCTURE ONLY; see oracle.h).
 *
 * src/bmo_cuda_kernels.cu:317-354 rotates, in every head of a row, the pairs
 * (x[2i], x[2i+1]) by the angle pos * theta^(-2i/head_dim), with theta the
 * model's rope_theta (src/bmo.cpp:301-303, default 10000), called on q and k
 * with the token's absolute position (src/bmo_compute.cpp:2329-2330).  The
 * reference evaluates theta^(-2i/d) and the sine/cosine with fp32 fast
 * intrinsics; here the frequency is r^i with r = theta^(-2/d) (binary powers,
 * the same IEEE double operations the kernel performs), the angle and its
 * cosine and sine are double, rounded once to fp32, and the rotation is fp32
 * with every product and sum rounded on its own.
 */
#include <math.h>

#include "oracle.h"

double orc_rope_freq(double r, int i) {
    double acc = 1.0, b = r;
    while (i) {
        if (i & 1) acc *= b;
        b *= b;
        i >>= 1;
    }
    return acc;
}

void orc_rope_cos_sin(int head_dim, int64_t pos, double theta, float *cs, float *sn) {
    const double r = pow(theta, -2.0 / (double) head_dim);
    for (int i = 0; i < head_dim / 2; ++i) {
        const double a = (double) pos * orc_rope_freq(r, i);
        cs[i] = (float) cos(a);
        sn[i] = (float) sin(a);
    }
}

void orc_rope_interleaved(const float *x, float *y, int n_rows, int head_dim, int64_t pos,
                          double theta) {
    float cs[512], sn[512];
    orc_rope_cos_sin(head_dim, pos, theta, cs, sn);
    for (int row = 0; row < n_rows; ++row) {
        const float *xr = x + (size_t) row * head_dim;
        float *yr = y + (size_t) row * head_dim;
        for (int i = 0; i < head_dim / 2; ++i) {
            const float a = xr[2 * i], b = xr[2 * i + 1];
            const float ac = a * cs[i], bs = b * sn[i];
            const float as = a * sn[i], bc = b * cs[i];
            yr[2 * i] = ac - bs;
            yr[2 * i + 1] = as + bc;
        }
    }
}
