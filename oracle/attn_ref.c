/*
 * attn_ref.c -- ring geometry, Q4_0 append, and double-precision sliding
 * window attention over the Q4_0 ring.  TEST INFRASTRUCTURE ONLY (see
 * oracle.h).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* src/bmo_cuda_kernels.cu:739-743 */
void orc_ring_window(int64_t pos, int n_ctx, int *window, int64_t *start,
                     int *cur_slot) {
    const int64_t total = pos + 1;
    const int64_t w = total > n_ctx ? n_ctx : total;
    if (window) *window = (int) w;
    if (start) *start = total - w;
    if (cur_slot) *cur_slot = (int) (pos % n_ctx);
}

static size_t blk_index(int h, int slot, int b, int n_ctx, int nblk) {
    return ((size_t) h * (size_t) n_ctx + (size_t) slot) * (size_t) nblk + (size_t) b;
}

/* src/bmo_cuda_kernels.cu:749-754: the current token's K and V rows go to
 * slot pos % n_ctx of every kv head; here they are Q4_0-quantized. */
void orc_ring_append(orc_block_q4_0 *kc, orc_block_q4_0 *vc, int n_kv_heads,
                     int head_dim, int n_ctx, int64_t pos, const float *k,
                     const float *v) {
    const int nblk = head_dim / ORC_QK4_0;
    const int slot = (int) (pos % n_ctx);
    for (int h = 0; h < n_kv_heads; ++h) {
        orc_quantize_row_q4_0(k + (size_t) h * head_dim,
                              kc + blk_index(h, slot, 0, n_ctx, nblk), head_dim);
        orc_quantize_row_q4_0(v + (size_t) h * head_dim,
                              vc + blk_index(h, slot, 0, n_ctx, nblk), head_dim);
    }
}

static void dequant_row(const orc_block_q4_0 *c, int h, int slot, int head_dim,
                        int n_ctx, float *row) {
    const int nblk = head_dim / ORC_QK4_0;
    orc_dequantize_row_q4_0(c + blk_index(h, slot, 0, n_ctx, nblk), row, head_dim);
}

/* Scores, softmax and weighted V sum of src/bmo_compute.cpp:937-969 (keys in
 * oldest -> newest order as src/bmo_cuda_kernels.cu:772-776 walks them), over
 * the ring window of src/bmo_cuda_kernels.cu:739-747, in double.  A window of
 * one key gives the dequantized cached V (src/bmo_compute.cpp:914-925). */
void orc_ring_decode_f64(const orc_block_q4_0 *kc, const orc_block_q4_0 *vc,
                         int n_heads, int n_kv_heads, int head_dim, int n_ctx,
                         int64_t pos, const float *q, double scale,
                         double *out) {
    int window;
    int64_t start;
    orc_ring_window(pos, n_ctx, &window, &start, NULL);
    const int q_per_kv = n_heads / n_kv_heads;
    double *sc = (double *) malloc(sizeof(double) * (size_t) window);
    float *row = (float *) malloc(sizeof(float) * (size_t) head_dim);
    for (int h = 0; h < n_heads; ++h) {
        const int kvh = (n_kv_heads == n_heads) ? h : h / q_per_kv;
        const float *qh = q + (size_t) h * head_dim;
        double mx = -INFINITY;
        for (int i = 0; i < window; ++i) {
            const int slot = (int) ((start + i) % n_ctx);
            dequant_row(kc, kvh, slot, head_dim, n_ctx, row);
            double dot = 0.0;
            for (int d = 0; d < head_dim; ++d) dot += (double) qh[d] * (double) row[d];
            sc[i] = dot * scale;
            if (sc[i] > mx) mx = sc[i];
        }
        double sum = 0.0;
        for (int i = 0; i < window; ++i) {
            sc[i] = exp(sc[i] - mx);
            sum += sc[i];
        }
        double *oh = out + (size_t) h * head_dim;
        for (int d = 0; d < head_dim; ++d) oh[d] = 0.0;
        for (int i = 0; i < window; ++i) {
            const int slot = (int) ((start + i) % n_ctx);
            dequant_row(vc, kvh, slot, head_dim, n_ctx, row);
            const double w = sc[i] / sum;
            for (int d = 0; d < head_dim; ++d) oh[d] += w * (double) row[d];
        }
    }
    free(row);
    free(sc);
}

void orc_ring_prefill_f64(orc_block_q4_0 *kc, orc_block_q4_0 *vc, int n_heads,
                          int n_kv_heads, int head_dim, int n_ctx, int64_t pos0,
                          int n_tok, const float *q, const float *k,
                          const float *v, double scale, double *out) {
    const int nblk = head_dim / ORC_QK4_0;
    const int q_per_kv = n_heads / n_kv_heads;
    /* Quantize the chunk rows once: these exact blocks are what attention
     * sees for chunk positions and what is appended afterwards. */
    const size_t rows = (size_t) n_tok * (size_t) n_kv_heads;
    orc_block_q4_0 *kq = (orc_block_q4_0 *) malloc(sizeof(orc_block_q4_0) * rows * nblk);
    orc_block_q4_0 *vq = (orc_block_q4_0 *) malloc(sizeof(orc_block_q4_0) * rows * nblk);
    orc_quantize_row_q4_0(k, kq, (int64_t) rows * head_dim);
    orc_quantize_row_q4_0(v, vq, (int64_t) rows * head_dim);
    float *row = (float *) malloc(sizeof(float) * (size_t) head_dim);
    double *sc = (double *) malloc(sizeof(double) * (size_t) n_ctx);
    for (int i = 0; i < n_tok; ++i) {
        const int64_t p = pos0 + i;
        int window;
        int64_t start;
        orc_ring_window(p, n_ctx, &window, &start, NULL);
        for (int h = 0; h < n_heads; ++h) {
            const int kvh = (n_kv_heads == n_heads) ? h : h / q_per_kv;
            const float *qh = q + ((size_t) i * n_heads + h) * head_dim;
            double mx = -INFINITY;
            for (int j = 0; j < window; ++j) {
                const int64_t t = start + j;
                if (t < pos0) {
                    dequant_row(kc, kvh, (int) (t % n_ctx), head_dim, n_ctx, row);
                } else {
                    orc_dequantize_row_q4_0(kq + ((size_t) (t - pos0) * n_kv_heads + kvh) * nblk,
                                            row, head_dim);
                }
                double dot = 0.0;
                for (int d = 0; d < head_dim; ++d) dot += (double) qh[d] * (double) row[d];
                sc[j] = dot * scale;
                if (sc[j] > mx) mx = sc[j];
            }
            double sum = 0.0;
            for (int j = 0; j < window; ++j) {
                sc[j] = exp(sc[j] - mx);
                sum += sc[j];
            }
            double *oh = out + ((size_t) i * n_heads + h) * head_dim;
            for (int d = 0; d < head_dim; ++d) oh[d] = 0.0;
            for (int j = 0; j < window; ++j) {
                const int64_t t = start + j;
                if (t < pos0) {
                    dequant_row(vc, kvh, (int) (t % n_ctx), head_dim, n_ctx, row);
                } else {
                    orc_dequantize_row_q4_0(vq + ((size_t) (t - pos0) * n_kv_heads + kvh) * nblk,
                                            row, head_dim);
                }
                const double w = sc[j] / sum;
                for (int d = 0; d < head_dim; ++d) oh[d] += w * (double) row[d];
            }
        }
    }
    /* Commit the chunk to the ring. */
    for (int i = 0; i < n_tok; ++i) {
        const int slot = (int) ((pos0 + i) % n_ctx);
        for (int h = 0; h < n_kv_heads; ++h) {
            memcpy(kc + blk_index(h, slot, 0, n_ctx, nblk),
                   kq + ((size_t) i * n_kv_heads + h) * nblk, sizeof(orc_block_q4_0) * nblk);
            memcpy(vc + blk_index(h, slot, 0, n_ctx, nblk),
                   vq + ((size_t) i * n_kv_heads + h) * nblk, sizeof(orc_block_q4_0) * nblk);
        }
    }
    free(sc);
    free(row);
    free(vq);
    free(kq);
}

/* src/bmo_api.cpp:315-331: out[(ti * n_heads + h) * head_dim + d] = K[d, slot
 * t_start + ti, h] as fp32. */
void orc_ring_copy_k_f32(const orc_block_q4_0 *kc, int n_heads, int head_dim,
                         int n_ctx, int t_start, int n_pos, float *out) {
    for (int ti = 0; ti < n_pos; ++ti) {
        for (int h = 0; h < n_heads; ++h) {
            dequant_row(kc, h, t_start + ti, head_dim, n_ctx,
                        out + ((size_t) ti * n_heads + h) * head_dim);
        }
    }
}

/* ---- seeded synthetic inputs ----------------------------------------------- */

/* splitmix64 output function (Steele, Lea, Flood 2014). */
uint64_t orc_mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

void orc_fill_u64(uint64_t seed, uint64_t offset, uint64_t *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        out[i] = orc_mix64(seed ^ orc_mix64(offset + (uint64_t) i));
    }
}

/* The synthetic input stream of the benchmark configurations (the seeds and
 * layouts are listed with the configurations): element c of stream `seed` is
 * a Box-Muller normal of two splitmix64 words, cosine branch only,
 *   a = mix64(seed ^ mix64(2c)),  b = mix64(seed ^ mix64(2c + 1)),
 *   u1 = (a >> 11) + 0.5) 2^-53,  u2 = (b >> 11) 2^-53,
 *   z = (float) (sqrt(-2 ln u1) cos(2 pi u2)),
 * with ln and cos(2 pi .) evaluated from +, -, *, / and sqrt alone (no fused
 * multiply-add, no library transcendental), each correctly rounded in
 * IEEE double, so that a device implementation of the same steps gives the
 * same bits.  The "kv" variant multiplies an element by 8 when a third word,
 * mix64((seed ^ 0xD1B54A32D192ED03) ^ mix64(c)), has its top 32 bits below
 * 42949673 (probability 0.0100000000093). */

/* ln x for x in [2^-54, 1]: x = m 2^e with m in [sqrt(1/2), sqrt(2)], ln x =
 * e ln 2 + 2 atanh(s), s = (m - 1)/(m + 1), |s| <= 0.1716, the atanh series
 * to s^21 (the next term is below 2^-55 of the sum). */
static double synth_ln(double x) {
    uint64_t bits;
    memcpy(&bits, &x, sizeof bits);
    int e = (int) ((bits >> 52) & 0x7FF) - 1023;
    bits = (bits & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull;
    double m;
    memcpy(&m, &bits, sizeof m);
    if (m > 0x1.6a09e667f3bcdp+0) {  /* sqrt(2) */
        m = m * 0.5;
        e = e + 1;
    }
    const double s = (m - 1.0) / (m + 1.0);
    const double s2 = s * s;
    double p = 0x1.8618618618618p-5;            /* 1/21 */
    p = p * s2 + 0x1.af286bca1af28p-5;          /* 1/19 */
    p = p * s2 + 0x1.e1e1e1e1e1e1ep-5;          /* 1/17 */
    p = p * s2 + 0x1.1111111111111p-4;          /* 1/15 */
    p = p * s2 + 0x1.3b13b13b13b14p-4;          /* 1/13 */
    p = p * s2 + 0x1.745d1745d1746p-4;          /* 1/11 */
    p = p * s2 + 0x1.c71c71c71c71cp-4;          /* 1/9 */
    p = p * s2 + 0x1.2492492492492p-3;          /* 1/7 */
    p = p * s2 + 0x1.999999999999ap-3;          /* 1/5 */
    p = p * s2 + 0x1.5555555555555p-2;          /* 1/3 */
    p = p * s2 + 1.0;
    return (double) e * 0x1.62e42fefa39efp-1 + 2.0 * (s * p);   /* ln 2 */
}

/* cos(2 pi t) for t in [0, 1): quadrant n = floor(4t), g = 4t - n (both
 * exact), cos(pi/2 (n + g)) = cos y, -sin y, -cos y, sin y for n = 0..3 with
 * y = pi/2 g; g > 1/2 is folded to 1 - g with cos and sin swapped, so
 * y <= pi/4 and the Taylor series to y^16 (cos) or y^17 (sin) suffice. */
static double synth_cos2pi(double t) {
    const double t4 = t * 4.0;
    const int n = (int) t4;
    double g = t4 - (double) n;
    int use_sin = n & 1;
    const int neg = n == 1 || n == 2;
    if (g > 0.5) {
        g = 1.0 - g;
        use_sin ^= 1;
    }
    const double y = g * 0x1.921fb54442d18p+0;  /* pi/2 */
    const double y2 = y * y;
    double r;
    if (use_sin) {
        double p = 0x1.952c77030ad4ap-49;       /* 1/17! */
        p = 0x1.ae7f3e733b81fp-41 - y2 * p;     /* 1/15! */
        p = 0x1.6124613a86d09p-33 - y2 * p;     /* 1/13! */
        p = 0x1.ae64567f544e4p-26 - y2 * p;     /* 1/11! */
        p = 0x1.71de3a556c734p-19 - y2 * p;     /* 1/9! */
        p = 0x1.a01a01a01a01ap-13 - y2 * p;     /* 1/7! */
        p = 0x1.1111111111111p-7 - y2 * p;      /* 1/5! */
        p = 0x1.5555555555555p-3 - y2 * p;      /* 1/3! */
        p = 1.0 - y2 * p;
        r = y * p;
    } else {
        double p = 0x1.ae7f3e733b81fp-45;       /* 1/16! */
        p = 0x1.93974a8c07c9dp-37 - y2 * p;     /* 1/14! */
        p = 0x1.1eed8eff8d898p-29 - y2 * p;     /* 1/12! */
        p = 0x1.27e4fb7789f5cp-22 - y2 * p;     /* 1/10! */
        p = 0x1.a01a01a01a01ap-16 - y2 * p;     /* 1/8! */
        p = 0x1.6c16c16c16c17p-10 - y2 * p;     /* 1/6! */
        p = 0x1.5555555555555p-5 - y2 * p;      /* 1/4! */
        p = 0.5 - y2 * p;                       /* 1/2! */
        r = 1.0 - y2 * p;
    }
    return neg ? -r : r;
}

static float synth_normal(uint64_t seed, uint64_t c) {
    const uint64_t a = orc_mix64(seed ^ orc_mix64(2 * c));
    const uint64_t b = orc_mix64(seed ^ orc_mix64(2 * c + 1));
    const double u1 = ((double) (a >> 11) + 0.5) * 0x1p-53;
    const double u2 = (double) (b >> 11) * 0x1p-53;
    return (float) (sqrt(-2.0 * synth_ln(u1)) * synth_cos2pi(u2));
}

void orc_fill_normal(uint64_t seed, uint64_t offset, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = synth_normal(seed, offset + (uint64_t) i);
}

void orc_fill_kv(uint64_t seed, uint64_t offset, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const uint64_t c = offset + (uint64_t) i;
        const float z = synth_normal(seed, c);
        const uint64_t w = orc_mix64((seed ^ 0xD1B54A32D192ED03ull) ^ orc_mix64(c));
        out[i] = (w >> 32) < 42949673u ? z * 8.0f : z;
    }
}

double orc_synth_ln(double x) { return synth_ln(x); }
double orc_synth_cos2pi(double t) { return synth_cos2pi(t); }
