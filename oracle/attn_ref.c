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

/* Box-Muller on two splitmix64 words per element (cosine branch only). */
void orc_fill_normal(uint64_t seed, uint64_t offset, float *out, int64_t n) {
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; ++i) {
        const uint64_t c = offset + (uint64_t) i;
        const uint64_t a = orc_mix64(seed ^ orc_mix64(2 * c));
        const uint64_t b = orc_mix64(seed ^ orc_mix64(2 * c + 1));
        const double u1 = ((double) (a >> 11) + 0.5) * (1.0 / 9007199254740992.0);
        const double u2 = (double) (b >> 11) * (1.0 / 9007199254740992.0);
        out[i] = (float) (sqrt(-2.0 * log(u1)) * cos(two_pi * u2));
    }
}
