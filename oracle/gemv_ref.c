/*
 * gemv_ref.c -- oracle restatement of the reference's Q4_0 x Q8_1 GEMV
 * (TEST INFRASTRUCTURE ONLY; see oracle.h).
 *
 * launch_gemv_q4_0_q8_1 (src/bmo_cuda_kernels.cu:685-711) quantizes the fp32
 * activation row into Q8_1 blocks (bmo_quantize_row_q8_1_kernel, :529-558)
 * and multiplies every Q4_0 weight row by it (bmo_gemv_q4_0_q8_1_kernel,
 * :560-683).  Per 32-element block of x: amax = max |x_j| (strict running
 * compare from 0), d = amax / 127, id = d ? 1/d : 0, q_j = clamp(roundf(x_j *
 * id), -128, 127), and the block's second field is fp16 of the sequential
 * fp32 sum of the ORIGINAL x_j (this reference's choice; ggml's own Q8_1
 * stores d * sum(q)).  Per weight block: sumi = sum_j code_j * q_j over the
 * unsigned codes (dp4a, :641-660), term = d4 * (sumi * d8 - 8 * s8) (the two
 * half-block lanes' 4 * s8 corrections, :662-665, summed), y = sum of terms.
 * Here the terms and their sum are evaluated in double from the fp16 fields.
 */
#include <math.h>
#include <string.h>

#include "oracle.h"

void orc_quantize_row_q8_1_bmo(const float *x, orc_block_q8_1 *y, int64_t k) {
    const int64_t nb = k / ORC_QK8_1;
    for (int64_t i = 0; i < nb; ++i) {
        const float *src = x + i * ORC_QK8_1;
        float amax = 0.0f;
        for (int j = 0; j < ORC_QK8_1; ++j) {
            const float v = fabsf(src[j]);
            if (v > amax) amax = v;
        }
        const float d = amax / 127.0f;
        const float id = (d != 0.0f) ? (1.0f / d) : 0.0f;
        float sum = 0.0f;
        for (int j = 0; j < ORC_QK8_1; ++j) {
            const float v = src[j];
            const float p = v * id;
            int q0 = (int) roundf(p);
            if (q0 > 127) q0 = 127;
            if (q0 < -128) q0 = -128;
            y[i].qs[j] = (int8_t) q0;
            sum += v;
        }
        y[i].d = orc_fp32_to_fp16(d);
        y[i].s = orc_fp32_to_fp16(sum);
    }
}

double orc_vec_dot_q4_0_q8_1_f64(const orc_block_q4_0 *w, const orc_block_q8_1 *x, int64_t nb) {
    double acc = 0.0;
    for (int64_t b = 0; b < nb; ++b) {
        int sumi = 0;
        for (int j = 0; j < ORC_QK4_0 / 2; ++j) {
            sumi += (int) (w[b].qs[j] & 0x0F) * (int) x[b].qs[j];
            sumi += (int) (w[b].qs[j] >> 4) * (int) x[b].qs[j + ORC_QK4_0 / 2];
        }
        const double d4 = orc_fp16_to_fp32(w[b].d);
        const double d8 = orc_fp16_to_fp32(x[b].d);
        const double s8 = orc_fp16_to_fp32(x[b].s);
        acc += d4 * ((double) sumi * d8 - 8.0 * s8);
    }
    return acc;
}

void orc_gemv_q4_0_q8_1_f64(const orc_block_q4_0 *w, const orc_block_q8_1 *x, int rows,
                            int cols, double *y) {
    const int64_t nb = cols / ORC_QK4_0;
    for (int r = 0; r < rows; ++r) y[r] = orc_vec_dot_q4_0_q8_1_f64(w + (int64_t) r * nb, x, nb);
}

void orc_gemv_term_abs_f64(const orc_block_q4_0 *w, const orc_block_q8_1 *x, int rows, int cols,
                           double *y) {
    const int64_t nb = cols / ORC_QK4_0;
    for (int r = 0; r < rows; ++r) {
        double acc = 0.0;
        for (int64_t b = 0; b < nb; ++b) {
            const orc_block_q4_0 *wb = w + (int64_t) r * nb + b;
            int sumi = 0;
            for (int j = 0; j < ORC_QK4_0 / 2; ++j) {
                sumi += (int) (wb->qs[j] & 0x0F) * (int) x[b].qs[j];
                sumi += (int) (wb->qs[j] >> 4) * (int) x[b].qs[j + ORC_QK4_0 / 2];
            }
            const double d4 = orc_fp16_to_fp32(wb->d);
            acc += fabs(d4) * (fabs((double) sumi * orc_fp16_to_fp32(x[b].d)) +
                               fabs(8.0 * orc_fp16_to_fp32(x[b].s)));
        }
        y[r] = acc;
    }
}
