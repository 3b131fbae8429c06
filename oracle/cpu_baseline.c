/*
 * cpu_baseline.c -- the timed CPU baseline for bench.py: an fp32 restatement
 * of the reference's eager CPU decode attention (src/bmo_compute.cpp:927-970,
 * single threaded in the reference) reading the Q4_0 ring with the window of
 * src/bmo_cuda_kernels.cu:739-747.  Each cached row is dequantized to fp32
 * right before use, as the reference converts each fp16 element with
 * ggml_fp16_to_fp32 inside its loops.  TEST INFRASTRUCTURE ONLY (see oracle.h):
 * it is the baseline the GPU numbers are reported next to, never the product.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define MAX_HEAD_DIM 256

static void decode_head(const orc_block_q4_0 *kc, const orc_block_q4_0 *vc,
                        int kvh, int head_dim, int n_ctx, int64_t pos,
                        const float *qh, float *oh, float *scores) {
    const int nblk = head_dim / ORC_QK4_0;
    const int64_t total = pos + 1;
    const int window = (int) (total > n_ctx ? n_ctx : total);
    const int64_t start = total - window;
    const float scale = 1.0f / sqrtf((float) head_dim);
    float row[MAX_HEAD_DIM];
    for (int i = 0; i < window; ++i) {
        const int slot = (int) ((start + i) % n_ctx);
        orc_dequantize_row_q4_0(kc + ((size_t) kvh * n_ctx + slot) * nblk, row, head_dim);
        float dot = 0.0f;
        for (int d = 0; d < head_dim; ++d) dot += qh[d] * row[d];
        scores[i] = dot * scale;
    }
    float mx = scores[0];
    for (int i = 1; i < window; ++i) if (scores[i] > mx) mx = scores[i];
    float sum = 0.0f;
    for (int i = 0; i < window; ++i) {
        const float e = expf(scores[i] - mx);
        scores[i] = e;
        sum += e;
    }
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (int i = 0; i < window; ++i) scores[i] *= inv;
    for (int d = 0; d < head_dim; ++d) oh[d] = 0.0f;
    for (int i = 0; i < window; ++i) {
        const int slot = (int) ((start + i) % n_ctx);
        orc_dequantize_row_q4_0(vc + ((size_t) kvh * n_ctx + slot) * nblk, row, head_dim);
        const float w = scores[i];
        for (int d = 0; d < head_dim; ++d) oh[d] += w * row[d];
    }
}

void orc_cpu_decode_f32(const orc_block_q4_0 *kc, const orc_block_q4_0 *vc,
                        int n_heads, int n_kv_heads, int head_dim, int n_ctx,
                        int64_t pos, const float *q, float *out,
                        float *scores_scratch) {
    const int q_per_kv = n_heads / n_kv_heads;
    for (int h = 0; h < n_heads; ++h) {
        const int kvh = (n_kv_heads == n_heads) ? h : h / q_per_kv;
        decode_head(kc, vc, kvh, head_dim, n_ctx, pos, q + (size_t) h * head_dim,
                    out + (size_t) h * head_dim, scores_scratch);
    }
}

typedef struct {
    const orc_block_q4_0 *kc, *vc;
    int n_sess, n_heads, n_kv_heads, head_dim, n_ctx;
    const int64_t *pos;
    const float *q;
    float *out;
    int unit_begin, unit_end, iters;
} job_t;

static void *worker(void *arg) {
    job_t *j = (job_t *) arg;
    const int nblk = j->head_dim / ORC_QK4_0;
    const size_t sess_blocks = (size_t) j->n_kv_heads * j->n_ctx * nblk;
    const int q_per_kv = j->n_heads / j->n_kv_heads;
    float *scores = (float *) malloc(sizeof(float) * (size_t) j->n_ctx);
    for (int it = 0; it < j->iters; ++it) {
        for (int u = j->unit_begin; u < j->unit_end; ++u) {
            const int s = u / j->n_heads;
            const int h = u % j->n_heads;
            const int kvh = (j->n_kv_heads == j->n_heads) ? h : h / q_per_kv;
            const size_t row = ((size_t) s * j->n_heads + h) * j->head_dim;
            decode_head(j->kc + s * sess_blocks, j->vc + s * sess_blocks, kvh,
                        j->head_dim, j->n_ctx, j->pos[s], j->q + row, j->out + row,
                        scores);
        }
    }
    free(scores);
    return NULL;
}

double orc_cpu_baseline_run(const orc_block_q4_0 *kc, const orc_block_q4_0 *vc,
                            int n_sess, int n_heads, int n_kv_heads,
                            int head_dim, int n_ctx, const int64_t *pos,
                            const float *q, float *out, int n_threads,
                            int iters) {
    if (n_threads < 1) n_threads = 1;
    if (head_dim > MAX_HEAD_DIM) return -1.0;
    const int units = n_sess * n_heads;
    if (n_threads > units) n_threads = units;
    job_t *jobs = (job_t *) calloc((size_t) n_threads, sizeof(job_t));
    pthread_t *tids = (pthread_t *) calloc((size_t) n_threads, sizeof(pthread_t));
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int t = 0; t < n_threads; ++t) {
        jobs[t] = (job_t){kc, vc, n_sess, n_heads, n_kv_heads, head_dim, n_ctx, pos, q, out,
                          (int) ((int64_t) units * t / n_threads),
                          (int) ((int64_t) units * (t + 1) / n_threads), iters};
        if (n_threads == 1) {
            worker(&jobs[0]);
        } else {
            pthread_create(&tids[t], NULL, worker, &jobs[t]);
        }
    }
    if (n_threads > 1) {
        for (int t = 0; t < n_threads; ++t) pthread_join(tids[t], NULL);
    }
    clock_gettime(CLOCK_MONOTONIC, &t1);
    free(tids);
    free(jobs);
    return (double) (t1.tv_sec - t0.tv_sec) + 1e-9 * (double) (t1.tv_nsec - t0.tv_nsec);
}
