/*
 * cpu_ggml_style.c -- a SIMD CPU baseline restating the arithmetic of ggml's
 * CPU flash attention over a Q4_0 K/V cache, the backend the reference's lazy
 * path reaches through ggml_flash_attn_ext (src/bmo_compute.cpp:2410-2412;
 * ggml itself is fetched at configure time, CMakeLists.txt:45-55, and is not
 * available here).  TEST INFRASTRUCTURE ONLY (see oracle.h): it is a timed
 * baseline reported next to the GPU numbers, never the product.
 *
 * Steps, per (session, query head), as ggml's CPU flash attention runs them
 * for a quantized K (from its published algorithm):
 *   - q is converted to the vec-dot type of Q4_0, Q8_0: per 32 elements
 *     d = max|x| / 127 stored as fp16, codes roundf(x / d);
 *   - each key's score is the Q4_0 x Q8_0 dot product, sum over blocks of
 *     d_k * d_q * sum((c - 8) * q8), times the softmax scale;
 *   - online softmax with expf: when a score exceeds the running max M, the
 *     accumulator and the sum are scaled by expf(M_old - M), else the key's
 *     weight is expf(s - M);
 *   - the V row is dequantized to fp32 ((c - 8) * d) and accumulated with
 *     that weight; the output is the accumulator over the weight sum.
 * The window is the ring's (src/bmo_cuda_kernels.cu:739-747).  The dot product
 * and the V accumulation are vectorized with AVX2 (the build targets
 * x86-64-v3), one thread per contiguous range of (session, head) units.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define GG_MAX_HEAD_DIM 256
#define GG_MAX_BLOCKS (GG_MAX_HEAD_DIM / 32)

typedef struct {
    uint16_t d;   /* fp16 scale */
    int8_t qs[32];
} q8_block;

static void quantize_q8_0(const float *x, q8_block *y, int n_blocks) {
    for (int b = 0; b < n_blocks; ++b) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float a = fabsf(x[b * 32 + j]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[b].d = _cvtss_sh(d, 0);
        for (int j = 0; j < 32; ++j) y[b].qs[j] = (int8_t) roundf(x[b * 32 + j] * id);
    }
}

/* 16 code bytes -> 32 signed bytes c - 8 in element order (low nibbles are
 * elements 0..15, high nibbles 16..31). */
static inline __m256i unpack_q4_0(const uint8_t *qs) {
    const __m128i raw = _mm_loadu_si128((const __m128i *) qs);
    const __m256i both = _mm256_set_m128i(_mm_srli_epi16(raw, 4), raw);
    return _mm256_sub_epi8(_mm256_and_si256(both, _mm256_set1_epi8(0x0F)), _mm256_set1_epi8(8));
}

static inline float hsum8(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

/* sum over blocks of d_k * d_q * sum((c - 8) * q8) */
static float dot_q4_0_q8_0(const orc_block_q4_0 *k, const q8_block *q, int n_blocks) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i ones = _mm256_set1_epi16(1);
    for (int b = 0; b < n_blocks; ++b) {
        const __m256i x = unpack_q4_0(k[b].qs);
        const __m256i y = _mm256_loadu_si256((const __m256i *) q[b].qs);
        /* |x| * (y with x's sign): unsigned x signed products in pairs */
        const __m256i ax = _mm256_sign_epi8(x, x);
        const __m256i sy = _mm256_sign_epi8(y, x);
        const __m256i s32 = _mm256_madd_epi16(_mm256_maddubs_epi16(ax, sy), ones);
        const __m256 d = _mm256_set1_ps(_cvtsh_ss(k[b].d) * _cvtsh_ss(q[b].d));
        acc = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(s32), acc);
    }
    return hsum8(acc);
}

/* row (head_dim fp32) of (c - 8) * d */
static void dequant_row(const orc_block_q4_0 *v, float *row, int n_blocks) {
    for (int b = 0; b < n_blocks; ++b) {
        const __m256i x = unpack_q4_0(v[b].qs);
        const __m256 d = _mm256_set1_ps(_cvtsh_ss(v[b].d));
        const __m128i lo = _mm256_castsi256_si128(x), hi = _mm256_extracti128_si256(x, 1);
        _mm256_storeu_ps(row + b * 32 + 0, _mm256_mul_ps(d, _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(lo))));
        _mm256_storeu_ps(row + b * 32 + 8,
                         _mm256_mul_ps(d, _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(lo, 8)))));
        _mm256_storeu_ps(row + b * 32 + 16, _mm256_mul_ps(d, _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(hi))));
        _mm256_storeu_ps(row + b * 32 + 24,
                         _mm256_mul_ps(d, _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(hi, 8)))));
    }
}

static void attend_head(const orc_block_q4_0 *kc, const orc_block_q4_0 *vc, int kvh, int head_dim,
                        int n_ctx, int64_t pos, const float *qh, float *oh) {
    const int nblk = head_dim / ORC_QK4_0;
    const int64_t total = pos + 1;
    const int window = (int) (total > n_ctx ? n_ctx : total);
    const int64_t start = total - window;
    const float scale = 1.0f / sqrtf((float) head_dim);
    q8_block q8[GG_MAX_BLOCKS];
    quantize_q8_0(qh, q8, nblk);
    float acc[GG_MAX_HEAD_DIM] __attribute__((aligned(32)));
    float row[GG_MAX_HEAD_DIM] __attribute__((aligned(32)));
    memset(acc, 0, sizeof(float) * (size_t) head_dim);
    float M = -INFINITY, S = 0.0f;
    for (int i = 0; i < window; ++i) {
        const int slot = (int) ((start + i) % n_ctx);
        const size_t off = ((size_t) kvh * n_ctx + slot) * nblk;
        const float s = dot_q4_0_q8_0(kc + off, q8, nblk) * scale;
        float ms = 1.0f, vs = 1.0f;
        if (s > M) {
            const float m_old = M;
            M = s;
            ms = expf(m_old - M);
            const __m256 f = _mm256_set1_ps(ms);
            for (int e = 0; e < head_dim; e += 8)
                _mm256_store_ps(acc + e, _mm256_mul_ps(_mm256_load_ps(acc + e), f));
        } else {
            vs = expf(s - M);
        }
        dequant_row(vc + off, row, nblk);
        const __m256 w = _mm256_set1_ps(vs);
        for (int e = 0; e < head_dim; e += 8)
            _mm256_store_ps(acc + e, _mm256_fmadd_ps(_mm256_load_ps(row + e), w, _mm256_load_ps(acc + e)));
        S = S * ms + vs;
    }
    const float inv = S > 0.0f ? 1.0f / S : 0.0f;
    for (int e = 0; e < head_dim; ++e) oh[e] = acc[e] * inv;
}

typedef struct {
    const orc_block_q4_0 *kc, *vc;
    int n_heads, n_kv_heads, head_dim, n_ctx;
    const int64_t *pos;
    const float *q;
    float *out;
    int unit_begin, unit_end, iters;
} gg_job;

static void *gg_worker(void *arg) {
    gg_job *j = (gg_job *) arg;
    const int nblk = j->head_dim / ORC_QK4_0;
    const size_t sess_blocks = (size_t) j->n_kv_heads * j->n_ctx * nblk;
    const int q_per_kv = j->n_heads / j->n_kv_heads;
    for (int it = 0; it < j->iters; ++it) {
        for (int u = j->unit_begin; u < j->unit_end; ++u) {
            const int s = u / j->n_heads;
            const int h = u % j->n_heads;
            const size_t row = ((size_t) s * j->n_heads + h) * j->head_dim;
            attend_head(j->kc + s * sess_blocks, j->vc + s * sess_blocks, h / q_per_kv, j->head_dim,
                        j->n_ctx, j->pos[s], j->q + row, j->out + row);
        }
    }
    return NULL;
}

double orc_cpu_ggml_style_run(const orc_block_q4_0 *kc, const orc_block_q4_0 *vc, int n_sess,
                              int n_heads, int n_kv_heads, int head_dim, int n_ctx,
                              const int64_t *pos, const float *q, float *out, int n_threads,
                              int iters) {
    if (n_threads < 1) n_threads = 1;
    if (head_dim > GG_MAX_HEAD_DIM || head_dim % 32 != 0) return -1.0;
    const int units = n_sess * n_heads;
    if (n_threads > units) n_threads = units;
    gg_job *jobs = (gg_job *) calloc((size_t) n_threads, sizeof(gg_job));
    pthread_t *tids = (pthread_t *) calloc((size_t) n_threads, sizeof(pthread_t));
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int t = 0; t < n_threads; ++t) {
        jobs[t] = (gg_job){kc, vc, n_heads, n_kv_heads, head_dim, n_ctx, pos, q, out,
                           (int) ((int64_t) units * t / n_threads),
                           (int) ((int64_t) units * (t + 1) / n_threads), iters};
        if (n_threads == 1)
            gg_worker(&jobs[0]);
        else
            pthread_create(&tids[t], NULL, gg_worker, &jobs[t]);
    }
    if (n_threads > 1)
        for (int t = 0; t < n_threads; ++t) pthread_join(tids[t], NULL);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    free(tids);
    free(jobs);
    return (double) (t1.tv_sec - t0.tv_sec) + 1e-9 * (double) (t1.tv_nsec - t0.tv_nsec);
}
