/*
 * oracle.h -- CPU restatement of bmo_jetson's sliding-window decode attention
 * over a Q4_0 ring KV cache.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the parity tests,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py compare the
 * HIP path against.  Nothing in the product (bmo_jetson_amd/, include/) links,
 * loads or calls it, and the product never falls back to it.
 *
 * Functions and what pins each one (reference citations are path:line into
 * utkarshyadav009/bmo_jetson):
 *
 *   orc_fp32_to_fp16 / orc_fp16_to_fp32
 *       GGML_FP32_TO_FP16 / ggml_fp16_to_fp32 as used at
 *       src/bmo_compute.cpp:885-886,921,941,967 (IEEE-754 binary16,
 *       round-to-nearest-even).  Pinned by an exhaustive comparison over all
 *       2^32 fp32 bit patterns against the host's F16C instruction
 *       (orc_selftest_fp16_exhaustive) and against numpy's float16 cast.
 *   orc_quantize_row_q4_0 / orc_dequantize_row_q4_0
 *       ggml quantize_row_q4_0_ref / dequantize_row_q4_0 (ggml is fetched at
 *       configure time with GIT_TAG master, CMakeLists.txt:45-55, and is not
 *       in the reference tree; the published algorithm is restated).  Block
 *       format from src/bmo_cuda_kernels.cu:496-499; dequant (q-8)*d pinned by
 *       src/bmo_kernel_bench.cu:92-93 and nibble order by
 *       src/bmo_cuda_kernels.cu:626-629.  Pinned by hand-derived known answers,
 *       a brute-force nearest-code check and error-bound invariants
 *       (tests/test_oracle_q4_0.py).
 *   orc_ring_window
 *       src/bmo_cuda_kernels.cu:739-743.  Pinned by closed forms and a brute
 *       force enumeration (tests/test_oracle_ring.py).
 *   orc_ring_append
 *       KV write of src/bmo_cuda_kernels.cu:749-754 (slot pos % n_ctx) with the
 *       F16 conversion replaced by Q4_0 quantization.
 *   orc_ring_decode_f64
 *       attention math of src/bmo_compute.cpp:927-970 with the ring window of
 *       src/bmo_cuda_kernels.cu:739-747, evaluated in double precision.
 *       Pinned by closed forms (window 1, uniform scores, dominant key,
 *       q = 0) and by a float64 numpy evaluation on dequantized K/V.
 *   orc_ring_prefill_f64
 *       chunked prefill with a causal + sliding-window mask over the ring
 *       (new semantics; the reference's lazy path at
 *       src/bmo_compute.cpp:2376-2418 is linear and unmasked).  Pinned by the
 *       identity "prefill of C tokens == C successive decode steps".
 *   orc_rope_interleaved / orc_rope_cos_sin / orc_rope_freq
 *       interleaved RoPE of src/bmo_cuda_kernels.cu:317-354 (pairs (2i, 2i+1),
 *       angle pos * theta^(-2i/head_dim)), cosine and sine in double rounded
 *       to fp32, fp32 rotation.  Pinned by a complex-exponential evaluation
 *       in numpy, pos = 0 identity, pair-norm preservation, composition of
 *       rotations, and the relative-position property of rotated dot
 *       products (tests/test_oracle_rope.py).
 *   orc_quantize_row_q8_1_bmo / orc_gemv_q4_0_q8_1_f64
 *       the reference's activation quantizer and Q4_0 x Q8_1 GEMV
 *       (src/bmo_cuda_kernels.cu:529-711), terms summed in double.  Pinned
 *       by hand-derived known answers (round half away from zero, clamp,
 *       the sum field), nearest-code and range invariants, and an
 *       independent numpy evaluation from the raw block bytes
 *       (tests/test_oracle_gemv.py).
 *   orc_cpu_decode_f32 / orc_cpu_baseline_*
 *       timed CPU baseline: fp32 restatement of the reference's single
 *       threaded eager path src/bmo_compute.cpp:927-970 over dequantized Q4_0.
 */
#ifndef BMO_ORACLE_H
#define BMO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK4_0 32

/* 18-byte Q4_0 block, byte-identical to ggml block_q4_0
 * (src/bmo_cuda_kernels.cu:496-499): fp16 scale then 16 nibble bytes.
 * Element j (0..15) is the low nibble of qs[j], element j+16 the high one. */
typedef struct {
    uint16_t d;
    uint8_t qs[ORC_QK4_0 / 2];
} orc_block_q4_0;

/* ---- fp16 ---------------------------------------------------------------- */
uint16_t orc_fp32_to_fp16(float f);
float orc_fp16_to_fp32(uint16_t h);
/* Returns the number of fp32 bit patterns (non-NaN) whose conversion differs
 * from the host F16C instruction, or -1 if the host lacks F16C. */
int64_t orc_selftest_fp16_exhaustive(void);

/* ---- Q4_0 ------------------------------------------------------------------ */
void orc_quantize_row_q4_0(const float *x, orc_block_q4_0 *y, int64_t k);
void orc_dequantize_row_q4_0(const orc_block_q4_0 *x, float *y, int64_t k);

/* ---- ring geometry -------------------------------------------------------- */
/* total = pos+1, window = min(total, n_ctx), start = total-window,
 * cur_slot = pos % n_ctx. */
void orc_ring_window(int64_t pos, int n_ctx, int *window, int64_t *start,
                     int *cur_slot);

/* Ring stripe layout used by every oracle routine (the reference's ggml
 * ne = [head_dim, n_ctx, n_heads] order with Q4_0 blocks along head_dim):
 *   block (h, slot, b) at index (h * n_ctx + slot) * (head_dim/32) + b. */

/* Quantize k, v ([n_kv_heads][head_dim] fp32) into slot pos % n_ctx. */
void orc_ring_append(orc_block_q4_0 *kc, orc_block_q4_0 *vc, int n_kv_heads,
                     int head_dim, int n_ctx, int64_t pos, const float *k,
                     const float *v);

/* Decode attention of q ([n_heads][head_dim] fp32) over the window that ends
 * at pos.  out is [n_heads][head_dim] double. */
void orc_ring_decode_f64(const orc_block_q4_0 *kc, const orc_block_q4_0 *vc,
                         int n_heads, int n_kv_heads, int head_dim, int n_ctx,
                         int64_t pos, const float *q, double scale,
                         double *out);

/* Chunked prefill of n_tok tokens at positions pos0 .. pos0+n_tok-1
 * (n_tok <= n_ctx).  q: [n_tok][n_heads][head_dim] fp32 (bf16 values),
 * k, v: [n_tok][n_kv_heads][head_dim] fp32 (bf16 values).  Query i attends to
 * positions max(0, pos0+i-n_ctx+1) .. pos0+i: older ones from the ring as it
 * was before the call, chunk ones from the Q4_0-quantized k/v rows.  After
 * the attention the chunk is appended to the ring.  out is
 * [n_tok][n_heads][head_dim] double. */
void orc_ring_prefill_f64(orc_block_q4_0 *kc, orc_block_q4_0 *vc, int n_heads,
                          int n_kv_heads, int head_dim, int n_ctx, int64_t pos0,
                          int n_tok, const float *q, const float *k,
                          const float *v, double scale, double *out);

/* ---- Q4_0 x Q8_1 GEMV ------------------------------------------------------ */
#define ORC_QK8_1 32
/* 36-byte Q8_1 block, byte-identical to the reference's bmo_block_q8_1
 * (src/bmo_cuda_kernels.cu:501-504): fp16 d, fp16 s, 32 int8. */
typedef struct {
    uint16_t d;
    uint16_t s;
    int8_t qs[ORC_QK8_1];
} orc_block_q8_1;

void orc_quantize_row_q8_1_bmo(const float *x, orc_block_q8_1 *y, int64_t k);
double orc_vec_dot_q4_0_q8_1_f64(const orc_block_q4_0 *w, const orc_block_q8_1 *x, int64_t nb);
/* y[r] = row r of w (rows x cols/32 blocks) dotted with x (cols/32 blocks). */
void orc_gemv_q4_0_q8_1_f64(const orc_block_q4_0 *w, const orc_block_q8_1 *x, int rows,
                            int cols, double *y);
/* Sum over blocks of |d4| * (|sumi * d8| + |8 * s8|): the scale of the
 * rounding error of any fp32 evaluation of row r (tolerance helper). */
void orc_gemv_term_abs_f64(const orc_block_q4_0 *w, const orc_block_q8_1 *x, int rows, int cols,
                           double *y);

/* ---- RoPE ------------------------------------------------------------------ */
/* r^i by binary powers (square-and-multiply from the low bit), the frequency
 * of pair i for r = theta^(-2/head_dim). */
double orc_rope_freq(double r, int i);
/* cos and sin (fp32) of pos * theta^(-2i/head_dim), i < head_dim/2 <= 512. */
void orc_rope_cos_sin(int head_dim, int64_t pos, double theta, float *cs, float *sn);
/* y = x rotated pairwise (x, y: [n_rows][head_dim]; y may be x). */
void orc_rope_interleaved(const float *x, float *y, int n_rows, int head_dim, int64_t pos,
                          double theta);

/* Copy slots [t_start, t_start+n_pos) of K as fp32, layout (n_pos, n_heads,
 * head_dim), as bmo_copy_k_cache_f32 does (src/bmo_api.cpp:283-332). */
void orc_ring_copy_k_f32(const orc_block_q4_0 *kc, int n_heads, int head_dim,
                         int n_ctx, int t_start, int n_pos, float *out);

/* ---- seeded synthetic inputs ----------------------------------------------- */
uint64_t orc_mix64(uint64_t x);
/* n standard normals, element i a pure function of (seed, offset + i): the
 * synthetic input stream of the benchmark configurations (attn_ref.c). */
void orc_fill_normal(uint64_t seed, uint64_t offset, float *out, int64_t n);
/* The same normals, each multiplied by 8 with probability 1% (a third word
 * per element decides): the K/V of configurations 3 and 4. */
void orc_fill_kv(uint64_t seed, uint64_t offset, float *out, int64_t n);
/* The stream's ln (x in [2^-54, 1]) and cos(2 pi t) (t in [0, 1)). */
double orc_synth_ln(double x);
double orc_synth_cos2pi(double t);
/* uniform 64-bit words, element i a pure function of (seed, offset + i). */
void orc_fill_u64(uint64_t seed, uint64_t offset, uint64_t *out, int64_t n);
/* fp32 -> bf16 -> fp32, round to nearest even (NaN kept quiet). */
float orc_round_bf16(float x);

/* ---- CPU baseline (timed) --------------------------------------------------- */
/* fp32 restatement of src/bmo_compute.cpp:927-970 over the Q4_0 ring, one
 * (session) stripe set: all heads.  scores_scratch holds >= n_ctx floats. */
void orc_cpu_decode_f32(const orc_block_q4_0 *kc, const orc_block_q4_0 *vc,
                        int n_heads, int n_kv_heads, int head_dim, int n_ctx,
                        int64_t pos, const float *q, float *out,
                        float *scores_scratch);
/* Runs orc_cpu_decode_f32 over n_sess sessions (each with its own ring
 * stripe set, q and pos) on n_threads threads, iters times; returns seconds. */
double orc_cpu_baseline_run(const orc_block_q4_0 *kc, const orc_block_q4_0 *vc,
                            int n_sess, int n_heads, int n_kv_heads,
                            int head_dim, int n_ctx, const int64_t *pos,
                            const float *q, float *out, int n_threads,
                            int iters);

/* A SIMD baseline restating ggml's CPU flash attention over Q4_0 K/V
 * (cpu_ggml_style.c): q to Q8_0, Q4_0 x Q8_0 dot products, online softmax
 * with expf, V dequantized to fp32.  Same arguments and result as
 * orc_cpu_baseline_run. */
double orc_cpu_ggml_style_run(const orc_block_q4_0 *kc, const orc_block_q4_0 *vc, int n_sess,
                              int n_heads, int n_kv_heads, int head_dim, int n_ctx,
                              const int64_t *pos, const float *q, float *out, int n_threads,
                              int iters);

#ifdef __cplusplus
}
#endif

#endif /* BMO_ORACLE_H */
