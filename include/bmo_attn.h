/*
 * bmo_attn.h -- C ABI of the MI355X (gfx950) Q4_0 ring KV cache and its
 * sliding-window attention kernels.
 *
 * Drop-in for the decode-attention path of utkarshyadav009/bmo_jetson:
 *   - the KV allocator   bmo_init_kv_cache / bmo_reset_depth_kv
 *                        (src/bmo.cpp:1348-1508, :1558-1565),
 *   - the node launcher  launch_decode_attention (src/bmo.h:412-426,
 *                        src/bmo_cuda_kernels.cu:713-884),
 *   - the KV-touching parts of the public ABI bmo_reset and
 *                        bmo_copy_k_cache_f32 (src/bmo_api.h:47,61-67).
 *
 * Conventions
 *   - Plain C types only.  Device pointers are HIP device addresses, streams
 *     are hipStream_t passed as void* (NULL = the null stream), exactly as the
 *     reference passes cudaStream_t as void*.
 *   - Every call is asynchronous on its stream unless it says otherwise.  A
 *     call that writes slots (append, fused append+decode, write, reset,
 *     import) must be ordered with the calls that read those slots, as on one
 *     stream; decode calls alone may overlap.  Only bmo_kv_ring_create,
 *     bmo_attn_session_create and bmo_kv_ring_prefill (its staging buffer,
 *     when a staged call needs a larger one than the ring holds) allocate
 *     device memory.
 *   - Functions returning int return BMO_ATTN_OK (0) or an error code below;
 *     bmo_kv_ring_last_error() then describes the most recent failure on that
 *     ring (as bmo_last_error does per handle, src/bmo_api.h:145).
 *   - Q4_0 is ggml's block format (src/bmo_cuda_kernels.cu:496-499): 32
 *     elements share one fp16 scale d, element j is (code_j - 8) * d, codes
 *     are nibbles, element j in the low and j+16 in the high nibble of byte j.
 *     Appends quantize bit-exactly as ggml quantize_row_q4_0_ref.
 *
 * Ring layout in HBM (what the kernels read; export/import convert to and
 * from ggml's 18-byte AoS blocks): the n_ctx slots of one (layer, session,
 * kv head) -- a stripe -- are cut into groups of G = 2048/head_dim slots; a
 * group is 2304 bytes: K codes [G][head_dim/2] (stored as code ^ 8 per
 * nibble), V codes [G][head_dim/2], then one dword per (slot, block) holding
 * the K scale (fp16, low half) and the V scale (high half).  One allocation
 * holds the groups as [n_layers][groups per stripe][n_sessions][n_kv_heads].
 * Slot of absolute position p is p % n_ctx.  A fresh or reset slot holds the
 * ggml block with d = 0 and all codes 0.
 */
#ifndef BMO_ATTN_H
#define BMO_ATTN_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define BMO_ATTN_API __attribute__((visibility("default")))
#else
#define BMO_ATTN_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  1, 2 and 9 keep the meaning bmo_forward_temporal2 gives
 * them (src/bmo_api.cpp:394-413, :504-510). */
#define BMO_ATTN_OK 0
#define BMO_ATTN_ERR_NULL 1      /* a required pointer argument is NULL */
#define BMO_ATTN_ERR_ARG 2       /* an argument is out of range */
#define BMO_ATTN_ERR_HIP 8       /* the HIP runtime reported an error */
#define BMO_ATTN_ERR_INTERNAL 9  /* unexpected failure (exception) */

/* Readout return codes of bmo_copy_k_cache_f32 (src/bmo_api.cpp:290-311). */
#define BMO_ATTN_READ_ERR_NULL (-1)
#define BMO_ATTN_READ_ERR_SMALL (-2)
#define BMO_ATTN_READ_ERR_RANGE (-3)

typedef struct bmo_kv_ring bmo_kv_ring_t;

/* ---- allocation (replaces bmo_init_kv_cache, src/bmo.cpp:1348-1508) ------- */

/* Bytes of one (layer, session, kv head) stripe (its K and V, in groups that
 * are not contiguous); 0 for an unsupported head_dim or n_ctx <= 0. */
BMO_ATTN_API int64_t bmo_kv_ring_stripe_bytes(int head_dim, int n_ctx);

/* Allocates and zeroes a ring on the current HIP device.  head_dim must be 64
 * or 128; n_ctx in [1, 65536] (no 1024 cap: that clamp, src/bmo.cpp:1362-1367,
 * is an Orin memory budget).  The temporal cache of the reference is
 * (32 layers, 1 session, 32 heads, 128, n_ctx); the depformer cache is
 * (6, 1, 16, 64, 8).  Returns NULL on failure; bmo_kv_ring_last_error(NULL)
 * then gives the reason (the calling thread's last create error). */
BMO_ATTN_API bmo_kv_ring_t *bmo_kv_ring_create(int n_layers, int n_sessions,
                                               int n_kv_heads, int head_dim,
                                               int n_ctx);

/* Releases the ring.  NULL-safe; never fails (src/bmo_api.cpp:210-256). */
BMO_ATTN_API void bmo_kv_ring_free(bmo_kv_ring_t *ring);

/* Geometry and allocation size; any output pointer may be NULL. */
BMO_ATTN_API int bmo_kv_ring_geometry(const bmo_kv_ring_t *ring, int *n_layers,
                                      int *n_sessions, int *n_kv_heads,
                                      int *head_dim, int *n_ctx);
BMO_ATTN_API int64_t bmo_kv_ring_bytes(const bmo_kv_ring_t *ring);

/* The two cache pointers bmo_launch_decode_attention takes for this ring:
 * k_base is the ring allocation, v_base = k_base + 1024 (the V codes' offset
 * inside a slot group).  They are not separate regions. */
BMO_ATTN_API void *bmo_kv_ring_k_base(bmo_kv_ring_t *ring);
BMO_ATTN_API void *bmo_kv_ring_v_base(bmo_kv_ring_t *ring);

/* Zeroes every layer of one session (session >= 0) or of all sessions
 * (session == -1), asynchronously on stream.  A zeroed block dequantizes to
 * 0.  Replaces the K/V memset of bmo_reset (src/bmo_api.cpp:258-272) and
 * bmo_reset_depth_kv (src/bmo.cpp:1558-1565). */
BMO_ATTN_API int bmo_kv_ring_reset(bmo_kv_ring_t *ring, int session,
                                   void *stream);

/* Message for the most recent failed call on ring, or for the calling
 * thread's last failed bmo_kv_ring_create when ring is NULL.  NULL if none.
 * Owned by the library (a per-thread copy), valid until this thread's next
 * call of bmo_kv_ring_last_error (src/bmo_api.h:142-145). */
BMO_ATTN_API const char *bmo_kv_ring_last_error(const bmo_kv_ring_t *ring);

/* ---- decode path ------------------------------------------------------------ */
/*
 * Batched forms: batch entry b (0 <= b < n_batch <= n_sessions) works on ring
 * session session_ids[b] (or b when session_ids is NULL) at absolute position
 * pos[b] >= 0.  session_ids and pos are DEVICE int arrays, so a captured graph
 * can be replayed with new positions (the role of pos_dev in
 * src/bmo_api.cpp:168-171).  An entry whose session id or position is out of
 * range is skipped: nothing is written to the ring and its output rows are
 * set to zero.  The entries of one call that writes slots (append, fused
 * append + decode, with or without RoPE) must name distinct sessions: one
 * entry's write of slot pos % n_ctx would race with another entry of the same
 * session reading that slot in its window.
 *   q, out:        [n_batch][n_heads][head_dim] fp32 (q after RoPE)
 *   k_new, v_new:  [n_batch][n_kv_heads][head_dim] fp32
 *   scale:         softmax scale; <= 0 selects 1/sqrt(head_dim)
 *                  (src/bmo_cuda_kernels.cu:867)
 * The window of position p is the min(p+1, n_ctx) most recent positions
 * (src/bmo_cuda_kernels.cu:739-743).  n_heads must be a multiple of
 * n_kv_heads, and n_batch * n_heads at most INT_MAX; query head h reads kv
 * head h / (n_heads / n_kv_heads) (src/bmo_cuda_kernels.cu:736-737).
 */

/* Quantizes k_new/v_new into slot pos[b] % n_ctx (the KV write of
 * src/bmo_cuda_kernels.cu:749-754, to Q4_0 instead of fp16). */
BMO_ATTN_API int bmo_kv_ring_append(bmo_kv_ring_t *ring, int layer, int n_batch,
                                    const int *session_ids, const int *pos,
                                    const float *k_new, const float *v_new,
                                    void *stream);

/* Attention of q over each entry's window as it stands in the ring (the
 * current token must already have been appended). */
BMO_ATTN_API int bmo_kv_ring_decode(bmo_kv_ring_t *ring, int layer, int n_batch,
                                    const int *session_ids, const int *pos,
                                    int n_heads, const float *q, float *out,
                                    float scale, void *stream);

/* Fused append + attention in one launch (the reference kernel's fused
 * write-then-attend, src/bmo_cuda_kernels.cu:749-847): the current token's
 * K/V are quantized, written to slot pos % n_ctx and attended to with their
 * quantized values, together with the rest of the window. */
BMO_ATTN_API int bmo_kv_ring_append_decode(bmo_kv_ring_t *ring, int layer,
                                           int n_batch, const int *session_ids,
                                           const int *pos, int n_heads,
                                           const float *q, const float *k_new,
                                           const float *v_new, float *out,
                                           float scale, void *stream);

/* Quantizes n_tok consecutive rows (positions pos0 .. pos0+n_tok-1, host
 * values, 1 <= n_tok <= n_ctx) of one session into the ring.  k, v:
 * [n_tok][n_kv_heads][head_dim] fp32 on the device.  This is the multi-token
 * KV write of the reference's lazy path (src/bmo_compute.cpp:2390-2401), on
 * ring slots. */
BMO_ATTN_API int bmo_kv_ring_write(bmo_kv_ring_t *ring, int layer, int session,
                                   int64_t pos0, int n_tok, const float *k,
                                   const float *v, void *stream);

/* bmo_kv_ring_append_decode with RoPE fused in front (the rotation the
 * reference launches separately on q and k before attention,
 * src/bmo_cuda_kernels.cu:317-368, called at src/bmo_compute.cpp:2329-2330):
 * q and k_new are the pre-RoPE rows; in every head, pair (x[2i], x[2i+1])
 * turns by pos[b] * rope_theta^(-2i/head_dim) (rope_theta > 0; the model's
 * rope_theta, default 10000, src/bmo.cpp:301-303).  The ring receives the
 * rotated K, as the reference's cache does.  The cosine and sine are the
 * exact values rounded to fp32 (the reference uses fp32 fast intrinsics);
 * v_new is not rotated. */
BMO_ATTN_API int bmo_kv_ring_append_decode_rope(bmo_kv_ring_t *ring, int layer, int n_batch,
                                                const int *session_ids, const int *pos,
                                                int n_heads, const float *q,
                                                const float *k_new, const float *v_new,
                                                float *out, float scale, float rope_theta,
                                                void *stream);

/* Chunked prefill (multi-token attention node of the reference's lazy path,
 * src/bmo_compute.cpp:2376-2418, here over the ring with a causal +
 * sliding-window mask).  Entry b writes n_tok tokens at positions pos0[b] ..
 * pos0[b]+n_tok-1 (pos0 a DEVICE array, 1 <= n_tok <= n_ctx) of session
 * session_ids[b] (or b).  Query i, at position p = pos0[b] + i, attends to
 * positions max(0, p-n_ctx+1) .. p: those before pos0[b] from the ring as it
 * stands, chunk positions from the chunk's own K/V quantized to Q4_0 exactly
 * as bmo_kv_ring_append quantizes them.  Then the chunk's blocks go to slots
 * (pos0[b]+i) % n_ctx.  The ring must hold the session's positions up to
 * pos0[b]-1 (or pos0[b] == 0).  Entries with a bad session, pos0 < 0 or
 * pos0 + n_tok > INT_MAX are skipped (output zeroed, ring untouched).  The
 * entries of one call must name distinct sessions.
 *   q:    [n_batch][n_tok][n_heads][head_dim] bf16 (bit patterns)
 *   k, v: [n_batch][n_tok][n_kv_heads][head_dim] bf16
 *   out:  [n_batch][n_tok][n_heads][head_dim] fp32
 * Attention runs on matrix cores with scores as close as fp32 arithmetic on
 * the bf16 q: each query row enters scaled by its own power of two (exact in
 * fp16 whatever the row's range), K as its exact codes (c - 8) with each
 * block's fp16 scale applied in fp32; V and the softmax weights in fp16,
 * fp32 accumulation (K and V values must lie in fp16 range, as the
 * reference's F16 cache requires).  A query row holding a NaN or an
 * infinity gets a NaN output row; the other rows are unaffected.  With
 * n_heads == n_kv_heads, n_tok <= 256 and n_ctx a multiple of 32, one kernel
 * quantizes, attends and commits; otherwise the call stages the chunk's
 * Q4_0 blocks in the ring's staging buffer (n_batch * n_kv_heads stripes of
 * n_tok slots), grown on first use with a synchronization of stream; staged
 * calls on one ring share that buffer and must therefore be ordered on one
 * stream. */
BMO_ATTN_API int bmo_kv_ring_prefill(bmo_kv_ring_t *ring, int layer, int n_batch,
                                     const int *session_ids, const int *pos0,
                                     int n_tok, int n_heads, const uint16_t *q,
                                     const uint16_t *k, const uint16_t *v,
                                     float *out, float scale, void *stream);

/* bmo_kv_ring_prefill that allocates nothing, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  Same
 * arguments, results and errors as bmo_kv_ring_prefill; a staged call (GQA, or
 * more than 256 tokens) stages the chunk in a fixed 32 MiB array that each
 * GPU holds for the life of the process, instead of the ring's growable
 * buffer.  A staged chunk needing more than 32 MiB (n_batch * n_kv_heads *
 * ceil(n_tok / (2048 / head_dim)) * 2304 bytes) is rejected with
 * BMO_ATTN_ERR_ARG and nothing is launched.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (on different streams or
 * from different threads) race and must be ordered by the caller. */
BMO_ATTN_API int bmo_kv_ring_prefill_noalloc(bmo_kv_ring_t *ring, int layer, int n_batch,
                                             const int *session_ids, const int *pos0,
                                             int n_tok, int n_heads, const uint16_t *q,
                                             const uint16_t *k, const uint16_t *v,
                                             float *out, float scale, void *stream);

/* ---- readout / export ------------------------------------------------------- */

/* Copies slots [t_start, t_start+n_positions) of layer's K for one session as
 * fp32 into HOST memory, layout (n_positions, n_kv_heads, head_dim); blocks
 * until the copy is done (synchronizes the null stream's work on the ring's
 * device first).  Returns the number of floats written, or -1 (NULL ring/out,
 * n_positions <= 0, max_floats <= 0, bad session), -2 (max_floats too small),
 * -3 (layer or slot range out of bounds), as bmo_copy_k_cache_f32 does
 * (src/bmo_api.cpp:283-332; t_start is a slot index, not a position). */
BMO_ATTN_API int bmo_kv_ring_copy_k_f32(bmo_kv_ring_t *ring, int layer,
                                        int session, int t_start,
                                        int n_positions, float *out,
                                        int max_floats);

/* Copies slots [t_start, t_start+n_positions) of K (which == 0) or V
 * (which == 1) as ggml block_q4_0 (18 bytes per block, layout
 * [n_positions][n_kv_heads][head_dim/32]) into HOST memory; synchronous.
 * Returns bytes written or a negative readout code as above. */
BMO_ATTN_API int64_t bmo_kv_ring_export_q4_0(bmo_kv_ring_t *ring, int layer,
                                             int session, int which,
                                             int t_start, int n_positions,
                                             void *out, int64_t max_bytes);

/* Inverse of export: writes host ggml blocks into the ring; synchronous. */
BMO_ATTN_API int64_t bmo_kv_ring_import_q4_0(bmo_kv_ring_t *ring, int layer,
                                             int session, int which,
                                             int t_start, int n_positions,
                                             const void *in, int64_t n_bytes);

/* ---- graph replay ----------------------------------------------------------- */

/* pos_dev[i] += delta for i < n, asynchronously on stream.  Every entry point
 * above reads positions from device memory when each kernel runs, and none
 * allocates, synchronizes or records a memset on a decode step, so a whole
 * step (the L layers' bmo_kv_ring_append_decode[_rope] calls followed by this
 * advance) can be captured once into a HIP graph and replayed per token: each
 * replay attends, appends and rotates at the current positions.  (The
 * reference's static capture froze RoPE at the capture-time position and was
 * disabled, src/bmo_api.cpp:334-350.)  bmo_kv_ring_prefill allocates only
 * when a staged call needs a larger staging buffer than the ring holds; call
 * it once eagerly before capturing it. */
BMO_ATTN_API int bmo_positions_advance(int *pos_dev, int n, int delta, void *stream);

/* ---- per-session handle ------------------------------------------------------ */
/*
 * The attention part of the reference's bmo_handle (src/bmo_api.cpp:164-172):
 * one session of a ring, a HIP stream of its own (non-blocking, default
 * priority), a device-resident position that every launch reads (the
 * reference's pos_dev), and a mutex that serializes the handle's calls
 * (src/bmo_api.cpp:28, :415).  A token step runs the fused append +
 * attention of every layer of the ring at one position (with RoPE when
 * rope_theta > 0) and advances the position, as bmo_forward_temporal2 does
 * with h->pos = pos + 1 (src/bmo_api.cpp:501).  For a step:
 *   q, out:  [n_layers][n_heads][head_dim] fp32, device
 *   k, v:    [n_layers][n_kv_heads][head_dim] fp32, device
 * The ring must outlive its handles; one handle per ring session (two handles
 * on one session race on its slots).  Handles on distinct sessions of one
 * ring may run concurrently.  Functions returning int return BMO_ATTN_OK or
 * an error code; bmo_attn_session_last_error() gives the message.
 */
typedef struct bmo_attn_session bmo_attn_session_t;

/* Creates a handle for `session` of `ring` with n_heads query heads (a
 * multiple of the ring's n_kv_heads), softmax scale (<= 0: 1/sqrt(head_dim))
 * and rope_theta (0: q and k arrive with RoPE applied).  The position starts
 * at 0; the ring is not cleared.  Returns NULL on failure;
 * bmo_attn_session_last_error(NULL) then gives the calling thread's reason
 * (the reference prints init failures to stderr, src/bmo_api.cpp:196-205;
 * this does both). */
BMO_ATTN_API bmo_attn_session_t *bmo_attn_session_create(bmo_kv_ring_t *ring, int session,
                                                         int n_heads, float scale,
                                                         float rope_theta);

/* Waits for the handle's work and releases it.  NULL-safe. */
BMO_ATTN_API void bmo_attn_session_free(bmo_attn_session_t *s);

/* Position 0 and the session's K/V zeroed in every layer; synchronous (the
 * K/V part of bmo_reset, src/bmo_api.cpp:258-272). */
BMO_ATTN_API int bmo_attn_session_reset(bmo_attn_session_t *s);

/* The position the next step uses once the queued work has run (the one
 * after the last step run or queued); -1 for NULL. */
BMO_ATTN_API int64_t bmo_attn_session_pos(bmo_attn_session_t *s);

/* The handle's HIP stream (hipStream_t as void*). */
BMO_ATTN_API void *bmo_attn_session_stream(bmo_attn_session_t *s);

/* One token step at position pos (0 <= pos <= 2^31 - 2; any position, not
 * only the next one, as bmo_forward_temporal2 takes it,
 * src/bmo_api.cpp:365-511), launched eagerly on the handle's stream;
 * returns when out is written.  Afterwards the position is pos + 1. */
BMO_ATTN_API int bmo_attn_session_forward(bmo_attn_session_t *s, int pos, const float *q,
                                          const float *k, const float *v, float *out);

/* Records one token step over these buffers into a HIP graph; the graph
 * reads the position from device memory and ends by advancing it.  Nothing
 * runs and the position does not change.  The buffers must stay valid while
 * the graph is kept.  A previous graph is replaced only once the new one is
 * instantiated (a failed capture keeps it).  Stands in for
 * bmo_capture_graphs (src/bmo_api.cpp:334-351). */
BMO_ATTN_API int bmo_attn_session_capture(bmo_attn_session_t *s, const float *q, const float *k,
                                          const float *v, float *out);

/* 1 when a step is captured, else 0 (bmo_has_cuda_graphs,
 * src/bmo_api.cpp:353-359). */
BMO_ATTN_API int bmo_attn_session_has_graph(bmo_attn_session_t *s);

/* Replays the captured graph (bmo_attn_session_capture, or _capture_begin /
 * _end) on the handle's stream and returns when it is done; the captured
 * buffers hold the inputs on entry and the outputs on return.  A graph that
 * does not begin with a reset runs at position pos (same range as forward;
 * replaying at the handle's current position costs one graph launch, another
 * position first sets the device position) and leaves the position at pos +
 * its steps; a graph that begins with bmo_attn_session_reset_async ignores
 * pos and leaves the position at its steps. */
BMO_ATTN_API int bmo_attn_session_replay(bmo_attn_session_t *s, int pos);

/* ---- the handle at a model's layer granularity ----
 * The reference's layer loop (src/bmo_compute.cpp:2188-2641, driven by
 * bmo_forward_temporal2, src/bmo_api.cpp:384-511) computes layer l+1's q/k/v
 * from layer l's attention output: the output projection (:2423), the FFN
 * and the next QKV projection (:2232) run between two attention calls.  These
 * calls queue one layer at a time on the handle's stream
 * (bmo_attn_session_stream), so the caller's own kernels on that stream fall
 * between them in stream order; none of them waits for the GPU.  A step is
 *   begin_step(pos), then layer(l, ...) for the layers in any order, then
 *   end_step();
 * every layer call of a step reads the same device position.  Between
 * capture_begin and capture_end the calls (and the caller's kernels on the
 * handle's stream) are recorded instead of run; replay then runs them. */

/* Sets the position the next layer calls use to pos (0 <= pos <= 2^31 - 2),
 * queued on the stream (nothing is queued when it already holds pos).  Not
 * allowed during a capture: a captured step takes its position from replay. */
BMO_ATTN_API int bmo_attn_session_begin_step(bmo_attn_session_t *s, int pos);

/* Queues layer `layer`'s fused append + attention at the current device
 * position (with RoPE when the handle has rope_theta > 0): the arguments of
 * one layer of bmo_attn_session_forward, q/out [n_heads][head_dim] and k/v
 * [n_kv_heads][head_dim] fp32 device buffers, read and written when the
 * stream reaches the call (the attention node of src/bmo_compute.cpp:2293-2418,
 * and of the depth loop, :2945-2991). */
BMO_ATTN_API int bmo_attn_session_layer(bmo_attn_session_t *s, int layer, const float *q,
                                        const float *k, const float *v, float *out);

/* Queues the advance of the device position by one that ends a step
 * (h->pos = pos + 1, src/bmo_api.cpp:501); bmo_attn_session_pos reports the
 * advanced position at once. */
BMO_ATTN_API int bmo_attn_session_end_step(bmo_attn_session_t *s);

/* Queues the zeroing of the session's K/V in every layer and position 0:
 * bmo_attn_session_reset without the wait, so that a capture can begin with
 * it (the depformer's per-frame reset in bmo_forward_depth_cascade,
 * src/bmo_api.cpp:668-743 with the reset at :682). */
BMO_ATTN_API int bmo_attn_session_reset_async(bmo_attn_session_t *s);

/* Waits for everything queued on the handle's stream; reports a HIP error
 * the queued work raised. */
BMO_ATTN_API int bmo_attn_session_sync(bmo_attn_session_t *s);

/* Starts recording the handle's stream into a HIP graph (thread-local
 * capture mode: the caller's other HIP calls on this thread must not
 * allocate or synchronize until capture_end).  forward, capture, replay,
 * reset, begin_step and sync are rejected until capture_end. */
BMO_ATTN_API int bmo_attn_session_capture_begin(bmo_attn_session_t *s);

/* Ends the recording and keeps it as the handle's graph (replacing a previous
 * one only once the new one is instantiated).  If a handle call inside the
 * capture failed, the recording is discarded, the previous graph kept and an
 * error returned.  The position does not change. */
BMO_ATTN_API int bmo_attn_session_capture_end(bmo_attn_session_t *s);

/* Message of the handle's most recent failed call, or (s == NULL) of the
 * calling thread's last failed create; NULL if none.  Owned by the library
 * (a per-thread copy), valid until this thread's next call of
 * bmo_attn_session_last_error (src/bmo_api.h:142-145). */
BMO_ATTN_API const char *bmo_attn_session_last_error(bmo_attn_session_t *s);

/* ---- Q4_0 weight GEMV (the projections around attention) -------------------- */

/* Same arguments as the reference's launch_gemv_q4_0_q8_1
 * (src/bmo_cuda_kernels.cu:685-711, the QKV projection before attention and
 * the output projection after it, src/bmo_compute.cpp:2232,2423):
 * y[r] = row r of W (rows x cols, ggml block_q4_0 AoS, 18 bytes per 32
 * elements, device memory) times x (cols fp32), with x quantized to the
 * reference's Q8_1 (d = amax/127, q = roundf(x/d) clamped, s = fp16 of the
 * fp32 sum of the x values) and every block contributing
 * d4 * (sum(code*q) * d8 - 8 * s8).  One launch: each workgroup quantizes x
 * itself.  q8_scratch may be NULL; when given (cols/32 * 36 bytes) it receives
 * the Q8_1 blocks, as the reference's scratch does.  cols must be a multiple
 * of 64 (at most 52428); W_dev and q8_scratch 4-byte aligned, x_dev 16-byte
 * aligned.  A 16-byte aligned W_dev with cols a multiple of 256, at most 6144,
 * and at most 16384 rows takes a faster streaming kernel; the outputs are
 * the same bit for bit either way.  Asynchronous on stream.  Returns
 * BMO_ATTN_OK or an error code; rejected arguments launch nothing and are
 * reported once on stderr (the reference's launcher returns nothing). */
BMO_ATTN_API int bmo_launch_gemv_q4_0_q8_1(const void *W_dev, const float *x_dev,
                                           float *y_dev, int rows, int cols,
                                           void *q8_scratch, void *stream);

/* ---- node-level drop-in ------------------------------------------------------ */

/* Same signature and semantics as the reference's launch_decode_attention
 * (src/bmo.h:412-426, src/bmo_cuda_kernels.cu:850-884): fused write of the
 * current k/v to slot (pos % n_ctx) and attention over the window, with
 * pos = *pos_dev when pos_dev is non-NULL, else n_past.  k_cache_dev and
 * v_cache_dev are bmo_kv_ring_k_base / bmo_kv_ring_v_base of a ring created
 * with n_sessions == 1 and n_kv_heads == n_heads (the reference allocates
 * n_heads head slots, src/bmo.cpp:1401-1402).  When k_cache_dev is a ring
 * from bmo_kv_ring_create its geometry is checked; arguments that do not fit
 * launch nothing and are reported once on stderr.
 * Returns nothing, as the reference does; launch errors surface through
 * hipGetLastError(). */
BMO_ATTN_API void bmo_launch_decode_attention(
    const float *q_dev, const float *k_dev, const float *v_dev,
    void *k_cache_dev, void *v_cache_dev, float *out_dev, int head_dim,
    int n_heads, int n_kv_heads, int n_ctx, int n_past, int layer,
    void *stream, const int *pos_dev);

#ifdef __cplusplus
}
#endif

#endif /* BMO_ATTN_H */
