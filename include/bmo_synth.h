/*
 * bmo_synth.h -- benchmark support (libbmo_synth.so): the device generator of
 * the synthetic inputs of the benchmark configurations, and a read probe.
 * Not part of the attention ABI (bmo_attn.h) and with no counterpart in the
 * reference: the generator exists so that the benchmark and the full-size
 * tests draw their q/k/v from the seeded stream the configurations name, on
 * the GPU, and the CPU can regenerate any part of them; the probe states the
 * memory ceiling of a single pass over the bytes a kernel reads.
 *
 * Stream: element c of stream `seed` is a Box-Muller normal of two
 * splitmix64 words (Steele, Lea, Flood 2014), cosine branch only:
 *   a = mix64(seed ^ mix64(2c)),  b = mix64(seed ^ mix64(2c + 1)),
 *   u1 = ((a >> 11) + 0.5) 2^-53,  u2 = (b >> 11) 2^-53,
 *   z = (float) (sqrt(-2 ln u1) cos(2 pi u2)),
 * where mix64(x) adds 0x9E3779B97F4A7C15 and applies splitmix64's output
 * function, and ln and cos(2 pi .) are evaluated from +, -, *, / and sqrt
 * alone (correctly rounded IEEE double, no fused multiply-add): ln x = e ln 2
 * + 2 atanh(s) over x = m 2^e, m in [sqrt(1/2), sqrt(2)], s = (m-1)/(m+1),
 * the atanh series to s^21; cos(2 pi t) by quadrant and half-quadrant
 * reduction of 4t and the Taylor series to y^16 (cos) or y^17 (sin).  With
 * outliers != 0 an element is multiplied by 8 when
 * mix64((seed ^ 0xD1B54A32D192ED03) ^ mix64(c)) has its top 32 bits below
 * 42949673 (probability 1%).  The CPU restatement is the oracle's
 * orc_fill_normal / orc_fill_kv; the two agree bit for bit.
 */
#ifndef BMO_SYNTH_H
#define BMO_SYNTH_H

#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define BMO_SYNTH_API __attribute__((visibility("default")))
#else
#define BMO_SYNTH_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* out[i] = element offset + i of stream seed, i < n (fp32, device memory),
 * asynchronously on stream (hipStream_t as void*).  Returns 0, 2 for n < 0
 * or a NULL out with n > 0, 8 for a HIP launch error. */
BMO_SYNTH_API int bmo_synth_fill_normal(float *out, int64_t n, uint64_t seed, uint64_t offset,
                                        int outliers, void *stream);

/* Reads `bytes` of device memory at buf once, asynchronously on stream, with
 * one 16-byte nontemporal load per thread in workgroups of 256 (of the read
 * patterns measured on MI355X, the fastest single pass), and discards the
 * data: the time of this launch is the ceiling for a kernel that reads the
 * same bytes in one launch.  sink: device memory of at least 1 KiB, written
 * only for one value in 2^32 of a piece's xor.  Returns 0, 2 for bytes < 0,
 * bytes not a multiple of 16, buf not 16-byte aligned or a NULL pointer with
 * bytes > 0, 8 for a HIP launch error. */
BMO_SYNTH_API int bmo_synth_read_probe(const void *buf, int64_t bytes, uint32_t *sink, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* BMO_SYNTH_H */
