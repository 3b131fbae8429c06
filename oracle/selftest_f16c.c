/*
 * selftest_f16c.c -- exhaustive check of orc_fp32_to_fp16 against the host's
 * F16C conversion instruction (the one GGML_FP32_TO_FP16 uses on x86).
 * TEST INFRASTRUCTURE ONLY.  Built with -mf16c; called only after a runtime
 * CPU feature check.
 */
#include "oracle.h"

#include <immintrin.h>
#include <string.h>

__attribute__((target("f16c")))
static uint16_t hw_fp32_to_fp16(float f) {
    return (uint16_t) _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT);
}

int64_t orc_selftest_fp16_exhaustive(void) {
    __builtin_cpu_init();
    if (!__builtin_cpu_supports("f16c")) return -1;
    int64_t bad = 0;
    uint32_t u = 0;
    do {
        float f;
        memcpy(&f, &u, sizeof f);
        const int is_nan = ((u & 0x7F800000u) == 0x7F800000u) && (u & 0x7FFFFFu);
        if (!is_nan) {
            if (orc_fp32_to_fp16(f) != hw_fp32_to_fp16(f)) ++bad;
        } else {
            const uint16_t h = orc_fp32_to_fp16(f);
            if ((h & 0x7C00u) != 0x7C00u || (h & 0x3FFu) == 0) ++bad;
        }
        ++u;
    } while (u != 0);
    return bad;
}
