/*
 * oracle_checks.c -- checks that pin the oracle's IEEE binary16 conversion.
 *
 * TEST INFRASTRUCTURE ONLY.  The independent side is the CPU's own F16C
 * conversion instruction (vcvtps2ph with round-to-nearest-even), which is a
 * hardware implementation of the same IEEE 754 rule.
 */
#include "gemma_oracle.h"

#include <immintrin.h>
#include <string.h>

static int is_nan_half(uint16_t h)
{
    return (h & 0x7C00u) == 0x7C00u && (h & 0x3FFu) != 0;
}

__attribute__((target("f16c")))
int64_t gor_check_half_exhaustive(void)
{
    int64_t mismatches = 0;

#pragma omp parallel for reduction(+ : mismatches) schedule(static)
    for (int64_t high = 0; high < 65536; ++high) {
        for (uint32_t low = 0; low < 65536u; ++low) {
            const uint32_t bits = ((uint32_t) high << 16) | low;
            float value;
            memcpy(&value, &bits, sizeof value);

            const uint16_t ours = gor_half_from_float(value);
            const uint16_t hardware = (uint16_t) _cvtss_sh(value, _MM_FROUND_TO_NEAREST_INT);

            if (value != value) {
                if (!is_nan_half(ours) || !is_nan_half(hardware))
                    ++mismatches;
            } else if (ours != hardware) {
                ++mismatches;
            }
        }
    }
    return mismatches;
}

__attribute__((target("f16c")))
int64_t gor_check_half_roundtrip(void)
{
    int64_t mismatches = 0;

    for (uint32_t h = 0; h < 65536u; ++h) {
        const float widened = gor_half_to_float((uint16_t) h);
        const float hardware = _cvtsh_ss((unsigned short) h);
        uint32_t a, b;
        memcpy(&a, &widened, 4);
        memcpy(&b, &hardware, 4);

        if (is_nan_half((uint16_t) h)) {
            if (widened == widened || gor_half_from_float(widened) == 0)
                ++mismatches;
            continue;
        }
        if (a != b || gor_half_from_float(widened) != (uint16_t) h)
            ++mismatches;
    }
    return mismatches;
}
