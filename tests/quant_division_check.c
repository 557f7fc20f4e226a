/*
 * Exhaustive check of the quantizer's division (nanochat_amd/csrc/nc_row.h: quant_code): for a row of bf16 values
 * with absmax amax, scale = amax / 448 (1 for amax = 0), the code of x is e4m3_encode(clamp(x / scale, +-448)).
 * quant_code computes it, for scale >= 2^-80, as q0 = |x| r, q = fma(fma(-q0, scale, |x|), r, q0) with r = 1 / scale,
 * encodes q and copies the sign of x. This program runs every finite bf16 amax >= 0 whose index is part mod parts
 * against every finite bf16 x with |x| <= amax, both ways, in IEEE fp32 (fmaf: one rounding; build with
 * -ffp-contract=off), and prints the count checked and the count whose codes differ. The full check is parts = 1:
 *     gcc -O2 -ffp-contract=off -o check tests/quant_division_check.c -lm && ./check 0 1
 * (1,065,402,240 pairs, 0 differing codes). Test infrastructure: nothing in the product builds or runs it.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bf16(uint32_t b) {
    const uint32_t u = b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* the kernels' e4m3_encode (nc_device.h), applied after the clamp */
static uint32_t e4m3(float x) {
    const uint32_t u = bits(x), sign = (u >> 24) & 0x80u, au = u & 0x7FFFFFFFu;
    float a;
    memcpy(&a, &au, 4);
    const uint32_t code = a >= 0x1p-6f ? ((au + 0x7FFFFu + ((au >> 20) & 1u)) >> 20) - ((127u - 7u) << 3)
                                       : (uint32_t)rintf(a * 512.0f);
    return code | sign;
}

static uint32_t by_division(float x, float scale) { return e4m3(fminf(fmaxf(x / scale, -448.0f), 448.0f)); }

static uint32_t by_reciprocal(float x, float scale) {
    if (!(scale >= 0x1p-80f)) return by_division(x, scale);
    const float r = 1.0f / scale, ax = fabsf(x);
    const float q0 = ax * r;
    const float q = fmaf(fmaf(-q0, scale, ax), r, q0);
    return e4m3(fminf(q, 448.0f)) | ((bits(x) >> 24) & 0x80u);
}

int main(int argc, char **argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: %s part parts\n", argv[0]);
        return 2;
    }
    const uint32_t part = (uint32_t)atoi(argv[1]), parts = (uint32_t)atoi(argv[2]);
    long long checked = 0, differ = 0;
    for (uint32_t ab = part; ab < 0x7F80u; ab += parts) {   /* amax: +0 and the positive finite bf16 values */
        const float amax = from_bf16(ab);
        const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
        for (uint32_t xb = 0; xb < 0x10000u; xb++) {
            const float x = from_bf16(xb);
            if (!isfinite(x) || fabsf(x) > amax) continue;
            checked++;
            if (by_reciprocal(x, scale) != by_division(x, scale)) {
                if (differ < 5) printf("differ: amax %a x %a\n", amax, x);
                differ++;
            }
        }
    }
    printf("%lld %lld\n", checked, differ);
    return differ != 0;
}
