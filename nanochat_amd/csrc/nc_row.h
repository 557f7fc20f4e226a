/*
 * The cache append's row math, shared by the append kernels (kv_append.hip) and the fused decode step
 * (attention.hip), so both produce the same bits: one (token, head) row per wave, lane l holding the rotation
 * pair (dims l, l + 64). Reference row math: model/kernels/qk_row.cuh:19-51 (qk_row_sum, qk_rstd, qk_rotate) and
 * model/kernels/decode.cu:481-494 (the value-embedding gate); the summation order is fixed here (lane partial
 * x[l]^2 + x[l+64]^2, then the xor butterfly over offsets 32..1) and 1/sqrt is correctly rounded where the
 * reference has rsqrtf. The value-embedding gate's exponential is exp_rn (below) where the reference has expf, so
 * the gate's bits follow from its fixed fp32 order alone.
 */
#pragma once

#include "nc_device.h"

namespace nc {

/* RMS norm (eps FLT_EPSILON), gain and -theta rotation of one row held as lane pairs (x1 = dim l,
 * x2 = dim l + 64); results before the bf16 rounding. Every operation is a single rounded fp32 op in the
 * order of the oracle's qk_norm_rope. All 64 lanes of the wave must call it together. */
__device__ __forceinline__ void norm_rope_pair(float x1, float x2, float g1, float g2, float c, float s, float &y1,
                                               float &y2) {
    const float part = x1 * x1 + x2 * x2;
    const float ss = wave_sum_butterfly(part);
    const float v = ss / 128.0f + FLT_EPS;
    const float r = 1.0f / __builtin_sqrtf(v);  /* correctly rounded (HIP's __fsqrt_rn is not, here) */
    const float n1 = (x1 * r) * g1;
    const float n2 = (x2 * r) * g2;
    y1 = n1 * c + n2 * s;
    y2 = n2 * c - n1 * s;
}

/* The code e4m3_encode(clamp(x / scale, +-448)) of a bf16 value x of a row whose scale is amax / 448 (|x| <= amax).
 * For scale >= 2^-80 (fast) the division becomes a product with r = 1 / scale (correctly rounded) and one FMA
 * correction of |x| (Markstein), the sign copied from x: every finite bf16 x with |x| <= amax, against every bf16
 * amax, gives the same code this way as by the division (an exhaustive check, tests/quant_division_check.c). Smaller
 * scales divide. */
__device__ __forceinline__ uint32_t quant_code(float x, float scale, float r, bool fast) {
    if (!fast) return e4m3_encode(fminf(fmaxf(x / scale, -FP8_MAX), FP8_MAX));
    const float ax = fabsf(x);
    const float q0 = ax * r;
    const float q = __builtin_fmaf(__builtin_fmaf(-q0, scale, ax), r, q0);
    return e4m3_encode(fminf(q, FP8_MAX)) | ((__float_as_uint(x) >> 24) & 0x80u);
}

constexpr float QUANT_FAST_SCALE = 0x1p-80f;   /* quant_code's fast path: scales from here up */

/* Absmax e4m3fn quantization of one row (lane pair x1 = dim l, x2 = dim l + 64, bf16 values): the row's scale
 * amax / 448 (1 for an all-zero row), returned in every lane, and this lane's two codes. */
__device__ __forceinline__ float quantize_pair(float x1, float x2, uint32_t &c1, uint32_t &c2) {
    const float amax = wave_max(fmaxf(fabsf(x1), fabsf(x2)));
    const float scale = amax > 0.0f ? amax / FP8_MAX : 1.0f;
    const bool fast = scale >= QUANT_FAST_SCALE;
    const float r = 1.0f / scale;
    c1 = quant_code(x1, scale, r, fast);
    c2 = quant_code(x2, scale, r, fast);
    return scale;
}

/* e^x of an fp32 x, rounded once to fp32: the double exponential (within an ulp of double precision) rounded to
 * float. This is the correctly rounded e^x except where e^x lies within about 2^-52 (relative) of the midpoint of two
 * floats, so it does not depend on a float exponential's own error. */
__device__ __forceinline__ float exp_rn(float x) { return (float)exp((double)x); }

/* Value-embedding mix of one value row: g = 2 sigmoid(w . h) from the token's normed stream h (C wide, lane-strided
 * FMAs, then the butterfly) and v = bf16(v + g e) with e the token's embedding row for this head. */
__device__ __forceinline__ void ve_mix_pair(const uint16_t *h, const float *w, int C, const uint16_t *e, int lane,
                                            float &v1, float &v2) {
    float d = 0.0f;
    for (int i = lane; i < C; i += WAVE) d = __builtin_fmaf(bf16_to_f32(h[i]), w[i], d);
    d = wave_sum_butterfly(d);
    const float g = 2.0f * (1.0f / (1.0f + exp_rn(-d)));
    v1 = bf16_to_f32(f32_to_bf16(v1 + g * bf16_to_f32(e[lane])));
    v2 = bf16_to_f32(f32_to_bf16(v2 + g * bf16_to_f32(e[lane + HALF])));
}

/* The same row math with 16 lanes a row, four rows a wave (the append kernel's form). Lane i of a 16-lane group
 * holds its row's dims i + 16 j, j = 0..7, as x[j]: its rotation pairs (x[j], x[j + 4]) are dims (i + 16 j, i + 16 j
 * + 64), and it stands for lanes l = i + 16 j (j < 4) of the one-row-a-wave form above. That form's butterfly steps 32
 * and 16 pair l with l ^ 32 (j with j ^ 2) and l ^ 16 (j with j ^ 1), so they are lane-local here, and steps 8 .. 1
 * are the same DPP exchanges within the group's 16 lanes: every sum is formed in the same order, and every result
 * has the same bits as the one-row-a-wave form's. All 64 lanes of the wave must call these together. */
__device__ __forceinline__ float quad_row_sum(const float (&p)[4]) {
    float v = (p[0] + p[2]) + (p[1] + p[3]);
    v = v + lane_xor_dpp<8>(v);
    v = v + lane_xor_dpp<4>(v);
    v = v + lane_xor_dpp<2>(v);
    return v + lane_xor_dpp<1>(v);
}

__device__ __forceinline__ float quad_row_max(const float (&m)[4]) {
    float v = fmaxf(fmaxf(m[0], m[2]), fmaxf(m[1], m[3]));
    v = fmaxf(v, lane_xor_dpp<8>(v));
    v = fmaxf(v, lane_xor_dpp<4>(v));
    v = fmaxf(v, lane_xor_dpp<2>(v));
    return fmaxf(v, lane_xor_dpp<1>(v));
}

/* norm_rope_pair in the 16-lane form: g, the gains of the lane's dims; c, s the rotation of its pairs. */
__device__ __forceinline__ void norm_rope_quad(const float (&x)[8], const float (&g)[8], const float (&c)[4],
                                               const float (&s)[4], float (&y)[8]) {
    float part[4];
#pragma unroll
    for (int j = 0; j < 4; j++) part[j] = x[j] * x[j] + x[j + 4] * x[j + 4];
    const float ss = quad_row_sum(part);
    const float v = ss / 128.0f + FLT_EPS;
    const float r = 1.0f / __builtin_sqrtf(v);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float n1 = (x[j] * r) * g[j];
        const float n2 = (x[j + 4] * r) * g[j + 4];
        y[j] = n1 * c[j] + n2 * s[j];
        y[j + 4] = n2 * c[j] - n1 * s[j];
    }
}

/* quantize_pair in the 16-lane form: the row's scale, and the lane's eight codes. */
__device__ __forceinline__ float quantize_quad(const float (&x)[8], uint32_t (&code)[8]) {
    float m[4];
#pragma unroll
    for (int j = 0; j < 4; j++) m[j] = fmaxf(fabsf(x[j]), fabsf(x[j + 4]));
    const float amax = quad_row_max(m);
    const float scale = amax > 0.0f ? amax / FP8_MAX : 1.0f;
    const bool fast = scale >= QUANT_FAST_SCALE;
    const float r = 1.0f / scale;
#pragma unroll
    for (int j = 0; j < 8; j++) code[j] = quant_code(x[j], scale, r, fast);
    return scale;
}

/* ve_mix_pair in the 16-lane form (i: the lane's index in its group): the lane runs the FMA chains of the four
 * one-row-a-wave lanes it stands for. */
__device__ __forceinline__ void ve_mix_quad(const uint16_t *h, const float *w, int C, const uint16_t *e, int i,
                                            float (&v)[8]) {
    float d[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        d[j] = 0.0f;
        for (int k = i + 16 * j; k < C; k += WAVE) d[j] = __builtin_fmaf(bf16_to_f32(h[k]), w[k], d[j]);
    }
    const float t = quad_row_sum(d);
    const float g = 2.0f * (1.0f / (1.0f + exp_rn(-t)));
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = bf16_to_f32(f32_to_bf16(v[j] + g * bf16_to_f32(e[i + 16 * j])));
}

}  // namespace nc
