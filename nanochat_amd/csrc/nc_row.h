/*
 * The cache append's row math, shared by the append kernels (kv_append.hip) and the fused decode step
 * (attention.hip), so both produce the same bits: one (token, head) row per wave, lane l holding the rotation
 * pair (dims l, l + 64). Reference row math: model/kernels/qk_row.cuh:19-51 (qk_row_sum, qk_rstd, qk_rotate) and
 * model/kernels/decode.cu:481-494 (the value-embedding gate); the summation order is fixed here (lane partial
 * x[l]^2 + x[l+64]^2, then the xor butterfly over offsets 32..1) and 1/sqrt is correctly rounded where the
 * reference has rsqrtf.
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

/* Absmax e4m3fn quantization of one row (lane pair x1 = dim l, x2 = dim l + 64, bf16 values): the row's scale
 * amax / 448 (1 for an all-zero row), returned in every lane, and this lane's two codes. */
__device__ __forceinline__ float quantize_pair(float x1, float x2, uint32_t &c1, uint32_t &c2) {
    const float amax = wave_max(fmaxf(fabsf(x1), fabsf(x2)));
    const float scale = amax > 0.0f ? amax / FP8_MAX : 1.0f;
    c1 = e4m3_encode(fminf(fmaxf(x1 / scale, -FP8_MAX), FP8_MAX));
    c2 = e4m3_encode(fminf(fmaxf(x2 / scale, -FP8_MAX), FP8_MAX));
    return scale;
}

/* Value-embedding mix of one value row: g = 2 sigmoid(w . h) from the token's normed stream h (C wide, lane-strided
 * FMAs, then the butterfly) and v = bf16(v + g e) with e the token's embedding row for this head. */
__device__ __forceinline__ void ve_mix_pair(const uint16_t *h, const float *w, int C, const uint16_t *e, int lane,
                                            float &v1, float &v2) {
    float d = 0.0f;
    for (int i = lane; i < C; i += WAVE) d = __builtin_fmaf(bf16_to_f32(h[i]), w[i], d);
    d = wave_sum_butterfly(d);
    const float g = 2.0f * (1.0f / (1.0f + expf(-d)));
    v1 = bf16_to_f32(f32_to_bf16(v1 + g * bf16_to_f32(e[lane])));
    v2 = bf16_to_f32(f32_to_bf16(v2 + g * bf16_to_f32(e[lane + HALF])));
}

}  // namespace nc
