/*
 * Device helpers shared by the gfx950 kernels of the fp8 KV-cache path: raw bf16 / e4m3fn formats in
 * integer arithmetic, wave-64 reductions, the paged-cache tile layout and the MFMA operand types.
 *
 * Every kernel file is built with -ffp-contract=off: an a*b+c written in these sources is two rounded
 * operations unless it is spelled __builtin_fmaf.
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifndef HEAD_DIM
#define HEAD_DIM 128
#endif
static_assert(HEAD_DIM == 128, "the page tiling and MFMA mapping assume 128-wide heads");

namespace nc {

constexpr int WAVE = 64;
constexpr int HALF = HEAD_DIM / 2;   /* rotation pairs: dims i and i + HALF, one pair per lane */
constexpr int PAGE = 16;             /* tokens per cache page */
constexpr int PAGE_BYTES = PAGE * HEAD_DIM;   /* one page of one KV head: 2 KiB of e4m3fn codes */
constexpr float FP8_MAX = 448.0f;
constexpr float FLT_EPS = 1.1920928955078125e-07f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

/* bf16 bits -> fp32 (exact). */
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

/* fp32 -> bf16 bits, round to nearest even (finite inputs). */
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
    const uint32_t u = __float_as_uint(x);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* fp32 with |x| <= 448 -> OCP e4m3fn code, round to nearest even; the sign bit is copied (so -0 -> 0x80).
 * Normal range: round the fp32 pattern to 3 mantissa bits (a carry moves into the exponent), rebias 127 -> 7.
 * Below 2^-6: |x| * 2^9 is exact and rounds to the subnormal count 0..8 (8 = the smallest normal, 0x08). */
__device__ __forceinline__ uint32_t e4m3_encode(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t au = u & 0x7FFFFFFFu;
    const float a = __uint_as_float(au);
    uint32_t code;
    if (a >= 0x1p-6f)
        code = ((au + 0x7FFFFu + ((au >> 20) & 1u)) >> 20) - ((127u - 7u) << 3);
    else
        code = (uint32_t)__builtin_rintf(a * 512.0f);
    return code | sign;
}

/* The pair of lanes (L, L ^ 32), or (L, L ^ 16), combined by one v_permlane32_swap / v_permlane16_swap (VALU, no
 * LDS round trip): the swap hands every lane both values of its pair, the lower lane's first, so the two lanes of a
 * pair compute the same result from the same operands in the same order. */
__device__ __forceinline__ float pair_max32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_max16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair_sum16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

/* This lane's value of lane L ^ M (M = 8, 4, 2, 1) by DPP, a VALU operand modifier with no LDS round trip:
 * row_ror:8 within each row of 16 lanes is xor 8; row_half_mirror (i -> 7 - i within 8 lanes) followed by
 * quad_perm [3,2,1,0] (j -> j ^ 3) is xor 4; quad_perm [2,3,0,1] and [1,0,3,2] are xor 2 and xor 1. */
template <int M>
__device__ __forceinline__ float lane_xor_dpp(float v) {
    static_assert(M == 8 || M == 4 || M == 2 || M == 1, "DPP xor partners within 16 lanes");
    const int x = __float_as_int(v);
    int r;
    if constexpr (M == 8) r = __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false);
    else if constexpr (M == 4)
        r = __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false), 0x1B, 0xF, 0xF, false);
    else if constexpr (M == 2) r = __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);
    else r = __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);
    return __int_as_float(r);
}

/* Sum over the wave by an xor butterfly (offsets 32, 16, ..., 1): at each offset o every lane L adds its value and
 * lane L ^ o's, so both lanes of a pair hold the same sum (a + b and b + a are the same fp32 value) and every lane
 * ends with the same result. The partners come from permlane swaps (32, 16) and DPP (8 .. 1), all 64 lanes active. */
__device__ __forceinline__ float wave_sum_butterfly(float v) {
    v = pair_sum32(v);
    v = pair_sum16(v);
    v = v + lane_xor_dpp<8>(v);
    v = v + lane_xor_dpp<4>(v);
    v = v + lane_xor_dpp<2>(v);
    return v + lane_xor_dpp<1>(v);
}

/* Max over the wave by the same butterfly. */
__device__ __forceinline__ float wave_max(float v) {
    v = pair_max32(v);
    v = pair_max16(v);
    v = fmaxf(v, lane_xor_dpp<8>(v));
    v = fmaxf(v, lane_xor_dpp<4>(v));
    v = fmaxf(v, lane_xor_dpp<2>(v));
    return fmaxf(v, lane_xor_dpp<1>(v));
}

/* Byte offset of (slot, dim) inside a K page: the 16x16x32 MFMA A-operand tiling (lane = group*16 + slot
 * holds dims group*32 + h*16 .. +15 at h*1024 + lane*16). */
__host__ __device__ __forceinline__ int k_page_offset(int slot, int dim) {
    return ((dim & 31) >> 4) * 1024 + (((dim >> 5) << 4) + slot) * 16 + (dim & 15);
}

/* Byte offset of (slot, dim) inside a V page: the transposed A-operand tiling of the PV MFMA (lane =
 * (slot/4)*16 + dim%16 holds, for tiles t = 4h..4h+3, the 4 slots of its group at dim 16t + dim%16). */
__host__ __device__ __forceinline__ int v_page_offset(int slot, int dim) {
    const int t = dim >> 4;
    return (t >> 2) * 1024 + (((slot >> 2) << 4) + (dim & 15)) * 16 + (t & 3) * 4 + (slot & 3);
}

/* Two e4m3fn codes (bytes 0-1, or 2-3 for the _hi form, of w) -> two bf16 (exact) packed in a dword, by one
 * v_cvt_scalef32_pk_bf16_fp8 with scale 1. The builtin's 2-element result is only ever reinterpreted whole: the
 * compiler mis-models an extracted element (it packs element 0 twice), while as a whole dword it emits the bare
 * instruction. It must stay a builtin (not inline asm) so the compiler sees a VALU write and inserts the wait
 * states an in-flight MFMA reading the same registers needs. */
typedef __bf16 bf16x2_cvt __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_fp8x2_bf16_lo(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, false));
}
__device__ __forceinline__ uint32_t cvt_fp8x2_bf16_hi(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, true));
}

/* Eight e4m3fn codes (dword a: codes 0-3, dword b: codes 4-7) -> an exact bf16x8 MFMA operand. */
__device__ __forceinline__ bf16x8 fp8x8_to_bf16(uint32_t a, uint32_t b) {
    const uint4 u = {cvt_fp8x2_bf16_lo(a), cvt_fp8x2_bf16_hi(a), cvt_fp8x2_bf16_lo(b), cvt_fp8x2_bf16_hi(b)};
    return __builtin_bit_cast(bf16x8, u);
}

__device__ __forceinline__ f32x4 mfma16x16x32(const bf16x8 &a, const bf16x8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

}  // namespace nc
