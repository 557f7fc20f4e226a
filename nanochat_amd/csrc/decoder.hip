/*
 * The decoder runtime on gfx950: the reference's dec_* ABI (model/kernels/decode.cu:904-1131, bound by
 * inference/decoder.py:132-148) over an fp8 paged KV cache.
 *
 * A step is a stream of kernels on the caller's stream, launched eagerly:
 *   body   norm_kernel(EMBED), norm_kernel(RESID) of layer 0 -> per layer { qkv GEMM, the fused decode step (q/k
 *          norm + RoPE + value embedding + fp8 append of the step's token, then split-K decode attention, one launch:
 *          attention.hip), o GEMM (+ residual: the bf16 rounding of the fp32 sum, and each 16-row tile's sum of
 *          squares), fc GEMM (+ ReLU^2 of the sum scaled by the rstd it takes from those tile sums), proj GEMM
 *          (K-slice partials), proj_norm_kernel (the partials + residual, then the next layer's residual norm) }
 *   head   norm_kernel(FINAL), lm_head GEMM (fp32 logits; prefill_gemm.hip's tiled kernel), choose_kernel (greedy,
 *          Gumbel-max or nucleus choice within the allowed tokens, then the commit), the tokens to pinned host memory.
 * A step's GEMMs are slot_gemm.hip's weight-streaming MFMA kernel with the epilogue fused (long-K GEMMs split into
 * K-slices whose partials a second kernel adds in order; a model wider than 2,048 computes the MLP's rstd in
 * rstd_kernel). Prefill's GEMMs (up to 16,384 rows a call) are prefill_gemm.hip's MFMA-tiled kernel over all the
 * call's rows at once, with the epilogue fused (bf16 out, the residual, ReLU^2 with the rstd); each row's sums run in
 * one fixed order, so they do not depend on how many rows the call holds. The o GEMM's residual sum needs its whole
 * row for the MLP's rstd, so it writes fp32 and rstd_kernel adds the residual. Every kernel covers the slots up to
 * the highest active one (dec_set_active) and skips inactive slots.
 *
 * Numerics, op by op as decode.cu: the epilogues round once (bf16(s + residual)); the MLP reads the un-normed stream
 * scaled by its rstd; every RMS norm is 1 / sqrt(mean x^2 + FLT_EPSILON), correctly rounded (the reference: rsqrtf).
 * The KV cache is fp8 e4m3fn with one absmax scale per (token, head) (the reference caches bf16); a step's own key
 * is read back from the cache like the others. Decode attention splits a slot's keys at fixed multiples of 1,024
 * positions (merged in position order in the same launch) and the step GEMMs sum every slot's row in one fixed order,
 * so a step's result for a slot depends only on the slot's own inputs and cache.
 *
 * Memory: one allocation per role, sized at dec_create. The KV pool of layer l is `pool` pages the slots draw from
 * (the same page index in every layer) followed by the prompt store's pages (store position s at page pool + s / 16,
 * slot s % 16). A slot's block-table entry is -1 until the slot first writes a position of that page, when a free
 * page is taken from the pool (host free list); a slot's pages return to the pool when it starts a new sequence (a
 * write at position 0), when dec_set_prompt moves it back to a shorter one, or on dec_release. dec_create sizes the
 * pool for every slot at max_len (the reference's reservation, so a step never runs out); dec_create_pool takes a
 * smaller pool, for more slots than full-length reservations allow, and then the host admits requests by the free
 * pages (dec_debug_pages). dec_save_prompt copies a slot's positions into the store; dec_load_prompt points the
 * slot's block-table entries at the store's whole pages (shared read-only, copied into a page of the slot's own on
 * its first write to one) and copies only partial pages.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <tuple>
#include <vector>

#include "nc_device.h"
#include "nanochat_amd.h"
#include "nanochat_decode.h"
#include "nc_internal.h"

namespace nc {
namespace dec {

constexpr int MAX_BATCH = 1024;            /* slots (the reference's limit, decode.cu:27-29) */
constexpr int MASK_BITS = 64;              /* slots per word of a slot mask */
constexpr int MASK_WORDS = MAX_BATCH / MASK_BITS;
constexpr int WORD_BITS = 32;              /* tokens per word of an allowed-token mask */
constexpr int PREFILL_ROWS = 16384;        /* rows per dec_prefill call */
constexpr int SPLIT_SLOTS = 64;            /* a step over more slots runs as two lanes (enqueue_body) */
constexpr int GLOBAL_PTRS = 4, LAYER_PTRS = 8;
constexpr int CHOICE_THREADS = 1024, CHOICE_WAVES = CHOICE_THREADS / WAVE;
constexpr float SM_SCALE = 0.08838834764831845f;  /* 1 / sqrt(128) */

/* A failed HIP call aborts, naming it: never silently wrong tokens (decode.cu:47-53). */
[[noreturn]] static void die(const char *what, const char *detail, int line) {
    fprintf(stderr, "decoder.hip:%d: %s: %s\n", line, what, detail);
    abort();
}
#define HIP_CHECK(call)                                                        \
    do {                                                                       \
        const hipError_t e_ = (call);                                          \
        if (e_ != hipSuccess) ::nc::dec::die(#call, hipGetErrorString(e_), __LINE__);    \
    } while (0)
#define NC_CHECK(call)                                                         \
    do {                                                                       \
        const int s_ = (call);                                                 \
        if (s_ != 0) ::nc::dec::die(#call, nc_status_string(s_), __LINE__);              \
    } while (0)
#define REQUIRE(cond, msg) \
    do {                   \
        if (!(cond)) ::nc::dec::die("dec_create", msg, __LINE__); \
    } while (0)

__device__ __forceinline__ bool live(const unsigned long long *mask, int b) {
    return (mask[b / MASK_BITS] >> (b % MASK_BITS)) & 1ull;
}

/* ---------------------------------------------------------------- norms and epilogues (a wave per row) */

enum { NORM_FINAL, NORM_RESID, NORM_EMBED };

struct NormArgs {
    int kind;
    const uint16_t *in;       /* RESID: the stream x (NULL at layer 0: x0 itself), FINAL: x */
    const float *wte;         /* EMBED: [vocab][C] fp32 */
    float *x0;                /* [rows][C] fp32: EMBED writes, RESID reads */
    int32_t *tokens;          /* EMBED: a token outside [0, vocab) is replaced by 0 here (embedded and read by
                                 the layers' value embeddings as 0), so no kernel reads outside a table */
    int vocab;
    float l1, l2;             /* RESID: resid and x0 lambdas */
    uint16_t *mixed, *out;    /* RESID: mixed = bf16(v); out = bf16(v r) */
    const unsigned long long *active;  /* NULL: every row */
    int rows, C;
    const int32_t *pos;       /* EMBED in a step: seq_lens = pos + 1 and num_new = 1 for active slots, else 0 */
    int32_t *seq_lens, *num_new;
};

/* Row kernels: a wave per row, four rows a 256-thread block, one pass. Lane l holds elements (j 64 + l) 8 .. + 7 for
 * j < NJ (NJ 512 >= C); every load is issued before the first use, the sum of squares is an FMA chain over the lane's
 * elements in order (j, then element) and then the wave butterfly, so the result is fixed for a given C. */
constexpr int ROW_CHUNK = WAVE * 8;   /* elements of a row per j */

__device__ __forceinline__ void load8(const float *p, float (&v)[8]) {
    const float4 a = *reinterpret_cast<const float4 *>(p), b = *reinterpret_cast<const float4 *>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ void load8(const uint16_t *p, float (&v)[8]) {
    const uint4 u = *reinterpret_cast<const uint4 *>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        v[2 * e] = bf16_to_f32((uint16_t)w[e]);
        v[2 * e + 1] = bf16_to_f32((uint16_t)(w[e] >> 16));
    }
}

__device__ __forceinline__ void store8(float *p, const float (&v)[8]) {
    *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4 *>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

__device__ __forceinline__ void store8(uint16_t *p, const float (&v)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; e++) w[e] = (uint32_t)f32_to_bf16(v[2 * e]) | ((uint32_t)f32_to_bf16(v[2 * e + 1]) << 16);
    *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}

/* RMS norm of a row (decode.cu:413-443): EMBED x0 = wte[token] r in fp32; RESID v = fma(l1, h, x0 l2),
 * mixed = bf16(v), out = bf16(v r); FINAL out = bf16(x r); r = 1 / sqrt(sum v^2 / C + FLT_EPSILON). */
template <int NJ>
__global__ void __launch_bounds__(256) norm_kernel(NormArgs a) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= a.rows) return;
    const bool on = !a.active || live(a.active, b);
    if (a.seq_lens && lane == 0) {
        a.seq_lens[b] = on ? a.pos[b] + 1 : 0;
        a.num_new[b] = on ? 1 : 0;
    }
    if (!on) return;
    const long long row = (long long)b * a.C;
    const float *emb = nullptr;
    if (a.kind == NORM_EMBED) {
        int token = a.tokens[b];   /* every lane reads it before lane 0 can store below */
        if (token < 0 || token >= a.vocab) {
            token = 0;
            if (lane == 0) a.tokens[b] = 0;
        }
        emb = a.wte + (long long)token * a.C;
    }
    float v[NJ][8];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int i = j * ROW_CHUNK + lane * 8;
#pragma unroll
        for (int e = 0; e < 8; e++) v[j][e] = 0.0f;
        if (i >= a.C) continue;
        if (a.kind == NORM_EMBED) {
            load8(emb + i, v[j]);
        } else if (a.kind == NORM_FINAL) {
            load8(a.in + row + i, v[j]);
        } else {
            float x0[8], h[8];
            load8(a.x0 + row + i, x0);
            if (a.in) load8(a.in + row + i, h);
#pragma unroll
            for (int e = 0; e < 8; e++) v[j][e] = __builtin_fmaf(a.l1, a.in ? h[e] : x0[e], x0[e] * a.l2);
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int e = 0; e < 8; e++) ss = __builtin_fmaf(v[j][e], v[j][e], ss);
    ss = wave_sum_butterfly(ss);
    const float r = 1.0f / __builtin_sqrtf(ss / (float)a.C + FLT_EPS);
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int i = j * ROW_CHUNK + lane * 8;
        if (i >= a.C) continue;
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; e++) y[e] = v[j][e] * r;
        if (a.kind == NORM_EMBED) {
            store8(a.x0 + row + i, y);
        } else {
            if (a.kind == NORM_RESID) store8(a.mixed + row + i, v[j]);
            store8(a.out + row + i, y);
        }
    }
}

/* The MLP's rstd of o_proj's fp32 residual sum (decode.cu:149-154, 445-456), a wave per row: x = s + xm when xm is
 * given (then xo = bf16(x) is written here), else x = s (the GEMM wrote xo and x); rstd = 1 / sqrt(sum x^2 (1 / C)
 * + FLT_EPSILON). */
template <int NJ>
__global__ void __launch_bounds__(256) rstd_kernel(const float *s, const uint16_t *xm, uint16_t *xo, float *rstd,
                                                   const unsigned long long *active, int rows, int C) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= rows || (active && !live(active, b))) return;
    const long long row = (long long)b * C;
    float x[NJ][8];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int i = j * ROW_CHUNK + lane * 8;
#pragma unroll
        for (int e = 0; e < 8; e++) x[j][e] = 0.0f;
        if (i >= C) continue;
        load8(s + row + i, x[j]);
        if (xm) {
            float m[8];
            load8(xm + row + i, m);
#pragma unroll
            for (int e = 0; e < 8; e++) x[j][e] = x[j][e] + m[e];
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int i = j * ROW_CHUNK + lane * 8;
        if (xm && i < C) store8(xo + row + i, x[j]);
#pragma unroll
        for (int e = 0; e < 8; e++) ss = __builtin_fmaf(x[j][e], x[j][e], ss);
    }
    ss = wave_sum_butterfly(ss);
    if (lane == 0) rstd[b] = 1.0f / __builtin_sqrtf(ss * (1.0f / (float)C) + FLT_EPS);
}

/* A step's layer boundary in one pass (decode.cu:149-154 and 413-443 for the same math): the proj GEMM's S K-slice
 * partials of one slot summed in slice order plus the residual, x = bf16(sum + xo); then, when the next layer's norm is
 * asked for (mixed non-NULL), NORM_RESID over x: v = fma(l1, x, x0 l2), mixed = bf16(v), out = bf16(v r),
 * r = 1 / sqrt(sum v^2 / C + FLT_EPSILON). A 256-thread block per slot; thread t holds the 8-element groups t, t + 256,
 * ... (NG of them); the sum of squares is each thread's FMA chain in group order, the wave butterfly, then the four
 * waves in order: fixed for a given C, whatever the other slots hold. */
struct ProjNormArgs {
    const float *part;        /* [S][N][C] fp32 partial sums (slot_gemm_partials) */
    int S, N, C;
    const uint16_t *res;      /* [N][C] bf16 residual (xo) */
    uint16_t *x;              /* [N][C] bf16: the layer's output stream */
    const float *x0;          /* [N][C] fp32 */
    float l1, l2;             /* the next layer's resid and x0 lambdas */
    uint16_t *mixed, *out;    /* NULL mixed: no norm */
    const unsigned long long *active;
};

constexpr int PN_MAX_S = 8;   /* K-slices proj_norm_kernel adds (F <= 16,384) */

template <int NG>
__global__ void __launch_bounds__(256) proj_norm_kernel(ProjNormArgs a) {
    __shared__ float wsum[256 / WAVE];
    const int n = blockIdx.x, t = threadIdx.x;
    if (a.active && !live(a.active, n)) return;
    const long long row = (long long)n * a.C, slice = (long long)a.N * a.C;
    float v[NG][8];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NG; j++) {
        const int i = (j * 256 + t) * 8;
#pragma unroll
        for (int e = 0; e < 8; e++) v[j][e] = 0.0f;
        if (i >= a.C) continue;
        float sum[8], r[8], q[PN_MAX_S - 1][8];
        load8(a.part + row + i, sum);
#pragma unroll
        for (int sl = 1; sl < PN_MAX_S; sl++)   /* every slice's loads before the first add */
            if (sl < a.S) load8(a.part + sl * slice + row + i, q[sl - 1]);
        load8(a.res + row + i, r);
#pragma unroll
        for (int sl = 1; sl < PN_MAX_S; sl++)
            if (sl < a.S)
#pragma unroll
                for (int e = 0; e < 8; e++) sum[e] = sum[e] + q[sl - 1][e];
#pragma unroll
        for (int e = 0; e < 8; e++) sum[e] = sum[e] + r[e];
        store8(a.x + row + i, sum);
        if (!a.mixed) continue;
        float x0[8];
        load8(a.x0 + row + i, x0);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            v[j][e] = __builtin_fmaf(a.l1, bf16_to_f32(f32_to_bf16(sum[e])), x0[e] * a.l2);
            ss = __builtin_fmaf(v[j][e], v[j][e], ss);
        }
        store8(a.mixed + row + i, v[j]);
    }
    if (!a.mixed) return;
    ss = wave_sum_butterfly(ss);
    if ((t & (WAVE - 1)) == 0) wsum[t / WAVE] = ss;
    __syncthreads();
    ss = wsum[0];
#pragma unroll
    for (int w = 1; w < 256 / WAVE; w++) ss = ss + wsum[w];
    const float r = 1.0f / __builtin_sqrtf(ss / (float)a.C + FLT_EPS);
#pragma unroll
    for (int j = 0; j < NG; j++) {
        const int i = (j * 256 + t) * 8;
        if (i >= a.C) continue;
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; e++) y[e] = v[j][e] * r;
        store8(a.out + row + i, y);
    }
}

/* ---------------------------------------------------------------- the choice */

/* Philox4x32-10 (Salmon et al., "Parallel random numbers: as easy as 1, 2, 3", SC'11; the Random123 constants):
 * ten rounds of two 32x32->64 multiplies, the key bumped by the Weyl constants between rounds. */
__host__ __device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
    for (int r = 0; r < 10; r++) {
        if (r) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint64_t p0 = (uint64_t)0xD2511F53u * c[0], p1 = (uint64_t)0xCD9E8D57u * c[2];
        const uint32_t y0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0, y1 = (uint32_t)p1;
        const uint32_t y2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1, y3 = (uint32_t)p0;
        c[0] = y0; c[1] = y1; c[2] = y2; c[3] = y3;
    }
}

/* Gumbel noise -log(-log(u)) for row `row` of generated position i under seed (decode.cu:98-105): Philox at counter
 * (row, i, 0, 0), key (seed low, seed high); the first two words give 52 bits r, u = (2 r + 1) 2^-53 in (0, 1);
 * the logs in fp64. */
__device__ __forceinline__ float gumbel(unsigned long long seed, int i, int row) {
    uint32_t c[4] = {(uint32_t)row, (uint32_t)i, 0u, 0u};
    philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    const unsigned long long r = ((unsigned long long)c[0] << 32 | c[1]) >> 12;
    const double u = ldexp(2.0 * (double)r + 1.0, -53);
    return (float)-log(-log(u));
}

/* The choice order (decode.cu:90-96): the score's bits mapped to an unsigned order, then ~row, so the largest key
 * has the largest score and, among equal scores, the lowest row. Key 0 means none. */
__device__ __forceinline__ unsigned long long choice_key(float score, int row) {
    const uint32_t bits = __float_as_uint(score);
    const uint32_t ordered = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
    return ((unsigned long long)ordered << 32) | (0xFFFFFFFFu - (uint32_t)row);
}

struct ChoiceArgs {
    const float *logits;       /* [B][vocab] fp32 */
    float *probs;              /* [B][vocab]: the nucleus path's exp(z / T - max) */
    const unsigned long long *active;  /* [2][MASK_WORDS]: active slots, then masked slots */
    const uint32_t *allow;     /* [B][vocab / 32] */
    const float *temperature, *top_p;
    const unsigned long long *seed;
    const int32_t *first;
    int32_t *tokens, *alt_tokens, *pos;
    float softcap;
    int vocab, lazy;
};

/* Block reductions: the wave butterfly, then the waves in order; every thread gets the result. */
__device__ float block_max(float v, float *scratch) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & (WAVE - 1)) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = -INFINITY;
    for (int w = 0; w < CHOICE_WAVES; w++) m = fmaxf(m, scratch[w]);
    return m;
}

__device__ unsigned long long block_max_key(unsigned long long v, unsigned long long *scratch) {
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) {
        const unsigned long long other = __shfl_xor(v, o, WAVE);
        v = other > v ? other : v;
    }
    __syncthreads();
    if ((threadIdx.x & (WAVE - 1)) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    unsigned long long m = 0;
    for (int w = 0; w < CHOICE_WAVES; w++) m = scratch[w] > m ? scratch[w] : m;
    return m;
}

/* ---------------------------------------------------------------- the nucleus threshold
 *
 * The nucleus (arXiv 1904.09751 §3.1, the rule of transformers' TopPLogitsWarper) keeps the rows whose probability
 * is at least e*, the least probability for which the rows at or below it hold more than (1 - top_p) of the mass.
 * The probabilities are e = exp(z / T - max z / T) in [0, 1], unnormalized. Masses are fixed point: a row weighs the
 * integer round(e 2^NUCLEUS_FRAC_BITS), so every sum below is exact and the same whatever order the adds run in (a
 * vocabulary under 2^25 rows keeps the total under 2^64). A row lighter than 2^-(NUCLEUS_FRAC_BITS + 1) of the largest
 * weighs 0 and is never kept.
 *
 * For e >= 0 the order of the values is the order of their IEEE bit patterns, so e*'s pattern is found digit by digit
 * from the top, 8 bits a round, as a weighted radix select. A round sums the weights of the rows that share the digits
 * chosen so far into 256 bins by their next digit (a private histogram per wave, so the integer LDS adds of different
 * waves never meet), merges the waves' bins, prefix-sums them, and picks the one bin in which the running mass, from
 * the weight of every row below the current range, first passes the drop. Four rounds fix all 32 bits. */
constexpr int NUCLEUS_FRAC_BITS = 38;
constexpr int NUCLEUS_BINS = 256;

struct NucleusShared {
    unsigned long long hist[CHOICE_WAVES][NUCLEUS_BINS];
    unsigned long long part[NUCLEUS_BINS / WAVE];   /* each bin-holding wave's bin total */
    unsigned long long base;                        /* weight below the chosen bin */
    uint32_t digit;
};

__device__ __forceinline__ unsigned long long nucleus_weight(float e) {
    return (unsigned long long)((double)e * (double)(1ull << NUCLEUS_FRAC_BITS) + 0.5);
}

__device__ unsigned long long wave_inclusive_scan(unsigned long long v) {
    const int lane = threadIdx.x & (WAVE - 1);
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const unsigned long long up = __shfl_up(v, d, WAVE);
        if (lane >= d) v += up;
    }
    return v;
}

/* e*'s bit pattern for one slot's probabilities e[0 .. vocab), each row read by the thread that wrote it
 * (rows tid, tid + CHOICE_THREADS, ...). Uniform over the block; every thread returns the same value. */
__device__ uint32_t nucleus_cut(const float *e, int vocab, float top_p, NucleusShared &sh) {
    const int tid = threadIdx.x, wave = tid / WAVE;
    uint32_t chosen = 0;               /* the digits fixed so far, in place */
    unsigned long long below = 0;      /* weight of every row whose pattern is under the current range */
    unsigned long long drop = 0;       /* the mass that may be dropped, fixed in the first round */
    for (int shift = 32 - 8; shift >= 0; shift -= 8) {
        for (int i = tid; i < CHOICE_WAVES * NUCLEUS_BINS; i += CHOICE_THREADS) (&sh.hist[0][0])[i] = 0ull;
        __syncthreads();
        const unsigned long long range = (unsigned long long)chosen >> (shift + 8);
        for (int r = tid; r < vocab; r += CHOICE_THREADS) {
            const uint32_t bits = __float_as_uint(e[r]);
            if (((unsigned long long)bits >> (shift + 8)) != range) continue;
            const unsigned long long w = nucleus_weight(e[r]);
            if (w != 0ull) atomicAdd(&sh.hist[wave][(bits >> shift) & (NUCLEUS_BINS - 1)], w);
        }
        __syncthreads();
        /* threads 0..255 hold a bin each: its total over the waves, then the running sums */
        unsigned long long bin = 0ull, upto = 0ull;
        if (tid < NUCLEUS_BINS) {
            for (int w = 0; w < CHOICE_WAVES; w++) bin += sh.hist[w][tid];
            upto = wave_inclusive_scan(bin);
            if ((tid & (WAVE - 1)) == WAVE - 1) sh.part[wave] = upto;
        }
        if (tid == 0) { sh.digit = NUCLEUS_BINS - 1; sh.base = below; }   /* kept only if nothing passes */
        __syncthreads();
        unsigned long long earlier = 0ull, range_total = 0ull;
        for (int w = 0; w < NUCLEUS_BINS / WAVE; w++) {
            if (w < wave) earlier += sh.part[w];
            range_total += sh.part[w];
        }
        if (shift == 32 - 8 && range_total != 0ull) {
            /* the first round's range is every row, so range_total is the whole mass. At most all but one unit of
             * it may go, so the largest row always stays (top_p <= 0 keeps exactly the rows at the maximum). With no
             * mass at all (no allowed row) nothing passes, and no row is kept. */
            const double keep_out = (1.0 - (double)top_p) * (double)range_total;
            drop = keep_out >= (double)(range_total - 1ull) ? range_total - 1ull : (unsigned long long)keep_out;
        }
        upto += earlier;
        if (tid < NUCLEUS_BINS && below + upto - bin <= drop && below + upto > drop) {
            sh.digit = (uint32_t)tid;
            sh.base = below + upto - bin;
        }
        __syncthreads();
        chosen |= sh.digit << shift;
        below = sh.base;
    }
    return chosen;
}

/* The cut alone, one block per row of e (a test hook: dec_debug_nucleus_cut). */
__global__ void __launch_bounds__(CHOICE_THREADS) nucleus_cut_kernel(const float *e, int vocab, const float *top_p,
                                                                     uint32_t *cut) {
    __shared__ NucleusShared sh;
    const uint32_t u = nucleus_cut(e + (long long)blockIdx.x * vocab, vocab, top_p[blockIdx.x], sh);
    if (threadIdx.x == 0) cut[blockIdx.x] = u;
}

/* A block per slot: its token among the allowed rows of its logits, then the commit (decode.cu:170-229, 361-411,
 * 677-688). Temperature 0: the largest logit. T > 0: the largest z / T + gumbel, z = c tanh(s / c) (Gumbel-max
 * sampling of softmax(z / T)). T > 0 and top_p < 1: Gumbel-max within the nucleus that nucleus_cut fixes. The
 * alternative is the best key but the lazy row's (none for a nucleus slot). */
__global__ void __launch_bounds__(CHOICE_THREADS) choose_kernel(ChoiceArgs c) {
    __shared__ float fscratch[CHOICE_WAVES];
    __shared__ unsigned long long kscratch[CHOICE_WAVES];
    __shared__ NucleusShared nucleus;
    const int b = blockIdx.x, tid = threadIdx.x;
    if (!live(c.active, b)) return;
    const float *s = c.logits + (long long)b * c.vocab;
    const float T = c.temperature[b], top_p = c.top_p[b];
    const bool masked = live(c.active + MASK_WORDS, b);
    const uint32_t *allow = c.allow + (long long)b * (c.vocab / WORD_BITS);
    const int gen = c.pos[b] - c.first[b];
    const unsigned long long seed = c.seed[b];
    auto allowed = [&](int r) { return !masked || ((allow[r / WORD_BITS] >> (r % WORD_BITS)) & 1u); };
    auto capped = [&](int r) { return c.softcap * tanhf(s[r] / c.softcap); };
    unsigned long long best = 0, alt = 0;
    if (T > 0.0f && top_p < 1.0f) {
        /* the slot's probabilities go to its row of c.probs; every pass over them visits a thread's own rows */
        float *prob = c.probs + (long long)b * c.vocab;
        float zmax = -INFINITY;
        for (int r = tid; r < c.vocab; r += CHOICE_THREADS)
            if (allowed(r)) zmax = fmaxf(zmax, capped(r) / T);
        zmax = block_max(zmax, fscratch);
        for (int r = tid; r < c.vocab; r += CHOICE_THREADS) prob[r] = allowed(r) ? expf(capped(r) / T - zmax) : 0.0f;
        const uint32_t cut = nucleus_cut(prob, c.vocab, top_p, nucleus);
        for (int r = tid; r < c.vocab; r += CHOICE_THREADS) {
            const float pr = prob[r];
            if (pr == 0.0f || __float_as_uint(pr) < cut) continue;
            const unsigned long long key = choice_key(capped(r) / T + gumbel(seed, gen, r), r);
            best = key > best ? key : best;
        }
    } else {
        /* four logits a thread a step by 16-byte reads, four reads in flight (the vocab is a multiple of 32); the result
         * is a maximum over keys unique per row, so the visiting order does not matter */
        const float4 *s4 = reinterpret_cast<const float4 *>(s);
#pragma unroll 4
        for (int q = tid; q < c.vocab / 4; q += CHOICE_THREADS) {
            const float4 v4 = s4[q];
            const float v[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int r = 4 * q + e;
                if (!allowed(r)) continue;
                const float score = T > 0.0f ? c.softcap * tanhf(v[e] / c.softcap) / T + gumbel(seed, gen, r) : v[e];
                const unsigned long long key = choice_key(score, r);
                best = key > best ? key : best;
                if (r != c.lazy) alt = key > alt ? key : alt;
            }
        }
    }
    best = block_max_key(best, kscratch);
    alt = block_max_key(alt, kscratch);
    if (tid == 0) {
        c.tokens[b] = (int32_t)(0xFFFFFFFFu - (uint32_t)best);   /* key 0 (nothing allowed) gives -1 */
        c.alt_tokens[b] = (int32_t)(0xFFFFFFFFu - (uint32_t)alt);
        c.pos[b] += 1;
    }
}

/* ---------------------------------------------------------------- small state kernels */

__global__ void set_slot_kernel(int32_t *tokens, int32_t *pos, int32_t *first, float *temperature, float *top_p,
                                unsigned long long *seeds, int b, int32_t token, int32_t last, float t, float p,
                                unsigned long long seed) {
    tokens[b] = token;
    pos[b] = last;
    first[b] = last;
    temperature[b] = t;
    top_p[b] = p;
    seeds[b] = seed;
}

struct SlotMasks {
    unsigned long long w[2 * MASK_WORDS];
};

__global__ void set_active_kernel(unsigned long long *active, SlotMasks m) {
    if (threadIdx.x < 2 * MASK_WORDS) active[threadIdx.x] = m.w[threadIdx.x];
}

__global__ void take_alt_kernel(int32_t *tokens, const int32_t *alt_tokens, int b) { tokens[b] = alt_tokens[b]; }

/* Copy n positions of every layer and head between two places of the same pools: position p of a side is slot p % 16
 * of page tab[p / 16] (a slot's block-table row) or, with tab NULL, of page page0 + p / 16 (the prompt store); codes
 * keep their tile layout, both scales move. A wave per (position, layer, head); lane l moves dims l and l + 64. */
__global__ void __launch_bounds__(256) copy_positions_kernel(uint8_t *k_pages, uint8_t *v_pages, float *kv_scale,
                                                             long long layer_pages, int H, int L, const int32_t *src_tab,
                                                             long long src_page0, int src_pos, const int32_t *dst_tab,
                                                             long long dst_page0, int dst_pos, int n) {
    const long long unit = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & (WAVE - 1);
    if (unit >= (long long)n * L * H) return;
    const int h = (int)(unit % H), l = (int)(unit / H % L), i = (int)(unit / ((long long)H * L));
    const int sp = src_pos + i, dp = dst_pos + i;
    const long long spage = src_tab ? src_tab[sp / PAGE] : src_page0 + sp / PAGE;
    const long long dpage = dst_tab ? dst_tab[dp / PAGE] : dst_page0 + dp / PAGE;
    const long long sa = ((long long)l * layer_pages + spage) * H + h;
    const long long da = ((long long)l * layer_pages + dpage) * H + h;
    const int ss = sp % PAGE, ds = dp % PAGE;
#pragma unroll
    for (int half = 0; half < 2; half++) {
        const int dim = lane + half * HALF;
        k_pages[da * PAGE_BYTES + k_page_offset(ds, dim)] = k_pages[sa * PAGE_BYTES + k_page_offset(ss, dim)];
        v_pages[da * PAGE_BYTES + v_page_offset(ds, dim)] = v_pages[sa * PAGE_BYTES + v_page_offset(ss, dim)];
    }
    if (lane < 2) kv_scale[(da * 2 + lane) * PAGE + ds] = kv_scale[(sa * 2 + lane) * PAGE + ss];
}

/* table[idx0 + i] = value0 + step i for i < count */
__global__ void set_table_kernel(int32_t *table, long long idx0, long long count, int value0, int step) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i < count) table[idx0 + i] = value0 + step * (int)i;
}

/* Runs of block-table entries written by one launch (kernel arguments, so the host's list is free once launched):
 * run r sets table[idx0 + i] = value0 + step i for i < count. The runs of a launch are disjoint. */
struct TableRun {
    int32_t idx0, count, value0, step;
};
constexpr int TABLE_RUNS = 224;
struct TableRuns {
    int32_t n;
    TableRun run[TABLE_RUNS];
};

__global__ void __launch_bounds__(256) set_table_runs_kernel(int32_t *table, TableRuns t) {
    if ((int)blockIdx.x >= t.n) return;
    const TableRun r = t.run[blockIdx.x];
    for (int i = threadIdx.x; i < r.count; i += 256) table[r.idx0 + i] = r.value0 + r.step * i;
}

/* Whole pages src_page0 + z -> dst_page0 + z of layer y and head x: 2 KiB of K codes, 2 KiB of V codes, 128 bytes of
 * scales. */
__global__ void __launch_bounds__(256) copy_pages_kernel(uint8_t *k_pages, uint8_t *v_pages, float *kv_scale,
                                                         long long layer_pages, int H, long long src_page0,
                                                         long long dst_page0) {
    const int h = blockIdx.x, l = blockIdx.y, t = threadIdx.x;
    const long long sa = ((long long)l * layer_pages + src_page0 + blockIdx.z) * H + h;
    const long long da = ((long long)l * layer_pages + dst_page0 + blockIdx.z) * H + h;
    if (t < 128)
        reinterpret_cast<uint4 *>(k_pages + da * PAGE_BYTES)[t] = reinterpret_cast<const uint4 *>(k_pages + sa * PAGE_BYTES)[t];
    else
        reinterpret_cast<uint4 *>(v_pages + da * PAGE_BYTES)[t - 128] =
            reinterpret_cast<const uint4 *>(v_pages + sa * PAGE_BYTES)[t - 128];
    if (t < 8) reinterpret_cast<float4 *>(kv_scale + da * 2 * PAGE)[t] = reinterpret_cast<const float4 *>(kv_scale + sa * 2 * PAGE)[t];
}

/* ---------------------------------------------------------------- the decoder */

struct Layer {
    const uint16_t *qkv, *o, *fc, *proj, *ve;  /* bf16 [3C][C], [C][C], [F][C], [C][F]; ve [vocab][C] or NULL */
    const float *ve_gate, *q_gain, *k_gain;   /* [H][C] or NULL; [128]; [128] */
    float resid, x0;
    int window;
};

/* Per-row activations of a step (slots) or of a prefill call (rows). */
struct Acts {
    float *x0;                 /* [rows][C] fp32 */
    uint16_t *x, *xm, *h, *hn, *qkv, *q, *att, *xo, *u;  /* bf16 [rows][C] (qkv [3C], u [F]) */
    float *acc;                /* [rows][max(C, F)]: fp32 GEMM outputs */
    float *rstd;               /* [rows] */
};

/* Where a stretch of work runs: a stream with its own scratch, so two lanes can run at once. */
struct Lane {
    hipStream_t stream;
    void *attn_ws;                       /* decode-attention partials (Decoder::attn_ws_bytes) */
    float *part;                         /* slot_gemm's split-K partial sums (Decoder::part_bytes) */
    float *ssq;                          /* [B][ceil(C / 16)]: the o GEMM's tile sums of squares for fc's rstd */
};

struct Decoder {
    int B, L, C, F, H, vocab, max_len, store, lazy, max_pages;
    long long pool, layer_pages;         /* pages the slots draw from; pages of a layer's pool (slots + store) */
    std::vector<int32_t> free_pages;     /* the pool's free pages, a stack (taken from the back) */
    float softcap;
    const float *wte, *cos, *sin;
    const uint16_t *lm_head;
    std::vector<Layer> layer;
    hipStream_t stream;                  /* the caller's stream: every call is ordered on it */
    Lane lane[2];                        /* lane 0 runs on `stream`; lane 1 on the decoder's own stream, forked from
                                            and joined back into `stream` within a step */
    hipEvent_t fork, join;
    std::vector<hipEvent_t> attn_done;   /* [2 L]: lane h's attention of layer l finished */
    uint8_t *k_pages, *v_pages;          /* [L][layer_pages][H][2048] */
    float *kv_scale;                     /* [L][layer_pages][H][2][16] */
    int32_t *block_table;                /* [B][max_pages]: slot b's entry e is -1, a pool page of its own, or a
                                            store page it shares read-only after dec_load_prompt */
    std::vector<int32_t> table;          /* host copy of block_table (what the enqueued work leaves there) */
    std::vector<int2> dirty;             /* [B]: slot b's entries [x, y) changed since the last flush_table */
    std::vector<int> dirty_slots;        /* the slots with changed entries, in the order first changed */
    std::vector<int32_t> hpos;           /* host copy of pos: the position a live slot's next step writes */
    std::vector<unsigned long long> live;  /* host copy of the live-slot mask of dec_set_active */
    int32_t *tokens, *alt_tokens, *pos, *first, *seq_lens, *num_new;  /* [B] */
    float *temperature, *top_p;
    unsigned long long *seed;
    unsigned long long *active;          /* [2][MASK_WORDS] */
    uint32_t *allow;                     /* [B][vocab / 32] */
    float *logits, *probs;               /* [B][vocab] */
    Acts slot, row;
    size_t attn_ws_bytes;
    int32_t *rows;                       /* device [7][PREFILL_ROWS]: token, position, slot; run row0, count, slot,
                                            start */
    int32_t *staging;                    /* pinned host, as rows */
    hipEvent_t staged;                   /* the last upload of staging has been read */
    int32_t *host_tokens;                /* pinned [2][B] */
    uint32_t *host_allow;                /* pinned [B][vocab / 32] */
    int narrow;                          /* a step's rows: the highest active slot + 1 */
    long long part_bytes;                /* each lane's slot_gemm partials, for SG_MAX_N slots */
    bool split;                          /* a step of more than SPLIT_SLOTS slots runs as two lanes */
    bool graphs;                         /* the body replays a captured graph per (narrow, split) */
    std::map<std::pair<int, int>, hipGraphExec_t> body_graphs;  /* nullptr: seen once, run eagerly */
    std::vector<void *> device_blocks;
};

static void *device_alloc(Decoder *d, size_t bytes) {
    void *p = nullptr;
    if (!bytes) return nullptr;
    HIP_CHECK(hipMalloc(&p, bytes));
    HIP_CHECK(hipMemsetAsync(p, 0, bytes, d->stream));
    d->device_blocks.push_back(p);
    return p;
}

static size_t acts_bytes(const Decoder *d, size_t rows) {
    const size_t C = d->C, F = d->F, W = F > C ? F : C;
    return rows * (C * 4 + 7 * C * 2 + 3 * C * 2 + F * 2 + W * 4 + 4) + 16 * 256;
}

static Acts carve_acts(Decoder *d, size_t rows) {
    const size_t C = d->C, F = d->F, W = F > C ? F : C;
    unsigned char *p = (unsigned char *)device_alloc(d, acts_bytes(d, rows));
    auto take = [&](size_t bytes) {
        void *q = p;
        p += (bytes + 255) / 256 * 256;
        return q;
    };
    Acts a;
    a.x0 = (float *)take(rows * C * 4);
    a.x = (uint16_t *)take(rows * C * 2);
    a.xm = (uint16_t *)take(rows * C * 2);
    a.h = (uint16_t *)take(rows * C * 2);
    a.hn = (uint16_t *)take(rows * C * 2);
    a.q = (uint16_t *)take(rows * C * 2);
    a.att = (uint16_t *)take(rows * C * 2);
    a.xo = (uint16_t *)take(rows * C * 2);
    a.qkv = (uint16_t *)take(rows * 3 * C * 2);
    a.u = (uint16_t *)take(rows * F * 2);
    a.acc = (float *)take(rows * W * 4);
    a.rstd = (float *)take(rows * 4);
    return a;
}

/* The activations of rows b0 .. of a. */
static Acts acts_from(const Decoder *d, const Acts &a, size_t b0) {
    const size_t C = d->C, F = d->F, W = F > C ? F : C;
    Acts r = a;
    r.x0 = a.x0 + b0 * C;
    r.x = a.x + b0 * C; r.xm = a.xm + b0 * C; r.h = a.h + b0 * C; r.hn = a.hn + b0 * C;
    r.q = a.q + b0 * C; r.att = a.att + b0 * C; r.xo = a.xo + b0 * C;
    r.qkv = a.qkv + b0 * 3 * C;
    r.u = a.u + b0 * F;
    r.acc = a.acc + b0 * W;
    r.rstd = a.rstd + b0;
    return r;
}

/* A prefill GEMM (prefill_gemm.hip) over all n rows of the call: out[r][rows] = epilogue(in[r][cols] . W[rows][cols]^T),
 * each row's sums in one fixed order whatever n is, so a row's result does not depend on how many rows share the call.
 * epi: SG_STORE (bf16), SG_RESID (bf16(s + resid)), SG_F32 (fp32) or SG_RELU2 (bf16(relu(p) p), p = s rstd[r]). */
static void gemm(const Lane &ln, const uint16_t *w, int rows, int cols, const uint16_t *in, int n, void *out, int epi,
                 const uint16_t *resid = nullptr, const float *rstd = nullptr) {
    if (n <= 0) return;
    if (n > PREFILL_ROWS) die("gemm", "more rows than the prefill buffers hold", __LINE__);
    PfGemm g = {in, w, n, rows, cols, epi == SG_F32 ? nullptr : (uint16_t *)out, epi == SG_F32 ? (float *)out : nullptr,
                resid, rstd};
    NC_CHECK(prefill_gemm(g, epi, ln.stream));
}

static NormArgs norm_args(Decoder *d, int kind, const Acts &a, int rows, int32_t *tokens,
                          const unsigned long long *active) {
    NormArgs n = {};
    n.kind = kind;
    n.wte = d->wte;
    n.x0 = a.x0;
    n.tokens = tokens;
    n.vocab = d->vocab;
    n.active = active;
    n.rows = rows;
    n.C = d->C;
    return n;
}

/* The row kernels' NJ: the fewest 512-element chunks covering C (C <= MAX_C). */
constexpr int MAX_C = 8 * ROW_CHUNK;

static void launch_norm(const Lane &ln, const NormArgs &n) {
    const dim3 grid((n.rows + 3) / 4), block(256);
    if (n.C <= 2 * ROW_CHUNK) hipLaunchKernelGGL(norm_kernel<2>, grid, block, 0, ln.stream, n);
    else if (n.C <= 4 * ROW_CHUNK) hipLaunchKernelGGL(norm_kernel<4>, grid, block, 0, ln.stream, n);
    else hipLaunchKernelGGL(norm_kernel<8>, grid, block, 0, ln.stream, n);
}

static void launch_rstd(Decoder *d, const Lane &ln, const float *s, const uint16_t *xm, uint16_t *xo, float *rstd,
                        const unsigned long long *active, int rows) {
    const dim3 grid((rows + 3) / 4), block(256);
    const int C = d->C;
    if (C <= 2 * ROW_CHUNK)
        hipLaunchKernelGGL(rstd_kernel<2>, grid, block, 0, ln.stream, s, xm, xo, rstd, active, rows, C);
    else if (C <= 4 * ROW_CHUNK)
        hipLaunchKernelGGL(rstd_kernel<4>, grid, block, 0, ln.stream, s, xm, xo, rstd, active, rows, C);
    else
        hipLaunchKernelGGL(rstd_kernel<8>, grid, block, 0, ln.stream, s, xm, xo, rstd, active, rows, C);
}

static uint8_t *layer_k(Decoder *d, int l) { return d->k_pages + (size_t)l * d->layer_pages * d->H * PAGE_BYTES; }
static uint8_t *layer_v(Decoder *d, int l) { return d->v_pages + (size_t)l * d->layer_pages * d->H * PAGE_BYTES; }
static float *layer_s(Decoder *d, int l) { return d->kv_scale + (size_t)l * d->layer_pages * d->H * 2 * PAGE; }

/* A GEMM with its epilogue. A decode step (step): slot_gemm over the slots in blocks of SG_MAX_N, each slot's sums in
 * the same order whatever the block holds, so a slot's result does not depend on the others; its split-K partials (long
 * K) are reduced in slice order. Prefill rows: prefill_gemm with the epilogue fused, except the o GEMM's residual sum,
 * whose rstd needs the whole row (fp32 out; rstd_kernel adds the residual). */
static void gemm_epi(Decoder *d, const Lane &ln, bool step, int epi, const uint16_t *w, int rows, int cols,
                     const uint16_t *in, int n, uint16_t *out, float *out_f32, const uint16_t *res, const float *rstd,
                     const unsigned long long *active, float *ssq = nullptr) {
    if (n <= 0) return;
    if (step) {
        const int S = slot_gemm_slices(rows, cols);
        const int ssq_cols = ((epi == SG_RELU2 ? cols : rows) + 15) / 16;   /* a slot's tile sums */
        for (int b0 = 0; b0 < n; b0 += SG_MAX_N) {
            const size_t o = (size_t)b0 * rows;
            SkinnyGemm g = {w, in + (size_t)b0 * cols, rows, cols, n - b0 < SG_MAX_N ? n - b0 : SG_MAX_N,
                            out ? out + o : nullptr, out_f32 ? out_f32 + o : nullptr, res ? res + o : nullptr,
                            rstd ? rstd + b0 : nullptr, active ? active + b0 / MASK_BITS : nullptr,
                            ssq ? ssq + (size_t)b0 * ssq_cols : nullptr};
            NC_CHECK(slot_gemm(g, epi, ln.part, d->part_bytes, S, ln.stream));
            if (S > 1) NC_CHECK(slot_gemm_reduce(g, epi, ln.part, d->part_bytes, S, ln.stream));
        }
        return;
    }
    switch (epi) {
    case SG_STORE: gemm(ln, w, rows, cols, in, n, out, SG_STORE); break;
    case SG_RESID: gemm(ln, w, rows, cols, in, n, out, SG_RESID, res); break;
    case SG_F32: gemm(ln, w, rows, cols, in, n, out_f32, SG_F32); break;
    case SG_RESID2:  /* fp32 s; the rstd kernel adds the residual and writes out */
        gemm(ln, w, rows, cols, in, n, out_f32, SG_F32);
        break;
    case SG_RELU2: gemm(ln, w, rows, cols, in, n, out, SG_RELU2, nullptr, rstd); break;
    }
}

/* A step's proj GEMM and the next layer's residual norm (next; NULL after the last layer: x alone): the GEMM's fp32
 * K-slice partials, then proj_norm_kernel adds them with the residual and normalizes the row. */
static void proj_norm(Decoder *d, const Lane &ln, const Layer &ly, const Layer *next, const Acts &a, int n,
                      const unsigned long long *active) {
    const int C = d->C, F = d->F;
    const int S = slot_gemm_slices(C, F);
    for (int b0 = 0; b0 < n; b0 += SG_MAX_N) {
        const int nn = n - b0 < SG_MAX_N ? n - b0 : SG_MAX_N;
        const size_t o = (size_t)b0 * C;
        SkinnyGemm g = {ly.proj, a.u + (size_t)b0 * F, C, F, nn, nullptr, nullptr, nullptr, nullptr,
                        active ? active + b0 / MASK_BITS : nullptr, nullptr};
        NC_CHECK(slot_gemm_partials(g, ln.part, d->part_bytes, S, ln.stream));
        ProjNormArgs pa = {ln.part, S, nn, C, a.xo + o, a.x + o, a.x0 + o, next ? next->resid : 0.0f,
                           next ? next->x0 : 0.0f, next ? a.xm + o : nullptr, next ? a.h + o : nullptr, g.active};
        if (C <= 256 * 8) hipLaunchKernelGGL(proj_norm_kernel<1>, dim3(nn), dim3(256), 0, ln.stream, pa);
        else hipLaunchKernelGGL(proj_norm_kernel<2>, dim3(nn), dim3(256), 0, ln.stream, pa);
    }
}

/* The rest of a layer after its attention: o_proj + residual, the MLP. In a step the o GEMM's epilogue adds the
 * residual itself (fp32 sum and its bf16 rounding), so the rstd kernel only reads the sum, and the proj GEMM's sums
 * go to proj_norm_kernel with the next layer's norm (next). */
static void mlp(Decoder *d, const Lane &ln, bool step, const Layer &ly, const Layer *next, const Acts &a, int n,
                const unsigned long long *active) {
    const int C = d->C, F = d->F;
    if (step && slot_gemm_slices(C, C) == 1) {   /* o and fc in one K slice: rstd from the o GEMM's tile sums */
        gemm_epi(d, ln, step, SG_RESID2, ly.o, C, C, a.att, n, a.xo, nullptr, a.xm, nullptr, active, ln.ssq);
        gemm_epi(d, ln, step, SG_RELU2, ly.fc, F, C, a.xo, n, a.u, nullptr, nullptr, nullptr, active, ln.ssq);
        proj_norm(d, ln, ly, next, a, n, active);
        return;
    }
    gemm_epi(d, ln, step, SG_RESID2, ly.o, C, C, a.att, n, a.xo, a.acc, a.xm, nullptr, active);
    launch_rstd(d, ln, a.acc, step ? nullptr : a.xm, a.xo, a.rstd, active, n);
    gemm_epi(d, ln, step, SG_RELU2, ly.fc, F, C, a.xo, n, a.u, a.acc, nullptr, a.rstd, active);
    if (step) proj_norm(d, ln, ly, next, a, n, active);
    else gemm_epi(d, ln, step, SG_RESID, ly.proj, C, F, a.u, n, a.x, nullptr, a.xo, nullptr, active);
}

/* Slots [b0, b0 + n) of a step (b0 a multiple of 64, so their active mask starts at word b0 / 64). */
struct Part {
    int b0, n;
    Acts a;
    const unsigned long long *active;
};

static Part step_part(Decoder *d, int b0, int n) {
    return Part{b0, n, acts_from(d, d->slot, b0), d->active + b0 / MASK_BITS};
}

static void body_embed(Decoder *d, const Lane &ln, const Part &p) {
    NormArgs n = norm_args(d, NORM_EMBED, p.a, p.n, d->tokens + p.b0, p.active);
    n.pos = d->pos + p.b0;
    n.seq_lens = d->seq_lens + p.b0;
    n.num_new = d->num_new + p.b0;
    launch_norm(ln, n);
}

/* Layer l up to its attention: the residual norm (layer 0's here; a later layer's is the previous layer's
 * proj_norm) and qkv. */
static void body_pre(Decoder *d, const Lane &ln, const Part &p, int l) {
    const Layer &ly = d->layer[l];
    const Acts &a = p.a;
    const int C = d->C;
    if (l == 0) {
        NormArgs r = norm_args(d, NORM_RESID, a, p.n, d->tokens + p.b0, p.active);
        r.in = nullptr;
        r.l1 = ly.resid;
        r.l2 = ly.x0;
        r.mixed = a.xm;
        r.out = a.h;
        launch_norm(ln, r);
    }
    gemm_epi(d, ln, true, SG_STORE, ly.qkv, 3 * C, C, a.h, p.n, a.qkv, nullptr, nullptr, nullptr, p.active);
}

/* Layer l's attention: the fused decode step (q/k norm + RoPE, value embedding, fp8 append of the step's k and v,
 * split-K attention) in one launch. Active slots have seq_lens = pos + 1; the others 0 (no append, zero rows). */
static void body_attn(Decoder *d, const Lane &ln, const Part &p, int l) {
    const Layer &ly = d->layer[l];
    StepArgs st = {};
    st.qkv = p.a.qkv;
    st.token_stride = 3LL * d->C;
    st.q_gain = ly.q_gain; st.k_gain = ly.k_gain; st.cos = d->cos; st.sin = d->sin;
    st.ve_h = p.a.h; st.ve = ly.ve; st.ve_gate = ly.ve_gate; st.ve_tokens = d->tokens + p.b0; st.C = d->C;
    st.ve_rows = d->vocab;
    st.k_pages = layer_k(d, l); st.v_pages = layer_v(d, l); st.kv_scale = layer_s(d, l);
    NC_CHECK(decode_step(st, layer_k(d, l), layer_v(d, l), layer_s(d, l), d->block_table + (size_t)p.b0 * d->max_pages,
                         d->max_pages, (int)d->layer_pages, d->seq_lens + p.b0, d->max_len, p.n, d->H, d->H, ly.window,
                         SM_SCALE, p.a.att, ln.attn_ws, d->attn_ws_bytes, ln.stream));
}

/* The step's body. Up to SPLIT_SLOTS slots, one lane. More: two lanes, slots [0, b1) on lane 0 and [b1, narrow) on
 * lane 1, forked from and joined into the caller's stream, with their attentions alternating (lane 1's attention
 * of layer l after lane 0's, lane 0's of layer l + 1 after lane 1's of layer l): attention is bound by HBM bandwidth
 * and the rest of a layer (norms, GEMMs over few rows, epilogues) by latency, so each half's attention runs while
 * the other half works through the rest of its layer. */
static void record_body(Decoder *d) {
    const int R = d->narrow;
    if (!d->split || R <= SPLIT_SLOTS) {
        const Part p = step_part(d, 0, R);
        const Lane &ln = d->lane[0];
        body_embed(d, ln, p);
        for (int l = 0; l < d->L; l++) {
            body_pre(d, ln, p, l);
            body_attn(d, ln, p, l);
            mlp(d, ln, true, d->layer[l], l + 1 < d->L ? &d->layer[l + 1] : nullptr, p.a, p.n, p.active);
        }
        return;
    }
    const int b1 = (R + 2 * MASK_BITS - 1) / (2 * MASK_BITS) * MASK_BITS;   /* half the rows, a multiple of 64 */
    const Part p[2] = {step_part(d, 0, b1), step_part(d, b1, R - b1)};
    const Lane *ln = d->lane;
    HIP_CHECK(hipEventRecord(d->fork, ln[0].stream));
    HIP_CHECK(hipStreamWaitEvent(ln[1].stream, d->fork, 0));
    for (int h = 0; h < 2; h++) body_embed(d, ln[h], p[h]);
    for (int l = 0; l < d->L; l++) {
        hipEvent_t *done = &d->attn_done[2 * l];
        body_pre(d, ln[0], p[0], l);
        if (l > 0) HIP_CHECK(hipStreamWaitEvent(ln[0].stream, d->attn_done[2 * l - 1], 0));
        body_attn(d, ln[0], p[0], l);
        HIP_CHECK(hipEventRecord(done[0], ln[0].stream));
        body_pre(d, ln[1], p[1], l);
        HIP_CHECK(hipStreamWaitEvent(ln[1].stream, done[0], 0));
        body_attn(d, ln[1], p[1], l);
        HIP_CHECK(hipEventRecord(done[1], ln[1].stream));
        for (int h = 0; h < 2; h++)
            mlp(d, ln[h], true, d->layer[l], l + 1 < d->L ? &d->layer[l + 1] : nullptr, p[h].a, p[h].n, p[h].active);
    }
    HIP_CHECK(hipEventRecord(d->join, ln[1].stream));
    HIP_CHECK(hipStreamWaitEvent(ln[0].stream, d->join, 0));
}

/* The body as a graph (the reference captures its step too, decode.cu:893-902): one launch instead of a few hundred
 * (two lanes: ~530 kernels and ~100 event edges a step). The first step of a given (narrow, split) runs eagerly, so
 * the library plans and occupancy queries it makes happen outside a capture; the second captures it (thread-local
 * mode, on the caller's stream, lane 1 joined through the fork event) and every later one replays it. The body
 * records no memset, and its kernels read every per-step value (tokens, positions, masks) from device memory. */
static void enqueue_body(Decoder *d) {
    if (d->narrow <= 0) return;
    if (!d->graphs) {
        record_body(d);
        return;
    }
    const auto key = std::make_pair(d->narrow, (int)d->split);
    auto it = d->body_graphs.find(key);
    if (it == d->body_graphs.end()) {
        d->body_graphs.emplace(key, nullptr);
        record_body(d);
        return;
    }
    if (!it->second) {
        hipGraph_t g = nullptr;
        HIP_CHECK(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal));
        record_body(d);
        HIP_CHECK(hipStreamEndCapture(d->stream, &g));
        HIP_CHECK(hipGraphInstantiate(&it->second, g, nullptr, nullptr, 0));
        HIP_CHECK(hipGraphDestroy(g));
    }
    HIP_CHECK(hipGraphLaunch(it->second, d->stream));
}

static void enqueue_head(Decoder *d) {
    const int R = d->narrow;
    if (R > 0) {
        const Acts &a = d->slot;
        NormArgs n = norm_args(d, NORM_FINAL, a, R, d->tokens, d->active);
        n.in = a.x;
        n.out = a.hn;
        launch_norm(d->lane[0], n);
        /* the vocabulary's rows are many: the tiled GEMM (128-row tiles up to 128 slots) takes in a tile's slots once
         * per 256 vocabulary rows, where the slot GEMM takes them in per 64 (config 5: 39 against 63 us). It writes
         * every row up to R; choose_kernel reads only the active slots'. Logits past its 2 GiB of 32-bit offsets
         * go through the slot GEMM. */
        if ((long long)R * d->vocab * 4 < (1LL << 31))
            gemm(d->lane[0], d->lm_head, d->vocab, d->C, a.hn, R, d->logits, SG_F32);
        else
            gemm_epi(d, d->lane[0], true, SG_F32, d->lm_head, d->vocab, d->C, a.hn, R, nullptr, d->logits, nullptr,
                     nullptr, d->active);
        ChoiceArgs c = {d->logits, d->probs, d->active, d->allow, d->temperature, d->top_p, d->seed, d->first,
                        d->tokens, d->alt_tokens, d->pos, d->softcap, d->vocab, d->lazy};
        hipLaunchKernelGGL(choose_kernel, dim3(R), dim3(CHOICE_THREADS), 0, d->stream, c);
    }
    HIP_CHECK(hipMemcpyAsync(d->host_tokens, d->tokens, (size_t)d->B * 4, hipMemcpyDeviceToHost, d->stream));
    HIP_CHECK(hipMemcpyAsync(d->host_tokens + d->B, d->alt_tokens, (size_t)d->B * 4, hipMemcpyDeviceToHost, d->stream));
}

/* pool_pages <= 0: a pool of max_pages per slot (every slot can reach max_len; slots as many as fit so);
 * pool_pages > 0: a pool of that many pages, the slots as many (<= max_slots) as fit beside it. */
static Decoder *create(const int *cfg, const uint64_t *ptrs, const float *scal, const int *window, void *stream,
                       int max_slots, long long pool_pages) {
    Decoder *d = new Decoder();
    d->L = cfg[0]; d->C = cfg[1]; d->F = cfg[2]; d->vocab = cfg[3]; d->max_len = cfg[4]; d->store = cfg[5];
    d->lazy = cfg[6];
    REQUIRE(d->L > 0 && d->C > 0 && d->C % HEAD_DIM == 0 && d->C <= MAX_C,
            "C must be a positive multiple of 128, at most 4096");
    REQUIRE(d->F > 0 && d->F % 128 == 0, "F must be a positive multiple of 128");
    REQUIRE(d->vocab > 0 && d->vocab % WORD_BITS == 0, "vocab must be a positive multiple of 32");
    REQUIRE(d->max_len > 0 && d->store >= 0, "max_len must be positive, store non-negative");
    REQUIRE(max_slots > 0 && max_slots <= MAX_BATCH, "slots must be in [1, 1024]");
    d->H = d->C / HEAD_DIM;
    d->max_pages = (d->max_len + PAGE - 1) / PAGE;
    d->wte = (const float *)ptrs[0];
    d->cos = (const float *)ptrs[1];
    d->sin = (const float *)ptrs[2];
    d->lm_head = (const uint16_t *)ptrs[3];
    REQUIRE(d->wte && d->cos && d->sin && d->lm_head, "null embedding, rotary table or lm_head");
    d->softcap = scal[2 * d->L];
    d->stream = (hipStream_t)stream;
    for (int l = 0; l < d->L; l++) {
        const uint64_t *p = ptrs + GLOBAL_PTRS + LAYER_PTRS * l;
        Layer ly = {(const uint16_t *)p[0], (const uint16_t *)p[1], (const uint16_t *)p[2], (const uint16_t *)p[3],
                    (const uint16_t *)p[4], (const float *)p[5], (const float *)p[6], (const float *)p[7],
                    scal[2 * l], scal[2 * l + 1], window[l]};
        REQUIRE(ly.qkv && ly.o && ly.fc && ly.proj && ly.q_gain && ly.k_gain, "null layer weight");
        REQUIRE(!ly.ve == !ly.ve_gate, "a value-embedding table needs its gate, and the gate its table");
        d->layer.push_back(ly);
    }
    /* lane 0 is the caller's stream; lane 1 a stream of the decoder's own (default priority) */
    d->lane[0].stream = d->stream;
    HIP_CHECK(hipStreamCreateWithFlags(&d->lane[1].stream, hipStreamNonBlocking));
    HIP_CHECK(hipEventCreateWithFlags(&d->fork, hipEventDisableTiming));
    HIP_CHECK(hipEventCreateWithFlags(&d->join, hipEventDisableTiming));
    d->attn_done.resize(2 * d->L);
    for (hipEvent_t &e : d->attn_done) HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));

    /* fixed blocks first (prefill rows, masks, the store's pages and, with pool_pages, the pool), then the slots: B,
     * the most slots (<= max_slots) whose activations, choice buffers and (without pool_pages) max_len worth of KV
     * pages fit the free memory less a reserve */
    const size_t store_pages = ((size_t)d->store + PAGE - 1) / PAGE;
    const size_t page_set = (size_t)d->H * (2 * PAGE_BYTES + 2 * PAGE * sizeof(float));  /* a page of every head */
    REQUIRE(pool_pages <= 0 || pool_pages >= d->max_pages, "a pool must hold at least one max_len sequence");
    const size_t per_slot = (pool_pages > 0 ? 0 : (size_t)d->L * d->max_pages * page_set) + acts_bytes(d, 1) +
                            (size_t)d->vocab * 8 + (size_t)d->vocab / 8 + (size_t)d->max_pages * 4 + 64 +
                            (size_t)d->H * (HEAD_DIM + 2) * 4 + (size_t)d->H * 8;
    d->row = carve_acts(d, PREFILL_ROWS);
    d->rows = (int32_t *)device_alloc(d, 7 * PREFILL_ROWS * sizeof(int32_t));
    d->active = (unsigned long long *)device_alloc(d, 2 * MASK_WORDS * sizeof(unsigned long long));
    size_t free_bytes = 0, total_bytes = 0;
    HIP_CHECK(hipStreamSynchronize(d->stream));
    HIP_CHECK(hipMemGetInfo(&free_bytes, &total_bytes));
    const size_t fixed = (size_t)d->L * (store_pages + (pool_pages > 0 ? (size_t)pool_pages : 0)) * page_set +
                         (size_t)4096 * d->H * (HEAD_DIM + 2) * 4;
    const size_t reserve = (size_t)2 << 30 > total_bytes / 64 ? (size_t)2 << 30 : total_bytes / 64;
    REQUIRE(free_bytes > fixed + reserve + per_slot, "no slot fits in free device memory");
    const size_t fit = (free_bytes - fixed - reserve) / per_slot;
    d->B = (int)(fit < (size_t)max_slots ? fit : (size_t)max_slots);

    d->pool = pool_pages > 0 ? pool_pages : (long long)d->B * d->max_pages;
    d->layer_pages = d->pool + (long long)store_pages;
    REQUIRE(d->layer_pages < (1LL << 31), "a layer's pool exceeds 2^31 pages");
    d->k_pages = (uint8_t *)device_alloc(d, (size_t)d->L * d->layer_pages * d->H * PAGE_BYTES);
    d->v_pages = (uint8_t *)device_alloc(d, (size_t)d->L * d->layer_pages * d->H * PAGE_BYTES);
    d->kv_scale = (float *)device_alloc(d, (size_t)d->L * d->layer_pages * d->H * 2 * PAGE * sizeof(float));
    const long long entries = (long long)d->B * d->max_pages;
    REQUIRE(entries < (1LL << 31), "the block table exceeds 2^31 entries");
    d->block_table = (int32_t *)device_alloc(d, (size_t)entries * sizeof(int32_t));
    hipLaunchKernelGGL(set_table_kernel, dim3((unsigned)((entries + 255) / 256)), dim3(256), 0, d->stream,
                       d->block_table, 0LL, entries, -1, 0);
    d->table.assign(entries, -1);
    d->dirty.assign(d->B, int2{0, 0});
    d->free_pages.resize(d->pool);
    for (long long i = 0; i < d->pool; i++) d->free_pages[i] = (int32_t)(d->pool - 1 - i);   /* page 0 on top */
    d->hpos.assign(d->B, 0);
    d->live.assign(MASK_WORDS, 0);
    const size_t B = d->B;
    int32_t *state = (int32_t *)device_alloc(d, B * 6 * sizeof(int32_t));
    d->tokens = state; d->alt_tokens = state + B; d->pos = state + 2 * B; d->first = state + 3 * B;
    d->seq_lens = state + 4 * B; d->num_new = state + 5 * B;
    d->temperature = (float *)device_alloc(d, B * sizeof(float));
    d->top_p = (float *)device_alloc(d, B * sizeof(float));
    d->seed = (unsigned long long *)device_alloc(d, B * sizeof(unsigned long long));
    d->allow = (uint32_t *)device_alloc(d, B * (d->vocab / WORD_BITS) * sizeof(uint32_t));
    d->logits = (float *)device_alloc(d, B * d->vocab * sizeof(float));
    d->probs = (float *)device_alloc(d, B * d->vocab * sizeof(float));
    d->slot = carve_acts(d, B);
    /* measured at config 5 (128 slots, 26 layers): one lane eager 6.12 ms a step, one lane with graphs 6.2-6.3 ms,
     * two lanes with graphs 6.6 ms: attention fills every CU, so the other lane's GEMMs cannot run beside it, and
     * the host stays ahead of a 6 ms step. Both stay available (dec_debug_set_split / dec_debug_set_graphs). */
    d->split = false;
    d->graphs = false;
    long long part_bytes = 0;
    const int C = d->C, F = d->F;
    const int shapes[5][2] = {{3 * C, C}, {C, C}, {F, C}, {C, F}, {d->vocab, C}};
    for (const auto &rk : shapes) {
        REQUIRE(slot_gemm_fits(rk[0], rk[1], SG_MAX_N), "a step GEMM shape the slot GEMM does not take");
        const long long bytes = slot_gemm_part_bytes(rk[0], SG_MAX_N, slot_gemm_slices(rk[0], rk[1]));
        part_bytes = bytes > part_bytes ? bytes : part_bytes;
    }
    REQUIRE(slot_gemm_slices(C, F) <= PN_MAX_S, "the FFN width (proj_norm adds at most 8 K-slices)");
    /* the step's proj GEMM always leaves its sums as partials (proj_norm), one slice or more */
    const long long proj_bytes = (long long)slot_gemm_slices(C, F) * SG_MAX_N * C * 4;
    part_bytes = proj_bytes > part_bytes ? proj_bytes : part_bytes;
    d->part_bytes = part_bytes;
    d->attn_ws_bytes = nc_decode_workspace_bytes(d->B, d->H, d->H, d->max_len, -1);
    REQUIRE(d->attn_ws_bytes > 0, "decode attention workspace");
    for (Lane &ln : d->lane) {
        ln.part = (float *)device_alloc(d, (size_t)part_bytes);
        ln.ssq = (float *)device_alloc(d, (size_t)B * ((C + 15) / 16) * sizeof(float));
        ln.attn_ws = device_alloc(d, d->attn_ws_bytes);
    }
    HIP_CHECK(hipHostMalloc((void **)&d->staging, 7 * PREFILL_ROWS * sizeof(int32_t), hipHostMallocDefault));
    HIP_CHECK(hipHostMalloc((void **)&d->host_tokens, 2 * B * sizeof(int32_t), hipHostMallocDefault));
    HIP_CHECK(hipHostMalloc((void **)&d->host_allow, B * (d->vocab / WORD_BITS) * sizeof(uint32_t),
                            hipHostMallocDefault));
    memset(d->host_tokens, 0, 2 * B * sizeof(int32_t));
    memset(d->host_allow, 0, B * (d->vocab / WORD_BITS) * sizeof(uint32_t));
    HIP_CHECK(hipEventCreateWithFlags(&d->staged, hipEventDisableTiming));
    HIP_CHECK(hipEventRecord(d->staged, d->stream));
    HIP_CHECK(hipStreamSynchronize(d->stream));
    d->narrow = 0;
    return d;
}

/* ---------------------------------------------------------------- pages: the pool and the prompt store
 *
 * A slot's block-table row maps its logical pages to pool pages taken on demand (own_pages) and returned when the
 * slot's sequence is dropped (release_pages); entries of positions the slot has not written are -1 (never read: a
 * pass reads only pages below its sequence's length). dec_load_prompt points a slot's entries at the store's pages
 * wherever the two ranges share their page phase ((store_at - at) % 16 == 0) and a page lies wholly inside the range:
 * the prompt's K and V are then read in place, with no copy (the reference copies the store into the slot,
 * decode.cu:1055-1075). Partial pages are copied. Nothing ever writes a shared page: before any write into a slot (a
 * prefill row, a live slot's step at its host-tracked position, a partial copy) the entry gets a pool page of the
 * slot's own, with the store page's content copied there (copy on write); before dec_save_prompt writes store pages,
 * every slot sharing them gets its own copy. Work is stream-ordered, so a page returned to the pool is reused only by
 * work enqueued after every earlier reader. */

static bool store_page(const Decoder *d, int32_t page) { return page >= d->pool; }

static int32_t *table_row(Decoder *d, int b) { return d->table.data() + (size_t)b * d->max_pages; }

/* Slot b's host entries [e0, e1) have changed: queued for the device table's next flush_table. */
static void upload_table(Decoder *d, int b, int e0, int e1) {
    if (e0 >= e1) return;
    int2 &r = d->dirty[b];
    if (r.x >= r.y) {
        d->dirty_slots.push_back(b);
        r = int2{e0, e1};
    } else {
        r = int2{e0 < r.x ? e0 : r.x, e1 > r.y ? e1 : r.y};
    }
}

/* The queued entries to the device table, each slot's changed range as runs of consecutive pages or of -1, up to
 * TABLE_RUNS runs a launch (a prefill call changes a page of every 16 rows: 512 entries in a few launches rather than
 * one each). Called before any launch that reads the table and at the end of each entry point that changes it. */
static void flush_table(Decoder *d) {
    TableRuns t;
    t.n = 0;
    auto launch = [&]() {
        hipLaunchKernelGGL(set_table_runs_kernel, dim3((unsigned)t.n), dim3(256), 0, d->stream, d->block_table, t);
        t.n = 0;
    };
    for (int b : d->dirty_slots) {
        const int32_t *row = table_row(d, b);
        const int e1 = d->dirty[b].y;
        for (int e = d->dirty[b].x; e < e1;) {
            const int step = row[e] < 0 ? 0 : 1;
            int f = e + 1;
            while (f < e1 && row[f] == row[f - 1] + step && (row[f] < 0) == (row[e] < 0)) f++;
            t.run[t.n++] = TableRun{(int32_t)((long long)b * d->max_pages + e), f - e, row[e], step};
            if (t.n == TABLE_RUNS) launch();
            e = f;
        }
        d->dirty[b] = int2{0, 0};
    }
    d->dirty_slots.clear();
    if (t.n) launch();
    HIP_CHECK(hipGetLastError());
}

static int32_t take_page(Decoder *d) {
    if (d->free_pages.empty())
        die("KV page pool", "no free page left (admit fewer or shorter sequences, or give dec_create_pool more)",
            __LINE__);
    const int32_t p = d->free_pages.back();
    d->free_pages.pop_back();
    return p;
}

/* Slot b's entries [e0, e1) become pages of its own: -1 takes a pool page; a shared store page takes one too, and with
 * keep the store page is first copied there, so the positions the slot does not rewrite keep their values. */
static void own_pages(Decoder *d, int b, int e0, int e1, bool keep) {
    int32_t *row = table_row(d, b);
    int lo = e1, hi = e0;
    for (int e = e0; e < e1; e++) {
        if (row[e] >= 0 && !store_page(d, row[e])) continue;
        const int32_t page = take_page(d);
        if (row[e] >= 0 && keep) {
            hipLaunchKernelGGL(copy_pages_kernel, dim3((unsigned)d->H, (unsigned)d->L, 1u), dim3(256), 0, d->stream,
                               d->k_pages, d->v_pages, d->kv_scale, d->layer_pages, d->H, (long long)row[e],
                               (long long)page);
            HIP_CHECK(hipGetLastError());
        }
        row[e] = page;
        lo = e < lo ? e : lo;
        hi = e + 1 > hi ? e + 1 : hi;
    }
    if (lo < hi) upload_table(d, b, lo, hi);
}

/* Slot b's entries from e0 on drop their pages: its own return to the pool, shared store pages are only unlinked. */
static void release_pages(Decoder *d, int b, int e0) {
    int32_t *row = table_row(d, b);
    int lo = d->max_pages, hi = e0;
    for (int e = e0 < 0 ? 0 : e0; e < d->max_pages; e++) {
        if (row[e] < 0) continue;
        if (!store_page(d, row[e])) d->free_pages.push_back(row[e]);
        row[e] = -1;
        lo = e < lo ? e : lo;
        hi = e + 1;
    }
    if (lo < hi) upload_table(d, b, lo, hi);
}

/* Positions [at, at + n) of slot b (through its block table) <-> store positions [store_at, store_at + n). The slot's
 * entries of those positions hold pages (the callers' checks). */
static void copy_positions(Decoder *d, int b, int at, int store_at, int n, bool to_store) {
    if (n <= 0) return;
    flush_table(d);   /* the kernel finds the slot's pages through the device table */
    const int32_t *tab = d->block_table + (size_t)b * d->max_pages;
    const long long units = (long long)n * d->L * d->H;
    hipLaunchKernelGGL(copy_positions_kernel, dim3((unsigned)((units + 3) / 4)), dim3(256), 0, d->stream, d->k_pages,
                       d->v_pages, d->kv_scale, d->layer_pages, d->H, d->L, to_store ? tab : nullptr, d->pool,
                       to_store ? at : store_at, to_store ? nullptr : tab, d->pool, to_store ? store_at : at, n);
    HIP_CHECK(hipGetLastError());
}

static void check_prompt_range(const Decoder *d, int b, int at, int store_at, int n) {
    if (b < 0 || b >= d->B || at < 0 || n < 0 || at + n > d->max_len || store_at < 0 || store_at + n > d->store)
        die("dec_save_prompt/dec_load_prompt", "slot or position range out of bounds", __LINE__);
}

static void save_prompt(Decoder *d, int b, int at, int store_at, int n) {
    check_prompt_range(d, b, at, store_at, n);
    if (n == 0) return;
    const int32_t *src = table_row(d, b);
    for (int e = at / PAGE; e <= (at + n - 1) / PAGE; e++)
        if (src[e] < 0) die("dec_save_prompt", "a position the slot has not cached", __LINE__);
    /* slots sharing the store pages about to change keep their own copies */
    const int32_t p0 = (int32_t)(d->pool + store_at / PAGE), p1 = (int32_t)(d->pool + (store_at + n - 1) / PAGE);
    for (int s = 0; s < d->B; s++) {
        const int32_t *row = table_row(d, s);
        for (int e = 0; e < d->max_pages; e++)
            if (row[e] >= p0 && row[e] <= p1) own_pages(d, s, e, e + 1, true);
    }
    copy_positions(d, b, at, store_at, n, true);
}

/* A load at position 0 starts the slot's sequence anew: its pages are released first. */
static void load_prompt(Decoder *d, int b, int at, int store_at, int n) {
    check_prompt_range(d, b, at, store_at, n);
    if (n == 0) return;
    if (at == 0) release_pages(d, b, 0);
    const int e_lo = (at + PAGE - 1) / PAGE, e_hi = (at + n) / PAGE;   /* pages wholly inside [at, at + n) */
    if ((store_at - at) % PAGE != 0 || e_lo >= e_hi) {
        own_pages(d, b, at / PAGE, (at + n - 1) / PAGE + 1, true);
        copy_positions(d, b, at, store_at, n, false);
        return;
    }
    if (at % PAGE) {   /* the leading partial page */
        own_pages(d, b, at / PAGE, at / PAGE + 1, true);
        copy_positions(d, b, at, store_at, e_lo * PAGE - at, false);
    }
    if ((at + n) % PAGE) {   /* the trailing partial page */
        own_pages(d, b, e_hi, e_hi + 1, true);
        copy_positions(d, b, e_hi * PAGE, store_at + (e_hi * PAGE - at), at + n - e_hi * PAGE, false);
    }
    int32_t *row = table_row(d, b);
    const long long shift = d->pool + (store_at - at) / PAGE;
    for (int e = e_lo; e < e_hi; e++) {
        if (row[e] >= 0 && !store_page(d, row[e])) d->free_pages.push_back(row[e]);
        row[e] = (int32_t)(shift + e);
    }
    upload_table(d, b, e_lo, e_hi);
}

static void prefill(Decoder *d, int n, const int32_t *rows) {
    if (n <= 0) return;
    if (n > PREFILL_ROWS) die("dec_prefill", "more rows than dec_prefill_rows", __LINE__);
    const int32_t *tok = rows, *pos = rows + n, *slot = rows + 2 * n;
    for (int r = 0; r < n; r++)
        if (slot[r] < 0 || slot[r] >= d->B || pos[r] < 0 || pos[r] >= d->max_len || tok[r] < 0 || tok[r] >= d->vocab)
            die("dec_prefill", "row with a slot, position or token out of range", __LINE__);
    /* a row at position 0 starts its slot's sequence anew (its pages are released); every row's page is the slot's
     * own before the rows are written */
    for (int r = 0; r < n; r++)
        if (pos[r] == 0) release_pages(d, slot[r], 0);
    for (int r = 0; r < n; r++) own_pages(d, slot[r], pos[r] / PAGE, pos[r] / PAGE + 1, true);
    flush_table(d);
    HIP_CHECK(hipEventSynchronize(d->staged));  /* the previous upload has been read */
    int32_t *s = d->staging;
    memcpy(s, tok, n * sizeof(int32_t));
    memcpy(s + PREFILL_ROWS, pos, n * sizeof(int32_t));
    memcpy(s + 2 * PREFILL_ROWS, slot, n * sizeof(int32_t));
    /* runs: maximal stretches of rows of one slot at consecutive positions */
    int32_t *row0 = s + 3 * PREFILL_ROWS, *count = s + 4 * PREFILL_ROWS, *rslot = s + 5 * PREFILL_ROWS,
            *start = s + 6 * PREFILL_ROWS;
    int runs = 0, max_count = 0;
    for (int r = 0; r < n; r++) {
        if (r == 0 || slot[r] != slot[r - 1] || pos[r] != pos[r - 1] + 1) {
            row0[runs] = r;
            count[runs] = 0;
            rslot[runs] = slot[r];
            start[runs] = pos[r];
            runs++;
        }
        count[runs - 1]++;
        if (count[runs - 1] > max_count) max_count = count[runs - 1];
    }
    HIP_CHECK(hipMemcpyAsync(d->rows, s, 7 * PREFILL_ROWS * sizeof(int32_t), hipMemcpyHostToDevice, d->stream));
    HIP_CHECK(hipEventRecord(d->staged, d->stream));
    int32_t *dtok = d->rows;
    const int32_t *drow0 = d->rows + 3 * PREFILL_ROWS, *dcount = d->rows + 4 * PREFILL_ROWS,
                  *drslot = d->rows + 5 * PREFILL_ROWS, *dstart = d->rows + 6 * PREFILL_ROWS;
    const int C = d->C;
    const Acts &a = d->row;
    const Lane &ln = d->lane[0];
    launch_norm(ln, norm_args(d, NORM_EMBED, a, n, dtok, nullptr));
    for (int l = 0; l < d->L; l++) {
        const Layer &ly = d->layer[l];
        NormArgs r = norm_args(d, NORM_RESID, a, n, dtok, nullptr);
        r.in = l == 0 ? nullptr : a.x;
        r.l1 = ly.resid;
        r.l2 = ly.x0;
        r.mixed = a.xm;
        r.out = a.h;
        launch_norm(ln, r);
        gemm(ln, ly.qkv, 3 * C, C, a.h, n, a.qkv, SG_STORE);
        NC_CHECK(append_runs(a.qkv, 3LL * C, runs, max_count, drow0, dcount, dstart, drslot, d->H, d->H, ly.q_gain,
                             ly.k_gain, d->cos, d->sin, d->max_len, a.q, d->block_table, d->max_pages, layer_k(d, l),
                             layer_v(d, l), layer_s(d, l), (int)d->layer_pages, a.h, ly.ve, ly.ve_gate, dtok, C,
                             d->stream));
        if (l == d->L - 1) break;  /* no row chooses a token: the last layer only caches its K and V */
        NC_CHECK(prefill_runs(a.q, layer_k(d, l), layer_v(d, l), layer_s(d, l), d->block_table, d->max_pages,
                              (int)d->layer_pages, dstart, drow0, dcount, drslot, runs, max_count, d->H, d->H, ly.window,
                              SM_SCALE, a.att, d->stream));
        mlp(d, ln, false, ly, nullptr, a, n, nullptr);
    }
}

static void destroy(Decoder *d) {
    hipStreamSynchronize(d->stream);
    for (void *p : d->device_blocks) hipFree(p);
    hipHostFree(d->staging);
    hipHostFree(d->host_tokens);
    hipHostFree(d->host_allow);
    hipEventDestroy(d->staged);
    hipStreamSynchronize(d->lane[1].stream);
    for (auto &kv : d->body_graphs)
        if (kv.second) hipGraphExecDestroy(kv.second);
    hipStreamDestroy(d->lane[1].stream);
    hipEventDestroy(d->fork);
    hipEventDestroy(d->join);
    for (hipEvent_t e : d->attn_done) hipEventDestroy(e);
    delete d;
}

}  // namespace dec
}  // namespace nc

using nc::dec::Decoder;

extern "C" void *dec_create_slots(const int *cfg, const uint64_t *ptrs, const float *scal, const int *window,
                                  void *stream, int max_slots) {
    return nc::dec::create(cfg, ptrs, scal, window, stream, max_slots, 0);
}

extern "C" void *dec_create_pool(const int *cfg, const uint64_t *ptrs, const float *scal, const int *window,
                                 void *stream, int max_slots, long long pool_pages) {
    if (pool_pages <= 0) nc::dec::die("dec_create_pool", "the pool needs at least one page", __LINE__);
    return nc::dec::create(cfg, ptrs, scal, window, stream, max_slots, pool_pages);
}

extern "C" void dec_release(void *handle, int b) {
    Decoder *d = (Decoder *)handle;
    if (b < 0 || b >= d->B) nc::dec::die("dec_release", "slot out of range", __LINE__);
    nc::dec::release_pages(d, b, 0);
    nc::dec::flush_table(d);
}

extern "C" void dec_debug_pages(void *handle, long long *out) {
    const Decoder *d = (const Decoder *)handle;
    out[0] = (long long)d->free_pages.size();
    out[1] = d->pool;
}

extern "C" void *dec_create(const int *cfg, const uint64_t *ptrs, const float *scal, const int *window, void *stream) {
    return nc::dec::create(cfg, ptrs, scal, window, stream, nc::dec::MAX_BATCH, 0);
}

extern "C" int dec_batch(void *handle) { return ((Decoder *)handle)->B; }

extern "C" void dec_set_prompt(void *handle, int b, int32_t token, int32_t last, float temperature, float top_p,
                               unsigned long long seed) {
    Decoder *d = (Decoder *)handle;
    if (b < 0 || b >= d->B || token < 0 || token >= d->vocab || last < 0 || last >= d->max_len)
        nc::dec::die("dec_set_prompt", "slot, token or position out of range", __LINE__);
    hipLaunchKernelGGL(nc::dec::set_slot_kernel, dim3(1), dim3(1), 0, d->stream, d->tokens, d->pos, d->first,
                       d->temperature, d->top_p, d->seed, b, token, last, temperature, top_p, seed);
    HIP_CHECK(hipGetLastError());
    d->hpos[b] = last;
    nc::dec::release_pages(d, b, last / nc::PAGE + 1);   /* pages past the slot's position hold an older sequence */
    nc::dec::flush_table(d);
}

extern "C" int dec_prefill_rows(void *) { return nc::dec::PREFILL_ROWS; }

extern "C" void dec_prefill(void *handle, int n, const int32_t *rows) { nc::dec::prefill((Decoder *)handle, n, rows); }

extern "C" void dec_save_prompt(void *handle, int b, int at, int store_at, int n) {
    nc::dec::save_prompt((Decoder *)handle, b, at, store_at, n);
    nc::dec::flush_table((Decoder *)handle);
}

extern "C" void dec_load_prompt(void *handle, int b, int at, int store_at, int n) {
    nc::dec::load_prompt((Decoder *)handle, b, at, store_at, n);
    nc::dec::flush_table((Decoder *)handle);
}

extern "C" uint32_t *dec_masks(void *handle) { return ((Decoder *)handle)->host_allow; }

extern "C" void dec_set_active(void *handle, const unsigned long long *slots) {
    using namespace nc::dec;
    Decoder *d = (Decoder *)handle;
    const int words = (d->B + MASK_BITS - 1) / MASK_BITS;
    SlotMasks m = {};
    int high = -1, lo = -1, hi = -1;
    for (int w = 0; w < words; w++) {
        m.w[w] = slots[w];
        m.w[MASK_WORDS + w] = slots[words + w];
        if (slots[w]) high = w * MASK_BITS + MASK_BITS - 1 - __builtin_clzll(slots[w]);
        if (slots[words + w]) {
            if (lo < 0) lo = w * MASK_BITS + __builtin_ctzll(slots[words + w]);
            hi = w * MASK_BITS + MASK_BITS - 1 - __builtin_clzll(slots[words + w]);
        }
    }
    if (high >= d->B) die("dec_set_active", "active slot beyond dec_batch", __LINE__);
    if (hi >= d->B) die("dec_set_active", "masked slot beyond dec_batch", __LINE__);
    hipLaunchKernelGGL(set_active_kernel, dim3(1), dim3(64), 0, d->stream, d->active, m);
    HIP_CHECK(hipGetLastError());
    d->narrow = high + 1;
    for (int w = 0; w < MASK_WORDS; w++) d->live[w] = w < words ? slots[w] : 0;
    if (lo >= 0) {
        const size_t n = d->vocab / WORD_BITS;
        HIP_CHECK(hipMemcpyAsync(d->allow + lo * n, d->host_allow + lo * n, (hi + 1 - lo) * n * sizeof(uint32_t),
                                 hipMemcpyHostToDevice, d->stream));
    }
}

extern "C" void dec_launch_body(void *handle) {
    Decoder *d = (Decoder *)handle;
    /* the step writes each live slot's K and V at its position: that page must be the slot's own */
    for (int b = 0; b < d->B; b++)
        if (((d->live[b / nc::dec::MASK_BITS] >> (b % nc::dec::MASK_BITS)) & 1ull) && d->hpos[b] < d->max_len)
            nc::dec::own_pages(d, b, d->hpos[b] / nc::PAGE, d->hpos[b] / nc::PAGE + 1, true);
    nc::dec::flush_table(d);
    nc::dec::enqueue_body(d);
    HIP_CHECK(hipGetLastError());
}

extern "C" void dec_launch_head(void *handle) {
    Decoder *d = (Decoder *)handle;
    nc::dec::enqueue_head(d);
    HIP_CHECK(hipGetLastError());
    for (int b = 0; b < d->B; b++)   /* choose_kernel's commit: pos += 1 for live slots */
        if ((d->live[b / nc::dec::MASK_BITS] >> (b % nc::dec::MASK_BITS)) & 1ull) d->hpos[b]++;
}

extern "C" void dec_tokens(void *handle, int32_t *out) {
    Decoder *d = (Decoder *)handle;
    HIP_CHECK(hipStreamSynchronize(d->stream));
    memcpy(out, d->host_tokens, 2 * (size_t)d->B * sizeof(int32_t));
}

extern "C" void dec_take_alt(void *handle, int b) {
    Decoder *d = (Decoder *)handle;
    if (b < 0 || b >= d->B) nc::dec::die("dec_take_alt", "slot out of range", __LINE__);
    hipLaunchKernelGGL(nc::dec::take_alt_kernel, dim3(1), dim3(1), 0, d->stream, d->tokens, d->alt_tokens, b);
    HIP_CHECK(hipGetLastError());
}

extern "C" void dec_destroy(void *handle) { nc::dec::destroy((Decoder *)handle); }

extern "C" void dec_debug_logits(void *handle, float *out, int rows) {
    Decoder *d = (Decoder *)handle;
    if (rows < 0 || rows > d->B) nc::dec::die("dec_debug_logits", "rows out of range", __LINE__);
    HIP_CHECK(hipStreamSynchronize(d->stream));
    HIP_CHECK(hipMemcpy(out, d->logits, (size_t)rows * d->vocab * sizeof(float), hipMemcpyDeviceToHost));
}

extern "C" void dec_debug_cache(void *handle, int layer, int b, int at, int n, uint8_t *k, uint8_t *v, float *scales) {
    using namespace nc;
    Decoder *d = (Decoder *)handle;
    const int limit = b < 0 ? d->store : d->max_len;
    if (layer < 0 || layer >= d->L || b >= d->B || at < 0 || n < 0 || at + n > limit)
        dec::die("dec_debug_cache", "layer, slot or position range out of bounds", __LINE__);
    if (n == 0) return;
    HIP_CHECK(hipStreamSynchronize(d->stream));
    const int first = at / PAGE, last = (at + n - 1) / PAGE, pages = last - first + 1, H = d->H;
    std::vector<uint8_t> kp((size_t)pages * H * PAGE_BYTES), vp(kp.size());
    std::vector<float> sp((size_t)pages * H * 2 * PAGE);
    for (int pg = 0; pg < pages; pg++) {   /* a slot's pages through its block table, the store's in order */
        const long long page = b < 0 ? d->pool + first + pg : d->table[(size_t)b * d->max_pages + first + pg];
        const size_t at_h = (size_t)pg * H;
        if (page < 0) {   /* a page the slot has not written: zeros */
            memset(kp.data() + at_h * PAGE_BYTES, 0, (size_t)H * PAGE_BYTES);
            memset(vp.data() + at_h * PAGE_BYTES, 0, (size_t)H * PAGE_BYTES);
            memset(sp.data() + at_h * 2 * PAGE, 0, (size_t)H * 2 * PAGE * sizeof(float));
            continue;
        }
        const size_t base = (size_t)(d->layer_pages * layer + page) * H;
        HIP_CHECK(hipMemcpy(kp.data() + at_h * PAGE_BYTES, d->k_pages + base * PAGE_BYTES, (size_t)H * PAGE_BYTES,
                            hipMemcpyDeviceToHost));
        HIP_CHECK(hipMemcpy(vp.data() + at_h * PAGE_BYTES, d->v_pages + base * PAGE_BYTES, (size_t)H * PAGE_BYTES,
                            hipMemcpyDeviceToHost));
        HIP_CHECK(hipMemcpy(sp.data() + at_h * 2 * PAGE, d->kv_scale + base * 2 * PAGE, (size_t)H * 2 * PAGE * sizeof(float),
                            hipMemcpyDeviceToHost));
    }
    for (int i = 0; i < n; i++) {
        const int p = at + i, pg = p / PAGE - first, slot = p % PAGE;
        for (int h = 0; h < H; h++) {
            const size_t unit = (size_t)pg * H + h;
            for (int dim = 0; dim < HEAD_DIM; dim++) {
                k[((size_t)i * H + h) * HEAD_DIM + dim] = kp[unit * PAGE_BYTES + k_page_offset(slot, dim)];
                v[((size_t)i * H + h) * HEAD_DIM + dim] = vp[unit * PAGE_BYTES + v_page_offset(slot, dim)];
            }
            scales[((size_t)i * H + h) * 2] = sp[(unit * 2) * PAGE + slot];
            scales[((size_t)i * H + h) * 2 + 1] = sp[(unit * 2 + 1) * PAGE + slot];
        }
    }
}

/* Slot b's block-table row (max_pages entries, host copy): entry e is b * max_pages + e (the slot's own page) or
 * B * max_pages + i (page i of the prompt store, shared after dec_load_prompt). */
extern "C" void dec_debug_table(void *handle, int b, int32_t *out) {
    Decoder *d = (Decoder *)handle;
    if (b < 0 || b >= d->B) nc::dec::die("dec_debug_table", "slot out of range", __LINE__);
    memcpy(out, d->table.data() + (size_t)b * d->max_pages, (size_t)d->max_pages * sizeof(int32_t));
}

extern "C" void dec_debug_set_split(void *handle, int on) {
    Decoder *d = (Decoder *)handle;
    HIP_CHECK(hipStreamSynchronize(d->stream));
    d->split = on != 0;
}

extern "C" void dec_debug_set_graphs(void *handle, int on) {
    Decoder *d = (Decoder *)handle;
    HIP_CHECK(hipStreamSynchronize(d->stream));
    d->graphs = on != 0;
}

extern "C" int dec_debug_slot_gemm(int epi, const void *w, int R, int K, const void *x, int N, void *out,
                                   float *out_f32, const void *res, const float *rstd, int slices, float *part,
                                   void *stream) {
    nc::SkinnyGemm g = {(const uint16_t *)w, (const uint16_t *)x, R, K, N, (uint16_t *)out, out_f32,
                        (const uint16_t *)res, rstd, nullptr, nullptr};
    if (!nc::slot_gemm_fits(R, K, N)) return -2;
    const int S = slices > 0 ? slices : nc::slot_gemm_slices(R, K);
    const long long part_bytes = nc::slot_gemm_part_bytes(R, N, S);   /* the caller allocates this much */
    const int e = nc::slot_gemm(g, epi, part, part_bytes, S, (hipStream_t)stream);
    if (e != 0 || S == 1) return e;
    return nc::slot_gemm_reduce(g, epi, part, part_bytes, S, (hipStream_t)stream);
}

extern "C" int dec_debug_slot_gemm_slices(int R, int K) { return nc::slot_gemm_slices(R, K); }

extern "C" long long dec_debug_slot_gemm_part_bytes(int R, int N, int slices) {
    return nc::slot_gemm_part_bytes(R, N, slices);
}

extern "C" int dec_debug_slot_gemm_ssq(int epi, const void *w, int R, int K, const void *x, int N, void *out,
                                       const void *res, float *ssq, void *stream) {
    if (!ssq || (epi != nc::SG_RESID2 && epi != nc::SG_RELU2)) return -2;
    nc::SkinnyGemm g = {(const uint16_t *)w, (const uint16_t *)x, R, K, N, (uint16_t *)out, nullptr,
                        (const uint16_t *)res, nullptr, nullptr, ssq};
    return nc::slot_gemm(g, epi, nullptr, 0, 1, (hipStream_t)stream);
}

extern "C" int dec_debug_slot_gemm_tile(int R, int K, int N, int slices) {
    if (!nc::slot_gemm_fits(R, K, N)) return -2;
    const int S = slices > 0 ? slices : nc::slot_gemm_slices(R, K);
    if (S > K / 128) return -2;
    return nc::slot_gemm_tile(R, K, N, S);
}

extern "C" int dec_debug_nucleus_cut(const float *e, int rows, int vocab, const float *top_p, uint32_t *cut,
                                     void *stream) {
    if (rows < 0 || vocab <= 0 || vocab >= (1 << 25) || !e || !top_p || !cut) return -2;
    if (rows == 0) return 0;
    hipLaunchKernelGGL(nc::dec::nucleus_cut_kernel, dim3(rows), dim3(nc::dec::CHOICE_THREADS), 0,
                       (hipStream_t)stream, e, vocab, top_p, cut);
    return (int)hipGetLastError();
}

extern "C" int dec_debug_append_runs(const void *qkv, long long token_stride, int runs, int max_count,
                                     const int32_t *row0, const int32_t *count, const int32_t *start,
                                     const int32_t *seq_slot, int Hq, int Hkv, const float *q_gain, const float *k_gain,
                                     const float *cos, const float *sin, int rope_len, void *q_out,
                                     const int32_t *block_table, int max_pages, void *k_pages, void *v_pages,
                                     float *kv_scale, int num_pages, const void *ve_h, const void *ve,
                                     const float *ve_gate, const int32_t *tokens, int C, void *stream) {
    if (!qkv || !row0 || !count || !start || !seq_slot || !q_gain || !k_gain || !cos || !sin || !q_out ||
        !block_table || !k_pages || !v_pages || !kv_scale || runs < 0 || max_count < 0 || Hq <= 0 || Hkv <= 0 ||
        Hq % Hkv || rope_len <= 0 || max_pages <= 0 || num_pages <= 0 ||
        token_stride < (long long)(Hq + 2 * Hkv) * HEAD_DIM)
        return -2;
    if (ve && (!ve_h || !ve_gate || !tokens || C < Hkv * HEAD_DIM)) return -2;
    return nc::append_runs((const uint16_t *)qkv, token_stride, runs, max_count, row0, count, start, seq_slot, Hq, Hkv,
                           q_gain, k_gain, cos, sin, rope_len, (uint16_t *)q_out, block_table, max_pages,
                           (uint8_t *)k_pages, (uint8_t *)v_pages, kv_scale, num_pages, (const uint16_t *)ve_h,
                           (const uint16_t *)ve, ve_gate, tokens, C, (hipStream_t)stream);
}

extern "C" int dec_debug_prefill_gemm(int epi, const void *w, int N, int K, const void *a, int M, void *out,
                                      float *out_f32, const void *res, const float *rstd, void *stream) {
    nc::PfGemm g = {(const uint16_t *)a, (const uint16_t *)w, M, N, K, (uint16_t *)out, out_f32, (const uint16_t *)res,
                    rstd};
    return nc::prefill_gemm(g, epi, (hipStream_t)stream);
}
