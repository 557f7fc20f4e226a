/*
 * Training attention for gfx950: the varlen causal (optionally windowed) attention forward that the reference runs
 * through FlashAttention-4 (model/ops/flash_attn.py:325-347: _flash_attn_fwd over cu_seqlens with causal=True,
 * window_size_left = window, return_lse=True; window semantics fa4_window_left, flash_attn.py:309-311).
 *
 * Per segment s (tokens cu[s] .. cu[s+1]-1) and head h, row i attends keys j with j <= i and i - j <= window
 * (window < 0: no left limit):
 *   out[i] = sum_j softmax_j(scale q_i . k_j) v_j          bf16, fp32 accumulation
 *   lse[h][i] = ln sum_j exp(scale q_i . k_j)              fp32 (FA4's (H, total) layout)
 *
 * Mapping: a workgroup of four waves owns 128 query rows of one (segment, head), each wave two 16-row tiles. Keys
 * are visited in blocks of 64, staged in LDS for the four waves (K and V row-major with 16-byte chunks XOR-swizzled
 * by the key) by LDS DMA straight from HBM, in two LDS stages: block b+1 is fetched into one while block b is read
 * from the other, with no registers held for the fetch. Scores are S^T = K Q^T (v_mfma_f32_16x16x32_bf16, keys as
 * rows, queries as columns), so a lane's scores all belong to one query; the online softmax runs in the log2 domain
 * with the lazy rescale of the decode kernels (the reference max moves only when a column's max passes it by 2^8);
 * P^T then feeds O^T += V^T P^T with no shuffle: the V^T operand is read from the row-major tile by gfx950's
 * transposing LDS read (ds_read_b64_tr_b16) in P's key order. The backward stages its Q, dO (or K, V) tiles the
 * same way and reads their transposes the same way.
 */
#include "nc_device.h"
#include "nanochat_amd.h"

namespace nc {
namespace {

constexpr int FA_BM = 128;          /* query rows per workgroup */
constexpr int FA_BN = 64;           /* keys per block */
constexpr int FA_THREADS = 256;
constexpr float FA_LOG2E = 1.4426950408889634f;
constexpr float FA_LN2 = 0.6931471805599453f;
constexpr float FA_RESCALE = 8.0f;  /* lazy rescale threshold (log2 units) */

typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct FlashFwd {
    const uint16_t *q, *k, *v;      /* (total, H, 128) at token strides q_stride, k_stride, v_stride (elements) */
    long long q_stride, k_stride, v_stride;
    const int32_t *cu;              /* [segments + 1] */
    int segments, H, window;
    float scale_log2;               /* softmax scale * log2(e) */
    uint16_t *out;                  /* (total, H, 128) contiguous */
    float *lse;                     /* [H][lse_stride] */
    long long lse_stride;
};

struct FaStage {
    uint16_t k[FA_BN * HEAD_DIM];   /* [key][128], 16-byte chunk c of key j at chunk c ^ (j & 15) */
    uint16_t v[FA_BN * HEAD_DIM];   /* the same layout: read transposed by ds_read_b64_tr_b16 */
};

__device__ __forceinline__ int k_lds(int key, int chunk) { return key * HEAD_DIM + ((chunk ^ (key & 15)) << 3); }

__device__ __forceinline__ Rsrc make_rsrc(const void *p, unsigned bytes) {
    const unsigned long long u = (unsigned long long)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)u), hi = __builtin_amdgcn_readfirstlane((unsigned)(u >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void *)(((unsigned long long)hi << 32) | lo), (short)0,
                                             __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

__device__ __forceinline__ uint4 bload(Rsrc r, int off) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return uint4{v[0], v[1], v[2], v[3]};
}

/* Descriptor over `rows` rows of one head starting at token row0: row i at i * stride elements. */
__device__ __forceinline__ Rsrc rows_rsrc(const uint16_t *base, long long row0, long long stride, int h, int rows) {
    const unsigned bytes = rows > 0 ? (unsigned)(((long long)(rows - 1) * stride + HEAD_DIM) * 2) : 0u;
    return make_rsrc(base + row0 * stride + (long long)h * HEAD_DIM, bytes);
}

/* The A operand of a product over the dimension from a row-major tile: lane (g, c) holds dims 32 cc + 8 g .. +7 of
 * row 16 rt + c. */
__device__ __forceinline__ bf16x8 rows_operand(const uint16_t *lds, int rt, int cc, int g, int c) {
    return *reinterpret_cast<const bf16x8 *>(&lds[k_lds(rt * 16 + c, cc * 4 + g)]);
}

typedef __attribute__((address_space(3))) void LdsVoid;
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 LdsV4;

/* A 64-row tile of one head straight into LDS in the k_lds layout by LDS DMA (no registers held), shared by NW
 * waves: instruction i of a wave writes rows 4 i' .. 4 i' + 3 (i' = wave + NW i), lane l the 16 bytes at LDS chunk
 * l % 16 of row 4 i' + l / 16, fetched from the row's chunk (l % 16) ^ (row & 15). Rows past the descriptor's range
 * read zeros. */
template <int NW = 4>
__device__ __forceinline__ void tile_dma(const uint16_t *base, long long row0, long long stride, int h, int rows,
                                         uint16_t *lds, int wave, int lane) {
    const Rsrc rs = rows_rsrc(base, row0, stride, h, rows);
#pragma unroll
    for (int k = 0; k < FA_BN / 4 / NW; k++) {
        const int i = wave + NW * k, r = 4 * i + (lane >> 4), p = lane & 15;
        const int off = (int)((r * stride + ((p ^ (r & 15)) << 3)) * 2);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (LdsVoid *)(lds + i * 4 * HEAD_DIM), 16, off, 0, 0, 0);
    }
}

/* The A operand of a product over 32 rows of a row-major (k_lds) tile (V^T in O^T += V^T P^T; dO^T, Q^T, K^T in the
 * backward) for dim tile d and k-step s2, in the row order of a score MFMA's output pair: lane (g, c) gets rows
 * 32 s2 + 4 g .. + 3, then 32 s2 + 16 + 4 g .. + 3, of dim 16 d + c. ds_read_b64_tr_b16 hands lane i of a 16-lane group element i % 4 of the 8 bytes lane 4 t + i / 4 points
 * at, for t = 0..3: so lane j of group g points at dims 16 d + 4 (j % 4) .. + 3 of key base + j / 4. */
__device__ __forceinline__ bf16x8 tr_operand(const uint16_t *v, int d, int s2, int g, int c) {
    const int dim = 16 * d + 4 * (c & 3), chunk = dim >> 3, half = (dim >> 2) & 1;
    const int r0 = 32 * s2 + 4 * g + (c >> 2), r1 = r0 + 16;
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (LdsV4 *)(v + k_lds(r0, chunk) + 4 * half));
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (LdsV4 *)(v + k_lds(r1, chunk) + 4 * half));
    const uint2 a = __builtin_bit_cast(uint2, lo), b = __builtin_bit_cast(uint2, hi);
    return __builtin_bit_cast(bf16x8, uint4{a.x, a.y, b.x, b.y});
}

struct FaState {
    f32x4 o[2][8];   /* O^T tile d of query tile j: dims 16d + 4g + i of column (lane & 15) */
    float m[2];      /* the column's reference max (log2 domain), equal in the four groups */
    float l[2];      /* sum of exp2(s - m) over the keys this lane's group holds */
};

/* One key block for the wave's two query tiles. kb0: the block's first key (segment-relative); q0: the wave's first
 * query row (segment-relative). MASKED: apply causal, window and segment-end bounds per score. */
template <bool MASKED>
__device__ __forceinline__ void fa_block(const FlashFwd &a, const FaStage &s, const bf16x8 (&qb)[2][4], FaState &st,
                                         int kb0, int q0, int seglen, int lane) {
    const int g = lane >> 4, c = lane & 15;
    f32x4 sc[2][4];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int kt = 0; kt < 4; kt++) sc[j][kt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    /* raised priority while the scores issue: the SIMD's other wave runs its softmax between them (fa forward
     * 464 -> 471.5 TFLOP/s; the same around the PV products, or around the backward's S / dP products, was slower) */
    __builtin_amdgcn_s_setprio(1);
    /* tile 0's scores, then tile 1's (K operands read from LDS once per tile), so tile 1's products can issue among
     * tile 0's scale, mask and max instructions (the groups below): 471.8 -> 476.6 TFLOP/s; without the groups the
     * compiler issued them all first and the forward fell to 343.6 */
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int cc = 0; cc < 4; cc++) sc[j][kt] = mfma16x16x32(rows_operand(s.k, kt, cc, g, c), qb[j][cc], sc[j][kt]);
    __builtin_amdgcn_s_setprio(0);
    bf16x8 pv[2][2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int qi = q0 + 16 * j + c;
        /* raw scores: the scale is positive, so the max of the scaled scores is the scaled max, and it is folded into
         * one FMA per exponential below */
        float sv[16];
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float x = sc[j][kt][i];
                if (MASKED) {
                    const int key = kb0 + kt * 16 + 4 * g + i;
                    const bool ok = (key <= qi) & (key < seglen) & ((a.window < 0) | (qi - key <= a.window));
                    x = ok ? x : -INFINITY;
                }
                sv[kt * 4 + i] = x;
            }
        float mt = sv[0];
#pragma unroll
        for (int i = 1; i < 16; i++) mt = fmaxf(mt, sv[i]);
        mt = pair_max32(pair_max16(mt)) * a.scale_log2;
        if (j == 0) {
            __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
            }
        }
        const float mnew = fmaxf(st.m[j], mt);
        if (__any(mnew > st.m[j] + FA_RESCALE)) {
            const float alpha = mnew == st.m[j] ? 1.0f : __builtin_amdgcn_exp2f(st.m[j] - mnew);
#pragma unroll
            for (int d = 0; d < 8; d++) st.o[j][d] *= alpha;
            st.l[j] *= alpha;
            st.m[j] = mnew;
        }
        const float mbase = st.m[j] == -INFINITY ? 0.0f : st.m[j];
        float psum = 0.0f;
        float p[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[i], a.scale_log2, -mbase));
            psum += p[i];
        }
        st.l[j] += psum;
        /* k-step s2 covers key tiles 2 s2 and 2 s2 + 1: the group's keys 4g..4g+3 of each */
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
            for (int i = 0; i < 8; i++) pv[j][s2][i] = (__bf16)p[(2 * s2 + (i >> 2)) * 4 + (i & 3)];
    }
#pragma unroll
    for (int d = 0; d < 8; d++) {
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) {
            const bf16x8 vop = tr_operand(s.v, d, s2, g, c);
#pragma unroll
            for (int j = 0; j < 2; j++) st.o[j][d] = mfma16x16x32(vop, pv[j][s2], st.o[j][d]);
        }
    }
}

/* A workgroup's (rank, segment, head) from its place in the launch order: work-groups start in linear order (x,
 * then y, then z), so rank r = L / (segments heads) takes the r-th tile of every (segment, head) before any takes
 * the (r + 1)-th. The kernels map rank 0 to their longest tile, so the short ones of every head come last, where they
 * fill the CUs the long ones leave (the grid keeps x = tiles, y = segments, z = heads). */
struct FaBlock {
    int rank, seg, h;
};

__device__ __forceinline__ FaBlock fa_block_order() {
    const int yz = (int)(gridDim.y * gridDim.z);
    const int L = (int)blockIdx.x + (int)gridDim.x * ((int)blockIdx.y + (int)gridDim.y * (int)blockIdx.z);
    const int r = L % yz;
    return FaBlock{L / yz, r % (int)gridDim.y, r / (int)gridDim.y};
}

__global__ void __launch_bounds__(FA_THREADS, 2) flash_fwd_kernel(FlashFwd a) {
    __shared__ FaStage st0, st1;   /* distinct objects: a read of one never waits for DMA into the other */
    const FaBlock fb = fa_block_order();
    const int seg = fb.seg, h = fb.h;
    const long long start = a.cu[seg];
    const int seglen = a.cu[seg + 1] - a.cu[seg];
    const int tile = (int)gridDim.x - 1 - fb.rank;   /* the longest key ranges first */
    const int qa = tile * FA_BM;
    if (seglen <= 0 || qa >= seglen) return;
    const int t = threadIdx.x, lane = t & (WAVE - 1), wave = t >> 6, g = lane >> 4, c = lane & 15;
    const int qb = min(qa + FA_BM, seglen) - 1;
    const int q0 = qa + wave * 32;                                 /* the wave's first row */
    const bool active = q0 < seglen;
    const int qw1 = min(q0 + 31, seglen - 1);                       /* the wave's last valid row */

    /* the wave's queries: B operand of S^T = K Q^T, lane (g, c) holds dims 32 cc + 8 g .. +7 of row c */
    bf16x8 qb_[2][4];
    {
        const Rsrc rq = rows_rsrc(a.q, start + q0, a.q_stride, h, active ? min(32, seglen - q0) : 0);
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int cc = 0; cc < 4; cc++)
                qb_[j][cc] = __builtin_bit_cast(bf16x8, bload(rq, (int)(((16 * j + c) * a.q_stride + cc * 32 + g * 8) * 2)));
    }
    FaState st;
#pragma unroll
    for (int j = 0; j < 2; j++) {
#pragma unroll
        for (int d = 0; d < 8; d++) st.o[j][d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        st.m[j] = -INFINITY;
        st.l[j] = 0.0f;
    }

    const int klo = a.window >= 0 ? max(0, qa - a.window) : 0;
    const int kb_lo = klo / FA_BN, kb_hi = qb / FA_BN;
    /* block kb + 1 is fetched by LDS DMA into the other stage while block kb is computed; the barrier after the
     * compute (its fence waits for this wave's DMA) makes the fetched block visible and frees the one just read */
    auto fetch = [&](int kb, FaStage &stg) {
        const int n = min(FA_BN, seglen - kb * FA_BN);
        tile_dma(a.k, start + kb * FA_BN, a.k_stride, h, n, stg.k, wave, lane);
        tile_dma(a.v, start + kb * FA_BN, a.v_stride, h, n, stg.v, wave, lane);
    };
    auto compute = [&](int kb, const FaStage &stg) {
        if (!active) return;
        const int k0 = kb * FA_BN, k1 = k0 + FA_BN - 1;
        /* unmasked iff every key of the block is visible to every row of the wave */
        const bool interior = k1 <= q0 && k1 < seglen && (a.window < 0 || qw1 - k0 <= a.window);
        if (interior)
            fa_block<false>(a, stg, qb_, st, k0, q0, seglen, lane);
        else
            fa_block<true>(a, stg, qb_, st, k0, q0, seglen, lane);
    };
    fetch(kb_lo, st0);
    __syncthreads();
    for (int kb = kb_lo; kb <= kb_hi; kb += 2) {
        if (kb + 1 <= kb_hi) fetch(kb + 1, st1);
        compute(kb, st0);
        __syncthreads();
        if (kb + 1 > kb_hi) break;
        if (kb + 2 <= kb_hi) fetch(kb + 2, st0);
        compute(kb + 1, st1);
        __syncthreads();
    }
    if (!active) return;

    /* out = O^T / l, lse = (m + log2 l) ln 2 */
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int row = q0 + 16 * j + c;
        const float l = pair_sum32(pair_sum16(st.l[j]));
        if (row >= seglen) continue;
        const long long tok = start + row;
        const float inv = 1.0f / l;
        uint16_t *o = a.out + (tok * a.H + h) * HEAD_DIM + 4 * g;
#pragma unroll
        for (int d = 0; d < 8; d++) {
            const f32x4 v = st.o[j][d];
            *reinterpret_cast<uint2 *>(o + d * 16) =
                uint2{(uint32_t)f32_to_bf16(v[0] * inv) | ((uint32_t)f32_to_bf16(v[1] * inv) << 16),
                      (uint32_t)f32_to_bf16(v[2] * inv) | ((uint32_t)f32_to_bf16(v[3] * inv) << 16)};
        }
        if (g == 0) a.lse[(long long)h * a.lse_stride + tok] = (st.m[j] + __log2f(l)) * FA_LN2;
    }
}

/* ---------------------------------------------------------------------------------------------------------------
 * Backward (the reference's _flash_attn_bwd / bwd_bf16dq, model/ops/flash_attn.py:367-391), per segment and head:
 *   P = exp(scale S - lse), dV = P^T dO, dP = dO V^T, dS = P (dP - D) with D_i = dO_i . O_i (the caller's row
 *   statistics: the reference's `rows`, from the o_proj backward epilogue), dQ = scale dS K, dK = scale dS^T Q.
 * Two kernels and no atomics: flash_bwd_dkv_kernel owns 128 keys (a wave 16) and walks the query blocks that see them;
 * flash_bwd_dq_kernel owns 128 queries (a wave 32, as the forward) and walks their key blocks. S and dP are computed
 * in both (seven 128-deep products per (query, key) pair instead of five), the price of writing dQ once.
 * ------------------------------------------------------------------------------------------------------------- */

struct FlashBwd {
    const uint16_t *q, *k, *v, *dout;         /* (total, H, 128) at token strides */
    long long q_stride, k_stride, v_stride, do_stride;
    const float *lse;                          /* [H][lse_stride], natural log */
    long long lse_stride;
    const float *dpsum;                        /* (total, H): D = dO . O per row */
    const int32_t *cu;
    int segments, H, window;
    float scale, scale_log2;
    uint16_t *dq, *dk, *dv;                    /* (total, H, 128) at their token strides */
    long long dq_stride, dk_stride, dv_stride;
};

/* bitwise, not short-circuit: evaluated per element inside unrolled loops, a branch per term would split the wave */
__device__ __forceinline__ bool visible(int key, int q, int seglen, int window) {
    return (key <= q) & (q < seglen) & ((window < 0) | (q - key <= window));
}

__device__ __forceinline__ void store4(uint16_t *p, const f32x4 &v, float mul) {
    *reinterpret_cast<uint2 *>(p) = uint2{(uint32_t)f32_to_bf16(v[0] * mul) | ((uint32_t)f32_to_bf16(v[1] * mul) << 16),
                                          (uint32_t)f32_to_bf16(v[2] * mul) | ((uint32_t)f32_to_bf16(v[3] * mul) << 16)};
}

struct alignas(16) DkvStage {
    uint16_t q[FA_BN * HEAD_DIM], dout[FA_BN * HEAD_DIM];   /* k_lds layout; Q^T and dO^T read transposed */
    float lse2[FA_BN], dd[FA_BN];              /* the block's rows: lse log2(e) (+inf past the segment), D */
};

/* dK, dV of 128 keys: eight waves (two a SIMD) of 16 keys share each staged query block, so a CU takes in half the
 * Q and dO bytes per product that four waves of 16 would. S = Q K^T and dP = dO V^T with queries as rows (a lane holds
 * one key's column), so P and dS feed dV^T += dO^T P and dK^T += Q^T dS directly as B operands, with dO^T and Q^T read
 * from transposed LDS tiles. */
constexpr int DKV_WAVES = 8;
constexpr int DKV_KEYS = 16 * DKV_WAVES;

__global__ void __launch_bounds__(64 * DKV_WAVES, 2) flash_bwd_dkv_kernel(FlashBwd a) {
    __shared__ DkvStage s0, s1;   /* distinct objects: a read of one never waits for DMA into the other */
    const FaBlock fb = fa_block_order();
    const int seg = fb.seg, h = fb.h;
    const long long start = a.cu[seg];
    const int seglen = a.cu[seg + 1] - a.cu[seg];
    const int k0 = fb.rank * DKV_KEYS;          /* the most query blocks first */
    if (seglen <= 0 || k0 >= seglen) return;
    const int t = threadIdx.x, lane = t & (WAVE - 1), wave = t >> 6, g = lane >> 4, c = lane & 15;
    const int kw = k0 + wave * 16;              /* the wave's first key */
    const bool active = kw < seglen;
    const int key = kw + c;

    /* the wave's K and V as B operands: lane (g, c) holds dims 32 cc + 8 g .. +7 of key c */
    bf16x8 kb_[4], vb_[4];
    {
        const int n = active ? min(16, seglen - kw) : 0;
        const Rsrc rk = rows_rsrc(a.k, start + kw, a.k_stride, h, n), rv = rows_rsrc(a.v, start + kw, a.v_stride, h, n);
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            kb_[cc] = __builtin_bit_cast(bf16x8, bload(rk, (int)((c * a.k_stride + cc * 32 + g * 8) * 2)));
            vb_[cc] = __builtin_bit_cast(bf16x8, bload(rv, (int)((c * a.v_stride + cc * 32 + g * 8) * 2)));
        }
    }
    f32x4 dk[8], dv[8];
#pragma unroll
    for (int d = 0; d < 8; d++) dk[d] = dv[d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int qhi = a.window >= 0 ? min(seglen - 1, k0 + DKV_KEYS - 1 + a.window) : seglen - 1;
    /* query block qbk + 1 (Q and dO by LDS DMA, the row statistics through registers) is fetched into the other stage
     * while block qbk is computed; the barrier after the compute makes it visible and frees the one just read */
    float rl = INFINITY, rd = 0.0f;
    auto fetch = [&](int qbk, DkvStage &stg) {
        const int qs = qbk * FA_BN, nq = min(FA_BN, seglen - qs);
        tile_dma<DKV_WAVES>(a.q, start + qs, a.q_stride, h, nq, stg.q, wave, lane);
        tile_dma<DKV_WAVES>(a.dout, start + qs, a.do_stride, h, nq, stg.dout, wave, lane);
        if (t < FA_BN) {
            const bool ok = t < nq;
            rl = ok ? a.lse[(long long)h * a.lse_stride + start + qs + t] * FA_LOG2E : INFINITY;
            rd = ok ? a.dpsum[(start + qs + t) * a.H + h] : 0.0f;
        }
    };
    auto put_stats = [&](DkvStage &stg) {
        if (t < FA_BN) {
            stg.lse2[t] = rl;
            stg.dd[t] = rd;
        }
    };
    auto compute = [&](int qbk, const DkvStage &s) {
        if (!active) return;
        const int qs = qbk * FA_BN;
        const int kw1 = kw + 15, qe = qs + FA_BN - 1;
        if (kw > qe || (a.window >= 0 && qs - kw1 > a.window)) return;   /* no row of the block sees the wave's keys */
        const bool interior = kw1 <= qs && qe < seglen && kw1 < seglen && (a.window < 0 || qe - kw <= a.window);
        /* the four query tiles' S and dP first (eight independent accumulators, so the products pipeline), then
         * P and dS, then the dV and dK products of k-step 0 (query tiles 0, 1) and 1 (tiles 2, 3): each dv, dk element
         * adds k-step 0, then 1 */
        f32x4 sc[4], dp[4];
#pragma unroll
        for (int qt = 0; qt < 4; qt++) sc[qt] = dp[qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        /* step st = (cc, qt), cc-major; its Q and dO operands are read one step ahead of the products */
        bf16x8 qn = rows_operand(s.q, 0, 0, g, c), on = rows_operand(s.dout, 0, 0, g, c);
#pragma unroll
        for (int st = 0; st < 16; st++) {
            const int cc = st >> 2, qt = st & 3;
            const bf16x8 qo = qn, oo = on;
            if (st + 1 < 16) {
                qn = rows_operand(s.q, (st + 1) & 3, (st + 1) >> 2, g, c);
                on = rows_operand(s.dout, (st + 1) & 3, (st + 1) >> 2, g, c);
            }
            sc[qt] = mfma16x16x32(qo, kb_[cc], sc[qt]);
            dp[qt] = mfma16x16x32(oo, vb_[cc], dp[qt]);
        }
        /* the row statistics of the lane's 16 rows: one 16-byte LDS read per tile each, all issued together */
        float4 l2[4], dd[4];
#pragma unroll
        for (int qt = 0; qt < 4; qt++) {
            l2[qt] = *reinterpret_cast<const float4 *>(&s.lse2[qt * 16 + 4 * g]);
            dd[qt] = *reinterpret_cast<const float4 *>(&s.dd[qt * 16 + 4 * g]);
        }
        bf16x8 pb[2], db[2];
        /* P and dS of the lane's 16 (key, row) pairs; only a block on the diagonal, the window edge or the segment end
         * tests each pair (interior is uniform over the wave: one scalar branch) */
        auto stats = [&](bool masked) {
#pragma unroll
            for (int qt = 0; qt < 4; qt++) {
                /* lane (g, c): key c, query rows qs + 16 qt + 4 g + i */
                const float lv[4] = {l2[qt].x, l2[qt].y, l2[qt].z, l2[qt].w};
                const float dv_[4] = {dd[qt].x, dd[qt].y, dd[qt].z, dd[qt].w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = qt * 16 + 4 * g + i;
                    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[qt][i], a.scale_log2, -lv[i]));
                    const float p = !masked || visible(key, qs + r, seglen, a.window) ? e : 0.0f;
                    const float ds = p * (dp[qt][i] - dv_[i]);
                    pb[qt >> 1][(qt & 1) * 4 + i] = (__bf16)p;
                    db[qt >> 1][(qt & 1) * 4 + i] = (__bf16)ds;
                }
            }
        };
        if (interior)
            stats(false);
        else
            stats(true);
        /* step st = (s2, d); its dO^T and Q^T operands are read one step ahead of the products */
        bf16x8 vn = tr_operand(s.dout, 0, 0, g, c), kn = tr_operand(s.q, 0, 0, g, c);
#pragma unroll
        for (int st = 0; st < 16; st++) {
            const int s2 = st >> 3, d = st & 7;
            const bf16x8 vo = vn, ko = kn;
            if (st + 1 < 16) {
                vn = tr_operand(s.dout, (st + 1) & 7, (st + 1) >> 3, g, c);
                kn = tr_operand(s.q, (st + 1) & 7, (st + 1) >> 3, g, c);
            }
            dv[d] = mfma16x16x32(vo, pb[s2], dv[d]);
            dk[d] = mfma16x16x32(ko, db[s2], dk[d]);
        }
    };
    const int qb_lo = k0 / FA_BN, qb_hi = qhi / FA_BN;
    fetch(qb_lo, s0);
    put_stats(s0);
    __syncthreads();
    for (int qbk = qb_lo; qbk <= qb_hi; qbk += 2) {
        if (qbk + 1 <= qb_hi) fetch(qbk + 1, s1);
        compute(qbk, s0);
        if (qbk + 1 <= qb_hi) put_stats(s1);
        __syncthreads();
        if (qbk + 1 > qb_hi) break;
        if (qbk + 2 <= qb_hi) fetch(qbk + 2, s0);
        compute(qbk + 1, s1);
        if (qbk + 2 <= qb_hi) put_stats(s0);
        __syncthreads();
    }
    if (!active || key >= seglen) return;
    /* dK^T, dV^T tile d: lane (g, c) holds dims 16 d + 4 g .. +3 of key c */
    uint16_t *pk = a.dk + (start + key) * a.dk_stride + (long long)h * HEAD_DIM + 4 * g;
    uint16_t *pv = a.dv + (start + key) * a.dv_stride + (long long)h * HEAD_DIM + 4 * g;
#pragma unroll
    for (int d = 0; d < 8; d++) {
        store4(pk + d * 16, dk[d], a.scale);
        store4(pv + d * 16, dv[d], 1.0f);
    }
}

struct DqStage {
    uint16_t k[FA_BN * HEAD_DIM], v[FA_BN * HEAD_DIM];   /* k_lds layout; K^T read transposed */
};

/* dQ of 128 queries: as the forward, S^T = K Q^T and dP^T = V dO^T with queries as columns, so dS^T feeds
 * dQ^T += K^T dS^T as the B operand with K^T read from a transposed LDS tile. */
__global__ void __launch_bounds__(FA_THREADS, 2) flash_bwd_dq_kernel(FlashBwd a) {
    __shared__ DqStage s0, s1;   /* distinct objects: a read of one never waits for DMA into the other */
    const FaBlock fb = fa_block_order();
    const int seg = fb.seg, h = fb.h;
    const long long start = a.cu[seg];
    const int seglen = a.cu[seg + 1] - a.cu[seg];
    const int tile = (int)gridDim.x - 1 - fb.rank;
    const int qa = tile * FA_BM;
    if (seglen <= 0 || qa >= seglen) return;
    const int t = threadIdx.x, lane = t & (WAVE - 1), wave = t >> 6, g = lane >> 4, c = lane & 15;
    const int qb = min(qa + FA_BM, seglen) - 1;
    const int q0 = qa + wave * 32;
    const bool active = q0 < seglen;
    const int qw1 = min(q0 + 31, seglen - 1);

    /* queries and dO as B operands (lane (g, c): dims 32 cc + 8 g .. +7 of row c), each column's lse and D */
    bf16x8 qb_[2][4], ob_[2][4];
    float lse2[2], dd[2];
    {
        const int n = active ? min(32, seglen - q0) : 0;
        const Rsrc rq = rows_rsrc(a.q, start + q0, a.q_stride, h, n), ro = rows_rsrc(a.dout, start + q0, a.do_stride, h, n);
#pragma unroll
        for (int j = 0; j < 2; j++) {
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                qb_[j][cc] = __builtin_bit_cast(bf16x8, bload(rq, (int)(((16 * j + c) * a.q_stride + cc * 32 + g * 8) * 2)));
                ob_[j][cc] = __builtin_bit_cast(bf16x8, bload(ro, (int)(((16 * j + c) * a.do_stride + cc * 32 + g * 8) * 2)));
            }
            const int row = q0 + 16 * j + c;
            const bool ok = active && row < seglen;
            lse2[j] = ok ? a.lse[(long long)h * a.lse_stride + start + row] * FA_LOG2E : INFINITY;
            dd[j] = ok ? a.dpsum[(start + row) * a.H + h] : 0.0f;
        }
    }
    f32x4 dq[2][8];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int d = 0; d < 8; d++) dq[j][d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int klo = a.window >= 0 ? max(0, qa - a.window) : 0;
    /* key block kb + 1 (K and V by LDS DMA) is fetched into the other stage while block kb is computed */
    auto fetch = [&](int kb, DqStage &stg) {
        const int nk = min(FA_BN, seglen - kb * FA_BN);
        tile_dma(a.k, start + kb * FA_BN, a.k_stride, h, nk, stg.k, wave, lane);
        tile_dma(a.v, start + kb * FA_BN, a.v_stride, h, nk, stg.v, wave, lane);
    };
    auto compute = [&](int kb, const DqStage &s) {
        if (!active) return;
        const int k0 = kb * FA_BN, k1 = k0 + FA_BN - 1;
        const bool interior = k1 <= q0 && k1 < seglen && (a.window < 0 || qw1 - k0 <= a.window);
        /* k-step s2 (key tiles 2 s2, 2 s2 + 1): its dS^T half is formed, then consumed by the dQ products at once, so
         * only one half is ever live; each dq element still adds k-step 0, then 1 */
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) {
            bf16x8 db[2];
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                const int kt = 2 * s2 + kk;
                f32x4 sc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}}, dp[2] = {sc[0], sc[1]};
#pragma unroll
                for (int cc = 0; cc < 4; cc++) {
                    const bf16x8 kop = rows_operand(s.k, kt, cc, g, c), vop = rows_operand(s.v, kt, cc, g, c);
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        sc[j] = mfma16x16x32(kop, qb_[j][cc], sc[j]);
                        dp[j] = mfma16x16x32(vop, ob_[j][cc], dp[j]);
                    }
                }
                /* lane (g, c): query column c of tile j, keys k0 + 16 kt + 4 g + i; only a block on the diagonal, the
                 * window edge or the segment end tests each pair (interior is uniform: one scalar branch) */
                auto pds = [&](bool masked) {
#pragma unroll
                    for (int j = 0; j < 2; j++)
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][i], a.scale_log2, -lse2[j]));
                            const float p =
                                !masked || visible(k0 + 16 * kt + 4 * g + i, q0 + 16 * j + c, seglen, a.window) ? e : 0.0f;
                            db[j][kk * 4 + i] = (__bf16)(p * (dp[j][i] - dd[j]));
                        }
                };
                if (interior)
                    pds(false);
                else
                    pds(true);
            }
#pragma unroll
            for (int d = 0; d < 8; d++) {
                const bf16x8 kop = tr_operand(s.k, d, s2, g, c);
#pragma unroll
                for (int j = 0; j < 2; j++) dq[j][d] = mfma16x16x32(kop, db[j], dq[j][d]);
            }
        }
    };
    const int kb_lo = klo / FA_BN, kb_hi = qb / FA_BN;
    fetch(kb_lo, s0);
    __syncthreads();
    for (int kb = kb_lo; kb <= kb_hi; kb += 2) {
        if (kb + 1 <= kb_hi) fetch(kb + 1, s1);
        compute(kb, s0);
        __syncthreads();
        if (kb + 1 > kb_hi) break;
        if (kb + 2 <= kb_hi) fetch(kb + 2, s0);
        compute(kb + 1, s1);
        __syncthreads();
    }
    if (!active) return;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int row = q0 + 16 * j + c;
        if (row >= seglen) continue;
        uint16_t *p = a.dq + (start + row) * a.dq_stride + (long long)h * HEAD_DIM + 4 * g;
#pragma unroll
        for (int d = 0; d < 8; d++) store4(p + d * 16, dq[j][d], a.scale);
    }
}

/* D[row][h] = sum_d dO . O in fp32: one wave per (row, head), two dims per lane. */
__global__ void __launch_bounds__(256) flash_bwd_rows_kernel(const uint16_t *out, long long o_stride,
                                                             const uint16_t *dout, long long do_stride, long long n,
                                                             int H, float *dpsum) {
    const long long w = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (w >= n) return;
    const int lane = threadIdx.x & (WAVE - 1), h = (int)(w % H);
    const long long row = w / H;
    const uint32_t o = *reinterpret_cast<const uint32_t *>(out + row * o_stride + (long long)h * HEAD_DIM + 2 * lane);
    const uint32_t d = *reinterpret_cast<const uint32_t *>(dout + row * do_stride + (long long)h * HEAD_DIM + 2 * lane);
    const float v = __builtin_fmaf(__uint_as_float(o & 0xFFFF0000u), __uint_as_float(d & 0xFFFF0000u),
                                   __uint_as_float(o << 16) * __uint_as_float(d << 16));
    const float sum = wave_sum_butterfly(v);
    if (lane == 0) dpsum[w] = sum;
}

}  // namespace
}  // namespace nc

using namespace nc;

extern "C" int nc_flash_attn_fwd(const void *q, const void *k, const void *v, long long q_stride, long long k_stride,
                                 long long v_stride, const int32_t *cu_seqlens, int segments, int max_seqlen,
                                 int heads, int window, float softmax_scale, void *out, float *lse,
                                 long long lse_stride, void *stream) {
    if (segments < 0 || max_seqlen < 0 || heads < 1 || heads > 65535 || segments > 65535 || lse_stride < 0 ||
        !(softmax_scale > 0.0f))
        return NC_ERR_SHAPE;
    if (segments == 0 || max_seqlen == 0) return NC_OK;
    if (!q || !k || !v || !cu_seqlens || !out || !lse) return NC_ERR_NULL;
    const long long row = (long long)heads * HEAD_DIM;
    if (q_stride < row || k_stride < row || v_stride < row || q_stride % 8 || k_stride % 8 || v_stride % 8 ||
        ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15)
        return NC_ERR_SHAPE;
    /* a block of 64 rows of one head is one buffer descriptor with 32-bit signed offsets */
    if ((63 * max(max(q_stride, k_stride), v_stride) + HEAD_DIM) * 2 >= 0x7FFFFFFFLL) return NC_ERR_SHAPE;
    FlashFwd a;
    a.q = (const uint16_t *)q; a.k = (const uint16_t *)k; a.v = (const uint16_t *)v;
    a.q_stride = q_stride; a.k_stride = k_stride; a.v_stride = v_stride;
    a.cu = cu_seqlens; a.segments = segments; a.H = heads; a.window = window < 0 ? -1 : window;
    a.scale_log2 = softmax_scale * FA_LOG2E;
    a.out = (uint16_t *)out; a.lse = lse; a.lse_stride = lse_stride;
    const dim3 grid((unsigned)((max_seqlen + FA_BM - 1) / FA_BM), (unsigned)segments, (unsigned)heads);
    hipLaunchKernelGGL(flash_fwd_kernel, grid, dim3(FA_THREADS), 0, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

extern "C" int nc_flash_attn_bwd_rows(const void *out, long long o_stride, const void *dout, long long do_stride,
                                      long long total, int heads, float *dpsum, void *stream) {
    if (total < 0 || heads < 1 || o_stride < (long long)heads * HEAD_DIM || do_stride < (long long)heads * HEAD_DIM ||
        o_stride % 2 || do_stride % 2)
        return NC_ERR_SHAPE;
    if (total == 0) return NC_OK;
    if (!out || !dout || !dpsum) return NC_ERR_NULL;
    if (((uintptr_t)out | (uintptr_t)dout) & 3) return NC_ERR_SHAPE;
    const long long n = total * heads;
    hipLaunchKernelGGL(flash_bwd_rows_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)out, o_stride, (const uint16_t *)dout, do_stride, n, heads, dpsum);
    return (int)hipGetLastError();
}

extern "C" int nc_flash_attn_bwd(const void *q, const void *k, const void *v, const void *dout, long long q_stride,
                                 long long k_stride, long long v_stride, long long do_stride, const float *lse,
                                 long long lse_stride, const float *dpsum, const int32_t *cu_seqlens, int segments,
                                 int max_seqlen, int heads, int window, float softmax_scale, void *dq, void *dk,
                                 void *dv, long long dq_stride, long long dk_stride, long long dv_stride,
                                 void *stream) {
    if (segments < 0 || max_seqlen < 0 || heads < 1 || heads > 65535 || segments > 65535 || lse_stride < 0 ||
        !(softmax_scale > 0.0f))
        return NC_ERR_SHAPE;
    if (segments == 0 || max_seqlen == 0) return NC_OK;
    if (!q || !k || !v || !dout || !lse || !dpsum || !cu_seqlens || !dq || !dk || !dv) return NC_ERR_NULL;
    const long long row = (long long)heads * HEAD_DIM;
    const long long strides[] = {q_stride, k_stride, v_stride, do_stride, dq_stride, dk_stride, dv_stride};
    long long widest = 0;
    for (long long st : strides) {
        if (st < row || st % 8) return NC_ERR_SHAPE;
        widest = max(widest, st);
    }
    if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)dout | (uintptr_t)dq | (uintptr_t)dk | (uintptr_t)dv) & 15)
        return NC_ERR_SHAPE;
    if ((63 * widest + HEAD_DIM) * 2 >= 0x7FFFFFFFLL) return NC_ERR_SHAPE;
    FlashBwd a;
    a.q = (const uint16_t *)q; a.k = (const uint16_t *)k; a.v = (const uint16_t *)v; a.dout = (const uint16_t *)dout;
    a.q_stride = q_stride; a.k_stride = k_stride; a.v_stride = v_stride; a.do_stride = do_stride;
    a.lse = lse; a.lse_stride = lse_stride; a.dpsum = dpsum;
    a.cu = cu_seqlens; a.segments = segments; a.H = heads; a.window = window < 0 ? -1 : window;
    a.scale = softmax_scale; a.scale_log2 = softmax_scale * FA_LOG2E;
    a.dq = (uint16_t *)dq; a.dk = (uint16_t *)dk; a.dv = (uint16_t *)dv;
    a.dq_stride = dq_stride; a.dk_stride = dk_stride; a.dv_stride = dv_stride;
    hipLaunchKernelGGL(flash_bwd_dkv_kernel, dim3((unsigned)((max_seqlen + DKV_KEYS - 1) / DKV_KEYS),
                                                  (unsigned)segments, (unsigned)heads),
                       dim3(64 * DKV_WAVES), 0, (hipStream_t)stream, a);
    hipLaunchKernelGGL(flash_bwd_dq_kernel, dim3((unsigned)((max_seqlen + FA_BM - 1) / FA_BM), (unsigned)segments,
                                                 (unsigned)heads),
                       dim3(FA_THREADS), 0, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}
