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
 * are visited in blocks of 64, staged in LDS for the four waves (K row-major with 16-byte chunks XOR-swizzled by the
 * key, V transposed with 8-byte units swizzled by the dimension, so the MFMA operand reads are conflict-free), in
 * two LDS stages: block b+1 is written to one while block b is read from the other. Scores are S^T = K Q^T
 * (v_mfma_f32_16x16x32_bf16, keys as rows, queries as columns), so a lane's scores all belong to one query; the
 * online softmax runs in the log2 domain with the lazy rescale of the decode kernels (the reference max moves only
 * when a column's max passes it by 2^8); P^T then feeds O^T += V^T P^T with no shuffle, its key order matched by the
 * order of the transposed V operand.
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
    uint16_t vt[HEAD_DIM * FA_BN];  /* [dim][64], 8-byte unit u (keys 4u..4u+3) of dim d at unit u ^ (d & 15) */
};

__device__ __forceinline__ int k_lds(int key, int chunk) { return key * HEAD_DIM + ((chunk ^ (key & 15)) << 3); }
__device__ __forceinline__ int vt_lds(int d, int unit) { return d * FA_BN + ((unit ^ (d & 15)) << 2); }

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

/* One key block's K and V in registers: thread t holds K chunks 4(t%4) .. +3 of key t/4, and dims 8(t/16) .. +7 of
 * keys 4(t%16) .. +3 of V. Keys past the segment read zeros. */
struct StageRegs {
    uint4 k[4], v[4];
};

__device__ __forceinline__ void stage_load(const FlashFwd &a, long long key0, int nkeys, int h, StageRegs &r, int t) {
    const Rsrc rk = rows_rsrc(a.k, key0, a.k_stride, h, nkeys), rv = rows_rsrc(a.v, key0, a.v_stride, h, nkeys);
    const int kk = t >> 2, kc = (t & 3) * 4;
#pragma unroll
    for (int i = 0; i < 4; i++) r.k[i] = bload(rk, (int)((kk * a.k_stride + (kc + i) * 8) * 2));
    const int vk = (t & 15) * 4, vd = (t >> 4) * 8;
#pragma unroll
    for (int i = 0; i < 4; i++) r.v[i] = bload(rv, (int)(((vk + i) * a.v_stride + vd) * 2));
}

__device__ __forceinline__ uint32_t half_of(const uint4 &u, int j) {
    const uint32_t w = j < 2 ? (j == 0 ? u.x : u.y) : (j == 2 ? u.z : u.w);
    return w;
}

__device__ __forceinline__ void stage_store(FaStage &s, const StageRegs &r, int t) {
    const int kk = t >> 2, kc = (t & 3) * 4;
#pragma unroll
    for (int i = 0; i < 4; i++) *reinterpret_cast<uint4 *>(&s.k[k_lds(kk, kc + i)]) = r.k[i];
    /* V: r.v[i] = dims vd .. vd+7 of key vk + i; dim vd + j of the four keys -> one 8-byte unit of Vt */
    const int u = t & 15, vd = (t >> 4) * 8;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int sh = (j & 1) * 16;
        uint32_t e[4];
#pragma unroll
        for (int i = 0; i < 4; i++) e[i] = (half_of(r.v[i], j >> 1) >> sh) & 0xFFFFu;
        *reinterpret_cast<uint2 *>(&s.vt[vt_lds(vd + j, u)]) = uint2{e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
    }
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
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            const bf16x8 kop = *reinterpret_cast<const bf16x8 *>(&s.k[k_lds(kt * 16 + c, cc * 4 + g)]);
#pragma unroll
            for (int j = 0; j < 2; j++) sc[j][kt] = mfma16x16x32(kop, qb[j][cc], sc[j][kt]);
        }
    }
    bf16x8 pv[2][2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int qi = q0 + 16 * j + c;
        float sv[16];
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float x = sc[j][kt][i] * a.scale_log2;
                if (MASKED) {
                    const int key = kb0 + kt * 16 + 4 * g + i;
                    const bool ok = key <= qi && key < seglen && (a.window < 0 || qi - key <= a.window);
                    x = ok ? x : -INFINITY;
                }
                sv[kt * 4 + i] = x;
            }
        float mt = sv[0];
#pragma unroll
        for (int i = 1; i < 16; i++) mt = fmaxf(mt, sv[i]);
        mt = pair_max32(pair_max16(mt));
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
            p[i] = __builtin_amdgcn_exp2f(sv[i] - mbase);
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
            const int dim = d * 16 + c;
            const uint2 lo = *reinterpret_cast<const uint2 *>(&s.vt[vt_lds(dim, 8 * s2 + g)]);
            const uint2 hi = *reinterpret_cast<const uint2 *>(&s.vt[vt_lds(dim, 8 * s2 + 4 + g)]);
            const bf16x8 vop = __builtin_bit_cast(bf16x8, uint4{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
            for (int j = 0; j < 2; j++) st.o[j][d] = mfma16x16x32(vop, pv[j][s2], st.o[j][d]);
        }
    }
}

__global__ void __launch_bounds__(FA_THREADS, 2) flash_fwd_kernel(FlashFwd a) {
    __shared__ FaStage stage[2];
    const int seg = blockIdx.y, h = blockIdx.z;
    const long long start = a.cu[seg];
    const int seglen = a.cu[seg + 1] - a.cu[seg];
    const int tile = (int)gridDim.x - 1 - (int)blockIdx.x;   /* the longest key ranges first */
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
    StageRegs r;
    stage_load(a, start + kb_lo * FA_BN, min(FA_BN, seglen - kb_lo * FA_BN), h, r, t);
    stage_store(stage[0], r, t);
    __syncthreads();
    for (int kb = kb_lo; kb <= kb_hi; kb++) {
        const int cur = (kb - kb_lo) & 1;
        const bool more = kb < kb_hi;
        if (active) {
            const int k0 = kb * FA_BN, k1 = k0 + FA_BN - 1;
            /* unmasked iff every key of the block is visible to every row of the wave */
            const bool interior = k1 <= q0 && k1 < seglen && (a.window < 0 || qw1 - k0 <= a.window);
            if (interior)
                fa_block<false>(a, stage[cur], qb_, st, k0, q0, seglen, lane);
            else
                fa_block<true>(a, stage[cur], qb_, st, k0, q0, seglen, lane);
        }
        if (more) {
            stage_load(a, start + (kb + 1) * FA_BN, min(FA_BN, seglen - (kb + 1) * FA_BN), h, r, t);
            stage_store(stage[cur ^ 1], r, t);
        }
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
