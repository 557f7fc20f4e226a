/*
 * Value-embedding gate and mix of training, gfx950: the reference's model/kernels/ve_gate.cu (called through
 * model/ops/ve_gate.py by model/ops/flash_attn.py:340 and :391).
 *
 * Forward, per row r of the normed stream n (rows = B*T, C = 128 H for H heads):
 *   z[h]       = sum_c n[r][c] w[h][c]                           fp32 fused multiply-adds, then a wave reduction
 *   gate[r][h] = 2 * (1 / (1 + exp(-z[h])))                      fp32
 *   out[r][c]  = bf16(v[r][c] + gate[r][c / 128] * bf16(table[idx[r]][c]))   product and sum each rounded once
 * Backward, per row r, visited in token order (position p holds row order[p] and token ids[p]):
 *   dg[h]        = sum over head h's 128 columns of dout[r][c] * bf16(table[t][c])
 *   dz[r][h]     = bf16(2 dg[h] (1 - s) s) with s = gate[r][h] / 2   (dz_fp32, unrounded, feeds dn)
 *   dn[r][c]     = bf16(sum_h dz_fp32[h] w[h][c])
 *   dtable[t][c] += sum over the rows of token t of bf16(gate[r][c / 128] * dout[r][c])   (fp32, added in)
 * dw = dz^T n is a library GEMM on the host side, as in the reference. ids must hold equal tokens adjacently (sorted,
 * the reference's contract, model/ops/ve_gate.py:23-26): the table gradient of a token split into separate runs is
 * undefined.
 *
 * Mapping: one wave per row. Lane l holds the 8-column chunks c = (i*64 + l)*8, i < NCH = ceil(H/4), so chunk i of
 * lane l lies in head 4i + l/16 and a head's 128 columns are the 16 lanes of one DPP row: a per-head sum is four DPP
 * steps and a whole-row sum two permlane swaps more. w stays in LDS for the whole workgroup (fp32, zero-padded to
 * NCH*512 columns, in two planes holding columns 0-3 and 4-7 of every chunk, so a lane's 16-byte reads at 16-byte
 * stride are conflict-free). Every row access goes through a buffer descriptor of the row's exact size: the columns
 * past C of the last chunk read 0 and their stores are dropped, and a token outside the table (nc_ve_* entry points)
 * reads a zero-size descriptor, so it mixes in nothing and receives no gradient.
 */
#include "nc_device.h"
#include "nc_internal.h"
#include "nanochat_amd.h"

namespace nc {
namespace {

constexpr int VE_MAX_HEADS = 16;
constexpr int VE_THREADS = 512;
constexpr int VE_WAVES = VE_THREADS / WAVE;
constexpr int REF_HEADS = 6;   /* the reference kernel's compile-time H (C = 768, ve_gate.cu:34) */

typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int H>
struct VeShape {
    static constexpr int C = H * HEAD_DIM;
    static constexpr int NCH = (H + 3) / 4;        /* 8-column chunks per lane */
    static constexpr int Q = NCH * WAVE;           /* chunks per padded row */
    static constexpr int PLANE = H * Q * 4;        /* floats in one LDS plane */
};

/* A descriptor over [p, p + bytes): the wave-uniform operands are taken from the first lane so it lives in SGPRs. */
__device__ __forceinline__ Rsrc row_rsrc(const void *p, int bytes) {
    const unsigned long long u = (unsigned long long)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)u), hi = __builtin_amdgcn_readfirstlane((unsigned)(u >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void *)(((unsigned long long)hi << 32) | lo), (short)0,
                                             __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

__device__ __forceinline__ long long uniform64(long long v) {
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)((unsigned long long)v >> 32));
    return (long long)(((unsigned long long)hi << 32) | lo);
}

__device__ __forceinline__ uint4 ld16(Rsrc r, int off) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return uint4{v[0], v[1], v[2], v[3]};
}
/* non-temporal: rows streamed once */
__device__ __forceinline__ uint4 ld16_nt(Rsrc r, int off) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
    return uint4{v[0], v[1], v[2], v[3]};
}
__device__ __forceinline__ void st16(Rsrc r, int off, uint4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.x, v.y, v.z, v.w}, r, off, 0, 0);
}

__device__ __forceinline__ void unpack_bf16x8(uint4 u, float (&x)[8]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        x[2 * k] = __uint_as_float(w[k] << 16);
        x[2 * k + 1] = __uint_as_float(w[k] & 0xFFFF0000u);
    }
}

__device__ __forceinline__ uint4 pack_bf16x8(const float (&x)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; k++) w[k] = (uint32_t)f32_to_bf16(x[2 * k]) | ((uint32_t)f32_to_bf16(x[2 * k + 1]) << 16);
    return uint4{w[0], w[1], w[2], w[3]};
}

/* fp32 rounded to bf16 and back (round to nearest even). */
__device__ __forceinline__ float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }

/* Eight fp32 table values (two 16-byte words) rounded to bf16, packed. */
__device__ __forceinline__ uint4 table_bf16x8(uint4 a, uint4 b) {
    const float x[8] = {__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z), __uint_as_float(a.w),
                        __uint_as_float(b.x), __uint_as_float(b.y), __uint_as_float(b.z), __uint_as_float(b.w)};
    return pack_bf16x8(x);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

/* Sum over each 16-lane row (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror): every lane of
 * the row ends with the same bits, since each step adds the same two partial sums in either order. */
__device__ __forceinline__ float row16_sum(float v) {
    v = v + dpp<0xB1>(v);
    v = v + dpp<0x4E>(v);
    v = v + dpp<0x141>(v);
    v = v + dpp<0x140>(v);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return pair_sum32(pair_sum16(row16_sum(v))); }

/* w [H][C] fp32 -> LDS planes: column c of head h, chunk q = c / 8, at plane (c % 8) / 4, float (h Q + q) 4 + c % 4;
 * columns C .. Q*8 are zero. */
template <int H>
__device__ __forceinline__ void stage_w(float *ws, const float *w) {
    using S = VeShape<H>;
    for (int i = threadIdx.x; i < H * S::Q * 2; i += VE_THREADS) {
        const int h = i / (2 * S::Q), q = (i >> 1) % S::Q, half = i & 1, c = q * 8 + half * 4;
        float4 x = {0.0f, 0.0f, 0.0f, 0.0f};
        if (c < S::C) x = *reinterpret_cast<const float4 *>(w + (long long)h * S::C + c);
        *reinterpret_cast<float4 *>(ws + half * S::PLANE + (h * S::Q + q) * 4) = x;
    }
}

template <int H>
__device__ __forceinline__ void w_chunk(const float *ws, int h, int q, float (&wv)[8]) {
    using S = VeShape<H>;
    const float4 a = *reinterpret_cast<const float4 *>(ws + (h * S::Q + q) * 4);
    const float4 b = *reinterpret_cast<const float4 *>(ws + S::PLANE + (h * S::Q + q) * 4);
    wv[0] = a.x; wv[1] = a.y; wv[2] = a.z; wv[3] = a.w;
    wv[4] = b.x; wv[5] = b.y; wv[6] = b.z; wv[7] = b.w;
}

struct VeFwd {
    const uint16_t *n, *v;          /* n: [rows][C]; v: rows at v_stride elements */
    long long v_stride;
    const int32_t *idx;             /* [rows] tokens */
    const float *table;             /* [vocab][C] */
    long long vocab;
    const float *w;                 /* [H][C] */
    uint16_t *out;                  /* [rows][C] */
    float *gate;                    /* [rows][H] */
    long long rows;
};

template <int H>
__global__ void __launch_bounds__(VE_THREADS) ve_forward_kernel(VeFwd a) {
    using S = VeShape<H>;
    constexpr int C = S::C, NCH = S::NCH;
    __shared__ __attribute__((aligned(16))) float ws[2 * S::PLANE];
    stage_w<H>(ws, a.w);
    __syncthreads();
    const int lane = threadIdx.x & (WAVE - 1);
    const long long step = (long long)gridDim.x * VE_WAVES;
    for (long long rr = (long long)blockIdx.x * VE_WAVES + (threadIdx.x >> 6); rr < a.rows; rr += step) {
        const long long r = uniform64(rr);
        const int tok = __builtin_amdgcn_readfirstlane(a.idx[r]);
        const bool ok = tok >= 0 && (long long)tok < a.vocab;
        const Rsrc rn = row_rsrc(a.n + r * C, C * 2), rv = row_rsrc(a.v + r * a.v_stride, C * 2);
        const Rsrc re = row_rsrc(a.table + (ok ? (long long)tok * C : 0), ok ? C * 4 : 0);
        uint4 xn[NCH], xv[NCH], e0[NCH], e1[NCH];
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const int off = (i * WAVE + lane) * 16;
            xn[i] = ld16_nt(rn, off);
            xv[i] = ld16_nt(rv, off);
            e0[i] = ld16(re, 2 * off);
            e1[i] = ld16(re, 2 * off + 16);
        }
        float x[NCH][8];
#pragma unroll
        for (int i = 0; i < NCH; i++) unpack_bf16x8(xn[i], x[i]);
        /* one head at a time (a loop, not unrolled, so w's LDS reads are not all hoisted into registers); lane h
         * keeps gate h */
        float mine = 0.0f;
#pragma unroll 1
        for (int h = 0; h < H; h++) {
            float z = 0.0f;
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                float wv[8];
                w_chunk<H>(ws, h, i * WAVE + lane, wv);
#pragma unroll
                for (int j = 0; j < 8; j++) z = __builtin_fmaf(x[i][j], wv[j], z);
            }
            const float g = 2.0f * (1.0f / (1.0f + expf(-wave_sum(z))));
            if (lane == h) mine = g;
        }
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(mine), row_rsrc(a.gate + r * H, H * 4), lane * 4, 0, 0);
        const Rsrc ro = row_rsrc(a.out + r * C, C * 2);
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            /* chunk i's head 4i + lane/16 (a lane past the last head reads a gate it multiplies by zeros) */
            const float gh = __shfl(mine, min(4 * i + (lane >> 4), H - 1), WAVE);
            float x[8], e[8];
            unpack_bf16x8(xv[i], x);
            unpack_bf16x8(table_bf16x8(e0[i], e1[i]), e);
#pragma unroll
            for (int j = 0; j < 8; j++) x[j] = x[j] + gh * e[j];
            st16(ro, (i * WAVE + lane) * 16, pack_bf16x8(x));
        }
    }
}

struct VeBwd {
    const uint16_t *dout;           /* rows at dout_stride elements */
    long long dout_stride;
    const int32_t *ids;             /* [rows] tokens in visiting (sorted) order */
    const long long *order;         /* [rows] the row of each position */
    const float *table;             /* [vocab][C] */
    long long vocab;
    const float *w;                 /* [H][C] */
    const float *gate;              /* [rows][H] */
    uint16_t *dn;                   /* [rows][C] */
    float *dtable;                  /* [vocab][C], added into */
    uint16_t *dz;                   /* [rows][H] */
    long long rows;
};

/* w [H][C] fp32 -> LDS unchanged: the backward reads columns (2 lane, 2 lane + 1) of a head, 8 bytes at 8-byte
 * stride, conflict-free. */
template <int H>
__device__ __forceinline__ void stage_w_rows(float *ws, const float *w) {
    for (int i = threadIdx.x; i < H * H * HEAD_DIM / 4; i += VE_THREADS)
        reinterpret_cast<float4 *>(ws)[i] = reinterpret_cast<const float4 *>(w)[i];
}

/* A run's accumulated table gradient added into dtable row t. With equal tokens adjacent in `ids` (sorted, the
 * reference's contract), a run that neither starts at the wave's first position nor ends at its last one holds every
 * occurrence of its token, so no other wave touches that row: a plain read-add-write. The first and last run of a
 * wave's range may continue in the neighbouring waves' ranges: hardware fp32 atomics (two instructions per head,
 * each 64 dwords at 8-byte stride). */
template <int H>
__device__ __forceinline__ void flush_run(float *dtable, int t, const float (&acc)[H][2], int lane, bool shared) {
    float *row = dtable + (long long)t * (H * HEAD_DIM) + 2 * lane;
    if (shared) {
#pragma unroll
        for (int k = 0; k < H; k++) {
            unsafeAtomicAdd(row + k * HEAD_DIM, acc[k][0]);
            unsafeAtomicAdd(row + k * HEAD_DIM + 1, acc[k][1]);
        }
    } else {
        float2 cur[H];
#pragma unroll
        for (int k = 0; k < H; k++) cur[k] = *reinterpret_cast<const float2 *>(row + k * HEAD_DIM);
#pragma unroll
        for (int k = 0; k < H; k++)
            *reinterpret_cast<float2 *>(row + k * HEAD_DIM) = float2{cur[k].x + acc[k][0], cur[k].y + acc[k][1]};
    }
}

/* Backward mapping (unlike the forward's): lane l holds columns k*128 + 2l and k*128 + 2l + 1 of every head k, so a
 * head's gate is one scalar, dg is a whole-wave sum, and every access of dout, the table, dn and dtable is 4 or 8
 * contiguous bytes per lane, 256 or 512 contiguous bytes per instruction. */
template <int H>
__global__ void __launch_bounds__(VE_THREADS) ve_backward_kernel(VeBwd a) {
    constexpr int C = H * HEAD_DIM;
    __shared__ __attribute__((aligned(16))) float ws[H * C];
    stage_w_rows<H>(ws, a.w);
    __syncthreads();
    const int lane = threadIdx.x & (WAVE - 1);
    const long long nw = (long long)gridDim.x * VE_WAVES;
    const long long wid = uniform64((long long)blockIdx.x * VE_WAVES + (threadIdx.x >> 6));
    const long long p0 = a.rows * wid / nw, p1 = a.rows * (wid + 1) / nw;
    float acc[H][2];
    uint32_t eb[H];   /* the run's table columns as bf16x2 */
    int cur = -1;
    bool cur_ok = false, started = false, first = true;   /* first: the current run is the wave's first */
    for (long long p = p0; p < p1; p++) {
        const long long r = uniform64(a.order[p]);
        if (r < 0 || r >= a.rows) continue;   /* not a row: nothing to read or write */
        const int t = __builtin_amdgcn_readfirstlane(a.ids[p]);
        const Rsrc rd = row_rsrc(a.dout + r * a.dout_stride, C * 2);
        uint32_t d[H];
        float g[H];
#pragma unroll
        for (int k = 0; k < H; k++) {
            d[k] = __builtin_amdgcn_raw_buffer_load_b32(rd, (k * HEAD_DIM + 2 * lane) * 2, 0, 2);
            g[k] = a.gate[r * H + k];
        }
        if (!started || t != cur) {
            if (started) {
                if (cur_ok) flush_run<H>(a.dtable, cur, acc, lane, first);
                first = false;
            }
            started = true;
            cur = t;
            cur_ok = t >= 0 && (long long)t < a.vocab;
            const Rsrc re = row_rsrc(a.table + (cur_ok ? (long long)t * C : 0), cur_ok ? C * 4 : 0);
#pragma unroll
            for (int k = 0; k < H; k++) {
                const auto e = __builtin_amdgcn_raw_buffer_load_b64(re, (k * HEAD_DIM + 2 * lane) * 4, 0, 0);
                eb[k] = (uint32_t)f32_to_bf16(__uint_as_float(e[0])) | ((uint32_t)f32_to_bf16(__uint_as_float(e[1])) << 16);
                acc[k][0] = 0.0f;
                acc[k][1] = 0.0f;
            }
        }
        float dz[H], mine = 0.0f;
#pragma unroll
        for (int k = 0; k < H; k++) {
            const float d0 = __uint_as_float(d[k] << 16), d1 = __uint_as_float(d[k] & 0xFFFF0000u);
            const float e0 = __uint_as_float(eb[k] << 16), e1 = __uint_as_float(eb[k] & 0xFFFF0000u);
            acc[k][0] = acc[k][0] + bf16r(g[k] * d0);
            acc[k][1] = acc[k][1] + bf16r(g[k] * d1);
            const float dg = wave_sum(__builtin_fmaf(d1, e1, d0 * e0)), sg = g[k] * 0.5f;
            dz[k] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(2.0f * dg * (1.0f - sg) * sg)));
            if (lane == k) mine = dz[k];
        }
        __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(mine), row_rsrc(a.dz + r * H, H * 2), lane * 2, 0, 0);
        const Rsrc rn = row_rsrc(a.dn + r * C, C * 2);
        /* dn one head's columns at a time (a loop, so w's LDS reads are not all hoisted into registers) */
#pragma unroll 1
        for (int k = 0; k < H; k++) {
            float x0 = 0.0f, x1 = 0.0f;
#pragma unroll
            for (int h = 0; h < H; h++) {
                const float2 wv = *reinterpret_cast<const float2 *>(ws + h * C + k * HEAD_DIM + 2 * lane);
                x0 = __builtin_fmaf(dz[h], wv.x, x0);
                x1 = __builtin_fmaf(dz[h], wv.y, x1);
            }
            __builtin_amdgcn_raw_buffer_store_b32((uint32_t)f32_to_bf16(x0) | ((uint32_t)f32_to_bf16(x1) << 16), rn,
                                                  (k * HEAD_DIM + 2 * lane) * 2, 0, 0);
        }
    }
    if (started && cur_ok) flush_run<H>(a.dtable, cur, acc, lane, true);
}

/* Workgroups for `rows` rows: every row a wave, at most as many workgroups as the device holds at once (the
 * kernel's resident workgroups per device, cached per device in `resident`). */
template <typename K>
int ve_blocks(K kernel, long long rows, int (&resident)[64]) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -1;
    if (!resident[dev]) {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, VE_THREADS, 0) != hipSuccess)
            return -1;
        resident[dev] = max(1, cus) * max(1, per_cu);
    }
    const long long need = (rows + VE_WAVES - 1) / VE_WAVES;
    return (int)max(1LL, min(need, (long long)resident[dev]));
}

template <int H>
int launch_forward(const VeFwd &a, hipStream_t stream) {
    static int resident[64] = {0};
    const int blocks = ve_blocks(ve_forward_kernel<H>, a.rows, resident);
    if (blocks < 0) return (int)hipErrorInvalidDevice;
    hipLaunchKernelGGL(ve_forward_kernel<H>, dim3(blocks), dim3(VE_THREADS), 0, stream, a);
    return (int)hipGetLastError();
}

template <int H>
int launch_backward(const VeBwd &a, hipStream_t stream) {
    static int resident[64] = {0};
    const int blocks = ve_blocks(ve_backward_kernel<H>, a.rows, resident);
    if (blocks < 0) return (int)hipErrorInvalidDevice;
    hipLaunchKernelGGL(ve_backward_kernel<H>, dim3(blocks), dim3(VE_THREADS), 0, stream, a);
    return (int)hipGetLastError();
}

template <int H = 1>
int dispatch(int heads, bool fwd, const VeFwd &f, const VeBwd &b, hipStream_t stream) {
    if constexpr (H > VE_MAX_HEADS) {
        return NC_ERR_SHAPE;
    } else {
        if (heads == H) return fwd ? launch_forward<H>(f, stream) : launch_backward<H>(b, stream);
        return dispatch<H + 1>(heads, fwd, f, b, stream);
    }
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

int check_forward(const VeFwd &a, int heads) {
    if (heads < 1 || heads > VE_MAX_HEADS || a.rows < 0 || a.vocab < 1 || a.v_stride < (long long)heads * HEAD_DIM ||
        a.v_stride % 8)
        return NC_ERR_SHAPE;
    if (a.rows == 0) return NC_OK;
    if (!a.n || !a.v || !a.idx || !a.table || !a.w || !a.out || !a.gate) return NC_ERR_NULL;
    if (!aligned16(a.n) || !aligned16(a.v) || !aligned16(a.table) || !aligned16(a.w) || !aligned16(a.out) ||
        ((uintptr_t)a.gate & 3))
        return NC_ERR_SHAPE;
    return NC_OK;
}

int check_backward(const VeBwd &a, int heads) {
    if (heads < 1 || heads > VE_MAX_HEADS || a.rows < 0 || a.vocab < 1 ||
        a.dout_stride < (long long)heads * HEAD_DIM || a.dout_stride % 8)
        return NC_ERR_SHAPE;
    if (a.rows == 0) return NC_OK;
    if (!a.dout || !a.ids || !a.order || !a.table || !a.w || !a.gate || !a.dn || !a.dtable || !a.dz)
        return NC_ERR_NULL;
    if (!aligned16(a.dout) || !aligned16(a.table) || !aligned16(a.w) || !aligned16(a.dn) || !aligned16(a.dtable) ||
        ((uintptr_t)a.gate & 3) || ((uintptr_t)a.dz & 1) || ((uintptr_t)a.order & 7))
        return NC_ERR_SHAPE;
    return NC_OK;
}

int ve_forward_run(const VeFwd &a, int heads, hipStream_t stream) {
    const int st = check_forward(a, heads);
    if (st != NC_OK || a.rows == 0) return st;
    return dispatch(heads, true, a, VeBwd{}, stream);
}

int ve_backward_run(const VeBwd &a, int heads, hipStream_t stream) {
    const int st = check_backward(a, heads);
    if (st != NC_OK || a.rows == 0) return st;
    return dispatch(heads, false, VeFwd{}, a, stream);
}

VeFwd forward_args(const void *n, const void *v, long long v_stride, const void *idx, const void *table,
                   long long vocab, const void *w, void *out, void *gate, long long rows) {
    return VeFwd{(const uint16_t *)n, (const uint16_t *)v, v_stride, (const int32_t *)idx, (const float *)table, vocab,
                 (const float *)w, (uint16_t *)out, (float *)gate, rows};
}

VeBwd backward_args(const void *dout, long long dout_stride, const void *ids, const void *order, const void *table,
                    long long vocab, const void *w, const void *gate, void *dn, void *dtable, void *dz, long long rows) {
    return VeBwd{(const uint16_t *)dout, dout_stride, (const int32_t *)ids, (const long long *)order,
                 (const float *)table, vocab, (const float *)w, (const float *)gate, (uint16_t *)dn, (float *)dtable,
                 (uint16_t *)dz, rows};
}

}  // namespace
}  // namespace nc

using namespace nc;

/* The table's row count is not an argument of the reference's entry points: tokens are trusted, as there. */
static constexpr long long UNCHECKED_VOCAB = 0x7FFFFFFFLL;

extern "C" void ve_forward(const void *n, const void *v, long long v_stride, const void *idx, const void *table,
                           const void *w, void *out, void *gate, long long rows, void *stream) {
    set_last_error(ve_forward_run(forward_args(n, v, v_stride, idx, table, UNCHECKED_VOCAB, w, out, gate, rows),
                                  REF_HEADS, (hipStream_t)stream));
}

extern "C" void ve_backward(const void *dout, long long dout_stride, const void *ids, const void *order,
                            const void *table, const void *w, const void *gate, void *dn, void *dtable, void *dz,
                            long long rows, void *stream) {
    set_last_error(ve_backward_run(backward_args(dout, dout_stride, ids, order, table, UNCHECKED_VOCAB, w, gate, dn,
                                                 dtable, dz, rows),
                                   REF_HEADS, (hipStream_t)stream));
}

extern "C" int nc_ve_forward(const void *n, const void *v, long long v_stride, const int32_t *idx, const float *table,
                             long long vocab, const float *w, void *out, float *gate, long long rows, int heads,
                             void *stream) {
    return ve_forward_run(forward_args(n, v, v_stride, idx, table, vocab, w, out, gate, rows), heads,
                          (hipStream_t)stream);
}

extern "C" int nc_ve_backward(const void *dout, long long dout_stride, const int32_t *ids, const int64_t *order,
                              const float *table, long long vocab, const float *w, const float *gate, void *dn,
                              float *dtable, void *dz, long long rows, int heads, void *stream) {
    return ve_backward_run(backward_args(dout, dout_stride, ids, order, table, vocab, w, gate, dn, dtable, dz, rows),
                           heads, (hipStream_t)stream);
}
