/*
 * The decode step's GEMMs on gfx950: out[n][r] = epilogue(sum_k x[n][k] W[r][k]) for a few slots (n < N <= 128) and
 * many weight rows, bf16 operands, fp32 accumulation. Weight-streaming: every weight byte is read once from HBM.
 *
 * Grid: (R / 128 row blocks) x S K-slices. A workgroup (8 waves) owns 128 weight rows (16 per wave) and all N slots
 * over its K-slice, walked in 128-wide chunks. Each chunk of x (N x 128 bf16) is staged once in LDS (double
 * buffered) and shared by the eight waves; each wave streams its 16 weight rows from HBM into registers two chunks
 * ahead and accumulates with v_mfma_f32_16x16x32_bf16 (A = 16 weight rows, B = 16 slots from LDS). MFMA j of a
 * chunk at k0 contracts, in lane group g = lane / 16, over k = k0 + 8 (4 j + g) .. + 7 of both operands (any k order
 * common to A and B gives the same dot product), so each weight load instruction covers 64 contiguous bytes of a
 * row. Staged x rows are 256 bytes with their 16-byte blocks XOR-swizzled by the row (block b of row n
 * at b ^ (n % 16)), so the sixteen rows an operand read touches fall in distinct banks.
 *
 * Pipeline, step c: issue the loads of x(c + 2) and weights(c + 2); run chunk c's MFMAs (x(c) in LDS, weights(c) in
 * registers); store x(c + 1), loaded one step earlier, into the other LDS buffer; barrier. Vector-memory counters
 * retire in issue order, so a step only waits for loads issued a step earlier and this step's stay in flight.
 * Registers rotate by name (weights over three buffers, x over two: the loop is unrolled by six), so no copy ever
 * waits on a load.
 *
 * S = 1: the workgroup applies the epilogue itself:
 *   STORE   out = bf16(s)                           (qkv)
 *   RESID2  x = s + res (fp32); out = bf16(x); xf = x   (o_proj)
 *   RELU2   p = s rstd[n]; out = bf16(relu(p) p)    (fc)
 *   RESID   out = bf16(s + res)                     (proj)
 *   F32     xf = s                                  (lm_head logits)
 * S > 1: each workgroup stores its fp32 partial sums to part[s][n][r]; the consumer adds the S partials in slice
 * order (deterministic) before the same epilogue (sg_reduce_kernel here, or the decoder's rstd / ReLU^2 kernels).
 *
 * Reference: the slot GEMM and its epilogues, model/kernels/decode.cu:133-168, 295-359.
 */
#include <type_traits>

#include "nc_device.h"
#include "nc_internal.h"

namespace nc {

constexpr int SG_WAVES = 8;
constexpr int SG_THREADS = SG_WAVES * WAVE;
constexpr int SG_ROWS = 16 * SG_WAVES;  /* weight rows per workgroup */
constexpr int SG_CHUNK = 128;           /* k per chunk */
constexpr int SG_XROW = SG_CHUNK * 2;   /* bytes per staged x row */
constexpr int SG_TARGET_WGS = 256;      /* split K until about this many workgroups */

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bool sg_live(const unsigned long long *mask, int n) {
    return !mask || ((mask[n >> 6] >> (n & 63)) & 1ull);
}

/* A lane's four 16-byte pieces of a weight row's 256-byte chunk: piece j at bytes 64 j + 16 g (lane group g), so
 * one load instruction reads 64 contiguous bytes of each of its 16 rows. (Plain loads: a non-temporal hint let lines
 * leave the cache between the instructions that share them.) */
struct Frag {
    u32x4 v[4];
};

__device__ __forceinline__ Frag load_frag(const uint16_t *p) {
    const u32x4 *q = reinterpret_cast<const u32x4 *>(p);
    Frag f;
#pragma unroll
    for (int j = 0; j < 4; j++) f.v[j] = q[4 * j];
    return f;
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4 &u) { return __builtin_bit_cast(bf16x8, u); }

/* Apply the epilogue to four consecutive rows r .. r + 3 of slot n (sums s). */
template <int EPI>
__device__ __forceinline__ void sg_store(const SkinnyGemm &g, int n, int r, float s[4]) {
    const long long at = (long long)n * g.R + r;
    if (EPI == SG_F32) {
        *reinterpret_cast<float4 *>(g.out_f32 + at) = make_float4(s[0], s[1], s[2], s[3]);
        return;
    }
    if (EPI == SG_RESID || EPI == SG_RESID2) {
        const uint2 rr = *reinterpret_cast<const uint2 *>(g.res + at);
        const float res[4] = {bf16_to_f32((uint16_t)rr.x), bf16_to_f32((uint16_t)(rr.x >> 16)),
                              bf16_to_f32((uint16_t)rr.y), bf16_to_f32((uint16_t)(rr.y >> 16))};
#pragma unroll
        for (int i = 0; i < 4; i++) s[i] = s[i] + res[i];
        if (EPI == SG_RESID2) *reinterpret_cast<float4 *>(g.out_f32 + at) = make_float4(s[0], s[1], s[2], s[3]);
    } else if (EPI == SG_RELU2) {
        const float r_ = g.rstd[n];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float p = s[i] * r_;
            s[i] = fmaxf(p, 0.0f) * p;
        }
    }
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = f32_to_bf16(s[i]);
    *reinterpret_cast<uint2 *>(g.out + at) =
        make_uint2((uint32_t)o[0] | (uint32_t)o[1] << 16, (uint32_t)o[2] | (uint32_t)o[3] << 16);
}

/* EPI < 0: store partial sums (S > 1). */
template <int CT, int EPI>
__global__ void __launch_bounds__(SG_THREADS) skinny_gemm_kernel(SkinnyGemm g, float *part, int S) {
    constexpr int NP = 16 * CT;                         /* staged slot rows (zeros past N) */
    constexpr int PIECES = NP * SG_XROW / 16 / SG_THREADS;   /* 16-byte pieces of a chunk per thread */
    constexpr int PIECES_T = PIECES > 0 ? PIECES : 1;
    __shared__ __align__(16) unsigned char xs[2][NP * SG_XROW];
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    const int row_in = lane & 15, grp = lane >> 4;
    const int r0 = blockIdx.x * SG_ROWS + wave * 16;
    const int chunks = g.K / SG_CHUNK, s = blockIdx.y;
    const int c_begin = s * chunks / S, c_end = (s + 1) * chunks / S;

    f32x4 acc[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ct++) acc[ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    /* weight rows past R read row R - 1 (in bounds; their sums are never stored) */
    const uint16_t *wrow = g.w + (long long)min(r0 + row_in, g.R - 1) * g.K + grp * 8;

    /* staging: piece p = tid + 512 i is slot row p / 16, logical block p % 16, stored at block (p % 16) ^ (row % 16);
     * slot rows past N load row N - 1 and store zeros (branch-free). With NP * 16 < 512 pieces (N <= 16), threads
     * past the chunk repeat a piece (same bytes, same place). */
    auto load_x = [&](int c, u32x4 *v) {
#pragma unroll
        for (int i = 0; i < PIECES_T; i++) {
            const int p = (tid + SG_THREADS * i) % (NP * 16), n = min(p >> 4, g.N - 1), blk = p & 15;
            v[i] = *reinterpret_cast<const u32x4 *>(g.x + (long long)n * g.K + c * SG_CHUNK + blk * 8);
        }
    };
    auto store_x = [&](int buf, const u32x4 *v) {
#pragma unroll
        for (int i = 0; i < PIECES_T; i++) {
            const int p = (tid + SG_THREADS * i) % (NP * 16), n = p >> 4, blk = p & 15;
            const u32x4 val = n < g.N ? v[i] : u32x4{0u, 0u, 0u, 0u};
            *reinterpret_cast<u32x4 *>(&xs[buf][n * SG_XROW + ((blk ^ (n & 15)) << 4)]) = val;
        }
    };

    if (c_begin < c_end) {
        u32x4 xa[PIECES_T], xb[PIECES_T];
        Frag f0 = {}, f1 = {}, f2 = {};
        load_x(c_begin, xa);
        f0 = load_frag(wrow + c_begin * SG_CHUNK);
        if (c_begin + 1 < c_end) {
            load_x(c_begin + 1, xb);
            f1 = load_frag(wrow + (c_begin + 1) * SG_CHUNK);
        }
        store_x(c_begin & 1, xa);
        __syncthreads();
        /* step c: xcur holds x(c + 1), xnext receives x(c + 2) */
        auto step = [&](auto full, int c, const Frag &use, Frag &fill, const u32x4 *xcur, u32x4 *xnext) {
            if (full || c + 2 < c_end) {
                load_x(c + 2, xnext);
                fill = load_frag(wrow + (c + 2) * SG_CHUNK);
            }
            __builtin_amdgcn_sched_barrier(0);
            const unsigned char *stage = xs[c & 1];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const bf16x8 aj = as_bf16x8(use.v[j]);
                const int blk = (j * 4 + grp) ^ row_in;   /* k block 4 j + g; (ct 16 + row_in) % 16 == row_in */
                u32x4 b[CT];
#pragma unroll
                for (int ct = 0; ct < CT; ct++)
                    b[ct] = *reinterpret_cast<const u32x4 *>(stage + (ct * 16 + row_in) * SG_XROW + (blk << 4));
#pragma unroll
                for (int ct = 0; ct < CT; ct++) acc[ct] = mfma16x16x32(aj, as_bf16x8(b[ct]), acc[ct]);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (full || c + 1 < c_end) store_x((c + 1) & 1, xcur);
            __syncthreads();
        };
        const std::true_type full{};
        const std::false_type guarded{};
        int c = c_begin;
        for (; c + 7 < c_end; c += 6) {
            step(full, c, f0, f2, xb, xa);
            step(full, c + 1, f1, f0, xa, xb);
            step(full, c + 2, f2, f1, xb, xa);
            step(full, c + 3, f0, f2, xa, xb);
            step(full, c + 4, f1, f0, xb, xa);
            step(full, c + 5, f2, f1, xa, xb);
        }
        for (int k = 0; c + k < c_end; k++) {   /* at most seven chunks remain */
            switch (k % 6) {
            case 0: step(guarded, c + k, f0, f2, xb, xa); break;
            case 1: step(guarded, c + k, f1, f0, xa, xb); break;
            case 2: step(guarded, c + k, f2, f1, xb, xa); break;
            case 3: step(guarded, c + k, f0, f2, xa, xb); break;
            case 4: step(guarded, c + k, f1, f0, xb, xa); break;
            default: step(guarded, c + k, f2, f1, xa, xb); break;
            }
        }
    }

    /* lane (group q = lane / 16, slot lane % 16) holds rows 4 q .. 4 q + 3 of the wave's tile */
    const int r = r0 + grp * 4;
    if (r >= g.R) return;
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
        const int n = ct * 16 + row_in;
        if (n >= g.N || !sg_live(g.active, n)) continue;
        float v[4] = {acc[ct][0], acc[ct][1], acc[ct][2], acc[ct][3]};
        if (EPI < 0)
            *reinterpret_cast<float4 *>(part + ((long long)s * g.N + n) * g.R + r) = make_float4(v[0], v[1], v[2], v[3]);
        else
            sg_store<EPI>(g, n, r, v);
    }
}

/* The S partials of each output summed in slice order, then the epilogue; a thread per four rows of one slot. */
template <int EPI>
__global__ void __launch_bounds__(256) sg_reduce_kernel(SkinnyGemm g, const float *part, int S) {
    const int n = blockIdx.y;
    const int r = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (r >= g.R || !sg_live(g.active, n)) return;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = 0; s < S; s++) {
        const float4 p = *reinterpret_cast<const float4 *>(part + ((long long)s * g.N + n) * g.R + r);
        v[0] = v[0] + p.x;
        v[1] = v[1] + p.y;
        v[2] = v[2] + p.z;
        v[3] = v[3] + p.w;
    }
    sg_store<EPI>(g, n, r, v);
}

template <int CT, int EPI>
static void launch_one(const SkinnyGemm &g, float *part, int S, hipStream_t stream) {
    const dim3 grid((g.R + SG_ROWS - 1) / SG_ROWS, S), block(SG_THREADS);
    hipLaunchKernelGGL((skinny_gemm_kernel<CT, EPI>), grid, block, 0, stream, g, part, S);
}

template <int CT>
static hipError_t launch_ct(const SkinnyGemm &g, int epi, float *part, int S, hipStream_t stream) {
    if (S > 1) {
        launch_one<CT, -1>(g, part, S, stream);
        return hipGetLastError();
    }
    switch (epi) {
    case SG_STORE: launch_one<CT, SG_STORE>(g, part, S, stream); break;
    case SG_RESID2: launch_one<CT, SG_RESID2>(g, part, S, stream); break;
    case SG_RELU2: launch_one<CT, SG_RELU2>(g, part, S, stream); break;
    case SG_RESID: launch_one<CT, SG_RESID>(g, part, S, stream); break;
    default: launch_one<CT, SG_F32>(g, part, S, stream); break;
    }
    return hipGetLastError();
}

bool skinny_gemm_fits(int R, int K, int N) {
    return N >= 1 && N <= SG_MAX_N && K >= SG_CHUNK && K % SG_CHUNK == 0 && R >= 1 && R % 4 == 0;
}

int skinny_gemm_slices(int R, int K) {
    const int blocks = (R + SG_ROWS - 1) / SG_ROWS, chunks = K / SG_CHUNK;
    int S = (SG_TARGET_WGS + blocks - 1) / blocks;
    S = S < 1 ? 1 : S;
    S = S > chunks / 2 ? chunks / 2 : S;   /* at least two chunks a slice */
    return S < 1 ? 1 : S;
}

int skinny_gemm(const SkinnyGemm &g, int epi, float *part, int S, hipStream_t stream) {
    if (!skinny_gemm_fits(g.R, g.K, g.N) || S < 1 || S > g.K / SG_CHUNK || (S > 1 && !part)) return -2;
    hipError_t e;
    if (g.N <= 16) e = launch_ct<1>(g, epi, part, S, stream);
    else if (g.N <= 32) e = launch_ct<2>(g, epi, part, S, stream);
    else if (g.N <= 64) e = launch_ct<4>(g, epi, part, S, stream);
    else e = launch_ct<8>(g, epi, part, S, stream);
    return (int)e;
}

int skinny_gemm_reduce(const SkinnyGemm &g, int epi, const float *part, int S, hipStream_t stream) {
    const dim3 grid((g.R / 4 + 255) / 256, g.N), block(256);
    switch (epi) {
    case SG_STORE: hipLaunchKernelGGL(sg_reduce_kernel<SG_STORE>, grid, block, 0, stream, g, part, S); break;
    case SG_RESID2: hipLaunchKernelGGL(sg_reduce_kernel<SG_RESID2>, grid, block, 0, stream, g, part, S); break;
    case SG_RELU2: hipLaunchKernelGGL(sg_reduce_kernel<SG_RELU2>, grid, block, 0, stream, g, part, S); break;
    case SG_RESID: hipLaunchKernelGGL(sg_reduce_kernel<SG_RESID>, grid, block, 0, stream, g, part, S); break;
    default: hipLaunchKernelGGL(sg_reduce_kernel<SG_F32>, grid, block, 0, stream, g, part, S); break;
    }
    return (int)hipGetLastError();
}

}  // namespace nc
