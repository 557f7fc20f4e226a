/*
 * The decode step's GEMMs on gfx950: out[n][r] = epilogue(sum_k x[n][k] w[r][k]) for a step's slots (n < N <= 128)
 * and many weight rows, bf16 operands, fp32 accumulation, every weight byte read once from HBM.
 *
 * Every global access goes through a buffer resource whose range is the exact extent of its array, so the hardware
 * range check turns any access outside an operand into a zero read or a dropped write (never a fault); the stores'
 * row and slot masks keep ragged tiles out of the neighbouring rows of the same array.
 *
 * Grid (ceil(R / 128) row blocks, S K-slices of at most GM_KC 128-wide chunks), 4 waves. A workgroup loads its whole
 * slice at once and waits once (a slab: no software pipeline, every load is in flight together):
 *   - the slots' x over the slice (CT * 16 slots x up to 512 k, up to 128 KiB) goes straight to LDS by buffer loads
 *     with the LDS destination (16 bytes a lane, 1 KiB an instruction); slot row n's 16-byte block b lands at block
 *     b ^ (n % 16) (each lane picks the global block that belongs at its LDS position), so the 16 rows of one MFMA
 *     operand read fall in distinct banks;
 *   - a wave owns 32 weight rows (two 16-row MFMA tiles) and loads all of them for the slice into registers: lane
 *     (g = lane / 16, i = lane % 16) of tile t holds row 32 w + 16 t + i, bytes 64 j + 16 g of each chunk's 256
 *     (piece j), so load instruction j covers 64 contiguous bytes of each of 16 rows and MFMA j
 *     (v_mfma_f32_16x16x32_bf16) contracts k = 32 j .. 32 j + 31 of the chunk.
 * Chunks past the slice are read at GM_PAST, beyond every operand's range (zeros, no memory access), so no load is
 * conditional; the chunks are added in order.
 *
 * S = 1: the workgroup applies the epilogue itself (SkinnyGemm's SG_* kinds, nc_internal.h). S > 1: fp32 partial
 * sums to part[s][n][r], reduced in slice order (deterministic) by stream_gemm_reduce before the same epilogue.
 *
 * Reference: the slot GEMM and its epilogues, model/kernels/decode.cu:133-168, 295-359.
 */
#include "nc_device.h"
#include "nc_internal.h"

namespace nc {

constexpr int GM_WAVES = 4;
constexpr int GM_THREADS = GM_WAVES * WAVE;
constexpr int GM_WAVE_ROWS = 32;                        /* two 16-row MFMA tiles */
constexpr int GM_ROWS = GM_WAVE_ROWS * GM_WAVES;        /* weight rows per workgroup */
constexpr int GM_CHUNK = 128;                           /* k per pipeline step */
constexpr int GM_XROW = GM_CHUNK * 2;                   /* bytes of one staged slot row */
constexpr int GM_KC = 4;                                /* chunks per slice at most (x: 128 KiB of LDS) */
constexpr int GM_TARGET_WGS = 128;                      /* more slices than the minimum until this many workgroups */
constexpr int GM_PAST = 0x7FFF0000;   /* a byte offset past every operand's range (operands stay below it) */

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t Rsrc;

/* A raw buffer over `bytes` bytes from p (bytes < 2^31, checked by the host). */
__device__ __forceinline__ Rsrc rsrc(const void *p, long long bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ u32x4 bload16(Rsrc r, int off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }
__device__ __forceinline__ u32x2 bload8(Rsrc r, int off) { return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0); }
__device__ __forceinline__ float bloadf(Rsrc r, int off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ void bstore16(Rsrc r, int off, u32x4 v) { __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 0); }
__device__ __forceinline__ void bstore8(Rsrc r, int off, u32x2 v) { __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, 0); }

__device__ __forceinline__ bool gm_live(const unsigned long long *mask, int n) {
    return !mask || ((mask[n >> 6] >> (n & 63)) & 1ull);
}

/* A wave's weights of one chunk: [tile][piece]. */
struct WChunk {
    u32x4 v[2][4];
};

typedef __attribute__((address_space(3))) void LdsPtr;

/* The operand views of one launch. */
struct GemmViews {
    Rsrc w, x, out, out_f32, res, rstd, part;
};

/* part_bytes: the partial-sum buffer's allocation (the caller's), so its range is the allocation itself. */
__device__ __forceinline__ GemmViews views(const SkinnyGemm &g, const float *part, long long part_bytes) {
    GemmViews v;
    v.w = rsrc(g.w, (long long)g.R * g.K * 2);
    v.x = rsrc(g.x, (long long)g.N * g.K * 2);
    v.out = rsrc(g.out, g.out ? (long long)g.N * g.R * 2 : 0);
    v.out_f32 = rsrc(g.out_f32, g.out_f32 ? (long long)g.N * g.R * 4 : 0);
    v.res = rsrc(g.res, g.res ? (long long)g.N * g.R * 2 : 0);
    v.rstd = rsrc(g.rstd, g.rstd ? (long long)g.N * 4 : 0);
    v.part = rsrc(part, part ? part_bytes : 0);
    return v;
}

/* The epilogue of four consecutive rows r .. r + 3 of slot n (sums s); at = (n R + r). */
template <int EPI>
__device__ __forceinline__ void gm_store(const GemmViews &v, const SkinnyGemm &g, int n, int at, float s[4]) {
    if (EPI == SG_F32) {
        bstore16(v.out_f32, at * 4, u32x4{__float_as_uint(s[0]), __float_as_uint(s[1]), __float_as_uint(s[2]),
                                          __float_as_uint(s[3])});
        return;
    }
    if (EPI == SG_RESID || EPI == SG_RESID2) {
        const u32x2 rr = bload8(v.res, at * 2);
        const float res[4] = {bf16_to_f32((uint16_t)rr[0]), bf16_to_f32((uint16_t)(rr[0] >> 16)),
                              bf16_to_f32((uint16_t)rr[1]), bf16_to_f32((uint16_t)(rr[1] >> 16))};
#pragma unroll
        for (int i = 0; i < 4; i++) s[i] = s[i] + res[i];
        if (EPI == SG_RESID2)
            bstore16(v.out_f32, at * 4, u32x4{__float_as_uint(s[0]), __float_as_uint(s[1]), __float_as_uint(s[2]),
                                              __float_as_uint(s[3])});
    } else if (EPI == SG_RELU2) {
        const float r_ = bloadf(v.rstd, n * 4);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float p = s[i] * r_;
            s[i] = fmaxf(p, 0.0f) * p;
        }
    }
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = f32_to_bf16(s[i]);
    bstore8(v.out, at * 2, u32x2{(uint32_t)o[0] | (uint32_t)o[1] << 16, (uint32_t)o[2] | (uint32_t)o[3] << 16});
}

/* EPI < 0: store partial sums (S > 1). */
template <int CT, int EPI>
__global__ void __launch_bounds__(GM_THREADS) stream_gemm_kernel(SkinnyGemm g, float *part, long long part_bytes,
                                                                  int S) {
    constexpr int NP = 16 * CT;   /* staged slot rows (buffer reads past N return zeros) */
    __shared__ __align__(16) unsigned char xs[GM_KC][NP * GM_XROW];
    const GemmViews v = views(g, part, part_bytes);
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    const int i16 = lane & 15, grp = lane >> 4;
    const int r0 = blockIdx.x * GM_ROWS + wave * GM_WAVE_ROWS;
    const int chunks = g.K / GM_CHUNK, s = blockIdx.y;
    const int c_begin = s * chunks / S, c_end = (s + 1) * chunks / S;   /* at most GM_KC chunks (host-checked) */
    const int rowb = g.K * 2;   /* bytes of a weight or slot row */

    /* x: instruction i of chunk q fills LDS bytes [1024 i, 1024 i + 1024) of xs[q], slot rows 4 i .. 4 i + 3; the
     * four waves take i = wave, wave + 4, ... */
#pragma unroll
    for (int q = 0; q < GM_KC; q++) {
        const int c = c_begin + q;
#pragma unroll
        for (int k = 0; k < CT; k++) {
            const int i = wave + 4 * k, n = 4 * i + grp, lb = i16 ^ (n & 15);
            const int off = c < c_end ? n * rowb + c * GM_XROW + lb * 16 : GM_PAST;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(v.x, (LdsPtr *)&xs[q][i * 1024], 16, off, 0, 0, 0);
        }
    }
    /* weights: all of the slice's chunks in registers */
    const int woff0 = (r0 + i16) * rowb + grp * 16;
    const int woff1 = woff0 + 16 * rowb;
    WChunk f[GM_KC];
#pragma unroll
    for (int q = 0; q < GM_KC; q++) {
        const int c = c_begin + q;
        const int o0 = c < c_end ? woff0 + c * GM_XROW : GM_PAST, o1 = c < c_end ? woff1 + c * GM_XROW : GM_PAST;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            f[q].v[0][j] = bload16(v.w, o0 + 64 * j);
            f[q].v[1][j] = bload16(v.w, o1 + 64 * j);
        }
    }

    f32x4 acc[2][CT];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int ct = 0; ct < CT; ct++) acc[t][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    __syncthreads();   /* waits for the LDS loads of every wave */
#pragma unroll
    for (int q = 0; q < GM_KC; q++) {
        if (c_begin + q >= c_end) break;
        const unsigned char *stage = xs[q];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int blk = (4 * j + grp) ^ i16;   /* k block 4 j + g of slot row ct 16 + i16 */
            u32x4 b[CT];
#pragma unroll
            for (int ct = 0; ct < CT; ct++)
                b[ct] = *reinterpret_cast<const u32x4 *>(stage + (ct * 16 + i16) * GM_XROW + (blk << 4));
            const bf16x8 a0 = __builtin_bit_cast(bf16x8, f[q].v[0][j]);
            const bf16x8 a1 = __builtin_bit_cast(bf16x8, f[q].v[1][j]);
#pragma unroll
            for (int ct = 0; ct < CT; ct++) {
                acc[0][ct] = mfma16x16x32(a0, __builtin_bit_cast(bf16x8, b[ct]), acc[0][ct]);
                acc[1][ct] = mfma16x16x32(a1, __builtin_bit_cast(bf16x8, b[ct]), acc[1][ct]);
            }
        }
    }

    /* lane (g, i16) holds rows 4 g .. 4 g + 3 of each tile for slot ct 16 + i16 */
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int r = r0 + 16 * t + 4 * grp;
        if (r >= g.R) continue;
#pragma unroll
        for (int ct = 0; ct < CT; ct++) {
            const int n = ct * 16 + i16;
            if (n >= g.N || !gm_live(g.active, n)) continue;
            float sv[4] = {acc[t][ct][0], acc[t][ct][1], acc[t][ct][2], acc[t][ct][3]};
            if (EPI < 0)
                bstore16(v.part, ((s * g.N + n) * g.R + r) * 4,
                         u32x4{__float_as_uint(sv[0]), __float_as_uint(sv[1]), __float_as_uint(sv[2]),
                               __float_as_uint(sv[3])});
            else
                gm_store<EPI < 0 ? SG_STORE : EPI>(v, g, n, n * g.R + r, sv);
        }
    }
}

/* The S partials of four rows of one slot summed in slice order, then the epilogue; a thread per four rows. */
template <int EPI>
__global__ void __launch_bounds__(256) stream_gemm_reduce_kernel(SkinnyGemm g, const float *part,
                                                                  long long part_bytes, int S) {
    const int n = blockIdx.y;
    const int r = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (r >= g.R || !gm_live(g.active, n)) return;
    const GemmViews v = views(g, part, part_bytes);
    float sv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = 0; s < S; s++) {
        const u32x4 p = bload16(v.part, ((s * g.N + n) * g.R + r) * 4);
#pragma unroll
        for (int i = 0; i < 4; i++) sv[i] = sv[i] + __uint_as_float(p[i]);
    }
    gm_store<EPI>(v, g, n, n * g.R + r, sv);
}

template <int CT, int EPI>
static void gm_launch(const SkinnyGemm &g, float *part, long long part_bytes, int S, hipStream_t stream) {
    const dim3 grid((g.R + GM_ROWS - 1) / GM_ROWS, S), block(GM_THREADS);
    hipLaunchKernelGGL((stream_gemm_kernel<CT, EPI>), grid, block, 0, stream, g, part, part_bytes, S);
}

template <int CT>
static hipError_t gm_launch_ct(const SkinnyGemm &g, int epi, float *part, long long part_bytes, int S,
                               hipStream_t stream) {
    if (S > 1) {
        gm_launch<CT, -1>(g, part, part_bytes, S, stream);
        return hipGetLastError();
    }
    switch (epi) {
    case SG_STORE: gm_launch<CT, SG_STORE>(g, part, part_bytes, S, stream); break;
    case SG_RESID2: gm_launch<CT, SG_RESID2>(g, part, part_bytes, S, stream); break;
    case SG_RELU2: gm_launch<CT, SG_RELU2>(g, part, part_bytes, S, stream); break;
    case SG_RESID: gm_launch<CT, SG_RESID>(g, part, part_bytes, S, stream); break;
    default: gm_launch<CT, SG_F32>(g, part, part_bytes, S, stream); break;
    }
    return hipGetLastError();
}

bool stream_gemm_fits(int R, int K, int N) {
    /* every byte offset, including those of the rows and slots past R and N a tile covers, fits an int */
    return N >= 1 && N <= SG_MAX_N && K >= GM_CHUNK && K % GM_CHUNK == 0 && R >= 1 && R % 4 == 0 &&
           (long long)(R + GM_ROWS) * K * 2 <= GM_PAST && (long long)SG_MAX_N * K * 2 <= GM_PAST &&
           (long long)N * R * 4 <= GM_PAST;
}

int stream_gemm_min_slices(int K) { return (K / GM_CHUNK + GM_KC - 1) / GM_KC; }

int stream_gemm_slices(int R, int K) {
    const int blocks = (R + GM_ROWS - 1) / GM_ROWS, chunks = K / GM_CHUNK;
    int S = stream_gemm_min_slices(K);
    const int want = (GM_TARGET_WGS + blocks - 1) / blocks;
    if (want > S) S = want > chunks ? chunks : want;
    return S;
}

long long stream_gemm_part_bytes(int R, int N, int S) { return S > 1 ? (long long)S * N * R * 4 : 0; }

/* The partial sums of S slices fit the caller's part_bytes (and an int offset). */
static bool part_fits(const SkinnyGemm &g, const float *part, long long part_bytes, int S) {
    const long long need = stream_gemm_part_bytes(g.R, g.N, S);
    return part && need <= part_bytes && part_bytes < (1LL << 31);
}

int stream_gemm(const SkinnyGemm &g, int epi, float *part, long long part_bytes, int S, hipStream_t stream) {
    if (!stream_gemm_fits(g.R, g.K, g.N) || S < stream_gemm_min_slices(g.K) || S > g.K / GM_CHUNK) return -2;
    if (S > 1 && !part_fits(g, part, part_bytes, S)) return -2;
    if (epi < SG_STORE || epi > SG_F32) return -2;
    if (S == 1) {
        const bool need_out = epi != SG_F32, need_f32 = epi == SG_F32 || epi == SG_RESID2;
        const bool need_res = epi == SG_RESID || epi == SG_RESID2;
        if ((need_out && !g.out) || (need_f32 && !g.out_f32) || (need_res && !g.res) || (epi == SG_RELU2 && !g.rstd))
            return -2;
    }
    hipError_t e;
    if (S == 1) part_bytes = 0;
    if (g.N <= 16) e = gm_launch_ct<1>(g, epi, part, part_bytes, S, stream);
    else if (g.N <= 32) e = gm_launch_ct<2>(g, epi, part, part_bytes, S, stream);
    else if (g.N <= 64) e = gm_launch_ct<4>(g, epi, part, part_bytes, S, stream);
    else e = gm_launch_ct<8>(g, epi, part, part_bytes, S, stream);
    return (int)e;
}

int stream_gemm_reduce(const SkinnyGemm &g, int epi, const float *part, long long part_bytes, int S,
                       hipStream_t stream) {
    if (!stream_gemm_fits(g.R, g.K, g.N) || S < 2 || !part_fits(g, part, part_bytes, S)) return -2;
    const bool need_out = epi != SG_F32, need_f32 = epi == SG_F32 || epi == SG_RESID2;
    const bool need_res = epi == SG_RESID || epi == SG_RESID2;
    if ((need_out && !g.out) || (need_f32 && !g.out_f32) || (need_res && !g.res) || (epi == SG_RELU2 && !g.rstd))
        return -2;
    const dim3 grid((g.R / 4 + 255) / 256, g.N), block(256);
    switch (epi) {
    case SG_STORE: hipLaunchKernelGGL(stream_gemm_reduce_kernel<SG_STORE>, grid, block, 0, stream, g, part, part_bytes, S);
        break;
    case SG_RESID2: hipLaunchKernelGGL(stream_gemm_reduce_kernel<SG_RESID2>, grid, block, 0, stream, g, part, part_bytes, S);
        break;
    case SG_RELU2: hipLaunchKernelGGL(stream_gemm_reduce_kernel<SG_RELU2>, grid, block, 0, stream, g, part, part_bytes, S);
        break;
    case SG_RESID: hipLaunchKernelGGL(stream_gemm_reduce_kernel<SG_RESID>, grid, block, 0, stream, g, part, part_bytes, S);
        break;
    case SG_F32: hipLaunchKernelGGL(stream_gemm_reduce_kernel<SG_F32>, grid, block, 0, stream, g, part, part_bytes, S);
        break;
    default: return -2;
    }
    return (int)hipGetLastError();
}

}  // namespace nc
