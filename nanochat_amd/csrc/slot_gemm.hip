/*
 * The decode step's GEMMs on gfx950: out[n][r] = epilogue(sum_k x[n][k] w[r][k]) for a step's slots (n < N <= 128) and
 * many weight rows r, bf16 operands, fp32 sums. At N <= 128 a GEMM is bound by moving bytes, not by the matrix cores:
 * every weight byte must come from HBM once, and every workgroup needs the activation rows x of its slots (N x K
 * bf16 is 426 KB at config 5), which come from L2.
 *
 * A workgroup owns 16 RT weight rows and 16 CT slots (a slot group) over its K range, walked in stages of 128 k. Each
 * stage's operands (x: 16 CT slot rows x 256 bytes; w: 16 RT rows x 256 bytes) go from memory into LDS by LDS DMA, 16
 * lanes per 256-byte row segment: a load instruction that covers long contiguous row pieces runs at about 3x the
 * per-CU rate of one scattering 16-byte pieces over 16 rows (measured: 16 rows x 64 B ~35 GB/s a CU, 8 rows x 128 B
 * 70-90 GB/s, 1 KB contiguous ~110 GB/s). A ring of RING stage buffers (3, or 4 for the smallest tile) keeps the next
 * RING - 1 stages in flight, with hand-placed waits and a barrier without a memory fence per stage (a fence would wait
 * for every DMA in flight). What
 * bounds it is the CU's ingress (about 40 GB/s a CU with every CU reading): a workgroup takes in its slots' x rows
 * besides its weights, so the host picks (RT, CT) per shape to make the bytes one CU takes in smallest, splitting the
 * slots into groups where x would outweigh the weights (sl_choose). The 4 waves split each stage's four 32-k steps
 * (wave w takes step w), so every LDS byte is read once; at the end the waves' sums meet in LDS and are added in wave
 * (K) order, then the epilogue is applied.
 *
 * Every global access goes through a buffer resource whose range is the exact extent of its array: rows past R and
 * slots past N read zeros, stages past the range read at SL_PAST (zeros, no memory access), and no load is
 * conditional. Each output's sum runs over its K range in a fixed order (stages in order, within a stage the wave's
 * 32-k step; then the four waves in order), the same for every slot, whatever N is and whatever tile shape holds it
 * (an MFMA output element is the sum of its own row and column products alone), so a slot's result depends on its own
 * x row only.
 *
 * Operand layout (v_mfma_f32_16x16x32_bf16): lane (g = lane / 16, i = lane % 16) of wave w holds, for stage k0,
 * A = w[row 16 t + i][k0 + 32 w + 8 g .. + 7] and B = x[slot n0 + 16 u + i][k0 + 32 w + 8 g .. + 7]; the result tile
 * holds rows 16 t + 4 g .. + 3 of slot n0 + 16 u + i. In LDS a row's 256 bytes (16 blocks of 16) keep block b at position
 * b ^ (row % 16), so the 16 rows of one operand read fall in distinct banks; each DMA lane fetches the global block
 * that belongs at its LDS position.
 *
 * S = 1: the workgroup applies the epilogue itself (the SG_* kinds of nc_internal.h). S > 1 (long K), or a caller that
 * finishes the sums itself (slot_gemm_partials): each of S K-slices stores fp32 partial sums to part[s][n][r], and
 * slot_gemm_reduce adds them in slice order before the same epilogue. With ssq (one slice), the residual epilogue also
 * writes each 16-row tile's sum of squares of its sums, and the ReLU^2 epilogue takes each slot's rstd from them, so
 * the MLP's rstd needs no kernel of its own.
 *
 * Reference: the slot GEMM and its epilogues, model/kernels/decode.cu:133-168, 295-359.
 */
#include "nc_device.h"
#include "nc_internal.h"

namespace nc {

constexpr int SL_WAVES = 4;
constexpr int SL_THREADS = SL_WAVES * WAVE;
constexpr int SL_KC = 128;                       /* k per stage: four 32-k MFMA steps, one per wave */
constexpr int SL_ROWB = SL_KC * 2;               /* bytes of a stage's row */
/* a stage's LDS bytes and DMA instructions a wave issues for 16 T rows (T 16-row tiles; each instruction moves 1 KiB) */
template <int T> constexpr int sl_buf() { return T * 16 * SL_ROWB; }
template <int T> constexpr int sl_tile_loads() { return sl_buf<T>() / 1024 / SL_WAVES; }
/* all of a stage's DMA a wave issues: the newer stage in flight at each wait */
template <int RT, int CT> constexpr int sl_loads() { return sl_tile_loads<RT>() + sl_tile_loads<CT>(); }
constexpr int SL_PAST = 0x7FFF0000;              /* a byte offset past every operand's range */
constexpr int SL_MAX_K_SLICE = 2048;             /* longer K is split into slices of at most this (then reduced) */

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef __attribute__((address_space(3))) void LdsPtr;

/* The sum of a 16-lane row by DPP (no LDS round trip, unlike a shuffle): adjacent lanes, then pairs, then the row
 * rotated by 4 and by 8; lane 0 of the row ends with ((v0 + v1) + (v2 + v3)) + ((v4 + v5) + (v6 + v7)) + ... in a
 * fixed association. */
__device__ __forceinline__ float dpp_add(float v, int ctrl_sel) {
    int o;
    switch (ctrl_sel) {
    case 0: o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false); break;   /* quad [1,0,3,2] */
    case 1: o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false); break;   /* quad [2,3,0,1] */
    case 2: o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false); break;  /* row_ror:4 */
    default: o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false); break; /* row_ror:8 */
    }
    return v + __int_as_float(o);
}
__device__ __forceinline__ float row16_sum(float v) { return dpp_add(dpp_add(dpp_add(dpp_add(v, 0), 1), 2), 3); }

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
__device__ __forceinline__ void bstore4(Rsrc r, int off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, 0);
}

__device__ __forceinline__ bool sl_live(const unsigned long long *mask, int n) {
    return !mask || ((mask[n >> 6] >> (n & 63)) & 1ull);
}

/* The operand views of one launch. */
struct SlotViews {
    Rsrc w, x, out, out_f32, res, rstd, part, ssq;
};

/* part_bytes: the partial-sum buffer's allocation (the caller's), so its range is the allocation itself; ssq_cols: the
 * tile sums a slot has (ceil(R / 16) written by RESID2, ceil(K / 16) read by RELU2). */
__device__ __forceinline__ SlotViews slot_views(const SkinnyGemm &g, const float *part, long long part_bytes,
                                                int ssq_cols) {
    SlotViews v;
    v.w = rsrc(g.w, (long long)g.R * g.K * 2);
    v.x = rsrc(g.x, (long long)g.N * g.K * 2);
    v.out = rsrc(g.out, g.out ? (long long)g.N * g.R * 2 : 0);
    v.out_f32 = rsrc(g.out_f32, g.out_f32 ? (long long)g.N * g.R * 4 : 0);
    v.res = rsrc(g.res, g.res ? (long long)g.N * g.R * 2 : 0);
    v.rstd = rsrc(g.rstd, g.rstd ? (long long)g.N * 4 : 0);
    v.part = rsrc(part, part ? part_bytes : 0);
    v.ssq = rsrc(g.ssq, g.ssq ? (long long)g.N * ssq_cols * 4 : 0);
    return v;
}

/* The epilogue of four consecutive rows r .. r + 3 of slot n (sums s); at = n R + r; rstd: slot n's (RELU2). */
template <int EPI>
__device__ __forceinline__ void sl_store(const SlotViews &v, int at, float s[4], float rstd) {
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
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float p = s[i] * rstd;
            s[i] = fmaxf(p, 0.0f) * p;
        }
    }
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = f32_to_bf16(s[i]);
    bstore8(v.out, at * 2, u32x2{(uint32_t)o[0] | (uint32_t)o[1] << 16, (uint32_t)o[2] | (uint32_t)o[3] << 16});
}

/* s_waitcnt: every vector-memory load but the newest (RING - 2) sl_loads<RT, CT>() has landed (the stages issued after
 * this one may stay in flight), and this wave's LDS reads are done. Encoding: vmcnt [3:0] and [15:14], expcnt [6:4]
 * (7: no wait), lgkmcnt [11:8]. */
template <int RT, int CT, int RING>
__device__ __forceinline__ void sl_wait_stage() {
    constexpr int n = (RING - 2) * sl_loads<RT, CT>();
    static_assert(n < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0x0 << 8));
}

/* A workgroup barrier with no memory fence; the empty asm statements keep memory accesses from moving across it. */
__device__ __forceinline__ void sl_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

/* The DMA of rows' stage j into buf (past the range: SL_PAST, zeros and no access). Instruction q fills the buffer's
 * rows 4 q .. 4 q + 3 (lane l: row 4 q + l / 16, LDS position l % 16, global block (l % 16) ^ (row % 16)); wave w issues
 * q = w, w + 4, ... */
template <int LOADS>
__device__ __forceinline__ void sl_fetch(Rsrc src, unsigned char *buf, int j, int nc, int kb0, int rowb, int row0,
                                         int wave, int lane) {
    const bool live = j < nc;
    const int kb = kb0 + j * SL_ROWB;
    const int pos = lane & 15;
#pragma unroll
    for (int m = 0; m < LOADS; m++) {
        const int q = wave + SL_WAVES * m, row = 4 * q + (lane >> 4);
        const int off = live ? (row0 + row) * rowb + kb + ((pos ^ (row & 15)) << 4) : SL_PAST;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(src, (LdsPtr *)(buf + q * 1024), 16, off, 0, 0, 0);
    }
}

/* The wave's 32-k step of a stage: A and B read from LDS (block 4 wave + grp of the row, at its swizzled position). */
template <int RT, int CT>
__device__ __forceinline__ void sl_compute(const unsigned char *xb, const unsigned char *wb, f32x4 (&acc)[RT][CT],
                                           int wave, int i16, int grp) {
    const int pos = (4 * wave + grp) ^ i16;   /* rows 16 t + i16 and 16 u + i16 all have row % 16 = i16 */
    bf16x8 a[RT];
#pragma unroll
    for (int t = 0; t < RT; t++)
        a[t] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(wb + (16 * t + i16) * SL_ROWB + pos * 16));
#pragma unroll
    for (int u = 0; u < CT; u++) {
        const bf16x8 b = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(xb + (16 * u + i16) * SL_ROWB + pos * 16));
#pragma unroll
        for (int t = 0; t < RT; t++) acc[t][u] = mfma16x16x32(a[t], b, acc[t][u]);
    }
}

/* One ring position: wait for stage j, barrier (every wave's DMA of stage j has landed and every wave is done with
 * stage j - 1), refill the buffers stage j - 1 used with stage j + RING - 1, compute stage j. */
#define SL_STEP(j, XB, WB, NXB, NWB)                                                     \
    do {                                                                                 \
        sl_wait_stage<RT, CT, RING>();                                                   \
        sl_barrier();                                                                    \
        sl_fetch<sl_tile_loads<CT>()>(v.x, NXB, (j) + RING - 1, nc, kb0, rowb, n0, wave, lane); \
        sl_fetch<sl_tile_loads<RT>()>(v.w, NWB, (j) + RING - 1, nc, kb0, rowb, r0, wave, lane); \
        sl_compute<RT, CT>(XB, WB, acc, wave, i16, grp);                                 \
    } while (0)

/* EPI < 0: store partial sums (S > 1). RT 16-row tiles and CT 16-slot tiles a workgroup, a ring of RING stage buffers
 * (RING - 1 stages in flight). Grid (ceil(R / (16 RT)), S, ceil(N / (16 CT))), 256 threads. */
template <int EPI, int RT, int CT, int RING>
__global__ void __launch_bounds__(SL_THREADS, 1) slot_gemm_kernel(SkinnyGemm g, float *part, long long part_bytes,
                                                                  int S) {
    constexpr int XB = sl_buf<CT>(), WB = sl_buf<RT>();
    static_assert(RING == 3 || RING == 4, "the loop below rotates three or four stage buffers");
    __shared__ __align__(16) unsigned char x0[XB], x1[XB], x2[XB], x3[RING == 4 ? XB : 16];
    __shared__ __align__(16) unsigned char w0[WB], w1[WB], w2[WB], w3[RING == 4 ? WB : 16];
    __shared__ float rs[EPI == SG_RELU2 ? 16 * CT : 1];   /* RELU2 from ssq: the group's slots' rstd */
    const SlotViews v = slot_views(g, part, part_bytes, EPI == SG_RELU2 ? (g.K + 15) / 16 : (g.R + 15) / 16);
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    const int i16 = lane & 15, grp = lane >> 4;
    const int r0 = blockIdx.x * 16 * RT, s = blockIdx.y, n0 = blockIdx.z * 16 * CT;
    const int chunks = g.K / SL_KC;
    const int c0 = s * chunks / S, nc = (s + 1) * chunks / S - c0;   /* the slice: stages [c0, c0 + nc) */
    const int rowb = g.K * 2, kb0 = c0 * SL_ROWB;

    /* RELU2 from tile sums: each slot's rstd from its row's tile sums (at most 128: K <= 2048, checked by the host).
     * Wave w takes slots n0 + 4 CT w + i; lane l holds tiles l and l + 64 of each. The loads go out before the first
     * DMA (loads complete in issue order, so the stage waits then cover them and stall nothing); the sums are made
     * after the main loop: (tile l + tile l + 64), then row16_sum within each 16 lanes and the rows' pair sums (lane
     * 0's order is fixed), the same for every slot. */
    constexpr int PW = EPI == SG_RELU2 ? 4 * CT : 1;
    float ts0[PW], ts1[PW];
    const int tiles = (g.K + 15) / 16;
    if (EPI == SG_RELU2 && g.ssq) {
#pragma unroll
        for (int i = 0; i < PW; i++) {
            const int n = n0 + PW * wave + i;   /* past N: zeros (the view's range) */
            ts0[i] = lane < tiles ? bloadf(v.ssq, (n * tiles + lane) * 4) : 0.0f;
            ts1[i] = lane + WAVE < tiles ? bloadf(v.ssq, (n * tiles + lane + WAVE) * 4) : 0.0f;
        }
    }

    f32x4 acc[RT][CT];
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int u = 0; u < CT; u++) acc[t][u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    sl_fetch<sl_tile_loads<CT>()>(v.x, x0, 0, nc, kb0, rowb, n0, wave, lane);
    sl_fetch<sl_tile_loads<RT>()>(v.w, w0, 0, nc, kb0, rowb, r0, wave, lane);
    sl_fetch<sl_tile_loads<CT>()>(v.x, x1, 1, nc, kb0, rowb, n0, wave, lane);
    sl_fetch<sl_tile_loads<RT>()>(v.w, w1, 1, nc, kb0, rowb, r0, wave, lane);
    int j = 0;
    if (RING == 3) {
        for (; j + 3 <= nc; j += 3) {
            SL_STEP(j, x0, w0, x2, w2);
            SL_STEP(j + 1, x1, w1, x0, w0);
            SL_STEP(j + 2, x2, w2, x1, w1);
        }
        if (j < nc) SL_STEP(j, x0, w0, x2, w2);           /* nc - j is 1 or 2: uniform over the workgroup */
        if (j + 1 < nc) SL_STEP(j + 1, x1, w1, x0, w0);
    } else {
        sl_fetch<sl_tile_loads<CT>()>(v.x, x2, 2, nc, kb0, rowb, n0, wave, lane);
        sl_fetch<sl_tile_loads<RT>()>(v.w, w2, 2, nc, kb0, rowb, r0, wave, lane);
        for (; j + 4 <= nc; j += 4) {
            SL_STEP(j, x0, w0, x3, w3);
            SL_STEP(j + 1, x1, w1, x0, w0);
            SL_STEP(j + 2, x2, w2, x1, w1);
            SL_STEP(j + 3, x3, w3, x2, w2);
        }
        if (j < nc) SL_STEP(j, x0, w0, x3, w3);           /* nc - j is 1, 2 or 3: uniform over the workgroup */
        if (j + 1 < nc) SL_STEP(j + 1, x1, w1, x0, w0);
        if (j + 2 < nc) SL_STEP(j + 2, x2, w2, x1, w1);
    }
    __builtin_amdgcn_s_waitcnt(0);                    /* no DMA may land in LDS after this */
    if (EPI == SG_RELU2 && g.ssq) {   /* read by the epilogue after the reduction's first barrier */
        static_assert(PW <= WAVE, "a lane per slot of the wave");
        float mine = 0.0f;             /* lane i: slot i's sum (lane 0's), so one sqrt and divide serve every slot */
#pragma unroll
        for (int i = 0; i < PW; i++) {
            const float ss = pair_sum32(pair_sum16(row16_sum(ts0[i] + ts1[i])));
            const float s0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 0));
            mine = lane == i ? s0 : mine;
        }
        if (lane < PW) rs[PW * wave + lane] = 1.0f / __builtin_sqrtf(mine * (1.0f / (float)g.K) + FLT_EPS);
    }
    sl_barrier();
    /* the four waves' sums, added in wave (K) order, up to two row tiles at a time: each wave writes its sums of the
     * round's (t, u) tiles (2 CT f32x4 a lane: waves 0, 1 into x0, waves 2, 3 into x1, which hold 4 CT), then wave w
     * finishes tiles q = w, w + 4, ... of the round's TT CT */
#pragma unroll
    for (int tt = 0; tt < RT; tt += 2) {
        constexpr int TT0 = RT < 2 ? RT : 2;
        const int TT = RT - tt < TT0 ? RT - tt : TT0;
        f32x4 *red = reinterpret_cast<f32x4 *>(wave < 2 ? x0 : x1) + (wave & 1) * 2 * CT * WAVE;
#pragma unroll
        for (int t = 0; t < TT0; t++)
#pragma unroll
            for (int u = 0; u < CT; u++)
                if (t < TT) red[(t * CT + u) * WAVE + lane] = acc[tt + t][u];
        sl_barrier();
#pragma unroll
        for (int q0 = 0; q0 < TT0 * CT; q0 += SL_WAVES) {
            const int q = q0 + wave;
            if (q >= TT * CT) continue;
            const int t = q / CT, u = q - t * CT;
            const int r = r0 + 16 * (tt + t) + 4 * grp, n = n0 + 16 * u + i16;
            f32x4 sum = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int w = 0; w < SL_WAVES; w++) {
                const f32x4 *rw = reinterpret_cast<const f32x4 *>(w < 2 ? x0 : x1) + (w & 1) * 2 * CT * WAVE;
                const f32x4 p = rw[(t * CT + u) * WAVE + lane];
                sum = w == 0 ? p : sum + p;
            }
            const bool ok = r < g.R && n < g.N && sl_live(g.active, n);
            float sv[4] = {sum[0], sum[1], sum[2], sum[3]};
            if (EPI == SG_RESID2 && g.ssq) {   /* wave-uniform: every lane takes part in the tile's sum of squares */
                if (ok) sl_store<SG_RESID2>(v, n * g.R + r, sv, 0.0f);   /* sv += the residual */
                float sq = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) sq = __builtin_fmaf(sv[i], sv[i], sq);
                sq = pair_sum32(pair_sum16(ok ? sq : 0.0f));   /* the tile's 16 rows (rows past R: 0) */
                const int tile = blockIdx.x * RT + tt + t;     /* a workgroup's last tiles may lie past R */
                if (grp == 0 && n < g.N && sl_live(g.active, n) && tile * 16 < g.R)
                    bstore4(v.ssq, (n * ((g.R + 15) / 16) + tile) * 4, sq);
                continue;
            }
            if (!ok) continue;
            if (EPI < 0)
                bstore16(v.part, ((s * g.N + n) * g.R + r) * 4,
                         u32x4{__float_as_uint(sv[0]), __float_as_uint(sv[1]), __float_as_uint(sv[2]),
                               __float_as_uint(sv[3])});
            else
                sl_store<EPI < 0 ? SG_STORE : EPI>(v, n * g.R + r, sv,
                                                   EPI == SG_RELU2 ? (g.ssq ? rs[n - n0] : bloadf(v.rstd, n * 4)) : 0.0f);
        }
        sl_barrier();   /* the reduction area is rewritten by the next round */
    }
}

/* The S partials of four rows of one slot summed in slice order, then the epilogue; a thread per four rows. */
template <int EPI>
__global__ void __launch_bounds__(256) slot_gemm_reduce_kernel(SkinnyGemm g, const float *part, long long part_bytes,
                                                                int S) {
    const int n = blockIdx.y;
    const int r = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (r >= g.R || !sl_live(g.active, n)) return;
    const SlotViews v = slot_views(g, part, part_bytes, 0);
    float sv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = 0; s < S; s++) {
        const u32x4 p = bload16(v.part, ((s * g.N + n) * g.R + r) * 4);
#pragma unroll
        for (int i = 0; i < 4; i++) sv[i] = sv[i] + __uint_as_float(p[i]);
    }
    sl_store<EPI>(v, n * g.R + r, sv, EPI == SG_RELU2 ? bloadf(v.rstd, n * 4) : 0.0f);
}

/* The tile shapes built, as (RT, CT). */
struct SlTile {
    int rt, ct;
};
constexpr SlTile SL_TILES[] = {{2, 2}, {3, 4}, {4, 4}, {4, 8}};
constexpr int SL_CUS = 256;   /* MI355X compute units */

/* The tile shape whose busiest CU takes in the fewest bytes: a workgroup takes in 16 (RT + CT) rows of 256 bytes a
 * stage, and the busiest CU runs ceil(workgroups / 256) of them; ties go to the earlier entry. The choice never
 * changes a result's bits (each output's sum order does not depend on the tile). */
static SlTile sl_choose(int R, int K, int N, int S) {
    SlTile best = SL_TILES[0];
    long long best_cost = 0;
    for (const SlTile &t : SL_TILES) {
        const long long wgs = (long long)((R + 16 * t.rt - 1) / (16 * t.rt)) * S * ((N + 16 * t.ct - 1) / (16 * t.ct));
        const long long cost = (wgs + SL_CUS - 1) / SL_CUS * (K / SL_KC / S) * (t.rt + t.ct);
        if (&t == SL_TILES || cost < best_cost) {
            best = t;
            best_cost = cost;
        }
    }
    return best;
}

/* A ring of four stages (three in flight) for the smallest tile, whose 16 KiB stages leave a CU's ingest idle behind
 * two in flight (config-5 o GEMM: 8.38 -> 7.63 us); three for the larger ones, whose stage time is their ingest
 * (measured with four: qkv 10.66 -> 10.92 us, fc 14.29 -> 14.42, proj 12.50 -> 12.71). */
template <int RT, int CT> constexpr int sl_ring() { return sl_buf<RT>() + sl_buf<CT>() <= 16 * 1024 ? 4 : 3; }

template <int EPI, int RT, int CT>
static void sl_launch_tile(const SkinnyGemm &g, float *part, long long part_bytes, int S, hipStream_t stream) {
    const dim3 grid((g.R + 16 * RT - 1) / (16 * RT), S, (g.N + 16 * CT - 1) / (16 * CT)), block(SL_THREADS);
    hipLaunchKernelGGL((slot_gemm_kernel<EPI, RT, CT, sl_ring<RT, CT>()>), grid, block, 0, stream, g, part, part_bytes,
                       S);
}

template <int EPI>
static void sl_launch(const SkinnyGemm &g, float *part, long long part_bytes, int S, hipStream_t stream) {
    const SlTile t = sl_choose(g.R, g.K, g.N, S);
    if (t.rt == 2 && t.ct == 2) sl_launch_tile<EPI, 2, 2>(g, part, part_bytes, S, stream);
    else if (t.rt == 3) sl_launch_tile<EPI, 3, 4>(g, part, part_bytes, S, stream);
    else if (t.ct == 4) sl_launch_tile<EPI, 4, 4>(g, part, part_bytes, S, stream);
    else sl_launch_tile<EPI, 4, 8>(g, part, part_bytes, S, stream);
}

bool slot_gemm_fits(int R, int K, int N) {
    /* every byte offset, including those of the rows and slots past R and N a tile covers, fits an int */
    return N >= 1 && N <= SG_MAX_N && K >= SL_KC && K % SL_KC == 0 && R >= 1 && R % 4 == 0 &&
           (long long)(R + 16 * 4) * K * 2 <= SL_PAST && (long long)SG_MAX_N * K * 2 <= SL_PAST &&
           (long long)N * R * 4 <= SL_PAST;
}

int slot_gemm_slices(int R, int K) {
    (void)R;
    const int chunks = K / SL_KC, per = SL_MAX_K_SLICE / SL_KC;
    return chunks > per ? (chunks + per - 1) / per : 1;
}

int slot_gemm_tile(int R, int K, int N, int S) {
    const SlTile t = sl_choose(R, K, N, S);
    return 100 * t.rt + t.ct;
}

long long slot_gemm_part_bytes(int R, int N, int S) { return S > 1 ? (long long)S * N * R * 4 : 0; }

static bool sl_part_fits(const SkinnyGemm &g, const float *part, long long part_bytes, int S) {
    const long long need = slot_gemm_part_bytes(g.R, g.N, S);
    return part && need <= part_bytes && part_bytes < (1LL << 31);
}

static bool sl_operands_fit(const SkinnyGemm &g, int epi) {
    const bool need_out = epi != SG_F32, need_f32 = epi == SG_F32 || (epi == SG_RESID2 && !g.ssq);
    const bool need_res = epi == SG_RESID || epi == SG_RESID2;
    return !((need_out && !g.out) || (need_f32 && !g.out_f32) || (need_res && !g.res) ||
             (epi == SG_RELU2 && !g.rstd && !g.ssq));
}

int slot_gemm(const SkinnyGemm &g, int epi, float *part, long long part_bytes, int S, hipStream_t stream) {
    if (!slot_gemm_fits(g.R, g.K, g.N) || S < 1 || S > g.K / SL_KC || epi < SG_STORE || epi > SG_F32) return -2;
    if (S > 1 && !sl_part_fits(g, part, part_bytes, S)) return -2;
    if (S == 1 && !sl_operands_fit(g, epi)) return -2;
    /* tile sums: one slice, a RELU2 row of at most 128 tiles */
    if (g.ssq && (S > 1 || (epi != SG_RESID2 && epi != SG_RELU2) || (epi == SG_RELU2 && (g.K + 15) / 16 > 2 * WAVE)))
        return -2;
    if (S > 1) {
        sl_launch<-1>(g, part, part_bytes, S, stream);
        return (int)hipGetLastError();
    }
    switch (epi) {
    case SG_STORE: sl_launch<SG_STORE>(g, nullptr, 0, 1, stream); break;
    case SG_RESID2: sl_launch<SG_RESID2>(g, nullptr, 0, 1, stream); break;
    case SG_RELU2: sl_launch<SG_RELU2>(g, nullptr, 0, 1, stream); break;
    case SG_RESID: sl_launch<SG_RESID>(g, nullptr, 0, 1, stream); break;
    default: sl_launch<SG_F32>(g, nullptr, 0, 1, stream); break;
    }
    return (int)hipGetLastError();
}

int slot_gemm_partials(const SkinnyGemm &g, float *part, long long part_bytes, int S, hipStream_t stream) {
    if (!slot_gemm_fits(g.R, g.K, g.N) || S < 1 || S > g.K / SL_KC || !part || g.ssq ||
        (long long)S * g.N * g.R * 4 > part_bytes || part_bytes >= (1LL << 31))
        return -2;
    sl_launch<-1>(g, part, part_bytes, S, stream);
    return (int)hipGetLastError();
}

int slot_gemm_reduce(const SkinnyGemm &g, int epi, const float *part, long long part_bytes, int S,
                     hipStream_t stream) {
    if (!slot_gemm_fits(g.R, g.K, g.N) || S < 2 || !sl_part_fits(g, part, part_bytes, S) || !sl_operands_fit(g, epi) ||
        g.ssq)
        return -2;
    const dim3 grid((g.R / 4 + 255) / 256, g.N), block(256);
    switch (epi) {
    case SG_STORE: hipLaunchKernelGGL(slot_gemm_reduce_kernel<SG_STORE>, grid, block, 0, stream, g, part, part_bytes, S);
        break;
    case SG_RESID2: hipLaunchKernelGGL(slot_gemm_reduce_kernel<SG_RESID2>, grid, block, 0, stream, g, part, part_bytes, S);
        break;
    case SG_RELU2: hipLaunchKernelGGL(slot_gemm_reduce_kernel<SG_RELU2>, grid, block, 0, stream, g, part, part_bytes, S);
        break;
    case SG_RESID: hipLaunchKernelGGL(slot_gemm_reduce_kernel<SG_RESID>, grid, block, 0, stream, g, part, part_bytes, S);
        break;
    case SG_F32: hipLaunchKernelGGL(slot_gemm_reduce_kernel<SG_F32>, grid, block, 0, stream, g, part, part_bytes, S);
        break;
    default: return -2;
    }
    return (int)hipGetLastError();
}

}  // namespace nc
