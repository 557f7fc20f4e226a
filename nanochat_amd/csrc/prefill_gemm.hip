/*
 * The prefill GEMMs of the decoder runtime on gfx950: out[m][n] = epilogue(sum_k a[m][k] w[n][k]) for the rows of a
 * dec_prefill call (M <= 16,384 prompt tokens), bf16 operands, fp32 sums. At these sizes a GEMM is bound by the matrix
 * cores, so it is tiled for them: a workgroup of 8 waves owns a 256 x 256 output tile (2 x 4 waves of 128 x 64, 32
 * accumulator tiles of 16 x 16 a wave; two waves a SIMD), walks K in stages of 32, and takes each
 * stage's operands (256 rows of a and 256 rows of w, 64 bytes each: 32 KiB) from memory into LDS by LDS DMA, in a ring
 * of four buffers: a buffer is refilled with the stage four on as soon as every wave holds its fragments in registers,
 * so three stages are in flight while one is computed. Hand-placed waits and one barrier without a memory fence per
 * stage order the ring.
 *
 * Per stage a wave issues 32 MFMAs (v_mfma_f32_16x16x32_bf16: A = 16 weight rows n, B = 16 activation rows m) on
 * fragments already in registers, and between them reads the next stage's 4 weight and 8 activation fragments (one
 * 16-byte LDS read each) into a second register set. Lane (g, i) of a
 * result tile holds columns n .. n + 3 (n = 16 t + 4 g) of row m = 16 u + i, and every epilogue writes 4 adjacent
 * columns of a row. In LDS a row's 64 bytes (4 blocks of 16) keep block b at position b ^ ((row / 4) % 4), so the 16
 * rows of a fragment read fall in distinct banks; each DMA lane fetches the global block that belongs at its LDS
 * position.
 *
 * Workgroups take their tiles in an XCD-aware order (pg_order), so the workgroups an XCD runs together share operand
 * tiles in its L2. The tiles that would leave the last round of workgroups part-filled (T mod CUs of T tiles) are cut
 * into halves (256 x 128) or quarters (128 x 128), so that round has a workgroup on every CU and each takes in half or
 * a quarter of the operands; the waves of a smaller tile hold fewer fragments (PgTile).
 *
 * Every output's sum runs over K in one fixed order (the stages in order, each stage one MFMA's own order), whatever M
 * is and whatever size of tile holds it, so a row's result depends on its own a row alone: a prompt's rows give the
 * same bits in any dec_prefill call.
 * Every global access goes through a buffer resource over the exact extent of its array, so rows past M read zeros
 * and store nothing; columns past N (a last partial tile of 256) are not stored.
 *
 * Epilogues (the SG_* kinds of nc_internal.h; decode.cu:133-168 for the math): SG_STORE bf16(s); SG_RESID
 * bf16(s + res); SG_F32 s; SG_RELU2 bf16(relu(p) p) with p = s rstd[m].
 *
 * Reference: the prefill rows of dec_prefill run through the step's GEMM body, model/kernels/decode.cu:170-230,
 * 295-359, 1041-1051.
 */
#include "nanochat_amd.h"
#include "nc_device.h"
#include "nc_internal.h"

namespace nc {

constexpr int PG_KC = 32;                      /* k per stage: one MFMA's depth */
constexpr int PG_ROWB = PG_KC * 2;             /* bytes of a row per stage */
constexpr int PG_STAGE = 512 * PG_ROWB;        /* a stage buffer: 256 a rows and 256 w rows */
constexpr int PG_RING = 4;                     /* stage buffers; three stages in flight */
constexpr int PG_WAVES = 8;
constexpr int PG_PAST = 0x7FFF0000;            /* a byte offset past every operand's range */

/* A workgroup's output tile: TM rows m x TN columns n, its 8 waves as 2 (m) x 4 (n), each wave WM x WN outputs, NU
 * activation and NT weight fragments a stage. A stage buffer holds the tile's TM a rows, then its TN w rows; its DMA
 * is ROWS / 16 instructions of 1 KiB, LOADS a wave, the first A_LOADS of them a's. */
template <int TM_, int TN_>
struct PgTile {
    static constexpr int TM = TM_, TN = TN_, WM = TM / 2, WN = TN / 4, NU = WM / 16, NT = WN / 16;
    static constexpr int ROWS = TM + TN, LOADS = ROWS / 16 / PG_WAVES, A_LOADS = TM / 16 / PG_WAVES;
    static_assert(ROWS * PG_ROWB <= PG_STAGE && ROWS % (16 * PG_WAVES) == 0 && TM % (16 * PG_WAVES) == 0, "DMA split");
    static_assert(NU % NT == 0, "a-fragment reads per weight fragment");
};
typedef PgTile<256, 256> PgFull;
typedef PgTile<256, 128> PgHalf;
typedef PgTile<128, 128> PgQuarter;
typedef PgTile<128, 256> PgThin;   /* calls of M <= 128 rows (a decode step's slots) */

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef __attribute__((address_space(3))) void LdsPtr;

__device__ __forceinline__ Rsrc pg_rsrc(const void *p, long long bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

/* Stage j's DMA into buf (j >= stages: offsets past the range, zeros and no memory access). Instruction q fills the
 * buffer's rows 16 q .. 16 q + 15 (rows below TM: a rows m0 + r; the rest: w rows n0 + r - TM); lane l writes row
 * 16 q + l / 4 at position l % 4 and fetches the global block (l % 4) ^ ((row / 4) % 4). Wave w issues q = w, w + 8,
 * ... (its first A_LOADS are a's). */
template <class P>
__device__ __forceinline__ void pg_fetch(Rsrc ra, Rsrc rw, unsigned char *buf, int j, int stages, int m0, int n0,
                                         int rowb, int wave, int lane) {
    const bool live = j < stages;
    const int kb = j * PG_ROWB, pos = lane & 3;
#pragma unroll
    for (int s = 0; s < P::LOADS; s++) {
        const int q = wave + PG_WAVES * s, row = 16 * q + (lane >> 2);
        const bool is_a = s < P::A_LOADS;
        const int grow = (is_a ? m0 : n0 - P::TM) + row;
        const int off = live ? grow * rowb + kb + ((pos ^ ((row >> 2) & 3)) << 4) : PG_PAST;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(is_a ? ra : rw, (LdsPtr *)(buf + q * 1024), 16, off, 0, 0, 0);
    }
}

/* s_waitcnt: all but this wave's DMA of the NEWER stages most recently issued have landed, and its LDS reads are
 * done. Encoding: vmcnt [3:0] and [15:14], expcnt [6:4] (7: no wait), lgkmcnt [11:8]. */
template <class P, int NEWER>
__device__ __forceinline__ void pg_wait_stage() {
    constexpr int n = NEWER * P::LOADS;
    static_assert(n < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0x0 << 8));
}

/* A workgroup barrier with no memory fence; the empty asm statements keep memory accesses from moving across it. */
__device__ __forceinline__ void pg_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

/* The LDS reads and the MFMAs are instructions of their own (inline assembly), in the order written. The compiler
 * cannot tell a read of one stage buffer from the DMA into the others, and with builtin reads it waited for most DMA
 * in flight before each stage's first read, which left one stage in flight instead of three. A read's result is used
 * only after the s_waitcnt lgkmcnt(0) at the head of the next ring position (pg_wait_stage), and the MFMAs, being
 * volatile too, stay after that wait.
 *
 * The compiler does not see the MFMAs as matrix instructions, so it inserts none of their wait states; the kernel
 * keeps their hazards by construction. Operands are written only by LDS reads, waited for as above, never by VALU
 * instructions (tests/test_prefill_gemm_isa.py checks the built code). An accumulator is used again 31 products
 * later. The accumulators are zeroed before the first stage's DMA is issued, and read only after the last product
 * and 32 wait states. Each accumulator tile stays in the same four AGPRs for the whole K walk ("+a"). */
__device__ __forceinline__ void pg_mfma(f32x4 &c, const bf16x8 &a, const bf16x8 &b) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

/* The LDS address of a lane's row of fragment 0 of a wave's rows row0 .. row0 + 16 F - 1 in buf (row0 a multiple of
 * 16, so rows 16 f on from it have the same swizzle and fragment f lies 16 f rows = 1 KiB further on). */
__device__ __forceinline__ uint32_t pg_base(const unsigned char *buf, int row0, int i16, int grp) {
    const int row = row0 + i16;
    const LdsPtr *p = (const LdsPtr *)(buf + row * PG_ROWB + ((grp ^ ((row >> 2) & 3)) << 4));
    return (uint32_t)reinterpret_cast<uintptr_t>(p);
}

__device__ __forceinline__ bf16x8 pg_frag(uint32_t base, int f) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(base), "i"(f * 16 * PG_ROWB));
    return __builtin_bit_cast(bf16x8, v);
}

/* One stage of a wave: the NT x NU products of its weight fragments cw (rows TM + WN wn + 16 t + i of the stage
 * buffer) and activation fragments ca (rows WM wm + 16 u + i), with the next stage's NU + NT fragment reads from the
 * bases nab, nwb into (nw, na) spread between them: for each t, NU / NT activation fragments and weight fragment t. */
template <class P>
__device__ __forceinline__ void pg_compute(uint32_t nab, uint32_t nwb, f32x4 (&acc)[P::NT][P::NU],
                                           const bf16x8 (&cw)[P::NT], const bf16x8 (&ca)[P::NU], bf16x8 (&nw)[P::NT],
                                           bf16x8 (&na)[P::NU]) {
    constexpr int R = P::NU / P::NT + 1;   /* reads per t */
#pragma unroll
    for (int t = 0; t < P::NT; t++) {
#pragma unroll
        for (int u = 0; u < P::NU; u++) {
            pg_mfma(acc[t][u], cw[t], ca[u]);
#pragma unroll
            for (int c = 0; c < R; c++) {
                /* read c after product 2 c + 1 where that fits (the whole tile), else spread evenly */
                if (u != (2 * R <= P::NU ? 2 * c + 1 : (2 * c + 1) * P::NU / (2 * R))) continue;
                if (c < R - 1) na[t * (R - 1) + c] = pg_frag(nab, t * (R - 1) + c);
                else nw[t] = pg_frag(nwb, t);
            }
        }
    }
}

/* One ring position j: wait for this wave's DMA of stage j + 1 and its reads of stage j (now in registers), barrier
 * (every wave's DMA of stage j + 1 has landed and every wave holds stage j), refill stage j's buffer with stage j + 4,
 * then compute stage j while reading stage j + 1 from the next buffer into the other register set. */
#define PG_STEP(j, CUR, NXT, C, N)                                                                  \
    do {                                                                                             \
        pg_wait_stage<P, 2>();                                                                       \
        pg_barrier();                                                                                \
        pg_fetch<P>(ra, rw, CUR, (j) + PG_RING, stages, m0, n0, rowb, wave, lane);                   \
        pg_compute<P>(pg_base(NXT, P::WM * wm, i16, grp), pg_base(NXT, P::TM + P::WN * wn, i16, grp), acc,  \
                      fw[C], fa[C], fw[N], fa[N]);                                                   \
    } while (0)

/* The output tile (rows m0.., columns n0..) of a workgroup, K walked and the epilogue applied. */
template <class P, int EPI>
__device__ __forceinline__ void pg_run(const PfGemm &g, int m0, int n0, unsigned char *b0, unsigned char *b1,
                                       unsigned char *b2, unsigned char *b3) {
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    const int i16 = lane & 15, grp = lane >> 4, wm = wave >> 2, wn = wave & 3;
    const int rowb = g.K * 2, stages = g.K / PG_KC;
    const Rsrc ra = pg_rsrc(g.a, (long long)g.M * rowb), rw = pg_rsrc(g.w, (long long)g.N * rowb);

    /* the accumulators start at zero in their AGPRs, before the first DMA is issued */
    f32x4 acc[P::NT][P::NU];
#pragma unroll
    for (int t = 0; t < P::NT; t++)
#pragma unroll
        for (int u = 0; u < P::NU; u++) asm volatile("" : "=a"(acc[t][u]) : "0"(f32x4{0.0f, 0.0f, 0.0f, 0.0f}));
    pg_fetch<P>(ra, rw, b0, 0, stages, m0, n0, rowb, wave, lane);
    pg_fetch<P>(ra, rw, b1, 1, stages, m0, n0, rowb, wave, lane);
    pg_fetch<P>(ra, rw, b2, 2, stages, m0, n0, rowb, wave, lane);
    pg_fetch<P>(ra, rw, b3, 3, stages, m0, n0, rowb, wave, lane);
    bf16x8 fw[2][P::NT], fa[2][P::NU];
    pg_wait_stage<P, 3>();
    pg_barrier();
#pragma unroll
    for (int u = 0; u < P::NU; u++) fa[0][u] = pg_frag(pg_base(b0, P::WM * wm, i16, grp), u);
#pragma unroll
    for (int t = 0; t < P::NT; t++) fw[0][t] = pg_frag(pg_base(b0, P::TM + P::WN * wn, i16, grp), t);
    for (int j = 0; j < stages; j += 4) {   /* stages is a multiple of 4 (K of 128, checked by the host) */
        PG_STEP(j, b0, b1, 0, 1);
        PG_STEP(j + 1, b1, b2, 1, 0);
        PG_STEP(j + 2, b2, b3, 0, 1);
        PG_STEP(j + 3, b3, b0, 1, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);                 /* no DMA may land in LDS after this */
    /* 32 wait states: every product has written its accumulator before the epilogue reads it (each accumulator is
     * tied to this point, so no read moves above it) */
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int t = 0; t < P::NT; t++)
#pragma unroll
        for (int u = 0; u < P::NU; u++) asm volatile("" : "+a"(acc[t][u]));

    const Rsrc ro = pg_rsrc(EPI == SG_F32 ? (const void *)g.out_f32 : (const void *)g.out,
                            (long long)g.M * g.N * (EPI == SG_F32 ? 4 : 2));
    const Rsrc rr = pg_rsrc(g.res, EPI == SG_RESID ? (long long)g.M * g.N * 2 : 0);
    const Rsrc rs = pg_rsrc(g.rstd, EPI == SG_RELU2 ? (long long)g.M * 4 : 0);
#pragma unroll
    for (int u = 0; u < P::NU; u++) {
        const int m = m0 + P::WM * wm + 16 * u + i16;
        const float r = EPI == SG_RELU2 ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, m * 4, 0, 0))
                                        : 0.0f;
#pragma unroll
        for (int t = 0; t < P::NT; t++) {
            const int n = n0 + P::WN * wn + 16 * t + 4 * grp;
            if (n >= g.N) continue;
            const int at = m * g.N + n;   /* rows past M lie outside the views' ranges: no access */
            float s[4] = {acc[t][u][0], acc[t][u][1], acc[t][u][2], acc[t][u][3]};
            if (EPI == SG_F32) {
                __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(s[0]), __float_as_uint(s[1]),
                                                             __float_as_uint(s[2]), __float_as_uint(s[3])},
                                                       ro, at * 4, 0, 0);
                continue;
            }
            if (EPI == SG_RESID) {
                const u32x2 rv = __builtin_amdgcn_raw_buffer_load_b64(rr, at * 2, 0, 0);
                const float res[4] = {bf16_to_f32((uint16_t)rv[0]), bf16_to_f32((uint16_t)(rv[0] >> 16)),
                                      bf16_to_f32((uint16_t)rv[1]), bf16_to_f32((uint16_t)(rv[1] >> 16))};
#pragma unroll
                for (int e = 0; e < 4; e++) s[e] = s[e] + res[e];
            } else if (EPI == SG_RELU2) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float p = s[e] * r;
                    s[e] = fmaxf(p, 0.0f) * p;
                }
            }
            uint16_t o[4];
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = f32_to_bf16(s[e]);
            __builtin_amdgcn_raw_buffer_store_b64(
                u32x2{(uint32_t)o[0] | (uint32_t)o[1] << 16, (uint32_t)o[2] | (uint32_t)o[3] << 16}, ro, at * 2, 0, 0);
        }
    }
}

/* The order workgroups take work in. Workgroups are dispatched to the 8 XCDs in turn (L % 8), each XCD with its own
 * L2, so work items are numbered XCD by XCD: pg_order(l, count) gives XCD k a contiguous run of [0, count) (a
 * bijection, for a first workgroup that is a multiple of 8). Tile id is then placed in bands of PG_GROUP m-tiles walked
 * m-tile fastest, one n-tile at a time (pg_band), so the workgroups an XCD runs at once share a few a and w tiles,
 * read from its L2 rather than each from memory. */
constexpr int PG_XCDS = 8, PG_GROUP = 4;

__device__ __forceinline__ int pg_order(int l, int count) {
    const int k = l % PG_XCDS, r = l / PG_XCDS, per = count / PG_XCDS, extra = count % PG_XCDS;
    return k * per + min(k, extra) + r;
}

/* (n-tile, m-tile) of tile id of the T = nx * ny tiles. */
__device__ __forceinline__ int2 pg_band(int id, int T, int nx) {
    const int band = PG_GROUP * nx;                            /* tiles of a band of PG_GROUP m-tiles */
    const int y0 = (id / band) * PG_GROUP, ny = (T / nx) - y0, rows = ny < PG_GROUP ? ny : PG_GROUP;
    const int in = id - (id / band) * band;
    return int2{in / rows, y0 + in % rows};
}

/* Workgroups [0, full) take whole tiles 0 .. full - 1; the rest take pieces (2: halves by n, 4: quarters) of tiles
 * full .. T - 1, the pieces of a tile on consecutive items of one XCD. A piece past M or N has nothing to compute.
 * Launches with no pieces use the instantiation without them (MODE PG_WHOLE): the same whole-tile loop ran 3-6 %
 * slower in a kernel that also holds the pieces' code. Calls of M <= 128 rows take tiles of 128 rows (PG_THIN). */
enum { PG_WHOLE, PG_SPLIT, PG_THIN };

template <int EPI, int MODE>
__global__ void __launch_bounds__(PG_WAVES * WAVE, 1) prefill_gemm_kernel(PfGemm g, int full, int pieces) {
    __shared__ __align__(16) unsigned char b0[PG_STAGE], b1[PG_STAGE], b2[PG_STAGE], b3[PG_STAGE];
    const int nx = (g.N + 255) / 256, T = nx * ((g.M + 255) / 256), L = blockIdx.x;
    if (MODE == PG_THIN) {
        pg_run<PgThin, EPI>(g, 0, pg_order(L, nx) * 256, b0, b1, b2, b3);
        return;
    }
    if (MODE == PG_WHOLE || L < full) {
        const int2 tile = pg_band(pg_order(L, full), T, nx);
        pg_run<PgFull, EPI>(g, tile.y * 256, tile.x * 256, b0, b1, b2, b3);
        return;
    }
    const int id = pg_order(L - full, (T - full) * pieces), p = id % pieces;
    const int2 tile = pg_band(full + id / pieces, T, nx);
    if (pieces == 2) {
        const int m0 = tile.y * 256, n0 = tile.x * 256 + 128 * p;
        if (n0 < g.N) pg_run<PgHalf, EPI>(g, m0, n0, b0, b1, b2, b3);
    } else {
        const int m0 = tile.y * 256 + 128 * (p >> 1), n0 = tile.x * 256 + 128 * (p & 1);
        if (m0 < g.M && n0 < g.N) pg_run<PgQuarter, EPI>(g, m0, n0, b0, b1, b2, b3);
    }
}

/* The number of compute units of the current device (256 if it cannot be read), once per device. */
static int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n
                                                                                                                : 256;
    }
    return cus[dev];
}

int prefill_gemm(const PfGemm &g, int epi, hipStream_t stream) {
    if (g.M <= 0) return 0;
    if (!g.a || !g.w || g.N <= 0 || g.K <= 0 || g.K % (PG_RING * PG_KC) || g.N % 4 ||
        (long long)g.M * g.K * 2 >= (1LL << 31) || (long long)g.N * g.K * 2 >= (1LL << 31) ||
        (long long)g.M * g.N * 4 >= (1LL << 31))
        return NC_ERR_SHAPE;
    const bool f32 = epi == SG_F32;
    if ((f32 ? !g.out_f32 : !g.out) || (epi == SG_RESID && !g.res) || (epi == SG_RELU2 && !g.rstd) ||
        (epi != SG_STORE && epi != SG_RESID && epi != SG_F32 && epi != SG_RELU2))
        return NC_ERR_SHAPE;
    /* T tiles in rounds of one workgroup a CU: the R = T mod CUs tiles of a last part-filled round are cut into 4
     * (R <= CUs / 4) or 2 (R <= CUs / 2) pieces when there are earlier full rounds; otherwise every tile is whole. */
    const int cus = device_cus(), T = ((g.N + 255) / 256) * ((g.M + 255) / 256), R = T % cus;
    const bool cut = g.M > 128 && T > cus && R > 0;
    const int pieces = cut && 4 * R <= cus ? 4 : cut && 2 * R <= cus ? 2 : 1;
    const int full = pieces > 1 ? T - R : T;
    const dim3 grid(full + (T - full) * pieces), block(PG_WAVES * WAVE);
    const int mode = g.M <= 128 ? PG_THIN : pieces > 1 ? PG_SPLIT : PG_WHOLE;
#define PG_LAUNCH(E)                                                                                             \
    do {                                                                                                         \
        if (mode == PG_THIN) hipLaunchKernelGGL((prefill_gemm_kernel<E, PG_THIN>), grid, block, 0, stream, g, full,  \
                                                pieces);                                                         \
        else if (mode == PG_SPLIT) hipLaunchKernelGGL((prefill_gemm_kernel<E, PG_SPLIT>), grid, block, 0, stream, g, \
                                                      full, pieces);                                             \
        else hipLaunchKernelGGL((prefill_gemm_kernel<E, PG_WHOLE>), grid, block, 0, stream, g, full, pieces);     \
    } while (0)
    switch (epi) {
    case SG_STORE: PG_LAUNCH(SG_STORE); break;
    case SG_RESID: PG_LAUNCH(SG_RESID); break;
    case SG_F32: PG_LAUNCH(SG_F32); break;
    default: PG_LAUNCH(SG_RELU2); break;
    }
#undef PG_LAUNCH
    return (int)hipGetLastError();
}

}  // namespace nc
