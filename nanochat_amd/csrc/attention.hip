/*
 * Attention over the paged fp8 cache on gfx950: split-K flash-decode (one query token per sequence, the
 * Hq/Hkv query heads of a KV head served from one read of its pages) and chunked prefill (16 query rows
 * per wave), both on the same page-pair step.
 *
 * The step (attend_pair) streams two 16-token pages of one KV head straight from HBM into registers:
 * each lane issues four 16-byte loads per page pair per operand, every load instruction covering 1 KiB
 * contiguously, because the page tiling (nc_device.h) is the MFMA operand layout. Scores are
 * S^T = K Q^T by four v_mfma_f32_16x16x32_bf16 per page (fp8 codes converted exactly to bf16; the
 * per-token K scale multiplies the fp32 dot product), the online softmax runs in the log2 domain on the
 * MFMA result layout, and O^T += V^T P^T by eight MFMAs per pair with the V scale folded into P before
 * its bf16 rounding. Query columns (lane & 15) are query heads in decode and (token, head) rows in
 * prefill; the lane's four row groups (lane >> 4) hold keys 4g..4g+3 of each page.
 *
 * Reference semantics: model/kernels/decode.cu:567-675 (k_attn: keys [max(p - window, 0), p], scale
 * 1/sqrt(128), fp32 softmax) and 859-863 (prefill rows appended before any attends).
 */
#include <math.h>

#include "nc_device.h"
#include "nanochat_amd.h"

namespace nc {

constexpr float LOG2E = 1.4426950408889634f;
constexpr int WAVES = 4;
constexpr int O_PITCH = HEAD_DIM + 4;  /* LDS row pitch of a wave's merged output (floats) */

struct AttnArgs {
    const uint16_t *q;        /* [B][T][Hq][128] bf16 (T = 1 in decode) */
    const uint8_t *k_pages, *v_pages;
    const float *k_scale, *v_scale;
    const int32_t *block_table;
    int max_pages, num_pages;
    const int32_t *seq_lens;  /* decode */
    const int32_t *start_pos; /* prefill */
    int B, T, Hq, Hkv, G, window;
    float scale_log2;         /* sm_scale * log2(e) */
    int pages_per_split, n_splits;
    float *part_o;            /* [B][Hq][n_splits][128] */
    float *part_ml;           /* [B][Hq][n_splits][2]: max (log2 domain), sum */
    uint16_t *out;            /* [B][T][Hq][128] bf16 */
};

/* A wave's running state for its 16 query columns; lane (g, c) = (lane >> 4, lane & 15) holds column c. */
struct WaveState {
    f32x4 o[8];  /* O^T tile t: dims 16t + 4g + i of column c */
    float m;     /* running max of column c, log2 domain (equal in the four groups) */
    float l;     /* sum of exp2(s - m) over the keys this lane's group holds */
    bool bad;    /* a block-table entry fell outside the page pool */
};

__device__ __forceinline__ void state_init(WaveState &st) {
#pragma unroll
    for (int t = 0; t < 8; t++) st.o[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    st.m = -INFINITY;
    st.l = 0.0f;
    st.bad = false;
}

/* The query operand of column c (B operand of the score MFMAs): lane (g, c) holds dims g*32 + cc*8 .. +7 of
 * its row for MFMA cc; a NULL row gives zeros. */
__device__ __forceinline__ void load_q(const uint16_t *row, int g, bf16x8 (&qb)[4]) {
#pragma unroll
    for (int cc = 0; cc < 4; cc++) {
        if (row) {
            const uint4 u = *reinterpret_cast<const uint4 *>(row + g * 32 + cc * 8);
            qb[cc] = __builtin_bit_cast(bf16x8, u);
        } else {
            qb[cc] = __builtin_bit_cast(bf16x8, uint4{0u, 0u, 0u, 0u});
        }
    }
}

/* Scores S^T (keys 4g + i of one page, column c) = K Q^T from one page's two K loads. */
__device__ __forceinline__ f32x4 page_scores(const uint4 &k0, const uint4 &k1, const bf16x8 (&qb)[4]) {
    f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
    s = mfma16x16x32(fp8x8_to_bf16(k0.x, k0.y), qb[0], s);
    s = mfma16x16x32(fp8x8_to_bf16(k0.z, k0.w), qb[1], s);
    s = mfma16x16x32(fp8x8_to_bf16(k1.x, k1.y), qb[2], s);
    s = mfma16x16x32(fp8x8_to_bf16(k1.z, k1.w), qb[3], s);
    return s;
}

__device__ __forceinline__ uint32_t dword(const uint4 &u, int i) {
    return i == 0 ? u.x : i == 1 ? u.y : i == 2 ? u.z : u.w;
}

__device__ __forceinline__ uint4 and4(const uint4 &u, uint32_t m) { return uint4{u.x & m, u.y & m, u.z & m, u.w & m}; }

/*
 * One step over logical pages lpa and lpa + 1 (has_b: whether the second is in range) of KV head kvh of
 * sequence b. Keys of this lane's column outside [lo, hi] are masked; V codes of keys past written_hi (slots
 * the cache has not written, whose bytes may be anything) are zeroed before use.
 */
__device__ __forceinline__ void attend_pair(const AttnArgs &a, const int32_t *bt, int kvh, int lpa, bool has_b, int lo,
                                            int hi, int written_hi, const bf16x8 (&qb)[4], WaveState &st, int lane) {
    const int g = lane >> 4;
    int pa = bt[lpa];
    int pb = has_b ? bt[lpa + 1] : 0;
    if ((unsigned)pa >= (unsigned)a.num_pages) { st.bad = true; pa = 0; }
    if ((unsigned)pb >= (unsigned)a.num_pages) { st.bad = true; pb = 0; }
    const long long ha = (long long)pa * a.Hkv + kvh, hb = (long long)pb * a.Hkv + kvh;
    const uint4 *kA = reinterpret_cast<const uint4 *>(a.k_pages + ha * PAGE_BYTES) + lane;
    const uint4 *vA = reinterpret_cast<const uint4 *>(a.v_pages + ha * PAGE_BYTES) + lane;
    const uint4 ka0 = kA[0], ka1 = kA[64];
    uint4 va0 = vA[0], va1 = vA[64];
    const float4 ksa = *reinterpret_cast<const float4 *>(a.k_scale + ha * PAGE + g * 4);
    const float4 vsa = *reinterpret_cast<const float4 *>(a.v_scale + ha * PAGE + g * 4);
    uint4 kb0 = {0u, 0u, 0u, 0u}, kb1 = kb0, vb0 = kb0, vb1 = kb0;
    float4 ksb = {0.0f, 0.0f, 0.0f, 0.0f}, vsb = ksb;
    if (has_b) {
        const uint4 *kB = reinterpret_cast<const uint4 *>(a.k_pages + hb * PAGE_BYTES) + lane;
        const uint4 *vB = reinterpret_cast<const uint4 *>(a.v_pages + hb * PAGE_BYTES) + lane;
        kb0 = kB[0]; kb1 = kB[64];
        vb0 = vB[0]; vb1 = vB[64];
        ksb = *reinterpret_cast<const float4 *>(a.k_scale + hb * PAGE + g * 4);
        vsb = *reinterpret_cast<const float4 *>(a.v_scale + hb * PAGE + g * 4);
    }
    /* the tail page(s): zero V codes of unwritten slots (a dword holds slots 4g..4g+3 of one dim) */
    const int key_a = lpa * PAGE + g * 4, key_b = key_a + PAGE;
    if (lpa * PAGE + PAGE - 1 > written_hi) {
        const int n = min(max(written_hi - key_a + 1, 0), 4);
        const uint32_t m = n >= 4 ? 0xFFFFFFFFu : ((1u << (8 * n)) - 1u);
        va0 = and4(va0, m); va1 = and4(va1, m);
    }
    if (has_b && (lpa + 1) * PAGE + PAGE - 1 > written_hi) {
        const int n = min(max(written_hi - key_b + 1, 0), 4);
        const uint32_t m = n >= 4 ? 0xFFFFFFFFu : ((1u << (8 * n)) - 1u);
        vb0 = and4(vb0, m); vb1 = and4(vb1, m);
    }

    const f32x4 sa = page_scores(ka0, ka1, qb);
    f32x4 sb = {0.0f, 0.0f, 0.0f, 0.0f};
    if (has_b) sb = page_scores(kb0, kb1, qb);

    float s[8];
    const float ksA[4] = {ksa.x, ksa.y, ksa.z, ksa.w}, ksB[4] = {ksb.x, ksb.y, ksb.z, ksb.w};
    const float vsA[4] = {vsa.x, vsa.y, vsa.z, vsa.w}, vsB[4] = {vsb.x, vsb.y, vsb.z, vsb.w};
    bool ok[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        ok[i] = key_a + i >= lo && key_a + i <= hi;
        ok[4 + i] = has_b && key_b + i >= lo && key_b + i <= hi;
        s[i] = ok[i] ? sa[i] * ksA[i] * a.scale_log2 : -INFINITY;
        s[4 + i] = ok[4 + i] ? sb[i] * ksB[i] * a.scale_log2 : -INFINITY;
    }
    float mt = s[0];
#pragma unroll
    for (int i = 1; i < 8; i++) mt = fmaxf(mt, s[i]);
    mt = fmaxf(mt, __shfl_xor(mt, 16, WAVE));
    mt = fmaxf(mt, __shfl_xor(mt, 32, WAVE));
    const float mn = fmaxf(st.m, mt);
    const float ms = mn == -INFINITY ? 0.0f : mn;
    const float alpha = __builtin_amdgcn_exp2f(st.m - ms);
    float psum = 0.0f;
    bf16x8 pv;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float p = __builtin_amdgcn_exp2f(s[i] - ms);
        psum += p;
        const float w = ok[i] ? p * (i < 4 ? vsA[i] : vsB[i - 4]) : 0.0f;
        pv[i] = (__bf16)w;
    }
    st.l = st.l * alpha + psum;
    st.m = mn;
#pragma unroll
    for (int t = 0; t < 8; t++) {
        st.o[t] *= alpha;
        const bf16x8 va = fp8x8_to_bf16(dword(t < 4 ? va0 : va1, t & 3), dword(t < 4 ? vb0 : vb1, t & 3));
        st.o[t] = mfma16x16x32(va, pv, st.o[t]);
    }
}

/* Pages of sequence b's key range [begin, p]; sizing shared by the split and combine kernels. */
__device__ __forceinline__ void decode_range(const AttnArgs &a, int L, int &begin, int &pg0, int &pg1, int &ns) {
    const int p = L - 1;
    begin = a.window >= 0 ? max(p - a.window, 0) : 0;
    pg0 = begin / PAGE;
    pg1 = p / PAGE + 1;
    ns = (pg1 - pg0 + a.pages_per_split - 1) / a.pages_per_split;
}

__device__ __forceinline__ void store_bf16x4(uint16_t *dst, const float *v) {
    uint2 u;
    u.x = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
    u.y = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
    *reinterpret_cast<uint2 *>(dst) = u;
}

/* Grid (n_splits, Hkv, B), 4 waves: the split's page pairs go to the waves round-robin, the waves' states
 * merge in LDS, and the split writes either the final output (one split for this sequence) or a partial. */
__global__ void __launch_bounds__(256) decode_split_kernel(AttnArgs a) {
    __shared__ float sh_o[WAVES][16][O_PITCH];
    __shared__ float sh_m[WAVES][16], sh_l[WAVES][16];
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int L = a.seq_lens[b];
    if (L <= 0) {
        if (split == 0 && a.n_splits == 1)
            for (int e = threadIdx.x; e < a.G * HEAD_DIM; e += blockDim.x)
                a.out[((long long)b * a.Hq + kvh * a.G) * HEAD_DIM + e] = 0;
        return;
    }
    int begin, pg0, pg1, ns;
    decode_range(a, L, begin, pg0, pg1, ns);
    if (L > a.max_pages * PAGE || ns > a.n_splits) {  /* past the block table or the grid: NaN, no reads */
        if (split == 0 && a.n_splits == 1)
            for (int e = threadIdx.x; e < a.G * HEAD_DIM; e += blockDim.x)
                a.out[((long long)b * a.Hq + kvh * a.G) * HEAD_DIM + e] = (uint16_t)0x7FC0;
        return;
    }
    if (split >= ns) return;
    const int first = pg0 + split * a.pages_per_split;
    const int last = min(pg1, first + a.pages_per_split);
    const int npairs = (last - first + 1) / 2;

    bf16x8 qb[4];
    load_q(c < a.G ? a.q + ((long long)b * a.Hq + kvh * a.G + c) * HEAD_DIM : nullptr, g, qb);
    WaveState st;
    state_init(st);
    const int32_t *bt = a.block_table + (long long)b * a.max_pages;
    for (int k = wave; k < npairs; k += WAVES) {
        const int lpa = first + 2 * k;
        attend_pair(a, bt, kvh, lpa, lpa + 1 < last, begin, L - 1, L - 1, qb, st, lane);
    }
    st.l += __shfl_xor(st.l, 16, WAVE);
    st.l += __shfl_xor(st.l, 32, WAVE);
    if (c < a.G) {
#pragma unroll
        for (int t = 0; t < 8; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) sh_o[wave][c][16 * t + 4 * g + i] = st.o[t][i];
        if (g == 0) {
            sh_m[wave][c] = st.m;
            sh_l[wave][c] = st.l;
        }
    }
    const int bad = __syncthreads_or(st.bad ? 1 : 0);
    for (int e = threadIdx.x; e < a.G * HEAD_DIM; e += blockDim.x) {
        const int col = e / HEAD_DIM, d = e % HEAD_DIM;
        float M = sh_m[0][col];
        for (int w = 1; w < WAVES; w++) M = fmaxf(M, sh_m[w][col]);
        float ls = 0.0f, o = 0.0f;
        for (int w = 0; w < WAVES; w++) {
            const float f = __builtin_amdgcn_exp2f(sh_m[w][col] - M);
            ls += sh_l[w][col] * f;
            o += sh_o[w][col][d] * f;
        }
        const long long row = (long long)b * a.Hq + kvh * a.G + col;
        if (ns == 1 || a.n_splits == 1) {
            a.out[row * HEAD_DIM + d] = bad ? (uint16_t)0x7FC0 : f32_to_bf16(o / ls);
        } else {
            const long long at = row * a.n_splits + split;
            a.part_o[at * HEAD_DIM + d] = bad ? NAN : o;
            if (d == 0) {
                a.part_ml[at * 2] = bad ? NAN : M;
                a.part_ml[at * 2 + 1] = ls;
            }
        }
    }
}

/* Grid B*Hq, 128 threads (one per dim): merges a sequence's split partials (log-sum-exp in base 2). */
__global__ void __launch_bounds__(HEAD_DIM) decode_combine_kernel(AttnArgs a) {
    const int b = blockIdx.x / a.Hq, d = threadIdx.x;
    const long long row = blockIdx.x;
    const int L = a.seq_lens[b];
    if (L <= 0) {
        a.out[row * HEAD_DIM + d] = 0;
        return;
    }
    int begin, pg0, pg1, ns;
    decode_range(a, L, begin, pg0, pg1, ns);
    if (L > a.max_pages * PAGE || ns > a.n_splits) {
        a.out[row * HEAD_DIM + d] = (uint16_t)0x7FC0;
        return;
    }
    if (ns <= 1) return;
    const float *ml = a.part_ml + row * a.n_splits * 2;
    const float *po = a.part_o + row * a.n_splits * HEAD_DIM + d;
    float M = ml[0];
    for (int s = 1; s < ns; s++) M = fmaxf(M, ml[2 * s]);
    float ls = 0.0f, o = 0.0f;
    for (int s = 0; s < ns; s++) {
        const float f = __builtin_amdgcn_exp2f(ml[2 * s] - M);
        ls += ml[2 * s + 1] * f;
        o += po[(long long)s * HEAD_DIM] * f;
    }
    a.out[row * HEAD_DIM + d] = f32_to_bf16(o / ls);
}

/* Grid (ceil(T / (4 tpt)), Hkv, B), 4 waves; wave w owns tile blockIdx.x*4 + w of tpt = 16 / G consecutive
 * tokens x G heads (column c = token (c / G), head (c % G)) and streams every page its rows can see. */
__global__ void __launch_bounds__(256) prefill_kernel(AttnArgs a) {
    const int kvh = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int tpt = 16 / a.G;
    const int t0 = (blockIdx.x * WAVES + wave) * tpt;
    if (t0 >= a.T) return;
    const int tl = c / a.G, hg = c % a.G;
    const bool live = c < tpt * a.G && t0 + tl < a.T;
    const int start = a.start_pos[b];
    if (start < 0 || (long long)start + a.T > (long long)a.max_pages * PAGE) {  /* past the block table: NaN */
        if (c < tpt * a.G && t0 + tl < a.T) {
            uint16_t *dst = a.out + (((long long)b * a.T + t0 + tl) * a.Hq + kvh * a.G + hg) * HEAD_DIM;
            for (int d = g * 32; d < g * 32 + 32; d++) dst[d] = (uint16_t)0x7FC0;
        }
        return;
    }
    const int pos = start + t0 + tl;
    const int hi = live ? pos : -1;
    const int lo = live ? (a.window >= 0 ? max(pos - a.window, 0) : 0) : 0;
    const int written_hi = start + a.T - 1;
    const int w_hi = start + min(t0 + tpt, a.T) - 1;
    const int w_lo = a.window >= 0 ? max(start + t0 - a.window, 0) : 0;
    const int pg0 = w_lo / PAGE, pg1 = w_hi / PAGE + 1;

    bf16x8 qb[4];
    const long long qrow = ((long long)b * a.T + t0 + tl) * a.Hq + kvh * a.G + hg;
    load_q(live ? a.q + qrow * HEAD_DIM : nullptr, g, qb);
    WaveState st;
    state_init(st);
    const int32_t *bt = a.block_table + (long long)b * a.max_pages;
    for (int lpa = pg0; lpa < pg1; lpa += 2) attend_pair(a, bt, kvh, lpa, lpa + 1 < pg1, lo, hi, written_hi, qb, st, lane);
    st.l += __shfl_xor(st.l, 16, WAVE);
    st.l += __shfl_xor(st.l, 32, WAVE);
    if (!live) return;
    uint16_t *dst = a.out + qrow * HEAD_DIM;
    const float inv = 1.0f / st.l;
#pragma unroll
    for (int t = 0; t < 8; t++) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = st.bad ? NAN : st.o[t][i] * inv;
        store_bf16x4(dst + 16 * t + 4 * g, v);
    }
}

/* Pages per split when the caller passes 0: about 2048 work-groups in total, at least 8 pages. */
static int auto_pages_per_split(int units, int max_range_pages) {
    long long pps = ((long long)max_range_pages * units + 2047) / 2048;
    if (pps < 8) pps = 8;
    if (pps > 512) pps = 512;
    return (int)((pps + 1) & ~1LL);
}

static int max_range_pages(int max_seq_len, int window) {
    int n = (max_seq_len + PAGE - 1) / PAGE;
    if (window >= 0) n = min(n, window / PAGE + 2);
    return n;
}

}  // namespace nc

using namespace nc;

static int decode_splits(int B, int Hkv, int max_seq_len, int window, int pages_per_split, int &pps) {
    const int range = max_range_pages(max_seq_len, window);
    pps = pages_per_split > 0 ? ((pages_per_split + 1) & ~1) : auto_pages_per_split(B * Hkv, range);
    return (range + pps - 1) / pps;
}

extern "C" size_t nc_decode_workspace_bytes(int B, int Hq, int Hkv, int max_seq_len, int window, int pages_per_split) {
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || max_seq_len <= 0) return 0;
    int pps;
    const int splits = decode_splits(B, Hkv, max_seq_len, window, pages_per_split, pps);
    return splits > 1 ? (size_t)B * Hq * splits * (HEAD_DIM + 2) * sizeof(float) : 0;
}

extern "C" int nc_decode_attn_fp8(const void *q, const void *k_pages, const void *v_pages, const float *k_scale,
                                  const float *v_scale, const int32_t *block_table, int max_pages, int num_pages,
                                  const int32_t *seq_lens, int max_seq_len, int B, int Hq, int Hkv, int window,
                                  float sm_scale, int pages_per_split, void *out, void *workspace,
                                  size_t workspace_bytes, void *stream) {
    if (!q || !k_pages || !v_pages || !k_scale || !v_scale || !block_table || !seq_lens || !out) return NC_ERR_NULL;
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || Hq / Hkv > 16 || max_pages <= 0 || num_pages <= 0 ||
        max_seq_len <= 0 || (long long)max_seq_len > (long long)max_pages * PAGE || B > 65535 || Hkv > 65535)
        return NC_ERR_SHAPE;
    AttnArgs a = {};
    a.q = (const uint16_t *)q;
    a.k_pages = (const uint8_t *)k_pages; a.v_pages = (const uint8_t *)v_pages;
    a.k_scale = k_scale; a.v_scale = v_scale;
    a.block_table = block_table; a.max_pages = max_pages; a.num_pages = num_pages;
    a.seq_lens = seq_lens;
    a.B = B; a.T = 1; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv; a.window = window;
    a.scale_log2 = sm_scale * LOG2E;
    int pps;
    a.n_splits = decode_splits(B, Hkv, max_seq_len, window, pages_per_split, pps);
    a.pages_per_split = pps;
    a.out = (uint16_t *)out;
    if (a.n_splits > 1) {
        const size_t need = (size_t)B * Hq * a.n_splits * (HEAD_DIM + 2) * sizeof(float);
        if (!workspace) return NC_ERR_NULL;
        if (workspace_bytes < need) return NC_ERR_WORKSPACE;
        a.part_o = (float *)workspace;
        a.part_ml = a.part_o + (size_t)B * Hq * a.n_splits * HEAD_DIM;
    }
    hipLaunchKernelGGL(decode_split_kernel, dim3(a.n_splits, Hkv, B), dim3(256), 0, (hipStream_t)stream, a);
    if (a.n_splits > 1)
        hipLaunchKernelGGL(decode_combine_kernel, dim3(B * Hq), dim3(HEAD_DIM), 0, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

extern "C" int nc_prefill_attn_fp8(const void *q, const void *k_pages, const void *v_pages, const float *k_scale,
                                   const float *v_scale, const int32_t *block_table, int max_pages, int num_pages,
                                   const int32_t *start_pos, int B, int T, int Hq, int Hkv, int window,
                                   float sm_scale, void *out, void *stream) {
    if (!q || !k_pages || !v_pages || !k_scale || !v_scale || !block_table || !start_pos || !out) return NC_ERR_NULL;
    if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || Hq / Hkv > 16 || max_pages <= 0 || num_pages <= 0 ||
        B > 65535 || Hkv > 65535)
        return NC_ERR_SHAPE;
    AttnArgs a = {};
    a.q = (const uint16_t *)q;
    a.k_pages = (const uint8_t *)k_pages; a.v_pages = (const uint8_t *)v_pages;
    a.k_scale = k_scale; a.v_scale = v_scale;
    a.block_table = block_table; a.max_pages = max_pages; a.num_pages = num_pages;
    a.start_pos = start_pos;
    a.B = B; a.T = T; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv; a.window = window;
    a.scale_log2 = sm_scale * LOG2E;
    a.out = (uint16_t *)out;
    const int tpt = 16 / a.G;
    const int tiles = (T + tpt - 1) / tpt;
    hipLaunchKernelGGL(prefill_kernel, dim3((tiles + WAVES - 1) / WAVES, Hkv, B), dim3(256), 0, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}
