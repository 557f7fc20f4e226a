/*
 * Attention over the paged fp8 cache on gfx950: split-K flash-decode (one query token per sequence, the
 * Hq/Hkv query heads of a KV head served from one read of its pages) and chunked prefill (16 query rows
 * per wave), both on the same page-pair step.
 *
 * The step (attend_pair) streams two 16-token pages of one KV head straight from HBM into registers:
 * each lane issues four 16-byte loads per page pair per operand, every load instruction covering 1 KiB
 * contiguously, because the page tiling (nc_device.h) is the MFMA operand layout. Scores are
 * S^T = K Q^T by two v_mfma_scale_f32_16x16x128_f8f6f4 per page and tile, the cache's e4m3 K codes as they are
 * against the query split into two e4m3 parts whose sum is the (power-of-two scaled) bf16 query exactly; the
 * per-token K scale multiplies the fp32 dot product. The online softmax runs in the log2 domain on the MFMA
 * result layout, and O^T += V^T P^T by eight v_mfma_f32_16x16x32_bf16 per pair (V codes converted exactly to
 * bf16) with the V scale folded into P before its bf16 rounding. Query columns (lane & 15) are query heads in decode and (token, head) rows in
 * prefill; the lane's four row groups (lane >> 4) hold keys 4g..4g+3 of each page.
 *
 * Reference semantics: model/kernels/decode.cu:567-675 (k_attn: keys [max(p - window, 0), p], scale
 * 1/sqrt(128), fp32 softmax) and 859-863 (prefill rows appended before any attends).
 */
#include <limits.h>
#include <math.h>

#include <mutex>

#include "nc_device.h"
#include "nc_row.h"
#include "nanochat_amd.h"
#include "nc_internal.h"

namespace nc {

constexpr float LOG2E = 1.4426950408889634f;
constexpr int WAVES = 4;
constexpr int O_PITCH = HEAD_DIM + 4;  /* LDS row pitch of a wave's merged output (floats) */
constexpr float RESCALE_LOG2 = 8.0f;   /* lazy rescale threshold: exponentials stay <= 2^8 */

struct AttnArgs {
    const uint16_t *q;        /* [B][T][Hq][128] bf16 (T = 1 in decode) */
    const uint8_t *k_pages, *v_pages;
    const float *kv_scale;    /* [num_pages][Hkv][2][16]: K scales, then V scales */
    const int32_t *block_table;
    int max_pages, num_pages;
    const int32_t *seq_lens;  /* decode */
    const int32_t *start_pos; /* prefill: the first position of each sequence's (or run's) rows */
    const int32_t *run_row0;  /* NULL, or prefill runs: run b's rows are q/out rows run_row0[b] .. + run_count[b] */
    const int32_t *run_count;
    const int32_t *run_slot;  /* run b's block-table row */
    int B, T, Hq, Hkv, G, window;
    float scale_log2;         /* sm_scale * log2(e) */
    int workers;              /* decode: waves launched (whole work-groups of 4) */
    int max_len;              /* decode: the longest sequence the launch accepts (its workspace bound) */
    float *part_o;            /* decode partials [items][G][128] */
    float *part_ml;           /* [items][G][2]: reference max (log2 domain), sum */
    int *arrived;             /* [B*Hkv]: chunks of each (sequence, KV head) finished so far; zero between launches */
    uint16_t *out;            /* [B][T][Hq][128] bf16 */
    StepArgs step;            /* the fused decode step's append (decode_kernel<true>) */
};

/* A wave's running state for NT tiles of 16 query columns; lane (g, c) = (lane >> 4, lane & 15) holds column c
 * of every tile. */
template <int NT>
struct WaveState {
    f32x4 o[NT][8];  /* O^T tile d: dims 16d + 4g + i of column c, scaled by 2^-m */
    float m[NT];     /* column c's reference max (log2 domain, equal in the four groups); exponentials use it */
    float l[NT];     /* sum of exp2(s - m) over the keys this lane's group holds */
    float sl2;       /* score multiplier: sm_scale log2(e) */
    bool bad;        /* a block-table entry fell outside the page pool */
};

template <int NT>
__device__ __forceinline__ void state_init(WaveState<NT> &st) {
#pragma unroll
    for (int t = 0; t < NT; t++) {
#pragma unroll
        for (int d = 0; d < 8; d++) st.o[t][d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        st.m[t] = -INFINITY;
        st.l[t] = 0.0f;
    }
    st.bad = false;
}

/* The query operand of column c (B operand of the fp8 score MFMA v_mfma_scale_f32_16x16x128_f8f6f4): lane (g, c) holds
 * dims 32 g .. 32 g + 31 of its row as bytes 0..31, the same (lane, byte) -> k mapping as the K page's A operand
 * (lane (g, key) holds that key's dims 32 g .. + 31). The row times 2^e (e chosen per column, from the column's own
 * largest |q|, which lands in [128, 256)) is split into two e4m3 parts, hi = e4m3(x), lo = e4m3(x - hi): a bf16 value
 * has 8 significant bits and each part 4, so hi + lo = x exactly unless |x| < 2^-2 (then lo may lose bits below 2^-10,
 * at most 2^-18 of the column's largest element). The MFMA's E8M0 scale of the B operand, one per lane (a lane holds
 * exactly one 32-element block of one column), is 2^-e, so the products come out unscaled and one score multiplier
 * serves every column. The score MFMAs read the cache's K codes as they are, with no conversion. Since e depends on
 * the column alone, so do its scores: a row's result does not depend on the rows that share its wave. */
typedef int i32x8 __attribute__((ext_vector_type(8)));

struct QOp {
    i32x8 hi, lo;
    int scale;   /* E8M0 code of 2^-e: 127 - e */
};

__device__ __forceinline__ f32x4 mfma_fp8(const i32x8 &a, const i32x8 &b, int scale_b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, scale_b);   /* A: unit scale */
}

/* QOp of NT tiles from this lane's raw bf16 (raw[t][cc] = dims 32 g + 8 cc .. + 7 of its column in tile t). Every lane
 * of the wave must call it (a column's maximum combines its four row groups). */
template <int NT>
__device__ __forceinline__ void q8_from_raw(const uint4 (&raw)[NT][4], QOp (&q)[NT]) {
    float amax[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        amax[t] = 0.0f;
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            const uint32_t w[4] = {raw[t][cc].x, raw[t][cc].y, raw[t][cc].z, raw[t][cc].w};
#pragma unroll
            for (int i = 0; i < 4; i++)
                amax[t] = fmaxf(amax[t], fmaxf(fabsf(bf16_to_f32((uint16_t)w[i])), fabsf(bf16_to_f32((uint16_t)(w[i] >> 16)))));
        }
        amax[t] = pair_max32(pair_max16(amax[t]));   /* the column's four row groups */
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int E = amax[t] > 0.0f ? (int)((__float_as_uint(amax[t]) >> 23) & 0xFFu) - 127 : 0;
        const int e = min(max(7 - E, -120), 120);
        const float up = __uint_as_float((uint32_t)(127 + e) << 23);
        q[t].scale = 127 - e;
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            const uint32_t w[4] = {raw[t][cc].x, raw[t][cc].y, raw[t][cc].z, raw[t][cc].w};
#pragma unroll
            for (int h = 0; h < 2; h++) {   /* dwords 2 cc + h of the operand: dims 32 g + 8 cc + 4 h .. + 3 */
                float x[4];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    x[2 * i] = bf16_to_f32((uint16_t)w[2 * h + i]) * up;
                    x[2 * i + 1] = bf16_to_f32((uint16_t)(w[2 * h + i] >> 16)) * up;
                }
                int hi = __builtin_amdgcn_cvt_pk_fp8_f32(x[0], x[1], 0, false);
                hi = __builtin_amdgcn_cvt_pk_fp8_f32(x[2], x[3], hi, true);
                const float r[4] = {x[0] - __builtin_amdgcn_cvt_f32_fp8(hi, 0), x[1] - __builtin_amdgcn_cvt_f32_fp8(hi, 1),
                                    x[2] - __builtin_amdgcn_cvt_f32_fp8(hi, 2), x[3] - __builtin_amdgcn_cvt_f32_fp8(hi, 3)};
                int lo = __builtin_amdgcn_cvt_pk_fp8_f32(r[0], r[1], 0, false);
                lo = __builtin_amdgcn_cvt_pk_fp8_f32(r[2], r[3], lo, true);
                q[t].hi[2 * cc + h] = hi;
                q[t].lo[2 * cc + h] = lo;
            }
        }
    }
}

/* Stages NT rows (NULL: zeros) as QOp; every lane of the wave must call it. */
template <int NT>
__device__ __forceinline__ void load_q8(const uint16_t *const (&rows)[NT], int g, QOp (&q)[NT]) {
    uint4 raw[NT][4];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int cc = 0; cc < 4; cc++)
            raw[t][cc] = rows[t] ? *reinterpret_cast<const uint4 *>(rows[t] + g * 32 + cc * 8) : uint4{0u, 0u, 0u, 0u};
    q8_from_raw<NT>(raw, q);
}

/* Scores S^T (keys 4g + i of one page, column c of tile t) = K Q^T for every tile from one page's two K loads
 * (dims 32 g .. + 15, then + 16 .. + 31): two fp8 MFMAs a tile, hi then lo. */
template <int NT>
__device__ __forceinline__ void page_scores(const uint4 &k0, const uint4 &k1, const QOp (&qb)[NT], f32x4 (&s)[NT]) {
    const i32x8 k = {(int)k0.x, (int)k0.y, (int)k0.z, (int)k0.w, (int)k1.x, (int)k1.y, (int)k1.z, (int)k1.w};
#pragma unroll
    for (int t = 0; t < NT; t++) {
        s[t] = mfma_fp8(k, qb[t].hi, qb[t].scale, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        s[t] = mfma_fp8(k, qb[t].lo, qb[t].scale, s[t]);
    }
}

__device__ __forceinline__ uint32_t dword(const uint4 &u, int i) {
    return i == 0 ? u.x : i == 1 ? u.y : i == 2 ? u.z : u.w;
}

__device__ __forceinline__ uint4 and4(const uint4 &u, uint32_t m) { return uint4{u.x & m, u.y & m, u.z & m, u.w & m}; }

/* Two consecutive logical pages (lpa, lpa + 1) of one KV head: their (page, head) indices. Without a second
 * page in range (has_b false) the first is read twice and every key of the copy is masked. */
struct PairAddr {
    long long ha, hb;
    int lpa;
    bool has_b;
};

__device__ __forceinline__ PairAddr pair_addr(const AttnArgs &a, const int32_t *bt, int kvh, int lpa, int end,
                                              bool &bad) {
    PairAddr p;
    p.lpa = lpa;
    p.has_b = lpa + 1 < end;
    int pa = bt[lpa];
    int pb = p.has_b ? bt[lpa + 1] : pa;
    if ((unsigned)pa >= (unsigned)a.num_pages) { bad = true; pa = 0; }
    if ((unsigned)pb >= (unsigned)a.num_pages) { bad = true; pb = 0; }
    p.ha = (long long)pa * a.Hkv + kvh;
    p.hb = (long long)pb * a.Hkv + kvh;
    return p;
}

/* One operand (K or V) of a page pair as this lane loads it: two 1 KiB-contiguous 16-byte loads per page and
 * the four scales of the lane's keys 4g..4g+3. */
struct PairRegs {
    uint4 a0, a1, b0, b1;
    float4 sa, sb;
};

/* Page bytes are streamed once per launch: non-temporal loads (measured ~7 TB/s for a plain stream on MI355X,
 * against ~6.4 TB/s for ordinary loads). */
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 load_nt(const uint8_t *p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return uint4{v[0], v[1], v[2], v[3]};
}

__device__ __forceinline__ float4 load_nt(const float *p) {
    const f32x4v v = __builtin_nontemporal_load(reinterpret_cast<const f32x4v *>(p));
    return float4{v[0], v[1], v[2], v[3]};
}

/* scales: the K (or V) half of kv_scale, i.e. kv_scale (+ 16 for V); a (page, head)'s scales are 32 floats apart. */
__device__ __forceinline__ void load_pair(const uint8_t *pages, const float *scales, const PairAddr &p, int lane,
                                          PairRegs &r) {
    const uint8_t *A = pages + p.ha * PAGE_BYTES + lane * 16;
    const uint8_t *Bp = pages + p.hb * PAGE_BYTES + lane * 16;
    r.a0 = load_nt(A);
    r.a1 = load_nt(A + 1024);
    r.b0 = load_nt(Bp);
    r.b1 = load_nt(Bp + 1024);
    r.sa = load_nt(scales + p.ha * 2 * PAGE + (lane >> 4) * 4);
    r.sb = load_nt(scales + p.hb * 2 * PAGE + (lane >> 4) * 4);
}

/* Key bounds of a wave: in tile t a lane's column sees keys [lo[t], hi[t]]; pairs inside [full_lo, full_hi]
 * are unmasked for every column; V codes of keys past written_hi are not cache contents and are zeroed. */
template <int NT>
struct KeyBounds {
    int lo[NT], hi[NT];
    int full_lo, full_hi, written_hi;
};

/* Softmax update and PV of one pair from its scores. The lazy rescale keeps each column's reference max m until a
 * score passes it by RESCALE_LOG2 (so p <= 2^8). The common case costs one FMA and one exponential a score:
 * p = exp2(acc ks - m) against the current m. Only a column some of whose p exceed 2^8 (or whose m is still -inf) takes
 * the slow path, which moves the column to its new max, rescales it and recomputes its p; the wave enters the slow
 * block when any of its columns needs it, but every column's update depends on its own scores alone, so a query row's
 * result does not depend on the rows that share its wave. The pair's exponentials and PV MFMAs then form one straight
 * block. Each converted V operand feeds NT MFMAs. */
template <int NT, bool MASKED>
__device__ __forceinline__ void pair_update(const AttnArgs &a, const PairAddr &p, const f32x4 (&sa)[NT],
                                            const f32x4 (&sb)[NT], const float4 &ksa, const float4 &ksb, PairRegs &v,
                                            const KeyBounds<NT> &kb, WaveState<NT> &st, int lane) {
    const int g = lane >> 4;
    const int key_a = p.lpa * PAGE + g * 4, key_b = key_a + PAGE;
    if (MASKED) {
        const int na = min(max(kb.written_hi - key_a + 1, 0), 4), nb = p.has_b ? min(max(kb.written_hi - key_b + 1, 0), 4) : 0;
        const uint32_t ma = na >= 4 ? 0xFFFFFFFFu : ((1u << (8 * na)) - 1u);
        const uint32_t mb = nb >= 4 ? 0xFFFFFFFFu : ((1u << (8 * nb)) - 1u);
        v.a0 = and4(v.a0, ma); v.a1 = and4(v.a1, ma);
        v.b0 = and4(v.b0, mb); v.b1 = and4(v.b1, mb);
    }
    const float ks[8] = {ksa.x * st.sl2, ksa.y * st.sl2, ksa.z * st.sl2, ksa.w * st.sl2,
                         ksb.x * st.sl2, ksb.y * st.sl2, ksb.z * st.sl2, ksb.w * st.sl2};
    const float vs[8] = {v.sa.x, v.sa.y, v.sa.z, v.sa.w, v.sb.x, v.sb.y, v.sb.z, v.sb.w};
    bool ok[NT][8];
    float pr[NT][8];
    float pmax = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const float negm = -st.m[t];   /* +inf before the first key: every live p is +inf, the slow path */
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float acc = i < 4 ? sa[t][i] : sb[t][i - 4];
            if (MASKED) {
                const int key = (i < 4 ? key_a : key_b) + (i & 3);
                ok[t][i] = (i < 4 || p.has_b) && key >= kb.lo[t] && key <= kb.hi[t];
            } else {
                ok[t][i] = true;
            }
            pr[t][i] = ok[t][i] ? __builtin_amdgcn_exp2f(__builtin_fmaf(acc, ks[i], negm)) : 0.0f;
            pmax = fmaxf(pmax, pr[t][i]);
        }
    }
    if (__any(!(pmax <= 256.0f))) {   /* some column's max passed its reference by more than 2^8 (or has none yet) */
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float pc = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) pc = fmaxf(pc, pr[t][i]);
            pc = pair_max32(pair_max16(pc));   /* the column's largest p over its four row groups */
            if (pc <= 256.0f) continue;        /* this column keeps its reference and its p (NaN-free: pc >= 0) */
            float s[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float acc = i < 4 ? sa[t][i] : sb[t][i - 4];
                s[i] = ok[t][i] ? acc * ks[i] : -INFINITY;
            }
            float mt = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
            mt = pair_max32(pair_max16(mt));   /* the column's max over the four row groups */
            const float mnew = fmaxf(st.m[t], mt);
            const float alpha = mnew == st.m[t] ? 1.0f : __builtin_amdgcn_exp2f(st.m[t] - mnew);
#pragma unroll
            for (int d = 0; d < 8; d++) st.o[t][d] *= alpha;
            st.l[t] *= alpha;
            st.m[t] = mnew;
            const float mbase = mnew == -INFINITY ? 0.0f : mnew;  /* no key yet: every s is -inf */
#pragma unroll
            for (int i = 0; i < 8; i++) pr[t][i] = __builtin_amdgcn_exp2f(s[i] - mbase);
        }
    }
    bf16x8 pv[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            psum += pr[t][i];
            pv[t][i] = (__bf16)(pr[t][i] * vs[i]);
        }
        st.l[t] += psum;
    }
#pragma unroll
    for (int d = 0; d < 8; d++) {
        const bf16x8 va = fp8x8_to_bf16(dword(d < 4 ? v.a0 : v.a1, d & 3), dword(d < 4 ? v.b0 : v.b1, d & 3));
#pragma unroll
        for (int t = 0; t < NT; t++) st.o[t][d] = mfma16x16x32(va, pv[t], st.o[t][d]);
    }
}

template <int NT>
__device__ __forceinline__ void pair_step(const AttnArgs &a, const PairAddr &cur, const f32x4 (&sa)[NT],
                                          const f32x4 (&sb)[NT], const float4 &ksa, const float4 &ksb, PairRegs &vr,
                                          const KeyBounds<NT> &kb, WaveState<NT> &st, int lane) {
    const bool interior = cur.has_b && cur.lpa * PAGE >= kb.full_lo && cur.lpa * PAGE + 2 * PAGE - 1 <= kb.full_hi &&
                          cur.lpa * PAGE + 2 * PAGE - 1 <= kb.written_hi;
    if (interior)
        pair_update<NT, false>(a, cur, sa, sb, ksa, ksb, vr, kb, st, lane);
    else
        pair_update<NT, true>(a, cur, sa, sb, ksa, ksb, vr, kb, st, lane);
}

/* pair_step with the scores made inside each branch from the pair's K operands (k0, k1: page a; k2, k3: page b), so
 * the score MFMAs share a scheduling block with the exponentials: page a's products first, then page b's, one at a
 * time between groups of page a's softmax instructions, which do not wait for them (c4: 830-843 -> 868-875 TFLOP/s
 * against all eight products issued before the branch). The wave raises its priority while it issues them, so the
 * SIMD's other wave, when it is in its softmax, issues between them (870 -> 882 TFLOP/s; the same around the PV
 * products added nothing). */
template <int NT, bool MASKED>
__device__ __forceinline__ void pair_update_k(const AttnArgs &a, const PairAddr &p, const uint4 &k0, const uint4 &k1,
                                              const uint4 &k2, const uint4 &k3, const QOp (&qb)[NT],
                                              const float4 &ksa, const float4 &ksb, PairRegs &v,
                                              const KeyBounds<NT> &kb, WaveState<NT> &st, int lane) {
    f32x4 sa[NT], sb[NT];
    __builtin_amdgcn_s_setprio(1);   /* the other wave of the SIMD runs its VALU while these products issue */
    page_scores<NT>(k0, k1, qb, sa);
    page_scores<NT>(k2, k3, qb, sb);
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * NT, 0);
#pragma unroll
    for (int i = 0; i < 2 * NT; i++) {   /* groups of 2 to 10 VALU instructions measured the same */
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    }
    __builtin_amdgcn_s_setprio(0);
    pair_update<NT, MASKED>(a, p, sa, sb, ksa, ksb, v, kb, st, lane);
}

template <int NT>
__device__ __forceinline__ void pair_step_k(const AttnArgs &a, const PairAddr &cur, const uint4 &k0, const uint4 &k1,
                                            const uint4 &k2, const uint4 &k3, const QOp (&qb)[NT], const float4 &ksa,
                                            const float4 &ksb, PairRegs &vr, const KeyBounds<NT> &kb,
                                            WaveState<NT> &st, int lane) {
    const bool interior = cur.has_b && cur.lpa * PAGE >= kb.full_lo && cur.lpa * PAGE + 2 * PAGE - 1 <= kb.full_hi &&
                          cur.lpa * PAGE + 2 * PAGE - 1 <= kb.written_hi;
    if (interior)
        pair_update_k<NT, false>(a, cur, k0, k1, k2, k3, qb, ksa, ksb, vr, kb, st, lane);
    else
        pair_update_k<NT, true>(a, cur, k0, k1, k2, k3, qb, ksa, ksb, vr, kb, st, lane);
}

/*
 * A wave's pass over the page pairs lpa0, lpa0 + step, ... below `end` (logical pages of KV head kvh through
 * block-table row bt). PREFETCH: the next pair's K loads are issued as soon as this pair's scores are computed,
 * its V loads as soon as this pair's PV is issued, so one pair is always in flight per wave (both kernels use it;
 * measured 6% faster for prefill at two column tiles). Without it a pair's loads are issued at the top of its
 * step, which needs fewer registers.
 */
template <int NT, bool PREFETCH>
__device__ __forceinline__ void attend_pages(const AttnArgs &a, const int32_t *bt, int kvh, int lpa0, int step, int end,
                                             const KeyBounds<NT> &kb, const QOp (&qb)[NT], WaveState<NT> &st,
                                             int lane) {
    if (lpa0 >= end) return;
    if (PREFETCH) {
        PairAddr cur = pair_addr(a, bt, kvh, lpa0, end, st.bad);
        PairRegs kr, vr;
        load_pair(a.k_pages, a.kv_scale, cur, lane, kr);
        load_pair(a.v_pages, a.kv_scale + PAGE, cur, lane, vr);
        for (int lpa = lpa0; lpa < end; lpa += step) {
            const bool more = lpa + step < end;
            PairAddr nxt = cur;
            if (more) nxt = pair_addr(a, bt, kvh, lpa + step, end, st.bad);
            f32x4 sa[NT], sb[NT];
            page_scores<NT>(kr.a0, kr.a1, qb, sa);
            page_scores<NT>(kr.b0, kr.b1, qb, sb);
            const float4 ksa = kr.sa, ksb = kr.sb;
            if (more) load_pair(a.k_pages, a.kv_scale, nxt, lane, kr);
            pair_step<NT>(a, cur, sa, sb, ksa, ksb, vr, kb, st, lane);
            if (more) load_pair(a.v_pages, a.kv_scale + PAGE, nxt, lane, vr);
            cur = nxt;
        }
    } else {
        for (int lpa = lpa0; lpa < end; lpa += step) {
            const PairAddr cur = pair_addr(a, bt, kvh, lpa, end, st.bad);
            PairRegs kr, vr;
            load_pair(a.k_pages, a.kv_scale, cur, lane, kr);
            load_pair(a.v_pages, a.kv_scale + PAGE, cur, lane, vr);
            f32x4 sa[NT], sb[NT];
            page_scores<NT>(kr.a0, kr.a1, qb, sa);
            page_scores<NT>(kr.b0, kr.b1, qb, sb);
            pair_step<NT>(a, cur, sa, sb, kr.sa, kr.sb, vr, kb, st, lane);
        }
    }
}

/* The same pass with the page ids staged in registers by the caller (entry i is the page of logical page tab0 + i)
 * and the pages read through buffer descriptors. Inside the loop the only vector-memory loads are the K/V stream and
 * none is conditional: after the last pair the prefetch goes through zero-range descriptors (zeros, no memory access),
 * so every wait the compiler places counts only the stream (a conditional or table load in the loop made each pair
 * wait for every load in flight). */
typedef __amdgpu_buffer_rsrc_t Rsrc;

/* s_waitcnt operands (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8), expcnt and lgkmcnt left
 * at their maxima */
constexpr int VMCNT0 = 0x0F70;    /* vmcnt(0) */
constexpr int VMCNT12 = 0x0F7C;   /* vmcnt(12): all but the 12 most recent vector memory operations complete */

/* A descriptor over `bytes` bytes from p, p the same in every lane (its halves are read from the first lane, so the
 * descriptor lives in scalar registers and no load needs a per-lane loop). */
__device__ __forceinline__ Rsrc page_rsrc(const void *p, int bytes) {
    const unsigned long long u = (unsigned long long)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)u), hi = __builtin_amdgcn_readfirstlane((unsigned)(u >> 32));
    void *q = (void *)(((unsigned long long)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(q, (short)0, __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

/* non-temporal (aux bit 1: nt): page bytes are streamed once per launch */
__device__ __forceinline__ uint4 bload_nt(Rsrc r, int off) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
    return uint4{v[0], v[1], v[2], v[3]};
}

/* A wave's staged block-table entries of one chunk: lane j holds entries j (v) and 64 + j (v2), at most 128. Entry e
 * (wave-uniform) is read by v_readlane into a scalar register: no vector register or LDS access in the pair loop. */
struct TabRegs {
    int v, v2;
};

__device__ __forceinline__ int tab_entry(const TabRegs &t, int e) {
    const int lo = __builtin_amdgcn_readlane(t.v, e & (WAVE - 1)), hi = __builtin_amdgcn_readlane(t.v2, e & (WAVE - 1));
    return e < WAVE ? lo : hi;
}

__device__ __forceinline__ PairAddr pair_addr_tab(const AttnArgs &a, const TabRegs &tab, int tab0, int kvh, int lpa,
                                                  int end, bool &bad) {
    PairAddr p;
    p.lpa = lpa;
    p.has_b = lpa + 1 < end;
    int pa = tab_entry(tab, lpa - tab0);
    int pb = p.has_b ? tab_entry(tab, lpa + 1 - tab0) : pa;
    if ((unsigned)pa >= (unsigned)a.num_pages) { bad = true; pa = 0; }
    if ((unsigned)pb >= (unsigned)a.num_pages) { bad = true; pb = 0; }
    p.ha = (long long)pa * a.Hkv + kvh;
    p.hb = (long long)pb * a.Hkv + kvh;
    return p;
}

/* load_pair through descriptors of one (page, head) each; live false: zero-range descriptors (zeros, no access). */
__device__ __forceinline__ void load_pair_b(const uint8_t *pages, const float *scales, const PairAddr &p, bool live,
                                            int lane, PairRegs &r) {
    const int pb = live ? PAGE_BYTES : 0, sb = live ? PAGE * 4 : 0;
    const Rsrc A = page_rsrc(pages + p.ha * PAGE_BYTES, pb), B = page_rsrc(pages + p.hb * PAGE_BYTES, pb);
    r.a0 = bload_nt(A, lane * 16);
    r.a1 = bload_nt(A, 1024 + lane * 16);
    r.b0 = bload_nt(B, lane * 16);
    r.b1 = bload_nt(B, 1024 + lane * 16);
    const uint4 sa = bload_nt(page_rsrc(scales + p.ha * 2 * PAGE, sb), (lane >> 4) * 16);
    const uint4 sbv = bload_nt(page_rsrc(scales + p.hb * 2 * PAGE, sb), (lane >> 4) * 16);
    r.sa = float4{__uint_as_float(sa.x), __uint_as_float(sa.y), __uint_as_float(sa.z), __uint_as_float(sa.w)};
    r.sb = float4{__uint_as_float(sbv.x), __uint_as_float(sbv.y), __uint_as_float(sbv.z), __uint_as_float(sbv.w)};
}

/* One pair from registers already loaded: scores, softmax, PV. */
template <int NT>
__device__ __forceinline__ void pair_from_regs(const AttnArgs &a, const PairAddr &cur, const PairRegs &kr,
                                               PairRegs &vr, const KeyBounds<NT> &kb, const QOp (&qb)[NT],
                                               WaveState<NT> &st, int lane) {
    f32x4 sa[NT], sb[NT];
    page_scores<NT>(kr.a0, kr.a1, qb, sa);
    page_scores<NT>(kr.b0, kr.b1, qb, sb);
    pair_step<NT>(a, cur, sa, sb, kr.sa, kr.sb, vr, kb, st, lane);
}

/* Two register sets rotate by name (the loop is unrolled by two): a pair's K and V are issued as the pair before it
 * starts computing, so a whole pair's loads stay in flight behind every pair's math and no copy waits on a load.
 * The pass's first pair (c0, k0, v0: pages lpa0, lpa0 + 1) is issued by the caller, before it stages its query, so
 * the query's latency hides behind the first loads. lpa0 < end.
 */
template <int NT>
__device__ __forceinline__ void attend_pages_tab(const AttnArgs &a, const TabRegs &tab, int tab0, int kvh, int lpa0,
                                                 int end, const KeyBounds<NT> &kb, const QOp (&qb)[NT],
                                                 WaveState<NT> &st, int lane, PairAddr c0, PairRegs k0, PairRegs v0,
                                                 bool fence_stores) {
    /* wave-uniform in scalar registers, so a pair's address math is scalar and borrows no vector register a load in
     * flight still owns */
    lpa0 = __builtin_amdgcn_readfirstlane(lpa0);
    end = __builtin_amdgcn_readfirstlane(end);
    kvh = __builtin_amdgcn_readfirstlane(kvh);
    tab0 = __builtin_amdgcn_readfirstlane(tab0);
    bool more1 = lpa0 + 2 < end;
    PairAddr c1 = pair_addr_tab(a, tab, tab0, kvh, more1 ? lpa0 + 2 : lpa0, end, st.bad);
    PairRegs k1, v1;
    load_pair_b(a.k_pages, a.kv_scale, c1, more1, lane, k1);
    load_pair_b(a.v_pages, a.kv_scale + PAGE, c1, more1, lane, v1);
    /* the caller's stores (issued before this second pair's 12 loads) complete before any later page load issues */
    if (fence_stores) __builtin_amdgcn_s_waitcnt(VMCNT12);
    for (int lpa = lpa0;; lpa += 4) {
        pair_from_regs<NT>(a, c0, k0, v0, kb, qb, st, lane);
        if (!more1) break;
        const bool more0 = lpa + 4 < end;
        c0 = pair_addr_tab(a, tab, tab0, kvh, more0 ? lpa + 4 : lpa + 2, end, st.bad);
        load_pair_b(a.k_pages, a.kv_scale, c0, more0, lane, k0);
        load_pair_b(a.v_pages, a.kv_scale + PAGE, c0, more0, lane, v0);
        pair_from_regs<NT>(a, c1, k1, v1, kb, qb, st, lane);
        if (!more0) break;
        more1 = lpa + 6 < end;
        c1 = pair_addr_tab(a, tab, tab0, kvh, more1 ? lpa + 6 : lpa + 4, end, st.bad);
        load_pair_b(a.k_pages, a.kv_scale, c1, more1, lane, k1);
        load_pair_b(a.v_pages, a.kv_scale + PAGE, c1, more1, lane, v1);
    }
}

/* Split points of decode: a (sequence, KV head) unit's keys are cut at every multiple of SPLIT_PAGES pages (1,024
 * positions), except that a last piece of fewer than MIN_TAIL pages joins the chunk before it (a sequence one token
 * past a multiple of 1,024 would otherwise spend a work item, and a merge step, on one page). A unit that would be one
 * chunk (at most SPLIT_PAGES + MIN_TAIL - 1 pages) is cut at every multiple of SHORT_SPLIT pages instead, with the same
 * join, so a short context is streamed by several waves rather than one. The cuts depend on nothing but the sequence's
 * own length (and the window), whatever the rest of the batch holds, so a sequence's sums (and its output bits) depend
 * only on its own query, keys and length. */
constexpr int SPLIT_PAGES = 64;
constexpr int SHORT_SPLIT = 16;
constexpr int MIN_TAIL = 4;
constexpr int SHORT_UNIT = SPLIT_PAGES + MIN_TAIL - 1;   /* the most pages a unit of short chunks holds */
static_assert(SPLIT_PAGES + MIN_TAIL - 1 <= 2 * WAVE, "a chunk's block-table entries are staged in two lanes' worth");

/* Key range [begin, p] of a sequence of L keys and its logical pages [pg0, pg0 + npages); npages = 0 for an
 * inactive sequence (L <= 0) or one longer than max_len (the launch's bound; its output is NaN). */
__device__ __forceinline__ int decode_pages(const AttnArgs &a, int L, int &begin, int &pg0) {
    if (L <= 0 || L > a.max_len) return 0;
    const int p = L - 1;
    begin = a.window >= 0 ? max(p - a.window, 0) : 0;
    pg0 = begin / PAGE;
    return p / PAGE + 1 - pg0;
}

/* How a unit's logical pages [pg0, e) split (S = SPLIT_PAGES, or SHORT_SPLIT for a unit of at most SHORT_UNIT pages;
 * c0 = pg0 / S): chunk j covers [pg0 or (c0 + j) S, (c0 + j + 1) S or e), the first starting at pg0 and the last
 * ending at e; the pieces are cut at the multiples of S and a last piece shorter than MIN_TAIL joins the one before
 * it. A chunk is full when it covers at least SPLIT_PAGES pages; only the first and the last can be partial, and every
 * chunk of a unit of short chunks is. */
struct UnitSplit {
    int pg0, np, nch;   /* pages, chunks */
    int p0;             /* 1: chunk 0 is partial */
    int nfull, npart;   /* full and partial chunks */
    int s;              /* the cut: SPLIT_PAGES or SHORT_SPLIT */
};

__device__ __forceinline__ UnitSplit unit_split(const AttnArgs &a, int L, int &begin) {
    UnitSplit u = {0, 0, 0, 0, 0, 0, SPLIT_PAGES};
    const int np = decode_pages(a, L, begin, u.pg0);
    if (np <= 0) return u;
    const int S = np <= SHORT_UNIT ? SHORT_SPLIT : SPLIT_PAGES;
    const int e = u.pg0 + np, c0 = u.pg0 / S;
    u.np = np;
    u.s = S;
    const int pieces = (e - 1) / S - c0 + 1;
    const int tail = e - max(u.pg0, ((e - 1) / S) * S);
    u.nch = pieces - (pieces >= 2 && tail < MIN_TAIL);
    if (S == SHORT_SPLIT) {
        u.p0 = 1;
        u.npart = u.nch;
        u.nfull = 0;
        return u;
    }
    const int size0 = (u.nch == 1 ? e : (c0 + 1) * S) - u.pg0;
    const int sizel = e - (c0 + u.nch - 1) * S;
    u.p0 = size0 < S;
    u.npart = u.p0 + (u.nch > 1 && sizel < S);
    u.nfull = u.nch - u.npart;
    return u;
}

/* Logical pages [first, last) of chunk j. */
__device__ __forceinline__ void chunk_pages(const UnitSplit &u, int j, int &first, int &last) {
    const int c = u.pg0 / u.s + j;
    first = j == 0 ? u.pg0 : c * u.s;
    last = j == u.nch - 1 ? u.pg0 + u.np : (c + 1) * u.s;
}

__device__ __forceinline__ void store_bf16x4(uint16_t *dst, const float *v) {
    uint2 u;
    u.x = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
    u.y = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
    *reinterpret_cast<uint2 *>(dst) = u;
}

constexpr int MAX_DECODE_BATCH = 4096;  /* sequences per decode launch (the LDS chunk prefixes: 32 KiB) */

/* The last b in [0, B) with cum[b] <= k (cum non-decreasing, cum[0] = 0 <= k). */
__device__ __forceinline__ int find_sequence(const int *cum, int B, int k) {
    int lo = 0, hi = B - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cum[mid] <= k) lo = mid; else hi = mid - 1;
    }
    return lo;
}

/* Rows of the sequences with nothing to attend (found by their empty chunk ranges): zeros for an inactive sequence
 * (L <= 0), NaN for one longer than the launch's bound. Wave `id` of `waves` takes sequences id, id + waves, ... */
__device__ __forceinline__ void decode_fill_rows(const AttnArgs &a, const int *cf, const int *cp, int id, int waves,
                                                 int lane) {
    for (int b = id; b < a.B; b += waves) {
        if (cf[b + 1] != cf[b] || cp[b + 1] != cp[b]) continue;
        const uint32_t w = a.seq_lens[b] <= 0 ? 0u : 0x7FC07FC0u;
        uint2 *dst = reinterpret_cast<uint2 *>(a.out + (long long)b * a.Hq * HEAD_DIM);
        for (int i = lane; i < a.Hq * HEAD_DIM / 4; i += WAVE) dst[i] = uint2{w, w};
    }
}

/* The fused step's append work for one item of unit (b, kvh), the token at position p. Every item normalizes and
 * rotates the unit's G query rows into q_lds (bf16, row h at h * 128). The item that streams the token (own: the
 * unit's last chunk, the only one holding it) also normalizes and rotates k, mixes the value embedding into v,
 * quantizes both and stores codes and scales into the cache (unless the page is outside the pool); it also writes
 * q_out. Each row is the append kernel's arithmetic (nc_row.h), so the cache bytes and query bits equal those of the
 * separate append. Every load of the item is issued before any of its arithmetic (one round trip); the raw query
 * rows go through q_lds, where each lane's pair (dims l, l + 64) of a row is read and overwritten by the same lane.
 *
 * The pass reads the token's bytes back from the cache, so they must be stored before its page is loaded. The pass's
 * first page pair is issued before these stores (the query's work hides behind its latency) and its second right
 * after them; then the pass waits until all but the second pair's 12 loads have completed (vector memory operations
 * of a wave complete in issue order, one counter for loads and stores), which the first pair's use needs anyway, so
 * every later page load is issued after the stores have completed. A token in the first two pairs (first 4 pages)
 * is the exception: the caller then issues the first pair without access (zero-range descriptors), waits here for
 * the stores (`wait`) and issues it again. No other pass reads the token's page. */
constexpr int MAX_G = 16;
constexpr int Q_CHUNKS = MAX_G * HEAD_DIM * 2 / (16 * WAVE);   /* 16-byte loads a lane for the unit's query rows */

/* What step_rows reads, fetched before the pass's first page pair is issued: vector memory operations of a wave
 * complete in issue order, so a wait for anything issued after the page loads would wait for them too. */
struct StepLoads {
    uint4 raw[Q_CHUNKS];            /* the unit's raw query rows, 16 bytes a lane */
    float cr, sr, g1, g2, kg1, kg2; /* rotation of position p and gains (dims l, l + 64) */
    uint16_t kx1, kx2, vx1, vx2;    /* own: the token's k and v rows (dims l, l + 64) */
};

/* All through buffer (not flat) accesses: a flat access may address LDS, which would make the LDS accesses below wait
 * for every vector memory operation in flight. */
__device__ __forceinline__ StepLoads step_fetch(const AttnArgs &a, const StepArgs &s, int b, int kvh, int p, bool own,
                                                int lane) {
    StepLoads f;
    const uint16_t *row = s.qkv + (long long)b * s.token_stride;
    const Rsrc rq = page_rsrc(row + kvh * a.G * HEAD_DIM, a.G * HEAD_DIM * 2);
#pragma unroll
    for (int i = 0; i < Q_CHUNKS; i++) {   /* chunks past the G rows read zeros through the range (no access) */
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rq, (i * WAVE + lane) * 16, 0, 0);
        f.raw[i] = uint4{v[0], v[1], v[2], v[3]};
    }
    const Rsrc rc = page_rsrc(s.cos + (long long)p * HALF, HALF * 4), rs = page_rsrc(s.sin + (long long)p * HALF, HALF * 4);
    const Rsrc rqg = page_rsrc(s.q_gain, HEAD_DIM * 4), rkg = page_rsrc(s.k_gain, own ? HEAD_DIM * 4 : 0);
    f.cr = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rc, lane * 4, 0, 0));
    f.sr = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, lane * 4, 0, 0));
    f.g1 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rqg, lane * 4, 0, 0));
    f.g2 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rqg, (lane + HALF) * 4, 0, 0));
    f.kg1 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rkg, lane * 4, 0, 0));
    f.kg2 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rkg, (lane + HALF) * 4, 0, 0));
    /* own: the token's k and v rows (zero-range descriptors otherwise: no access) */
    const Rsrc rk = page_rsrc(row + (a.Hq + kvh) * HEAD_DIM, own ? HEAD_DIM * 2 : 0);
    const Rsrc rv = page_rsrc(row + (a.Hq + a.Hkv + kvh) * HEAD_DIM, own ? HEAD_DIM * 2 : 0);
    f.kx1 = __builtin_amdgcn_raw_buffer_load_b16(rk, lane * 2, 0, 0);
    f.kx2 = __builtin_amdgcn_raw_buffer_load_b16(rk, (lane + HALF) * 2, 0, 0);
    f.vx1 = __builtin_amdgcn_raw_buffer_load_b16(rv, lane * 2, 0, 0);
    f.vx2 = __builtin_amdgcn_raw_buffer_load_b16(rv, (lane + HALF) * 2, 0, 0);
    return f;
}

template <bool VE>
__device__ __forceinline__ void step_rows(const AttnArgs &a, const StepArgs &s, const StepLoads &f, int b, int kvh,
                                          int p, bool own, int page, bool wait, uint16_t *q_lds, int lane) {
#pragma unroll
    for (int i = 0; i < Q_CHUNKS; i++)
        if (i * WAVE * 8 < a.G * HEAD_DIM) *reinterpret_cast<uint4 *>(q_lds + (i * WAVE + lane) * 8) = f.raw[i];
    /* unrolled (forward branches only): a loop here would make the compiler wait for every load in flight at its
     * entry, the first page pair included */
#pragma unroll
    for (int h = 0; h < MAX_G; h++) {
        if (h >= a.G) break;
        float y1, y2;
        norm_rope_pair(bf16_to_f32(q_lds[h * HEAD_DIM + lane]), bf16_to_f32(q_lds[h * HEAD_DIM + lane + HALF]), f.g1,
                       f.g2, f.cr, f.sr, y1, y2);
        const uint16_t q1 = f32_to_bf16(y1), q2 = f32_to_bf16(y2);
        q_lds[h * HEAD_DIM + lane] = q1;
        q_lds[h * HEAD_DIM + lane + HALF] = q2;
        if (own && s.q_out) {
            const Rsrc ro = page_rsrc(s.q_out + ((long long)b * a.Hq + kvh * a.G + h) * HEAD_DIM, HEAD_DIM * 2);
            __builtin_amdgcn_raw_buffer_store_b16(q1, ro, lane * 2, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b16(q2, ro, (lane + HALF) * 2, 0, 0);
        }
    }
    if (!own) return;
    float y1, y2;
    norm_rope_pair(bf16_to_f32(f.kx1), bf16_to_f32(f.kx2), f.kg1, f.kg2, f.cr, f.sr, y1, y2);
    const float k1 = bf16_to_f32(f32_to_bf16(y1)), k2 = bf16_to_f32(f32_to_bf16(y2));
    float v1 = bf16_to_f32(f.vx1), v2 = bf16_to_f32(f.vx2);
    if (VE && s.ve) {
        const int token = s.ve_tokens[b];
        if ((unsigned)token < (unsigned)s.ve_rows)
            ve_mix_pair(s.ve_h + (long long)b * s.C, s.ve_gate + (long long)kvh * s.C, s.C,
                        s.ve + (long long)token * s.C + kvh * HEAD_DIM, lane, v1, v2);
    }
    uint32_t kc1, kc2, vc1, vc2;
    const int slot = p % PAGE;
    const float ks = quantize_pair(k1, k2, kc1, kc2);
    const float vs = quantize_pair(v1, v2, vc1, vc2);
    if ((unsigned)page >= (unsigned)a.num_pages) return;   /* the pass reports the bad entry */
    const long long at = (long long)page * a.Hkv + kvh;
    const Rsrc rkp = page_rsrc(s.k_pages + at * PAGE_BYTES, PAGE_BYTES);
    const Rsrc rvp = page_rsrc(s.v_pages + at * PAGE_BYTES, PAGE_BYTES);
    const Rsrc rsc = page_rsrc(s.kv_scale + at * 2 * PAGE, 2 * PAGE * 4);
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)kc1, rkp, k_page_offset(slot, lane), 0, 0);
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)kc2, rkp, k_page_offset(slot, lane + HALF), 0, 0);
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)vc1, rvp, v_page_offset(slot, lane), 0, 0);
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)vc2, rvp, v_page_offset(slot, lane + HALF), 0, 0);
    if (lane == 0) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(ks), rsc, slot * 4, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(vs), rsc, (PAGE + slot) * 4, 0, 0);
    }
    if (wait) __builtin_amdgcn_s_waitcnt(VMCNT0);
}

/* Partials cross work-groups (and XCDs, whose L2 caches are not coherent with each other) inside one launch. They
 * are written and read with the sc1 cache policy, the encoding of agent-scope atomic stores and loads (coherent
 * across the device: stores write through, loads miss stale lines), and the writer waits for its stores to complete
 * (vmcnt 0) before it counts its chunk, so the wave that sees the last count reads every partial as written. This
 * costs no cache-wide writeback or invalidate, which an agent-scope fence would (measured: twice the kernel time). */
constexpr int SC1 = 16;   /* cache-policy operand of the buffer builtins: sc1 */
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void part_store(Rsrc r, int off, const float4 &v) {
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                                                 __float_as_uint(v.w)}, r, off, 0, SC1);
}

__device__ __forceinline__ f32x4 part_load(Rsrc r, int off) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, SC1);
    return f32x4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
}

/* A partial slot's two descriptors: O [G][128] and (max, sum) [G][2]. */
__device__ __forceinline__ void part_rsrc(const AttnArgs &a, long long slot, Rsrc &ro, Rsrc &rm) {
    ro = page_rsrc(a.part_o + slot * a.G * HEAD_DIM, a.G * HEAD_DIM * 4);
    rm = page_rsrc(a.part_ml + slot * a.G * 2, a.G * 2 * 4);
}

/* The log-sum-exp (base 2) merge of a unit's nch partials, in chunk order, into its bf16 rows. The unit's G x 128
 * outputs are split into 16-byte pieces (piece p: column p / 32, dims 4 (p % 32) .. + 3); a call merges pieces
 * piece0 .. piece0 + 64 P - 1, lane l taking piece0 + l, piece0 + l + 64, ..., so every lane works for any G. Chunks are taken NB at a time with all their loads issued
 * together (the merge is latency-bound: it runs when the unit's last chunk ends): a batch raises the running maximum M
 * to the batch's largest chunk maximum, rescales the running (sum, O) by exp2(M_old - M) and adds each chunk's
 * (sum, O) times exp2(m_j - M), in chunk order. The order depends on nch alone, so the result does not depend on
 * which wave merges. Out-of-range pieces and chunks read zeros through the descriptors' ranges and store nothing. */
template <int P, int NB>
__device__ __forceinline__ void merge_pieces(const AttnArgs &a, long long slot0, int nch, long long row0, int piece0,
                                             int lane) {
    const int pieces = a.G * (HEAD_DIM / 4);
    float M[P], L[P];
    f32x4 O[P];
#pragma unroll
    for (int k = 0; k < P; k++) {
        M[k] = -INFINITY;
        L[k] = 0.0f;
        O[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    /* one descriptor pair over the unit's nch slots: chunk j's O at j G 512 bytes, its (max, sum) at j G 8 */
    const Rsrc ro = page_rsrc(a.part_o + slot0 * a.G * HEAD_DIM, nch * a.G * HEAD_DIM * 4);
    const Rsrc rm = page_rsrc(a.part_ml + slot0 * a.G * 2, nch * a.G * 2 * 4);
    for (int j0 = 0; j0 < nch; j0 += NB) {
        f32x4 oj[NB][P];
        float2 ml[NB][P];
#pragma unroll
        for (int jj = 0; jj < NB; jj++) {
#pragma unroll
            for (int k = 0; k < P; k++) {
                const int p = piece0 + lane + WAVE * k;
                oj[jj][k] = part_load(ro, (j0 + jj) * a.G * HEAD_DIM * 4 + p * 16);
                const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(rm, ((j0 + jj) * a.G + (p >> 5)) * 8, 0, SC1);
                ml[jj][k] = float2{__uint_as_float(w[0]), __uint_as_float(w[1])};
            }
        }
#pragma unroll
        for (int k = 0; k < P; k++) {
            float mb = M[k];
#pragma unroll
            for (int jj = 0; jj < NB; jj++)
                if (j0 + jj < nch) mb = fmaxf(mb, ml[jj][k].x);
            const float alpha = M[k] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M[k] - mb);
            L[k] *= alpha;
            O[k] *= alpha;
            M[k] = mb;
#pragma unroll
            for (int jj = 0; jj < NB; jj++) {
                if (j0 + jj >= nch) continue;
                const float w = ml[jj][k].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml[jj][k].x - mb);
                L[k] += ml[jj][k].y * w;
                O[k] += oj[jj][k] * w;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < P; k++) {
        const int p = piece0 + lane + WAVE * k;
        if (p >= pieces) continue;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = O[k][i] / L[k];
        store_bf16x4(a.out + (row0 + (p >> 5)) * HEAD_DIM + (p & 31) * 4, v);
    }
}

/* 128 pieces (4 columns) per pass: one instantiation serves every G, in at most 4 passes. */
__device__ __forceinline__ void merge_unit(const AttnArgs &a, long long slot0, int nch, long long row0, int lane) {
    for (int piece0 = 0; piece0 < a.G * (HEAD_DIM / 4); piece0 += 2 * WAVE)
        merge_pieces<2, 8>(a, slot0, nch, row0, piece0, lane);
}

/*
 * Split-K decode over fixed chunks. The work items are a unit's chunks (unit = (sequence, KV head)); every item starts
 * from a fresh softmax state and streams only its chunk's pages, so what is computed for an item does not depend on
 * which wave takes it or on what else the launch holds. A unit of one chunk is finished in place (bf16 output); a unit
 * of several leaves one partial per chunk, in slot cf[b] + cp[b] + kvh nch + j (the unit-order index of chunk j), and
 * counts its finished chunks in arrived[u]: the wave that finishes the last one merges the partials in chunk order
 * (merge_unit) and returns the count to zero. Partials are stored and loaded device-coherently (sc1) and complete
 * before they are counted, so the merging wave sees every other wave's partials whatever CU or XCD ran them; no
 * second launch is needed.
 *
 * Schedule: the full chunks (at least SPLIT_PAGES long) are numbered first, then the partial ones, each in (sequence, KV
 * head) order, a unit's full chunks rotated (its f-th full item takes full chunk (f + u + k0 / G) mod nfull, u the
 * unit's index, k0 its first full item); item k goes to work-group k % G (G = gridDim.x) and, within it, to wave
 * (k / G) % 4, round
 * k / (4 G). Equal full chunks land one per work-group before any doubles up, and the short partial chunks fill in
 * last: every compute unit streams about the same number of pages (a CU's bandwidth, not a wave's, is the limit once
 * it holds more than one wave), and a wave that finishes early leaves the HBM bandwidth to the others.
 *
 * STEP (the fused decode step): the sequence's token at position L - 1 is appended in the same launch (step_rows):
 * every item normalizes and rotates its query rows from the raw qkv row, and the item holding the token quantizes and
 * stores its K and V before its pass reads them back. VE: the step mixes value embeddings into v; a step without them
 * runs an instantiation without that code (243 VGPRs against 256: the gate's double exponential holds its constants
 * in registers).
 */
template <bool STEP, bool VE = false>
__global__ void __launch_bounds__(256, 2) decode_kernel(AttnArgs a) {
    extern __shared__ int sh_cum[];  /* [2][B + 1]: full, then partial chunks of the sequences < b */
    __shared__ __align__(16) uint16_t sh_q[WAVES][STEP ? MAX_G * HEAD_DIM : 8];   /* the step's query rows */
    __shared__ StepArgs sh_step;   /* the step's arguments, read per item (kept in registers they would spill) */
    int *cf = sh_cum, *cp = sh_cum + a.B + 1;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    if (wave == 0) {  /* exclusive prefixes over sequences of Hkv * (full, partial) chunks, 64 sequences per step */
        int run_f = 0, run_p = 0;
        for (int b0 = 0; b0 < a.B; b0 += WAVE) {
            const int b = b0 + lane;
            int vf = 0, vp = 0;
            if (b < a.B) {
                int begin = 0;
                const UnitSplit u = unit_split(a, a.seq_lens[b], begin);
                vf = a.Hkv * u.nfull;
                vp = a.Hkv * u.npart;
            }
#pragma unroll
            for (int o = 1; o < WAVE; o <<= 1) {
                const int tf = __shfl_up(vf, o, WAVE), tp = __shfl_up(vp, o, WAVE);
                if (lane >= o) {
                    vf += tf;
                    vp += tp;
                }
            }
            if (b < a.B) {
                cf[b + 1] = run_f + vf;
                cp[b + 1] = run_p + vp;
            }
            run_f += __shfl(vf, WAVE - 1, WAVE);
            run_p += __shfl(vp, WAVE - 1, WAVE);
        }
        if (lane == 0) cf[0] = cp[0] = 0;
        if (STEP && lane == 0) sh_step = a.step;
    }
    __syncthreads();
    decode_fill_rows(a, cf, cp, blockIdx.x * WAVES + wave, gridDim.x * WAVES, lane);
    const int NF = cf[a.B], N = NF + cp[a.B];
    const long long G = gridDim.x;
    for (long long kk = blockIdx.x + G * wave; kk < N; kk += 4 * G) {
        const int k = (int)kk;
        int b, kvh, j, begin = 0;
        UnitSplit us;
        if (k < NF) {   /* full chunk: the (k - cf[b])-th of sequence b, in (KV head, chunk) order */
            b = find_sequence(cf, a.B, k);
            us = unit_split(a, a.seq_lens[b], begin);
            const int local = k - cf[b];
            kvh = local / us.nfull;
            /* The unit's full chunks in a rotated order. Consecutive items run on successive XCDs (work-group L on XCD
             * L % 8) and successive work-groups, so unrotated, chunk j of every unit would share an XCD, and the last
             * chunks (the token's append, most merges) would run on one XCD and a few work-groups. Rotating by the
             * unit's index u spreads them over the XCDs; adding the round (first item / work-groups) spreads units
             * whose items fall on the same work-groups in successive rounds. */
            const int first_item = cf[b] + kvh * us.nfull;
            const int rot = (b * a.Hkv + kvh + (int)(first_item / G)) % us.nfull;
            j = (local - kvh * us.nfull + rot) % us.nfull + us.p0;
        } else {        /* partial chunk: the first and / or the last of a unit */
            const int k2 = k - NF;
            b = find_sequence(cp, a.B, k2);
            us = unit_split(a, a.seq_lens[b], begin);
            const int local = k2 - cp[b];
            kvh = local / us.npart;
            const int jp = local - kvh * us.npart;
            /* a unit of short chunks lists them all; any other unit its partial first and / or last chunk */
            j = us.s == SHORT_SPLIT ? jp : (us.p0 && jp == 0) ? 0 : us.nch - 1;
        }
        const long long slot = (long long)cf[b] + cp[b] + (long long)kvh * us.nch + j;
        const int L = a.seq_lens[b];
        int first, last;
        chunk_pages(us, j, first, last);
        const long long row0 = (long long)b * a.Hq + kvh * a.G;
        const int32_t *bt = a.block_table + (long long)b * a.max_pages;
        TabRegs tab;
        tab.v = first + lane < last ? bt[first + lane] : 0;
        tab.v2 = first + WAVE + lane < last ? bt[first + WAVE + lane] : 0;

        WaveState<1> st;
        state_init(st);
        st.sl2 = a.scale_log2;
        const bool own = j == us.nch - 1, late = STEP && own && (L - 1) / PAGE - first < 4;
        /* the query's loads first, then the first page pair (see StepLoads) */
        StepLoads sl;
        StepArgs sa;
        uint4 qraw[1][4];
        if (STEP) {
            asm volatile("" ::: "memory");   /* sh_step is read here, per item, not hoisted out of the loop */
            sa = sh_step;
            sl = step_fetch(a, sa, b, kvh, L - 1, own, lane);
        } else {
            const Rsrc rq = page_rsrc(a.q + row0 * HEAD_DIM, a.G * HEAD_DIM * 2);   /* columns c >= G read zeros */
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rq, (c * HEAD_DIM + g * 32 + cc * 8) * 2, 0, 0);
                qraw[0][cc] = uint4{v[0], v[1], v[2], v[3]};
            }
        }
        PairAddr c0 = pair_addr_tab(a, tab, first, kvh, first, last, st.bad);
        PairRegs k0, v0;
        load_pair_b(a.k_pages, a.kv_scale, c0, !late, lane, k0);
        load_pair_b(a.v_pages, a.kv_scale + PAGE, c0, !late, lane, v0);
        QOp qb[1];
        if (STEP) {
            const int p = L - 1;
            step_rows<VE>(a, sa, sl, b, kvh, p, own, own ? tab_entry(tab, p / PAGE - first) : 0, late, sh_q[wave], lane);
            uint4 raw[1][4];
#pragma unroll
            for (int cc = 0; cc < 4; cc++)
                raw[0][cc] = c < a.G ? *reinterpret_cast<const uint4 *>(&sh_q[wave][c * HEAD_DIM + g * 32 + cc * 8])
                                     : uint4{0u, 0u, 0u, 0u};
            q8_from_raw<1>(raw, qb);
            if (late) {
                load_pair_b(a.k_pages, a.kv_scale, c0, true, lane, k0);
                load_pair_b(a.v_pages, a.kv_scale + PAGE, c0, true, lane, v0);
            }
        } else {
            q8_from_raw<1>(qraw, qb);
        }
        KeyBounds<1> kb;
        kb.lo[0] = kb.full_lo = begin;
        kb.hi[0] = kb.full_hi = kb.written_hi = L - 1;
        attend_pages_tab<1>(a, tab, first, kvh, first, last, kb, qb, st, lane, c0, k0, v0, STEP && own);
        st.l[0] = pair_sum32(pair_sum16(st.l[0]));
        if (us.nch == 1) {
            if (c < a.G) {
                uint16_t *dst = a.out + (row0 + c) * HEAD_DIM;
                const float inv = 1.0f / st.l[0];
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    float v[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) v[i] = st.bad ? NAN : st.o[0][t][i] * inv;
                    store_bf16x4(dst + 16 * t + 4 * g, v);
                }
            }
            continue;
        }
        {
            Rsrc ro, rm;
            part_rsrc(a, slot, ro, rm);
            if (c < a.G) {
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const f32x4 o = st.o[0][t];
                    part_store(ro, (c * HEAD_DIM + 16 * t + 4 * g) * 4, float4{st.bad ? NAN : o[0], o[1], o[2], o[3]});
                }
                if (g == 0)
                    __builtin_amdgcn_raw_buffer_store_b64(
                        u32x2{__float_as_uint(st.bad ? NAN : st.m[0]), __float_as_uint(st.l[0])}, rm, c * 8, 0, SC1);
            }
        }
        const int u = b * a.Hkv + kvh;
        __builtin_amdgcn_s_waitcnt(VMCNT0);   /* the partial has reached the coherent level before it is counted */
        int prior = 0;
        if (lane == 0) prior = __hip_atomic_fetch_add(a.arrived + u, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prior = __builtin_amdgcn_readfirstlane(prior);
        if (prior == us.nch - 1) {   /* every other chunk of the unit has published its partial */
            merge_unit(a, slot - j, us.nch, row0, lane);
            if (lane == 0) __hip_atomic_store(a.arrived + u, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

/* Grid (ceil(T / (4 NT tpt)), Hkv, B), 4 waves. A wave owns NT tiles of 16 columns, each tile tpt = 16 / G
 * consecutive tokens x G heads (column c = token c / G, head c % G), and streams every page its rows can see;
 * each K/V operand it converts feeds its NT tiles. */
/* A prefill workgroup's (row tile, KV head, sequence) from its place in the launch order, the longest key ranges
 * first: work-groups start in linear order (x, then y, then z), and a row tile's keys grow with its index under the
 * causal bound, so the last tiles of every (head, sequence) go first and the shortest last, where they fill the CUs
 * the long ones leave (the grid keeps x = row tiles, y = KV heads, z = sequences). */
struct PrefillBlock {
    int tile, kvh, b;
};

__device__ __forceinline__ PrefillBlock prefill_block() {
    const int yz = (int)(gridDim.y * gridDim.z);
    const int L = (int)blockIdx.x + (int)gridDim.x * ((int)blockIdx.y + (int)gridDim.y * (int)blockIdx.z);
    const int r = L % yz;
    return PrefillBlock{(int)gridDim.x - 1 - L / yz, r % (int)gridDim.y, r / (int)gridDim.y};
}

template <int NT>
__global__ void __launch_bounds__(256, 2) prefill_kernel(AttnArgs a) {
    const PrefillBlock pb = prefill_block();
    const int kvh = pb.kvh, b = pb.b;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int tpt = 16 / a.G, tpw = tpt * NT;
    const int t0 = (pb.tile * WAVES + wave) * tpw;
    const int T = a.run_row0 ? a.run_count[b] : a.T;          /* this sequence's (run's) rows */
    if (t0 >= T) return;
    const long long row0 = a.run_row0 ? a.run_row0[b] : (long long)b * a.T;
    const int trow = a.run_row0 ? a.run_slot[b] : b;          /* its block-table row */
    const int start = a.start_pos[b];
    const int hg = c % a.G;
    bool live[NT];
    long long qrow[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int tok = t0 + t * tpt + c / a.G;
        live[t] = c < tpt * a.G && tok < T;
        qrow[t] = (row0 + tok) * a.Hq + kvh * a.G + hg;
    }
    if (start < 0 || (long long)start + T > (long long)a.max_pages * PAGE) {  /* past the block table: NaN */
#pragma unroll
        for (int t = 0; t < NT; t++)
            if (live[t])
                for (int d = g * 32; d < g * 32 + 32; d++) a.out[qrow[t] * HEAD_DIM + d] = (uint16_t)0x7FC0;
        return;
    }
    const int t_last = min(t0 + tpw, T) - 1;     /* the wave's last token */
    KeyBounds<NT> kb;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int pos = start + t0 + t * tpt + c / a.G;
        kb.hi[t] = live[t] ? pos : -1;
        kb.lo[t] = live[t] ? (a.window >= 0 ? max(pos - a.window, 0) : 0) : 0;
    }
    kb.full_hi = start + t0;                                                   /* the wave's first row */
    kb.full_lo = a.window >= 0 ? max(start + t_last - a.window, 0) : 0;       /* its last row's window start */
    kb.written_hi = start + T - 1;
    const int w_lo = a.window >= 0 ? max(start + t0 - a.window, 0) : 0;
    /* page pairs start at even logical pages, so a key's pair (and its place in a column's sums) depends on the key
     * alone, not on which rows share the wave */
    const int pg0 = (w_lo / PAGE) & ~1, pg1 = (start + t_last) / PAGE + 1;

    QOp qb[NT];
    const uint16_t *qrows[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) qrows[t] = live[t] ? a.q + qrow[t] * HEAD_DIM : nullptr;
    WaveState<NT> st;
    state_init(st);
    load_q8<NT>(qrows, g, qb);
    st.sl2 = a.scale_log2;
    attend_pages<NT, true>(a, a.block_table + (long long)trow * a.max_pages, kvh, pg0, 2, pg1, kb, qb, st, lane);
#pragma unroll
    for (int t = 0; t < NT; t++) {
        st.l[t] = pair_sum32(pair_sum16(st.l[t]));
        if (!live[t]) continue;
        uint16_t *dst = a.out + qrow[t] * HEAD_DIM;
        const float inv = 1.0f / st.l[t];
#pragma unroll
        for (int d = 0; d < 8; d++) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = st.bad ? NAN : st.o[t][d][i] * inv;
            store_bf16x4(dst + 16 * d + 4 * g, v);
        }
    }
}

/*
 * Chunked prefill with the workgroup's pages staged in LDS. The four waves of a workgroup serve the same (sequence, KV
 * head) and walk the same page pairs, so each pair is fetched once per workgroup, straight into LDS by
 * global_load_lds (K 4 KiB, V 4 KiB, the pair's scales 256 B; each wave fetches a quarter), PF_AHEAD pairs ahead of
 * the one being computed, with no registers held for the prefetch. The stage buffers are distinct LDS objects used in
 * a fixed rotation (the loop is unrolled by PF_BUFS), so the compiler's wait before reading a stage covers that
 * stage's fetches only; before the workgroup barrier each wave waits for its own fetches of the stage (the
 * PF_FETCHES (PF_AHEAD - 1) issued after them may stay in flight) and for its LDS reads of the stage it is about to
 * refill. The workgroup's block-table segment is read once into LDS. Each wave then runs the register kernel's pair
 * step (scores, online softmax, PV) on operands read from LDS. Pairs are aligned to the workgroup's first page; a
 * wave skips the pairs outside its own key range.
 */
constexpr int PF_AHEAD = 3;                    /* pairs in flight */
constexpr int PF_BUFS = PF_AHEAD + 1;          /* stage buffers */
constexpr int PF_FETCHES = 3;                  /* fetch instructions per wave per stage: K, V, scales */
constexpr int PF_SCALES = 2 * 2 * PAGE * 4;   /* a pair's scales: [page][K 16, V 16] fp32 */
constexpr int PF_STAGE = 2 * 2 * PAGE_BYTES;  /* K, then V, of two pages */
constexpr int PF_TAB = 4096;                   /* block-table entries a workgroup can stage (65,536 keys) */

struct PfStage {
    unsigned char b[PF_STAGE];
};
struct PfScales {
    float f[WAVES][PF_SCALES / 4];   /* each wave's copy of the pair's scales */
};
typedef __attribute__((address_space(3))) void LdsVoid;

/* s_waitcnt: this wave's fetches of the oldest stage landed (the later stages' may stay in flight) and its LDS
 * reads completed. Encoding: vmcnt [3:0] and [15:14], expcnt [6:4] (7: no wait), lgkmcnt [11:8]. */
__device__ __forceinline__ void pf_wait_stage() {
    constexpr int n = PF_FETCHES * (PF_AHEAD - 1);
    __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0x0 << 8));
}

/* A workgroup barrier without a memory fence (a fence would drain every fetch in flight); the empty asm statements
 * keep the compiler from moving memory accesses across it. */
__device__ __forceinline__ void pf_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

/* The pages of stage s (logical pages pg0 + 2 s, + 1; past the page range, the last pair again), each outside the
 * page pool replaced by page 0 (such a pair is only read: the waves that use it report NaN). */
struct PfPages {
    int pa, pb;
};

__device__ __forceinline__ PfPages pf_pages(const AttnArgs &a, const int *tab, int npages, int s) {
    const int ps = min(s, (npages - 1) / 2);
    const int la = 2 * ps, lb = la + 1 < npages ? la + 1 : la;
    PfPages p;
    p.pa = tab[la];
    p.pb = tab[lb];
    p.pa = (unsigned)p.pa < (unsigned)a.num_pages ? p.pa : 0;
    p.pb = (unsigned)p.pb < (unsigned)a.num_pages ? p.pb : 0;
    return p;
}

/* The fetches of one stage (pages pg) into buffer st: wave w fetches K bytes [1024 w, 1024 w + 1024) of the pair
 * (pages a, a, b, b), the same of V, and all 256 scale bytes into its own slot (4 bytes a lane: no lane is masked
 * off, so the compiler can count the fetches); every wave always issues PF_FETCHES. */
__device__ __forceinline__ void pf_fetch(const AttnArgs &a, PfPages pg, int kvh, PfStage &st, PfScales &sc, int wave,
                                         int lane) {
    const long long ph = (long long)(wave < 2 ? pg.pa : pg.pb) * a.Hkv + kvh;
    const int half = (wave & 1) * 1024;
    __builtin_amdgcn_global_load_lds((const void *)(a.k_pages + ph * PAGE_BYTES + half + lane * 16),
                                     (LdsVoid *)(st.b + wave * 1024), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void *)(a.v_pages + ph * PAGE_BYTES + half + lane * 16),
                                     (LdsVoid *)(st.b + 2 * 2048 + wave * 1024), 16, 0, 0);
    const long long sh = (long long)(lane < 32 ? pg.pa : pg.pb) * a.Hkv + kvh;
    __builtin_amdgcn_global_load_lds((const void *)(a.kv_scale + sh * 2 * PAGE + (lane & 31)), (LdsVoid *)sc.f[wave], 4,
                                     0, 0);
}

/* Whether a block-table entry of the pairs this wave computes (pairs la even with pg0 + la + 1 >= wpg0 and
 * pg0 + la < wpg1) lies outside the page pool: checked once, from the staged table. */
__device__ __forceinline__ bool pf_bad(const AttnArgs &a, const int *tab, int pg0, int npages, int wpg0, int wpg1,
                                       int lane) {
    const int la0 = (max(wpg0 - pg0 - 1, 0) + 1) & ~1;                  /* the first even la computed */
    const int end = min(npages, ((min(npages, wpg1 - pg0) + 1) & ~1));  /* one past its pairs' last page */
    bool bad = false;
    for (int i = la0 + lane; i < end; i += WAVE) bad = bad || (unsigned)tab[i] >= (unsigned)a.num_pages;
    return __any(bad);
}

/* One wave's step over stage s (buffer st) when the pair meets its key range. */
template <int NT>
__device__ __forceinline__ void pf_compute(const AttnArgs &a, int pg0, int npages, int s, const PfStage &st,
                                           const PfScales &scs, int wpg0, int wpg1, const KeyBounds<NT> &kb,
                                           const QOp (&qb)[NT], WaveState<NT> &st_w, int lane) {
    const int la = 2 * s;
    if (la >= npages || pg0 + la + 1 < wpg0 || pg0 + la >= wpg1) return;
    const int g = lane >> 4;
    PairAddr cur;
    cur.lpa = pg0 + la;
    cur.has_b = la + 1 < npages;
    cur.ha = cur.hb = 0;
    const uint4 *k4 = reinterpret_cast<const uint4 *>(st.b);
    const uint4 k0 = k4[lane], k1 = k4[64 + lane], k2 = k4[128 + lane], k3 = k4[192 + lane];
    const float *sc = scs.f[threadIdx.x >> 6];
    const float4 ksa = *reinterpret_cast<const float4 *>(sc + g * 4);
    const float4 ksb = *reinterpret_cast<const float4 *>(sc + 2 * PAGE + g * 4);
    const uint4 *v4 = reinterpret_cast<const uint4 *>(st.b + 2 * 2048);
    PairRegs vr;
    vr.a0 = v4[lane]; vr.a1 = v4[64 + lane]; vr.b0 = v4[128 + lane]; vr.b1 = v4[192 + lane];
    vr.sa = *reinterpret_cast<const float4 *>(sc + PAGE + g * 4);
    vr.sb = *reinterpret_cast<const float4 *>(sc + 3 * PAGE + g * 4);
    pair_step_k<NT>(a, cur, k0, k1, k2, k3, qb, ksa, ksb, vr, kb, st_w, lane);
}

/* Grid and columns as prefill_kernel. */
template <int NT>
__global__ void __launch_bounds__(256, 2) prefill_lds_kernel(AttnArgs a) {
    __shared__ __align__(16) PfStage pb0, pb1, pb2, pb3;
    __shared__ __align__(16) PfScales ps0, ps1, ps2, ps3;
    __shared__ int tab[PF_TAB];
    static_assert(PF_BUFS == 4, "the loop below rotates four stage buffers");
    const PrefillBlock pb = prefill_block();
    const int kvh = pb.kvh, b = pb.b;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int tpt = 16 / a.G, tpw = tpt * NT;
    const int T = a.run_row0 ? a.run_count[b] : a.T;          /* this sequence's (run's) rows */
    const int wg_t0 = pb.tile * WAVES * tpw;
    if (wg_t0 >= T) return;                                    /* the whole workgroup */
    const int t0 = wg_t0 + wave * tpw;
    const bool on = t0 < T;                                    /* this wave has rows */
    const long long row0 = a.run_row0 ? a.run_row0[b] : (long long)b * a.T;
    const int trow = a.run_row0 ? a.run_slot[b] : b;
    const int start = a.start_pos[b];
    const int hg = c % a.G;
    bool live[NT];
    long long qrow[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int tok = t0 + t * tpt + c / a.G;
        live[t] = on && c < tpt * a.G && tok < T;
        qrow[t] = (row0 + tok) * a.Hq + kvh * a.G + hg;
    }
    if (start < 0 || (long long)start + T > (long long)a.max_pages * PAGE) {  /* past the block table: NaN */
#pragma unroll
        for (int t = 0; t < NT; t++)
            if (live[t])
                for (int d = g * 32; d < g * 32 + 32; d++) a.out[qrow[t] * HEAD_DIM + d] = (uint16_t)0x7FC0;
        return;
    }
    /* the workgroup's pages [pg0, pg0 + npages) and this wave's [wpg0, wpg1) */
    const int wg_last = min(wg_t0 + WAVES * tpw, T) - 1;
    /* pairs start at even logical pages: a key's pair does not depend on which rows share the workgroup */
    const int pg0 = ((a.window >= 0 ? max(start + wg_t0 - a.window, 0) : 0) / PAGE) & ~1;
    const int npages = (start + wg_last) / PAGE + 1 - pg0;
    const int t_last = on ? min(t0 + tpw, T) - 1 : t0;
    const int wpg0 = (a.window >= 0 ? max(start + t0 - a.window, 0) : 0) / PAGE;
    const int wpg1 = on ? (start + t_last) / PAGE + 1 : 0;
    KeyBounds<NT> kb;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int pos = start + t0 + t * tpt + c / a.G;
        kb.hi[t] = live[t] ? pos : -1;
        kb.lo[t] = live[t] ? (a.window >= 0 ? max(pos - a.window, 0) : 0) : 0;
    }
    kb.full_hi = start + t0;
    kb.full_lo = a.window >= 0 ? max(start + t_last - a.window, 0) : 0;
    kb.written_hi = start + T - 1;

    const int32_t *bt = a.block_table + (long long)trow * a.max_pages + pg0;
    for (int i = threadIdx.x; i < npages; i += 256) tab[i] = bt[i];
    QOp qb[NT];
    const uint16_t *qrows[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) qrows[t] = live[t] ? a.q + qrow[t] * HEAD_DIM : nullptr;
    WaveState<NT> st;
    state_init(st);
    load_q8<NT>(qrows, g, qb);
    st.sl2 = a.scale_log2;
    __syncthreads();   /* the table is in LDS (no fetch is in flight yet, so this fence drains nothing) */

    const int stages = (npages + 1) / 2;
    st.bad = pf_bad(a, tab, pg0, npages, wpg0, wpg1, lane);
    pf_fetch(a, pf_pages(a, tab, npages, 0), kvh, pb0, ps0, wave, lane);
    pf_fetch(a, pf_pages(a, tab, npages, 1), kvh, pb1, ps1, wave, lane);
    pf_fetch(a, pf_pages(a, tab, npages, 2), kvh, pb2, ps2, wave, lane);
    PfPages next = pf_pages(a, tab, npages, 3);   /* the pages of the next fetch, read a step ahead */
    /* step s: wait for stage s, barrier, refill the buffer read at step s - 1 with stage s + 3, compute stage s */
    for (int s = 0; s < stages; s += PF_BUFS) {
        pf_wait_stage(); pf_barrier();
        pf_fetch(a, next, kvh, pb3, ps3, wave, lane);
        next = pf_pages(a, tab, npages, s + 4);
        pf_compute<NT>(a, pg0, npages, s, pb0, ps0, wpg0, wpg1, kb, qb, st, lane);
        pf_wait_stage(); pf_barrier();
        pf_fetch(a, next, kvh, pb0, ps0, wave, lane);
        next = pf_pages(a, tab, npages, s + 5);
        pf_compute<NT>(a, pg0, npages, s + 1, pb1, ps1, wpg0, wpg1, kb, qb, st, lane);
        pf_wait_stage(); pf_barrier();
        pf_fetch(a, next, kvh, pb1, ps1, wave, lane);
        next = pf_pages(a, tab, npages, s + 6);
        pf_compute<NT>(a, pg0, npages, s + 2, pb2, ps2, wpg0, wpg1, kb, qb, st, lane);
        pf_wait_stage(); pf_barrier();
        pf_fetch(a, next, kvh, pb2, ps2, wave, lane);
        next = pf_pages(a, tab, npages, s + 7);
        pf_compute<NT>(a, pg0, npages, s + 3, pb3, ps3, wpg0, wpg1, kb, qb, st, lane);
    }
    __builtin_amdgcn_s_waitcnt(0);   /* no fetch may land in LDS after the workgroup ends */
    pf_barrier();
#pragma unroll
    for (int t = 0; t < NT; t++) {
        st.l[t] = pair_sum32(pair_sum16(st.l[t]));
        if (!live[t]) continue;
        uint16_t *dst = a.out + qrow[t] * HEAD_DIM;
        const float inv = 1.0f / st.l[t];
#pragma unroll
        for (int d = 0; d < 8; d++) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = st.bad ? NAN : st.o[t][d][i] * inv;
            store_bf16x4(dst + 16 * d + 4 * g, v);
        }
    }
}

constexpr int PREFILL_TILES = 2;  /* 16-column tiles per prefill wave */

/* Chunked prefill of `rows` rows of `seqs` sequences (or runs): the LDS-staged kernel when a sequence's block-table
 * row fits its LDS segment, else the register kernel. */
static void launch_prefill(const AttnArgs &a, int rows, int seqs, hipStream_t stream) {
    const int tokens_per_block = WAVES * PREFILL_TILES * (16 / a.G);
    const dim3 grid((rows + tokens_per_block - 1) / tokens_per_block, a.Hkv, seqs), block(256);
    if (a.max_pages <= PF_TAB)
        hipLaunchKernelGGL(prefill_lds_kernel<PREFILL_TILES>, grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL(prefill_kernel<PREFILL_TILES>, grid, block, 0, stream, a);
}

/* Prefill over runs for the decoder runtime: run b = rows run_row0[b] .. + run_count[b] of q/out ([rows][Hq][128])
 * at positions start_pos[b] + t of block-table row run_slot[b]; max_count bounds run_count. Arguments are checked
 * by the caller. */
int prefill_runs(const uint16_t *q, const uint8_t *k_pages, const uint8_t *v_pages, const float *kv_scale,
                 const int32_t *block_table, int max_pages, int num_pages, const int32_t *start_pos,
                 const int32_t *run_row0, const int32_t *run_count, const int32_t *run_slot, int runs, int max_count,
                 int Hq, int Hkv, int window, float sm_scale, uint16_t *out, hipStream_t stream) {
    AttnArgs a = {};
    a.q = q;
    a.k_pages = k_pages; a.v_pages = v_pages; a.kv_scale = kv_scale;
    a.block_table = block_table; a.max_pages = max_pages; a.num_pages = num_pages;
    a.start_pos = start_pos;
    a.run_row0 = run_row0; a.run_count = run_count; a.run_slot = run_slot;
    a.B = runs; a.T = max_count; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv; a.window = window;
    a.scale_log2 = sm_scale * LOG2E;
    a.out = out;
    launch_prefill(a, max_count, runs, stream);
    return (int)hipGetLastError();
}

/* Decode workers (waves, launched as work-groups of 4): by default every wave slot the device holds at the kernel's
 * occupancy, at most 4 per item the launch can hold; workers > 0 asks for that many instead. */
constexpr int MAX_WORKERS = 1 << 20;

static long long max_unit_pages(int max_seq_len, int window) {
    long long n = (max_seq_len + PAGE - 1) / PAGE;
    if (window >= 0) n = min(n, (long long)(window / PAGE + 2));
    return n;
}

/* Items a launch can hold: a unit of n pages touches at most ceil(n / SPLIT_PAGES) + 1 chunks, or, cut into short
 * chunks (n <= SHORT_UNIT), ceil(n / SHORT_SPLIT) + 1. */
static long long item_bound(int B, int Hkv, int max_seq_len, int window) {
    const long long n = max_unit_pages(max_seq_len, window), ns = min(n, (long long)SHORT_UNIT);
    return (long long)B * Hkv * max((n + SPLIT_PAGES - 1) / SPLIT_PAGES + 1, (ns + SHORT_SPLIT - 1) / SHORT_SPLIT + 1);
}

static int device_wave_slots() {
    static int slots[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 2048;
    if (!slots[dev]) {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_kernel<true, true>, 256,
                                                         2 * (MAX_DECODE_BATCH + 1) * sizeof(int)) != hipSuccess)
            return 2048;
        slots[dev] = max(1, cus * per_cu * WAVES);
    }
    return slots[dev];
}

/* Workspace layout. Partial O [items][G][128] fp32 and partial (max, sum) [items][G][2] fp32 from the start (items =
 * item_bound(...)); the arrival counts, int32 per (sequence, KV head), in the last 1/256 of the workspace (from
 * count_region(bytes)). Where the counts sit depends on the workspace's size alone and no call writes partials there,
 * so a workspace zero-filled once and passed with the same size to every call keeps zero counts between calls (each
 * launch returns the counts it used to zero) whatever the shapes of the calls. Partials are written before they are
 * read in the same launch. */
static size_t partial_bytes(int Hq, int Hkv, long long items) {
    return (size_t)items * (Hq / Hkv) * (HEAD_DIM + 2) * sizeof(float);
}

static size_t count_region(size_t bytes) { return (bytes - ((bytes >> 8) & ~(size_t)3)) & ~(size_t)3; }

static bool workspace_fits(size_t bytes, int B, int Hq, int Hkv, long long items) {
    return partial_bytes(Hq, Hkv, items) <= count_region(bytes) &&
           (size_t)B * Hkv * sizeof(int) <= bytes - count_region(bytes);
}

/* The smallest multiple of 256 bytes that fits: 256 k with k >= P / 255 (partials below the count region) and
 * k >= 4 B Hkv (the counts), k a multiple of 4. */
static size_t workspace_bytes_for(int B, int Hq, int Hkv, long long items) {
    const size_t P = partial_bytes(Hq, Hkv, items);
    size_t k = max((P + 254) / 255, (size_t)B * Hkv * sizeof(int));
    k = (k + 3) & ~(size_t)3;
    return 256 * k;
}

static bool decode_shape_ok(int B, int Hq, int Hkv, int max_seq_len, int window) {
    return B > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= 16 && max_seq_len > 0 && B <= MAX_DECODE_BATCH &&
           item_bound(B, Hkv, max_seq_len, window) < (1LL << 31);
}

/* The launch itself (arguments checked by the caller); the workspace holds workspace_bytes_for(item_bound). step:
 * NULL for attention alone, else the fused step's append inputs (q is then unused). */
static int launch_decode(const void *q, const void *k_pages, const void *v_pages, const float *kv_scale,
                         const int32_t *block_table, int max_pages, int num_pages, const int32_t *seq_lens,
                         int max_seq_len, int B, int Hq, int Hkv, int window, float sm_scale, int workers, void *out,
                         void *workspace, size_t workspace_bytes, const StepArgs *step, hipStream_t stream) {
    AttnArgs a = {};
    a.q = (const uint16_t *)q;
    a.k_pages = (const uint8_t *)k_pages; a.v_pages = (const uint8_t *)v_pages;
    a.kv_scale = kv_scale;
    a.block_table = block_table; a.max_pages = max_pages; a.num_pages = num_pages;
    a.seq_lens = seq_lens;
    a.B = B; a.T = 1; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv; a.window = window;
    a.max_len = max_seq_len;
    a.scale_log2 = sm_scale * LOG2E;
    const long long items = item_bound(B, Hkv, max_seq_len, window);
    a.workers = (int)min((long long)(workers > 0 ? min(workers, MAX_WORKERS) : device_wave_slots()), 4 * items);
    a.out = (uint16_t *)out;
    a.part_o = (float *)workspace;
    a.part_ml = a.part_o + (size_t)items * a.G * HEAD_DIM;
    a.arrived = (int *)((char *)workspace + count_region(workspace_bytes));
    const int grid = (a.workers + WAVES - 1) / WAVES;
    const size_t lds = 2 * (B + 1) * sizeof(int);
    if (step) {
        a.step = *step;
        if (step->ve) hipLaunchKernelGGL((decode_kernel<true, true>), dim3(grid), dim3(256), lds, stream, a);
        else hipLaunchKernelGGL((decode_kernel<true, false>), dim3(grid), dim3(256), lds, stream, a);
    } else {
        hipLaunchKernelGGL(decode_kernel<false>, dim3(grid), dim3(256), lds, stream, a);
    }
    return (int)hipGetLastError();
}

int decode_step(const StepArgs &step, const void *k_pages, const void *v_pages, const float *kv_scale,
                const int32_t *block_table, int max_pages, int num_pages, const int32_t *seq_lens, int max_seq_len,
                int B, int Hq, int Hkv, int window, float sm_scale, void *out, void *workspace, size_t workspace_bytes,
                hipStream_t stream) {
    if (!workspace_fits(workspace_bytes, B, Hq, Hkv, item_bound(B, Hkv, max_seq_len, window))) return NC_ERR_WORKSPACE;
    return launch_decode(nullptr, k_pages, v_pages, kv_scale, block_table, max_pages, num_pages, seq_lens, max_seq_len,
                         B, Hq, Hkv, window, sm_scale, 0, out, workspace, workspace_bytes, &step, stream);
}

/* The allocation-free entry point's workspace: one static array per GPU, NC_DECODE_SCRATCH_BYTES long, held until the
 * process ends. In host code `scratch` names a host-side stand-in, not device memory: its device address on the current
 * GPU is looked up once (hipGetSymbolAddress with that GPU current) and only that address is ever passed to a kernel.
 * A device array without an initializer starts zero-filled, which is what the arrival counts need; every launch
 * leaves them zero. Calls that overlap on one GPU share the array and race. */
static __device__ __align__(256) unsigned char scratch[NC_DECODE_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;

/* The current GPU's address of `scratch` (NULL with *err set when the lookup fails). */
static void *scratch_on_current_device(int *err) {
    static std::mutex lock;
    static void *ptrs[MAX_DEVICES] = {nullptr};
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        *err = e != hipSuccess ? (int)e : (int)hipErrorInvalidDevice;
        return nullptr;
    }
    std::lock_guard<std::mutex> guard(lock);
    if (!ptrs[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            *err = e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
            return nullptr;
        }
        ptrs[dev] = p;
    }
    return ptrs[dev];
}

}  // namespace nc

using namespace nc;

extern "C" size_t nc_decode_workspace_bytes(int B, int Hq, int Hkv, int max_seq_len, int window) {
    if (!decode_shape_ok(B, Hq, Hkv, max_seq_len, window)) return 0;
    return workspace_bytes_for(B, Hq, Hkv, item_bound(B, Hkv, max_seq_len, window));
}

extern "C" int nc_decode_attn_fp8(const void *q, const void *k_pages, const void *v_pages, const float *kv_scale,
                                  const int32_t *block_table, int max_pages, int num_pages,
                                  const int32_t *seq_lens, int max_seq_len, int B, int Hq, int Hkv, int window,
                                  float sm_scale, int workers, void *out, void *workspace,
                                  size_t workspace_bytes, void *stream) {
    if (!q || !k_pages || !v_pages || !kv_scale || !block_table || !seq_lens || !out || !workspace)
        return NC_ERR_NULL;
    if (!decode_shape_ok(B, Hq, Hkv, max_seq_len, window) || max_pages <= 0 || num_pages <= 0 ||
        (long long)max_seq_len > (long long)max_pages * PAGE || workers < 0)
        return NC_ERR_SHAPE;
    if (!workspace_fits(workspace_bytes, B, Hq, Hkv, item_bound(B, Hkv, max_seq_len, window)))
        return NC_ERR_WORKSPACE;
    return launch_decode(q, k_pages, v_pages, kv_scale, block_table, max_pages, num_pages, seq_lens, max_seq_len, B,
                         Hq, Hkv, window, sm_scale, workers, out, workspace, workspace_bytes, nullptr,
                         (hipStream_t)stream);
}

extern "C" int nc_decode_step_fp8(const void *qkv, long long token_stride, int B, int Hq, int Hkv,
                                  const int32_t *seq_lens, const float *q_gain, const float *k_gain, const float *cos,
                                  const float *sin, int rope_len, void *q_out, const void *ve_h, const void *ve,
                                  const float *ve_gate, const int32_t *ve_tokens, int C, int ve_rows,
                                  const int32_t *block_table,
                                  int max_pages, void *k_pages, void *v_pages, float *kv_scale, int num_pages,
                                  int max_seq_len, int window, float sm_scale, int workers, void *out, void *workspace,
                                  size_t workspace_bytes, void *stream) {
    if (!qkv || !seq_lens || !q_gain || !k_gain || !cos || !sin || !block_table || !k_pages || !v_pages || !kv_scale ||
        !out || !workspace || (ve && (!ve_h || !ve_gate || !ve_tokens)))
        return NC_ERR_NULL;
    if (!decode_shape_ok(B, Hq, Hkv, max_seq_len, window) || max_pages <= 0 || num_pages <= 0 ||
        (long long)max_seq_len > (long long)max_pages * PAGE || workers < 0 || rope_len < max_seq_len ||
        token_stride < (long long)(Hq + 2 * Hkv) * HEAD_DIM || (ve && (C < Hkv * HEAD_DIM || ve_rows <= 0)))
        return NC_ERR_SHAPE;
    if (!workspace_fits(workspace_bytes, B, Hq, Hkv, item_bound(B, Hkv, max_seq_len, window)))
        return NC_ERR_WORKSPACE;
    StepArgs st = {};
    st.qkv = (const uint16_t *)qkv;
    st.token_stride = token_stride;
    st.q_gain = q_gain; st.k_gain = k_gain; st.cos = cos; st.sin = sin;
    st.q_out = (uint16_t *)q_out;
    st.ve_h = (const uint16_t *)ve_h; st.ve = (const uint16_t *)ve; st.ve_gate = ve_gate; st.ve_tokens = ve_tokens;
    st.C = C;
    st.ve_rows = ve_rows;
    st.k_pages = (uint8_t *)k_pages; st.v_pages = (uint8_t *)v_pages; st.kv_scale = kv_scale;
    return launch_decode(nullptr, k_pages, v_pages, kv_scale, block_table, max_pages, num_pages, seq_lens, max_seq_len,
                         B, Hq, Hkv, window, sm_scale, workers, out, workspace, workspace_bytes, &st,
                         (hipStream_t)stream);
}

extern "C" int nc_prefill_attn_fp8(const void *q, const void *k_pages, const void *v_pages, const float *kv_scale,
                                   const int32_t *block_table, int max_pages, int num_pages,
                                   const int32_t *start_pos, int B, int T, int Hq, int Hkv, int window,
                                   float sm_scale, void *out, void *stream) {
    if (!q || !k_pages || !v_pages || !kv_scale || !block_table || !start_pos || !out) return NC_ERR_NULL;
    if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || Hq / Hkv > 16 || max_pages <= 0 || num_pages <= 0 ||
        B > 65535 || Hkv > 65535)
        return NC_ERR_SHAPE;
    AttnArgs a = {};
    a.q = (const uint16_t *)q;
    a.k_pages = (const uint8_t *)k_pages; a.v_pages = (const uint8_t *)v_pages;
    a.kv_scale = kv_scale;
    a.block_table = block_table; a.max_pages = max_pages; a.num_pages = num_pages;
    a.start_pos = start_pos;
    a.B = B; a.T = T; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv; a.window = window;
    a.scale_log2 = sm_scale * LOG2E;
    a.out = (uint16_t *)out;
    launch_prefill(a, T, B, (hipStream_t)stream);
    return (int)hipGetLastError();
}

extern "C" int nc_decode_attn_fp8_noalloc(const void *q, const void *k_pages, const void *v_pages,
                                          const float *kv_scale, const int32_t *block_table, int max_pages,
                                          int num_pages, const int32_t *seq_lens, int max_seq_len, int B, int Hq,
                                          int Hkv, int window, float sm_scale, int workers, void *out, void *stream) {
    if (!q || !k_pages || !v_pages || !kv_scale || !block_table || !seq_lens || !out) return NC_ERR_NULL;
    if (!decode_shape_ok(B, Hq, Hkv, max_seq_len, window) || max_pages <= 0 || num_pages <= 0 ||
        (long long)max_seq_len > (long long)max_pages * PAGE || workers < 0)
        return NC_ERR_SHAPE;
    if (!workspace_fits(NC_DECODE_SCRATCH_BYTES, B, Hq, Hkv, item_bound(B, Hkv, max_seq_len, window)))
        return NC_ERR_WORKSPACE;
    int err = 0;
    void *ws = scratch_on_current_device(&err);
    if (!ws) return err;
    return launch_decode(q, k_pages, v_pages, kv_scale, block_table, max_pages, num_pages, seq_lens, max_seq_len, B,
                         Hq, Hkv, window, sm_scale, workers, out, ws, NC_DECODE_SCRATCH_BYTES, nullptr,
                         (hipStream_t)stream);
}

/*
 * The read-only ceiling of the decode step's access pattern: a kernel that only reads 2 KiB pages (the size of one
 * (page, head) of K or V codes) in a given order and folds them into a checksum. Each wave takes pages w, w + waves,
 * ... two at a time, each page as two 16-byte loads a lane, non-temporal like the decode stream. It does no
 * arithmetic beyond the XOR that keeps the loads, so its rate is what the memory system gives for that order of
 * pages; the XOR of every sink word is the XOR of every dword read. Entry i of `order` (NULL: i) names the page read i-th; an entry outside
 * [0, src_pages) reads page 0.
 */
__global__ void __launch_bounds__(256) read_pages_kernel(const u32x4 *src, int src_pages, const int32_t *order, int n,
                                                         uint32_t *sink) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int waves = gridDim.x * WAVES, w = blockIdx.x * WAVES + (threadIdx.x >> 6);
    uint32_t acc = 0;
    for (int c0 = 2 * w; c0 < n; c0 += 2 * waves) {
        u32x4 v[2][2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int c = c0 + u;
            const bool live = c < n;
            int p = live ? (order ? order[c] : c) : 0;
            p = (unsigned)p < (unsigned)src_pages ? p : 0;
            const u32x4 *b = src + (size_t)p * (PAGE_BYTES / 16);
            v[u][0] = live ? __builtin_nontemporal_load(b + lane) : u32x4{0u, 0u, 0u, 0u};
            v[u][1] = live ? __builtin_nontemporal_load(b + WAVE + lane) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int h = 0; h < 2; h++) acc ^= v[u][h][0] ^ v[u][h][1] ^ v[u][h][2] ^ v[u][h][3];
    }
    sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

extern "C" int nc_debug_read_pages(const void *src, long long src_bytes, const int32_t *order, int n, int grid,
                                   uint32_t *sink, void *stream) {
    if (!src || !sink) return NC_ERR_NULL;
    if (src_bytes < PAGE_BYTES || src_bytes % PAGE_BYTES || src_bytes / PAGE_BYTES > INT_MAX || n < 0 || grid <= 0 ||
        grid > 65535)
        return NC_ERR_SHAPE;
    hipLaunchKernelGGL(read_pages_kernel, dim3(grid), dim3(WAVES * WAVE), 0, (hipStream_t)stream,
                       (const u32x4 *)src, (int)(src_bytes / PAGE_BYTES), order, n, sink);
    return (int)hipGetLastError();
}
