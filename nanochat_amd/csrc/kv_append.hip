/*
 * Cache append for the fp8 KV path on gfx950: the fused q/k RMS norm + gain + -theta rotation, the
 * per-(token, KV head) absmax e4m3fn quantizer and the paged store; plus the training-form q/k prologue
 * (the reference's qkp_forward) on the same row math.
 *
 * One wave per (token, head) row: lane l holds the rotation pair (dims l, l + 64), so the rotation is
 * lane-local and the row's sum of squares is one xor butterfly over the wave. The row math (nc_row.h) is
 * shared with the fused decode step, which appends the step's token inside the attention kernel.
 */
#include "nc_device.h"
#include "nc_row.h"
#include "nanochat_amd.h"
#include "nc_internal.h"

namespace nc {

struct AppendArgs {
    const uint16_t *k, *v;     /* plain append: [B][T][Hkv][128] at token_stride */
    const uint16_t *qkv;       /* fused append: [B][T][(Hq + 2 Hkv) 128] at token_stride */
    long long token_stride;
    int B, T, Hq, Hkv;
    const int32_t *start_pos, *num_new;
    const int32_t *row0;       /* NULL: sequence b's tokens are rows b T + t; else rows row0[b] + t */
    const float *q_gain, *k_gain, *cos, *sin;
    int rope_len;
    uint16_t *q_out;           /* [rows][Hq][128] */
    const int32_t *block_table;
    const int32_t *seq_slot;   /* NULL, or sequence b's block-table row (the decoder's prefill runs) */
    /* value embeddings (fused append, NULL ve: none): v += 2 sigmoid(ve_gate[head] . h) ve[tokens[token]] */
    const uint16_t *ve_h, *ve;  /* h: [rows][C] the layer's normed input; ve: [vocab][C] */
    const float *ve_gate;       /* [Hkv][C] */
    const int32_t *ve_tokens;   /* [rows] */
    int C;
    int max_pages;
    uint8_t *k_pages, *v_pages;
    float *kv_scale;          /* [num_pages][Hkv][2][16]: K scales, then V scales */
    int num_pages;
    int pages_per_seq;        /* grid x = B pages_per_seq: the most cache pages T positions can touch */
};

/* Cache pages a run of T positions can touch: (T - 1) / 16 + 1 when aligned, one more when not. */
static inline int append_pages_per_seq(int T) { return (T + PAGE - 2) / PAGE + 1; }

/* Grid: x = (sequence b, k-th cache page its new positions touch), y = head groups; block = 4 waves.
 * The new positions of b are [max(start, 0), start + min(T, num_new[b])), cut at rope_len when FUSED (the rest are
 * skipped, as are all of b's positions on a page past max_pages or whose table entry lies outside the pool). The
 * work-group takes those of them on page k: slots [s_lo, s_hi) of that page. Rows are computed four a wave, 16 lanes
 * a row (nc_row.h's 16-lane form, the same bits as the one-row-a-wave form of the fused decode step).
 * y < Hkv: KV head y. Wave w computes the k rows of slots 4 w .. 4 w + 3 (norm and rotation when FUSED, then the
 * quantizer), then their v rows (the value-embedding mix when given, then the quantizer), and writes the codes into an
 * LDS image of the page in the cache's layout. The work-group then stores the image with one 16-byte store a lane; a
 * K block holds one slot, a V block four (slots 4 g .. 4 g + 3), and a V block holding slots outside [s_lo, s_hi) is
 * stored byte by byte, so the page's other slots keep their bytes. The 16 scales of K and of V go out the same way.
 * y >= Hkv (FUSED only): q head 4 (y - Hkv) + w a wave, four of the page's slots at a time, normed and rotated into
 * q_out. */
template <bool FUSED>
__global__ void __launch_bounds__(256) append_kernel(AppendArgs a) {
    __shared__ __align__(16) uint8_t img[2][PAGE_BYTES];
    __shared__ float img_scale[2][PAGE];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int r = lane >> 4, i = lane & 15;   /* the lane's row of the wave's four, its place in the row */
    const int b = blockIdx.x / a.pages_per_seq, k = blockIdx.x % a.pages_per_seq;
    const int sp = a.start_pos[b];
    const int n = a.num_new ? min(a.num_new[b], a.T) : a.T;
    const long long lo = max(sp, 0);
    long long hi = (long long)sp + n;
    if (FUSED && hi > a.rope_len) hi = a.rope_len;
    if (lo >= hi) return;
    const long long lp = lo / PAGE + k, pg0 = lp * PAGE;
    const int s_lo = (int)(max(lo, pg0) - pg0), s_hi = (int)(min(hi, pg0 + PAGE) - pg0);
    if (s_lo >= s_hi) return;
    const long long tok_at = (a.row0 ? (long long)a.row0[b] : (long long)b * a.T) - sp;   /* + position = row */

    if (FUSED && (int)blockIdx.y >= a.Hkv) {
        const int h = 4 * ((int)blockIdx.y - a.Hkv) + wave;
        if (h >= a.Hq) return;
        float g[8];
#pragma unroll
        for (int j = 0; j < 8; j++) g[j] = a.q_gain[i + 16 * j];
        for (int s0 = s_lo; s0 < s_hi; s0 += 4) {
            const int slot = s0 + r;   /* past s_hi: computes the last slot again and stores nothing */
            const long long p = pg0 + min(slot, s_hi - 1), tok = tok_at + p;
            const uint16_t *row = a.qkv + tok * a.token_stride + h * HEAD_DIM;
            float x[8], c[4], sn[4], y[8];
#pragma unroll
            for (int j = 0; j < 8; j++) x[j] = bf16_to_f32(row[i + 16 * j]);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                c[j] = a.cos[p * HALF + i + 16 * j];
                sn[j] = a.sin[p * HALF + i + 16 * j];
            }
            norm_rope_quad(x, g, c, sn, y);
            if (slot < s_hi) {
                uint16_t *q = a.q_out + (tok * a.Hq + h) * HEAD_DIM;
#pragma unroll
                for (int j = 0; j < 8; j++) q[i + 16 * j] = f32_to_bf16(y[j]);
            }
        }
        return;
    }

    const int kvh = blockIdx.y;
    if (lp >= a.max_pages) return;
    const int trow = a.seq_slot ? a.seq_slot[b] : b;
    const int page = a.block_table[(long long)trow * a.max_pages + lp];
    if (page < 0 || page >= a.num_pages) return;
    const long long at = (long long)page * a.Hkv + kvh;

    const int slot = 4 * wave + r;
    const bool live = slot >= s_lo && slot < s_hi;   /* rows of other slots compute a new one and store nothing */
    const long long p = pg0 + min(max(slot, s_lo), s_hi - 1), tok = tok_at + p;
    const uint16_t *kx = FUSED ? a.qkv + tok * a.token_stride + (a.Hq + kvh) * HEAD_DIM
                               : a.k + tok * a.token_stride + kvh * HEAD_DIM;
    const uint16_t *vx = FUSED ? a.qkv + tok * a.token_stride + (a.Hq + a.Hkv + kvh) * HEAD_DIM
                               : a.v + tok * a.token_stride + kvh * HEAD_DIM;
    float kr[8], vr[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        kr[j] = bf16_to_f32(kx[i + 16 * j]);
        vr[j] = bf16_to_f32(vx[i + 16 * j]);
    }
    if (FUSED) {
        float g[8], c[4], sn[4], y[8];
#pragma unroll
        for (int j = 0; j < 8; j++) g[j] = a.k_gain[i + 16 * j];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            c[j] = a.cos[p * HALF + i + 16 * j];
            sn[j] = a.sin[p * HALF + i + 16 * j];
        }
        norm_rope_quad(kr, g, c, sn, y);
#pragma unroll
        for (int j = 0; j < 8; j++) kr[j] = bf16_to_f32(f32_to_bf16(y[j]));
    }
    uint32_t code[8];
    float scale = quantize_quad(kr, code);
    if (live) {
#pragma unroll
        for (int j = 0; j < 8; j++) img[0][k_page_offset(slot, i + 16 * j)] = (uint8_t)code[j];
        if (i == 0) img_scale[0][slot] = scale;
    }
    if (FUSED && a.ve)
        ve_mix_quad(a.ve_h + tok * a.C, a.ve_gate + (long long)kvh * a.C, a.C,
                    a.ve + (long long)a.ve_tokens[tok] * a.C + kvh * HEAD_DIM, i, vr);
    scale = quantize_quad(vr, code);
    if (live) {
#pragma unroll
        for (int j = 0; j < 8; j++) img[1][v_page_offset(slot, i + 16 * j)] = (uint8_t)code[j];
        if (i == 0) img_scale[1][slot] = scale;
    }
    __syncthreads();

    const int t = threadIdx.x, blk = t & 127, kind = t >> 7;   /* kind 0: K block, 1: V block */
    uint8_t *dst = (kind ? a.v_pages : a.k_pages) + at * PAGE_BYTES + blk * 16;
    const uint8_t *src = img[kind] + blk * 16;
    const int s_first = kind ? 4 * ((blk >> 4) & 3) : (blk & 15), s_count = kind ? 4 : 1;
    if (s_first >= s_lo && s_first + s_count <= s_hi) {
        *reinterpret_cast<uint4 *>(dst) = *reinterpret_cast<const uint4 *>(src);
    } else if (kind && s_first < s_hi && s_first + s_count > s_lo) {
#pragma unroll
        for (int e = 0; e < 16; e++) {   /* byte e holds slot s_first + e % 4 */
            const int s = s_first + (e & 3);
            if (s >= s_lo && s < s_hi) dst[e] = src[e];
        }
    }
    if (t < 2 * PAGE) {
        const int s = t & (PAGE - 1), kv = t >> 4;
        if (s >= s_lo && s < s_hi) a.kv_scale[(at * 2 + kv) * PAGE + s] = img_scale[kv][s];
    }
}

/* The training-form prologue (reference model/kernels/qk_prologue.cu:8-32): token p = blockIdx.x of rows/H,
 * rows [0, H) q heads, [H, 2H) k heads; input token stride 3 H 128, output contiguous, position p % T. */
__global__ void __launch_bounds__(256) qkp_forward_kernel(const uint16_t *q, const uint16_t *k, const float *gq,
                                                          const float *gk, uint16_t *qo, uint16_t *ko,
                                                          const float *cos, const float *sin, int H, int T) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int row = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (row >= 2 * H) return;
    const long long p = blockIdx.x;
    const bool isq = row < H;
    const int h = isq ? row : row - H;
    const uint16_t *x = (isq ? q : k) + p * 3 * H * HEAD_DIM + h * HEAD_DIM;
    const float *g = isq ? gq : gk;
    const long long tab = (p % T) * HALF + lane;
    float y1, y2;
    norm_rope_pair(bf16_to_f32(x[lane]), bf16_to_f32(x[lane + HALF]), g[lane], g[lane + HALF], cos[tab], sin[tab], y1,
                   y2);
    uint16_t *y = (isq ? qo : ko) + (p * H + h) * HEAD_DIM;
    y[lane] = f32_to_bf16(y1);
    y[lane + HALF] = f32_to_bf16(y2);
}

/* The training-form prologue's backward (reference model/kernels/qk_prologue.cu:36-90): per (token, head) row, a
 * wave with lane l on dims l and l + 64, recomputing n = x r; the rotation's transpose gives dm (dm1 = dy1 c - dy2 s,
 * dm2 = dy1 s + dy2 c); dn = dm g; dx = r (dn - n b), b = sum(dn n) / 128 (the butterfly); the gain gradient
 * sum_rows dm n accumulates per lane in row order. Grid: QKB_BLOCKS blocks per tensor (q's, then k's), wave w of
 * block j taking rows j 4 + w, + QKB_BLOCKS 4, ...; each block writes its partial [128] (waves added in order). */
constexpr int QKB_BLOCKS = 512;   /* fixed, so the gain gradient's summation order is fixed */

__global__ void __launch_bounds__(256) qkp_backward_kernel(const uint16_t *q, const uint16_t *k, const float *gq,
                                                           const float *gk, const uint16_t *dqo, const uint16_t *dko,
                                                           uint16_t *dq, uint16_t *dk, const float *cos,
                                                           const float *sin, float *part, long long rows, int H,
                                                           int T) {
    __shared__ float wpart[4][HEAD_DIM];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const bool isq = blockIdx.x < QKB_BLOCKS;
    const long long first = (isq ? blockIdx.x : blockIdx.x - QKB_BLOCKS) * 4 + wave;
    const uint16_t *xin = isq ? q : k, *dyin = isq ? dqo : dko;
    uint16_t *dxout = isq ? dq : dk;
    const float *g = isq ? gq : gk;
    const float g1 = g[lane], g2 = g[lane + HALF];
    float a1 = 0.0f, a2 = 0.0f;
    for (long long i = first; i < rows; i += (long long)QKB_BLOCKS * 4) {
        const long long t = i / H, at = t * 3 * H * HEAD_DIM + (i % H) * HEAD_DIM;
        const long long tab = (t % T) * HALF + lane;
        const float x1 = bf16_to_f32(xin[at + lane]), x2 = bf16_to_f32(xin[at + lane + HALF]);
        const float d1 = bf16_to_f32(dyin[i * HEAD_DIM + lane]), d2 = bf16_to_f32(dyin[i * HEAD_DIM + lane + HALF]);
        const float c = cos[tab], s = sin[tab];
        const float ss = wave_sum_butterfly(x1 * x1 + x2 * x2);
        const float r = 1.0f / __builtin_sqrtf(ss / 128.0f + FLT_EPS);
        const float n1 = x1 * r, n2 = x2 * r;
        const float dm1 = d1 * c - d2 * s, dm2 = d1 * s + d2 * c;
        a1 = a1 + dm1 * n1;
        a2 = a2 + dm2 * n2;
        const float dn1 = dm1 * g1, dn2 = dm2 * g2;
        const float b = wave_sum_butterfly(dn1 * n1 + dn2 * n2) / 128.0f;
        dxout[at + lane] = f32_to_bf16(r * (dn1 - n1 * b));
        dxout[at + lane + HALF] = f32_to_bf16(r * (dn2 - n2 * b));
    }
    wpart[wave][lane] = a1;
    wpart[wave][lane + HALF] = a2;
    __syncthreads();
    if (threadIdx.x < HEAD_DIM)
        part[(long long)blockIdx.x * HEAD_DIM + threadIdx.x] =
            ((wpart[0][threadIdx.x] + wpart[1][threadIdx.x]) + wpart[2][threadIdx.x]) + wpart[3][threadIdx.x];
}

/* Block 0: q's gain gradient, block 1: k's; thread d adds dim d of the QKB_BLOCKS partials in block order
 * (reference qk_prologue.cu:92-97). */
__global__ void __launch_bounds__(HEAD_DIM) qkp_gain_sum_kernel(const float *part, float *dgq, float *dgk) {
    const float *p = part + (long long)blockIdx.x * QKB_BLOCKS * HEAD_DIM + threadIdx.x;
    float sum = 0.0f;
    for (int j = 0; j < QKB_BLOCKS; j++) sum = sum + p[(long long)j * HEAD_DIM];
    (blockIdx.x ? dgk : dgq)[threadIdx.x] = sum;
}

static thread_local int last_error = NC_OK;

static int launch_append(AppendArgs a, bool fused, hipStream_t stream) {
    a.pages_per_seq = append_pages_per_seq(a.T);
    const long long x = (long long)a.B * a.pages_per_seq;
    if (x * 256 >= (1LL << 32)) return NC_ERR_SHAPE;
    const dim3 grid((unsigned)x, (unsigned)(fused ? a.Hkv + (a.Hq + 3) / 4 : a.Hkv));
    if (fused)
        hipLaunchKernelGGL(append_kernel<true>, grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(append_kernel<false>, grid, dim3(256), 0, stream, a);
    return (int)hipGetLastError();
}

/* The fused append for the decoder runtime's prefill: runs of rows, run r being rows row0[r] .. + count[r] - 1 of
 * qkv (token_stride apart), at positions start[r] .. of block-table row seq_slot[r], max_count the longest run; with
 * ve non-NULL, v gets the layer's value embedding. Arguments are checked by the caller. */
int append_runs(const uint16_t *qkv, long long token_stride, int runs, int max_count, const int32_t *row0,
                const int32_t *count, const int32_t *start, const int32_t *seq_slot, int Hq, int Hkv,
                const float *q_gain, const float *k_gain, const float *cos, const float *sin, int rope_len,
                uint16_t *q_out, const int32_t *block_table, int max_pages, uint8_t *k_pages, uint8_t *v_pages,
                float *kv_scale, int num_pages, const uint16_t *ve_h, const uint16_t *ve, const float *ve_gate,
                const int32_t *tokens, int C, hipStream_t stream) {
    if (runs <= 0 || max_count <= 0) return NC_OK;
    AppendArgs a = {};
    a.qkv = qkv;
    a.token_stride = token_stride;
    a.B = runs; a.T = max_count; a.Hq = Hq; a.Hkv = Hkv;
    a.start_pos = start; a.num_new = count; a.row0 = row0; a.seq_slot = seq_slot;
    a.q_gain = q_gain; a.k_gain = k_gain; a.cos = cos; a.sin = sin; a.rope_len = rope_len;
    a.q_out = q_out;
    a.block_table = block_table; a.max_pages = max_pages;
    a.k_pages = k_pages; a.v_pages = v_pages; a.kv_scale = kv_scale; a.num_pages = num_pages;
    a.ve_h = ve_h; a.ve = ve; a.ve_gate = ve_gate; a.ve_tokens = tokens; a.C = C;
    return launch_append(a, true, stream);
}

}  // namespace nc

using namespace nc;

extern "C" int nc_kv_append_fp8(const void *k, const void *v, long long token_stride, int B, int T, int Hkv,
                                const int32_t *start_pos, const int32_t *num_new, const int32_t *block_table,
                                int max_pages, void *k_pages, void *v_pages, float *kv_scale, int num_pages,
                                void *stream) {
    if (!k || !v || !start_pos || !block_table || !k_pages || !v_pages || !kv_scale) return NC_ERR_NULL;
    if (B <= 0 || T <= 0 || Hkv <= 0 || max_pages <= 0 || num_pages <= 0 || token_stride < (long long)Hkv * HEAD_DIM)
        return NC_ERR_SHAPE;
    if ((long long)B * T > 0x7FFFFFFFLL) return NC_ERR_SHAPE;
    AppendArgs a = {};
    a.k = (const uint16_t *)k;
    a.v = (const uint16_t *)v;
    a.token_stride = token_stride;
    a.B = B; a.T = T; a.Hq = 0; a.Hkv = Hkv;
    a.start_pos = start_pos; a.num_new = num_new;
    a.block_table = block_table; a.max_pages = max_pages;
    a.k_pages = (uint8_t *)k_pages; a.v_pages = (uint8_t *)v_pages;
    a.kv_scale = kv_scale; a.num_pages = num_pages;
    return launch_append(a, false, (hipStream_t)stream);
}

extern "C" int nc_qk_norm_rope_append_fp8(const void *qkv, long long token_stride, int B, int T, int Hq, int Hkv,
                                          const int32_t *start_pos, const int32_t *num_new, const float *q_gain,
                                          const float *k_gain, const float *cos, const float *sin, int rope_len,
                                          void *q_out, const int32_t *block_table, int max_pages, void *k_pages,
                                          void *v_pages, float *kv_scale, int num_pages, void *stream) {
    if (!qkv || !start_pos || !q_gain || !k_gain || !cos || !sin || !q_out || !block_table || !k_pages || !v_pages ||
        !kv_scale)
        return NC_ERR_NULL;
    if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || max_pages <= 0 || num_pages <= 0 || rope_len <= 0 ||
        token_stride < (long long)(Hq + 2 * Hkv) * HEAD_DIM)
        return NC_ERR_SHAPE;
    if ((long long)B * T > 0x7FFFFFFFLL) return NC_ERR_SHAPE;
    AppendArgs a = {};
    a.qkv = (const uint16_t *)qkv;
    a.token_stride = token_stride;
    a.B = B; a.T = T; a.Hq = Hq; a.Hkv = Hkv;
    a.start_pos = start_pos; a.num_new = num_new;
    a.q_gain = q_gain; a.k_gain = k_gain; a.cos = cos; a.sin = sin; a.rope_len = rope_len;
    a.q_out = (uint16_t *)q_out;
    a.block_table = block_table; a.max_pages = max_pages;
    a.k_pages = (uint8_t *)k_pages; a.v_pages = (uint8_t *)v_pages;
    a.kv_scale = kv_scale; a.num_pages = num_pages;
    return launch_append(a, true, (hipStream_t)stream);
}

extern "C" int qkp_backward_blocks() { return QKB_BLOCKS; }

extern "C" void qkp_backward(const void *q, const void *k, const void *gq, const void *gk, const void *dqo,
                             const void *dko, void *dq, void *dk, void *dgq, void *dgk, void *part, const void *cos,
                             const void *sin, long long rows, int H, int T, void *stream) {
    if (!q || !k || !gq || !gk || !dqo || !dko || !dq || !dk || !dgq || !dgk || !part || !cos || !sin) {
        last_error = NC_ERR_NULL;
        return;
    }
    if (H <= 0 || T <= 0 || rows < 0 || rows % H) {
        last_error = NC_ERR_SHAPE;
        return;
    }
    hipLaunchKernelGGL(qkp_backward_kernel, dim3(2 * QKB_BLOCKS), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)q, (const uint16_t *)k, (const float *)gq, (const float *)gk,
                       (const uint16_t *)dqo, (const uint16_t *)dko, (uint16_t *)dq, (uint16_t *)dk,
                       (const float *)cos, (const float *)sin, (float *)part, rows, H, T);
    hipLaunchKernelGGL(qkp_gain_sum_kernel, dim3(2), dim3(HEAD_DIM), 0, (hipStream_t)stream, (const float *)part,
                       (float *)dgq, (float *)dgk);
    last_error = (int)hipGetLastError();
}

extern "C" void qkp_forward(const void *q, const void *k, const void *gq, const void *gk, void *qo, void *ko,
                            const void *cos, const void *sin, long long rows, int H, int T, void *stream) {
    if (!q || !k || !gq || !gk || !qo || !ko || !cos || !sin) {
        last_error = NC_ERR_NULL;
        return;
    }
    if (H <= 0 || T <= 0 || rows <= 0 || rows % H || rows / H > 0x7FFFFFFFLL) {
        last_error = NC_ERR_SHAPE;
        return;
    }
    const dim3 grid((unsigned)(rows / H), (unsigned)((2 * H + 3) / 4));
    hipLaunchKernelGGL(qkp_forward_kernel, grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t *)q,
                       (const uint16_t *)k, (const float *)gq, (const float *)gk, (uint16_t *)qo, (uint16_t *)ko,
                       (const float *)cos, (const float *)sin, H, T);
    last_error = (int)hipGetLastError();
}

void nc::set_last_error(int status) { last_error = status; }

extern "C" int nc_last_error(void) { return last_error; }

extern "C" const char *nc_status_string(int status) {
    switch (status) {
        case NC_OK: return "ok";
        case NC_ERR_NULL: return "a required pointer is NULL";
        case NC_ERR_SHAPE: return "a size or head count is out of the supported range";
        case NC_ERR_WORKSPACE: return "the workspace is smaller than nc_decode_workspace_bytes";
        default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown status";
    }
}

extern "C" int nc_abi_version(void) { return 4; }
