/*
 * nanochat_amd: the C ABI of the MI355X (gfx950) fp8 KV-cache decode path.
 *
 * Every pointer argument is a device address unless stated otherwise; sizes are element counts. Every
 * entry point is stream-ordered on `stream` (a hipStream_t; NULL = the null stream) and never
 * synchronizes. Entry points that return int return NC_OK (0), a negative NC_ERR_* code for an argument
 * the host can check, or a positive hipError_t from the launch.
 *
 * Data formats (the build's; the reference caches bf16, model/kernels/decode.cu:726):
 *   bf16             raw 16-bit patterns (torch.bfloat16 storage)
 *   k_pages, v_pages uint8 [num_pages][Hkv][2048]: one 16-token page of one KV head, OCP e4m3fn codes in
 *                    the MFMA tiling documented in nanochat_amd/csrc/nc_device.h (k/v_page_offset)
 *   kv_scale         fp32 [num_pages][Hkv][2][16]: one absmax/448 scale per (token, KV head), K scales then
 *                    V scales of a page's 16 slots (one 128-byte line per page and head)
 *   block_table      int32 [B][max_pages]: position p of sequence b is slot p % 16 of page
 *                    block_table[b][p / 16]
 * Query head h reads KV head h / (Hq / Hkv); Hq must be a multiple of Hkv with Hq / Hkv <= 16.
 */
#ifndef NANOCHAT_AMD_H
#define NANOCHAT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    NC_OK = 0,
    NC_ERR_NULL = -1,       /* a required pointer is NULL */
    NC_ERR_SHAPE = -2,      /* a size or head count out of the supported range */
    NC_ERR_WORKSPACE = -3,  /* the workspace is smaller than nc_decode_workspace_bytes */
};

/* Text of a status code (static storage). */
const char *nc_status_string(int status);

/* Version of this ABI (bumped on any signature or format change). */
int nc_abi_version(void);

/*
 * Training-form fused q/k prologue; same symbol, arguments and meaning as the reference's
 * model/kernels/qk_prologue.cu:111-118 (called by model/ops/qk_prologue.py:13-21 qk_forward):
 * q, k: bf16 (B, T, H, 128) views with token stride 3*H*128 (the fused projection); gq, gk: fp32 [128];
 * qo, ko: bf16 contiguous (B, T, H, 128); cos, sin: fp32 [T][64] indexed by the token's position t;
 * rows = B*T*H. Per row: RMS norm (eps FLT_EPSILON), gain, -theta rotation, one bf16 rounding.
 * Like the reference it returns nothing; nc_last_error() reports its launch status.
 */
void qkp_forward(const void *q, const void *k, const void *gq, const void *gk, void *qo, void *ko, const void *cos,
                 const void *sin, long long rows, int H, int T, void *stream);

/* The prologue's backward: the reference's qkp_backward (model/kernels/qk_prologue.cu:128-136), same arguments.
 * q, k as for qkp_forward; dqo, dko: the outputs' gradients, contiguous [rows][128] bf16; dq, dk: the inputs'
 * gradients at q's and k's strides (token stride 3 H 128); dgq, dgk: the gains' gradients fp32 [128], summed in a
 * fixed order (bitwise reproducible); part: fp32 [2 qkp_backward_blocks()][128] scratch. rows = 0 is allowed (the
 * gain gradients are zero). Returns nothing; nc_last_error() reports the status. */
void qkp_backward(const void *q, const void *k, const void *gq, const void *gk, const void *dqo, const void *dko,
                  void *dq, void *dk, void *dgq, void *dgk, void *part, const void *cos, const void *sin,
                  long long rows, int H, int T, void *stream);

/* Blocks per tensor of qkp_backward's partial gain gradients (reference qk_prologue.cu:120-125): fixed. */
int qkp_backward_blocks(void);

/*
 * Value-embedding gate and mix of training; same symbols, arguments and meaning as the reference's
 * model/kernels/ve_gate.cu:199-214 (called by model/ops/ve_gate.py:13-33), with the reference's fixed shape H = 6
 * heads, C = 768. Forward: n bf16 [rows][C] (the normed stream), v bf16 rows at v_stride elements, idx int32 [rows],
 * table fp32 [vocab][C], w fp32 [H][C] -> out bf16 [rows][C] = v + gate[head] * bf16(table[idx]),
 * gate fp32 [rows][H] = 2 sigmoid(n w^T). Backward: dout bf16 rows at dout_stride, ids int32 [rows] sorted tokens
 * (equal tokens must be adjacent, else the table gradient is undefined), order int64 [rows] their rows (a row
 * outside [0, rows) is skipped), gate from the forward -> dn bf16 [rows][C], dz bf16 [rows][H] (dw = dz^T n is the
 * caller's GEMM), and the table's gradient added into dtable fp32 [vocab][C]. Tokens are trusted (negative ones
 * read as a zero embedding). Like the reference they return nothing; nc_last_error() reports the status.
 */
void ve_forward(const void *n, const void *v, long long v_stride, const void *idx, const void *table, const void *w,
                void *out, void *gate, long long rows, void *stream);
void ve_backward(const void *dout, long long dout_stride, const void *ids, const void *order, const void *table,
                 const void *w, const void *gate, void *dn, void *dtable, void *dz, long long rows, void *stream);

/* ve_forward / ve_backward for any head count 1 <= heads <= 16 (C = 128 heads) and a table of `vocab` rows: a token
 * outside [0, vocab) mixes in nothing and receives no gradient. Strides are multiples of 8 elements and at least C;
 * n, v, table, w, out, dout, dn and dtable are 16-byte aligned. rows = 0 launches nothing. */
int nc_ve_forward(const void *n, const void *v, long long v_stride, const int32_t *idx, const float *table,
                  long long vocab, const float *w, void *out, float *gate, long long rows, int heads, void *stream);
int nc_ve_backward(const void *dout, long long dout_stride, const int32_t *ids, const int64_t *order,
                   const float *table, long long vocab, const float *w, const float *gate, void *dn, float *dtable,
                   void *dz, long long rows, int heads, void *stream);

/*
 * Training attention forward: the varlen causal attention the reference runs through FlashAttention-4
 * (model/ops/flash_attn.py:340-345, _flash_attn_fwd(q, k, v, cu_seqlens, cu_seqlens, T, T, causal=True,
 * window_size_left=window, return_lse=True)). q, k, v: bf16 (total, heads, 128) with contiguous heads at token strides
 * q_stride, k_stride, v_stride (elements, multiples of 8); cu_seqlens: int32 [segments + 1] (segment s is tokens
 * cu[s] .. cu[s+1] - 1, at most max_seqlen of them). Row i of a segment attends keys j of the same segment with
 * j <= i and i - j <= window (window < 0: no left limit), scores scaled by softmax_scale.
 * out: bf16 (total, heads, 128) contiguous; lse: fp32 [heads][lse_stride], ln of the row's sum of exponentials.
 */
int nc_flash_attn_fwd(const void *q, const void *k, const void *v, long long q_stride, long long k_stride,
                      long long v_stride, const int32_t *cu_seqlens, int segments, int max_seqlen, int heads,
                      int window, float softmax_scale, void *out, float *lse, long long lse_stride, void *stream);

/*
 * Training attention backward (the reference's _flash_attn_bwd and bwd_bf16dq, model/ops/flash_attn.py:367-391):
 * q, k, v, dout as the forward's inputs and the output's gradient (token strides in elements); lse from
 * nc_flash_attn_fwd; dpsum fp32 (total, heads): D = dout . out per row (the reference's `rows`; see
 * nc_flash_attn_bwd_rows). Writes dq, dk, dv: bf16 (total, heads, 128) with contiguous heads at their token strides.
 * No atomics: the result does not depend on scheduling.
 */
int nc_flash_attn_bwd(const void *q, const void *k, const void *v, const void *dout, long long q_stride,
                      long long k_stride, long long v_stride, long long do_stride, const float *lse, long long lse_stride,
                      const float *dpsum, const int32_t *cu_seqlens, int segments, int max_seqlen, int heads,
                      int window, float softmax_scale, void *dq, void *dk, void *dv, long long dq_stride,
                      long long dk_stride, long long dv_stride, void *stream);

/* dpsum (total, heads) fp32 = sum over the 128 dims of dout * out (token strides in elements, even). */
int nc_flash_attn_bwd_rows(const void *out, long long o_stride, const void *dout, long long do_stride,
                           long long total, int heads, float *dpsum, void *stream);

/* Status of the last void entry point's launch on this host thread (NC_OK or a hipError_t). */
int nc_last_error(void);

/*
 * Quantize and append T new tokens per sequence to the paged fp8 cache. Replaces the cache store of the
 * reference's k_prologue (model/kernels/decode.cu:551-565, `kc/vc[cs][p] = bf16(k/v)`).
 * k, v: bf16 [B][T][Hkv][128] at token stride `token_stride` elements (batch stride T*token_stride);
 * token t of sequence b is written at position start_pos[b] + t; num_new (nullable) limits sequence b to
 * its first num_new[b] tokens. Per (token, KV head): scale = max|x| / 448 (1 if all zero),
 * code = e4m3fn_rne(clamp(x / scale, +-448)). Tokens whose page lies outside the block table or the
 * page pool are skipped.
 */
int nc_kv_append_fp8(const void *k, const void *v, long long token_stride, int B, int T, int Hkv,
                     const int32_t *start_pos, const int32_t *num_new, const int32_t *block_table, int max_pages,
                     void *k_pages, void *v_pages, float *kv_scale, int num_pages, void *stream);

/*
 * The fused append of a decode or prefill step: the reference's attn_prologue q/k math
 * (model/kernels/decode.cu:478-507 via qk_row.cuh:26-51) followed by nc_kv_append_fp8's quantized store.
 * qkv: bf16 [B][T][(Hq + 2*Hkv)*128] at token stride `token_stride` elements: q heads, then k heads, then
 * v heads. q and k rows are RMS-normed (eps FLT_EPSILON), multiplied by q_gain / k_gain (fp32 [128]) and
 * rotated by -theta with cos, sin (fp32 [rope_len][64]) at the token's position, then rounded to bf16;
 * q goes to q_out (bf16 [B][T][Hq][128], contiguous), k and v (unchanged) are quantized into the cache.
 * Tokens at positions >= rope_len are skipped.
 */
int nc_qk_norm_rope_append_fp8(const void *qkv, long long token_stride, int B, int T, int Hq, int Hkv,
                               const int32_t *start_pos, const int32_t *num_new, const float *q_gain,
                               const float *k_gain, const float *cos, const float *sin, int rope_len, void *q_out,
                               const int32_t *block_table, int max_pages, void *k_pages, void *v_pages,
                               float *kv_scale, int num_pages, void *stream);

/* Workspace bytes nc_decode_attn_fp8 and nc_decode_step_fp8 need for these sizes (0 for unsupported sizes): fp32
 * partial results from its start and, in its last 1/256, one int32 arrival count per (sequence, KV head). The
 * workspace must be zero-filled before its first call and passed with the same workspace_bytes to every call: the
 * counts' place depends on that size alone, partials never go there and every call returns the counts it used to
 * zero, so one zero fill serves any number of calls of any sizes that fit, ordered on one stream. */
size_t nc_decode_workspace_bytes(int B, int Hq, int Hkv, int max_seq_len, int window);

/*
 * Single-token decode attention over the paged fp8 cache. Replaces the reference's k_attn
 * (model/kernels/decode.cu:567-675): sequence b's query at position p = seq_lens[b] - 1 attends keys
 * [max(p - window, 0), p] (window < 0: all), scores (q . k) * sm_scale, fp32 softmax, out bf16.
 * The current token must already be appended (nc_kv_append_fp8 / nc_qk_norm_rope_append_fp8).
 * q: bf16 [B][Hq][128]; out: bf16 [B][Hq][128]; seq_lens: int32 [B] (<= 0: inactive, output zeros; more
 * than max_seq_len: output NaN); max_seq_len <= max_pages * 16; B <= 4096.
 * Work split: a (sequence, KV head)'s keys are cut at every multiple of 1,024 positions, or of 256 positions when its
 * keys span at most 67 pages (1,072 positions); a last piece under 64 positions joins the one before it. Each piece
 * is one work item with its own softmax state; the wave that finishes a unit's last piece merges its pieces in
 * position order, in the same launch (one kernel). The split points depend on nothing but the sequence's own length, so its
 * output bits do not depend on the other sequences of the launch, on its place in the batch or on `workers` (waves
 * taking the items; 0: every wave slot of the device). The workspace (at least nc_decode_workspace_bytes) must be
 * zero-filled before its first use and keep one workspace_bytes value across calls.
 * A block-table entry outside [0, num_pages) makes that sequence's output NaN instead of reading outside
 * the pool.
 */
int nc_decode_attn_fp8(const void *q, const void *k_pages, const void *v_pages, const float *kv_scale,
                       const int32_t *block_table, int max_pages, int num_pages,
                       const int32_t *seq_lens, int max_seq_len, int B, int Hq, int Hkv, int window, float sm_scale,
                       int workers, void *out, void *workspace, size_t workspace_bytes, void *stream);

/*
 * The fused decode step: nc_qk_norm_rope_append_fp8 with T = 1 followed by nc_decode_attn_fp8, in one launch, with
 * the same results bit for bit (query rows, cache bytes and scales, attention output). Replaces the reference's
 * k_prologue + k_attn pair of a decode step (model/kernels/decode.cu:551-675, launched at 861-863). Sequence b's
 * token sits at position p = seq_lens[b] - 1 (seq_lens <= 0: inactive, nothing appended, output zeros); its row of
 * qkv (bf16 [B][(Hq + 2 Hkv) 128] at token_stride elements) is normed, rotated (q_gain, k_gain, cos, sin as in
 * nc_qk_norm_rope_append_fp8; rope_len >= max_seq_len) and, when ve is not NULL, its value row gets the value
 * embedding of token ve_tokens[b] (ve bf16 [ve_rows][C], ve_gate fp32 [Hkv][C], ve_h bf16 [B][C] the layer's normed
 * input; v += 2 sigmoid(ve_gate[kvh] . h) ve[token][kvh 128 ..]; a token outside [0, ve_rows) mixes nothing); k and v are quantized into the cache and q goes to
 * q_out (bf16 [B][Hq][128]) unless q_out is NULL; then the query attends as in nc_decode_attn_fp8. A sequence longer
 * than max_seq_len gets NaN and no append. The page receiving a sequence's token must not appear in another
 * sequence's block-table row (the work item that streams that page takes the token from registers while it stores
 * it). Workspace as for nc_decode_attn_fp8.
 */
int nc_decode_step_fp8(const void *qkv, long long token_stride, int B, int Hq, int Hkv, const int32_t *seq_lens,
                       const float *q_gain, const float *k_gain, const float *cos, const float *sin, int rope_len,
                       void *q_out, const void *ve_h, const void *ve, const float *ve_gate, const int32_t *ve_tokens,
                       int C, int ve_rows, const int32_t *block_table, int max_pages, void *k_pages, void *v_pages, float *kv_scale,
                       int num_pages, int max_seq_len, int window, float sm_scale, int workers, void *out,
                       void *workspace, size_t workspace_bytes, void *stream);

/* Bytes of the static device workspace of nc_decode_attn_fp8_noalloc (one array per GPU, held until the process
 * ends). */
#define NC_DECODE_SCRATCH_BYTES (16u << 20)

/*
 * No counterpart in the reference. For callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): nc_decode_attn_fp8 with the same arguments, results and
 * errors, but its workspace is a static device array of NC_DECODE_SCRATCH_BYTES per GPU instead of the caller's. It
 * calls no allocating routine. A launch that needs more than that (nc_decode_workspace_bytes) returns
 * NC_ERR_WORKSPACE. Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams, two
 * host threads) race and give undefined results; calls ordered on one stream do not.
 */
int nc_decode_attn_fp8_noalloc(const void *q, const void *k_pages, const void *v_pages, const float *kv_scale,
                               const int32_t *block_table, int max_pages, int num_pages, const int32_t *seq_lens,
                               int max_seq_len, int B, int Hq, int Hkv, int window, float sm_scale, int workers,
                               void *out, void *stream);

/*
 * Chunked-prefill attention over the paged fp8 cache (MFMA). Replaces the reference's prefill rows
 * (model/kernels/decode.cu:1041-1051 with enqueue_body's append-then-attend order, 859-863): row t of
 * sequence b sits at position start_pos[b] + t and attends keys [max(p - window, 0), p]; the chunk must
 * already be appended. q, out: bf16 [B][T][Hq][128].
 */
int nc_prefill_attn_fp8(const void *q, const void *k_pages, const void *v_pages, const float *kv_scale,
                        const int32_t *block_table, int max_pages, int num_pages,
                        const int32_t *start_pos, int B, int T, int Hq, int Hkv, int window, float sm_scale,
                        void *out, void *stream);

/*
 * Measurement only; no counterpart in the reference. Reads n pages of 2 KiB (one (page, head) of K or V codes) from
 * src (src_bytes, a multiple of 2,048), page order[i] as the i-th (order NULL: page i; an entry outside the buffer
 * reads page 0), with `grid` workgroups of 256 threads, and writes one checksum word per thread to sink
 * (grid x 256 uint32: their XOR is the XOR of every dword read). Its duration is the read-only ceiling of the decode
 * step's page stream. Returns 0, NC_ERR_NULL or NC_ERR_SHAPE (grid outside [1, 65535]).
 */
int nc_debug_read_pages(const void *src, long long src_bytes, const int32_t *order, int n, int grid, uint32_t *sink,
                        void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOCHAT_AMD_H */
