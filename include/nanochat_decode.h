/*
 * nanochat_amd decoder runtime (libnanochat_decode.so): the 14 dec_* symbols of the reference's decoder ABI,
 * model/kernels/decode.cu:904-1131, with the argument lists inference/decoder.py:132-148 binds, over an fp8
 * (e4m3fn) paged KV cache on gfx950. Every call is stream-ordered on the stream given to dec_create except
 * dec_create (synchronous allocation) and dec_tokens (synchronizes). A failed HIP call, or an argument out of
 * range, aborts with a message, as in the reference (decode.cu:47-53, 926-931).
 *
 * Differences from the reference, by design: the KV cache is fp8 with one scale per (token, head) (the reference
 * caches bf16); the prompt store lives in device memory, as pages of the same pools (the reference: pinned host
 * memory); dec_prefill takes up to 16384 rows (the reference: 1024); steps are launched eagerly, not as graphs.
 */
#ifndef NANOCHAT_DECODE_H
#define NANOCHAT_DECODE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* cfg [7]: L, C, F, vocab, max_len, store (prompt-store positions), lazy (the BOS row a host may reject).
 * ptrs [4 + 8 L]: wte fp32 [vocab][C], cos, sin fp32 [>= max_len][64], lm_head bf16 [vocab][C]; per layer qkv bf16
 * [3C][C], o [C][C], fc [F][C], proj [C][F], value-embedding table bf16 [vocab][C] and its gate fp32 [H][C] (both 0
 * on layers without value embeddings), q norm, k norm fp32 [128].
 * scal [2L + 1]: per layer (resid, x0) lambdas, then the logit cap. window [L]: keys before a query per layer.
 * Reference: decode.cu:950-1023. */
void *dec_create(const int *cfg, const uint64_t *ptrs, const float *scal, const int *window, void *stream);

/* Slots (decode.cu:948). */
int dec_batch(void *handle);

/* Start slot b at its prompt's last token `token`, position `last` (decode.cu:1026-1035). */
void dec_set_prompt(void *handle, int b, int32_t token, int32_t last, float temperature, float top_p,
                    unsigned long long seed);

/* Rows per dec_prefill call (decode.cu:1037). */
int dec_prefill_rows(void *handle);

/* Run n rows (host int32 [3][n]: token, position, slot; a slot's rows at consecutive positions) through the body,
 * caching each row's K and V, each row attending to its slot's positions up to its own (decode.cu:1041-1051). */
void dec_prefill(void *handle, int n, const int32_t *rows);

/* Copy slot b's positions [at, at + n) to / from prompt-store position store_at (decode.cu:1069-1075). */
void dec_save_prompt(void *handle, int b, int at, int store_at, int n);
void dec_load_prompt(void *handle, int b, int at, int store_at, int n);

/* Pinned host allowed-token masks [B][vocab / 32] (decode.cu:1079). */
uint32_t *dec_masks(void *handle);

/* Active and masked slots, host uint64 [2][ceil(B / 64)] (decode.cu:1083-1105). */
void dec_set_active(void *handle, const unsigned long long *slots);

/* One step: the body (embedding, layers), then the head (final norm, lm_head, choice, commit)
 * (decode.cu:1107-1116). */
void dec_launch_body(void *handle);
void dec_launch_head(void *handle);

/* Wait for the step; out [2B]: each slot's token, then its alternative (decode.cu:1120-1124). */
void dec_tokens(void *handle, int32_t *out);

/* Slot b's next input becomes its alternative (decode.cu:1128-1131). */
void dec_take_alt(void *handle, int b);

/* Free everything dec_create allocated (decode.cu:904-924). */
void dec_destroy(void *handle);

/* --- Extensions with no counterpart in the reference. */

/* dec_create with at most max_slots slots (1..1024): for callers that share the device with other work. dec_create
 * is dec_create_slots(..., 1024). */
void *dec_create_slots(const int *cfg, const uint64_t *ptrs, const float *scal, const int *window, void *stream,
                       int max_slots);

/* KV pages: every layer's pool holds `pool` pages the slots draw from on their first write of a page and return when
 * a slot starts a new sequence (a write at position 0), when dec_set_prompt moves it to an earlier position (the pages
 * past it), or on dec_release. dec_create / dec_create_slots size the pool for every slot at max_len; dec_create_pool
 * takes pool_pages (>= max_len / 16) and fits as many slots (<= max_slots) as the memory left allows, so a host can
 * run more sequences than full-length reservations would hold. A write that finds the pool empty aborts: such a host
 * admits sequences by dec_debug_pages. */
void *dec_create_pool(const int *cfg, const uint64_t *ptrs, const float *scal, const int *window, void *stream,
                      int max_slots, long long pool_pages);

/* Slot b's pages return to the pool (its shared store pages are unlinked); its next sequence starts at position 0. */
void dec_release(void *handle, int b);

/* out [2]: the pool's free pages, its size. */
void dec_debug_pages(void *handle, long long *out);

/* Test hooks (synchronize, then copy to host): the last head's fp32 logits of slots [0, rows), out [rows][vocab];
 * and the cached rows of slot b (b = -1: the prompt store) at positions [at, at + n) of one layer, k and v as
 * e4m3fn codes [n][H][128], scales [n][H][2] (K, V). */
void dec_debug_logits(void *handle, float *out, int rows);
void dec_debug_cache(void *handle, int layer, int b, int at, int n, uint8_t *k, uint8_t *v, float *scales);

/* Slot b's block-table row, max_length / 16 (rounded up) entries: -1 (no page yet), a pool page in [0, pool) of the
 * slot's own, or pool + i for page i of the prompt store, shared read-only after dec_load_prompt. */
void dec_debug_table(void *handle, int b, int32_t *out);

/* Whether a step over more than 64 slots runs as two concurrent lanes or as one (the default); whether the step's
 * body replays captured graphs or launches its kernels one by one (the default). Both synchronize. */
void dec_debug_set_split(void *handle, int on);
void dec_debug_set_graphs(void *handle, int on);

/* The decode step's GEMM alone (slot_gemm.hip): out[n][r] = epilogue(sum_k x[n][k] w[r][k]), bf16 w [R][K] and
 * x [N][K] (N <= 128), epi 0 bf16(s), 1 x = s + res: bf16 out and fp32 out_f32, 2 bf16(relu(p) p) with p = s rstd[n],
 * 3 bf16(s + res), 4 fp32 out_f32 = s; split over `slices` K-slices (0: the decoder's choice,
 * dec_debug_slot_gemm_slices) whose partial sums go to part (fp32 [slices][N][R], dec_debug_slot_gemm_part_bytes(R, N,
 * slices) bytes, none for one slice) and are added in slice order. Returns 0, a hipError_t, or -2 when the shape (K a
 * multiple of 128, R of 4), the slice count or an operand the epilogue needs does not fit. Stream-ordered. */
int dec_debug_slot_gemm(int epi, const void *w, int R, int K, const void *x, int N, void *out, float *out_f32,
                        const void *res, const float *rstd, int slices, float *part, void *stream);
int dec_debug_slot_gemm_slices(int R, int K);
long long dec_debug_slot_gemm_part_bytes(int R, int N, int slices);
/* The workgroup tile dec_debug_slot_gemm launches for (R, K, N, slices; slices 0 = the default): 100 RT + CT for RT
 * 16-row weight tiles and CT 16-slot tiles a workgroup, or -2 when the shape does not fit. */
int dec_debug_slot_gemm_tile(int R, int K, int N, int slices);
/* The step's MLP rstd path, one K slice: epi 1 (RESID2) writes bf16(s + res) to out and each 16-row tile's sum of
 * squares of s + res to ssq (fp32 [N][ceil(R / 16)]); epi 2 (RELU2) takes each slot's rstd from ssq (fp32
 * [N][ceil(K / 16)], summed over tiles in order: 1 / sqrt(sum / K + FLT_EPSILON)) and writes bf16(relu(s r) s r).
 * Returns 0, a hipError_t, or -2 when the shape or operands do not fit. Stream-ordered. */
int dec_debug_slot_gemm_ssq(int epi, const void *w, int R, int K, const void *x, int N, void *out, const void *res,
                            float *ssq, void *stream);

/* The prefill GEMM alone (prefill_gemm.hip): out[m][n] = epilogue(sum_k a[m][k] w[n][k]) for M rows, bf16 w [N][K]
 * and a [M][K]; epi 0 bf16(s) to out, 3 bf16(s + res) (res bf16 [M][N]), 4 fp32 s to out_f32, 2 bf16(relu(p) p) with
 * p = s rstd[m] (rstd fp32 [M]). Every row's sums run over K in one fixed order whatever M is. Returns 0, a hipError_t,
 * or -2 when the shape (K a multiple of 128, N of 4, every array under 2 GiB) or an operand the epilogue needs does
 * not fit. Stream-ordered. */
int dec_debug_prefill_gemm(int epi, const void *w, int N, int K, const void *a, int M, void *out, float *out_f32,
                           const void *res, const float *rstd, void *stream);

/* The prefill's cache append alone (kv_append.hip, as dec_prefill runs it): run r is rows row0[r] .. + count[r] - 1
 * of qkv (bf16 [rows][(Hq + 2 Hkv) 128] at token_stride elements) at positions start[r] .. of block-table row
 * seq_slot[r] (int32 [*][max_pages]); max_count bounds count. q is normed and rotated into q_out ([rows][Hq][128]),
 * k normed and rotated, v mixed with the value embedding when ve is non-NULL (v += 2 sigmoid(ve_gate[head] . ve_h[row])
 * ve[tokens[row]], ve_h bf16 [rows][C], ve bf16 [vocab][C], ve_gate fp32 [Hkv][C]), and both quantized into the pages
 * (k_pages, v_pages e4m3fn [num_pages][Hkv][2048], kv_scale fp32 [num_pages][Hkv][2][16]). Returns 0, a hipError_t,
 * or -2 for a NULL operand or a shape it does not take. Stream-ordered. */
int dec_debug_append_runs(const void *qkv, long long token_stride, int runs, int max_count, const int32_t *row0,
                          const int32_t *count, const int32_t *start, const int32_t *seq_slot, int Hq, int Hkv,
                          const float *q_gain, const float *k_gain, const float *cos, const float *sin, int rope_len,
                          void *q_out, const int32_t *block_table, int max_pages, void *k_pages, void *v_pages,
                          float *kv_scale, int num_pages, const void *ve_h, const void *ve, const float *ve_gate,
                          const int32_t *tokens, int C, void *stream);

/* The nucleus threshold of choose_kernel alone: for each of `rows` rows of probabilities e (fp32 [rows][vocab],
 * device; e = exp(z / T - max z / T) in [0, 1], 0 for rows not allowed) and its top_p (fp32 [rows], device), the
 * IEEE bit pattern of e*, the least e for which the rows with e' <= e* weigh more than (1 - top_p) of the total,
 * with each row weighing the integer round(e 2^38). Rows with e >= e* (and weight > 0) form the nucleus. cut:
 * uint32 [rows], device. Returns 0, a hipError_t, or -2 for a shape it does not take (vocab < 2^25).
 * Stream-ordered. */
int dec_debug_nucleus_cut(const float *e, int rows, int vocab, const float *top_p, uint32_t *cut, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOCHAT_DECODE_H */
