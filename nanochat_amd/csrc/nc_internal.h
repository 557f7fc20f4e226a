/*
 * Launchers shared between the kernel files and the decoder runtime (decoder.hip), not part of the C ABI.
 * Arguments are checked by the caller.
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nc {

/* kv_append.hip: the status nc_last_error() reports for the calling host thread (the void entry points set it). */
void set_last_error(int status);

/* kv_append.hip: the fused QK-norm/RoPE fp8 append of runs of rows: run r is rows row0[r] .. + count[r] - 1 of
 * qkv at positions start[r] .. of block-table row seq_slot[r] (max_count: the longest run); ve non-NULL adds the
 * value embedding 2 sigmoid(ve_gate[head] . ve_h[row]) ve[tokens[row]] to v before it is quantized (C: ve_h's
 * width). */
int append_runs(const uint16_t *qkv, long long token_stride, int runs, int max_count, const int32_t *row0,
                const int32_t *count, const int32_t *start, const int32_t *seq_slot, int Hq, int Hkv,
                const float *q_gain, const float *k_gain, const float *cos, const float *sin, int rope_len,
                uint16_t *q_out, const int32_t *block_table, int max_pages, uint8_t *k_pages, uint8_t *v_pages,
                float *kv_scale, int num_pages, const uint16_t *ve_h, const uint16_t *ve, const float *ve_gate,
                const int32_t *tokens, int C, hipStream_t stream);

/* The fused decode step's inputs: each sequence's token row as the qkv projection left it, and what the cache
 * append needs (the fused append's arguments, for one token per sequence at position seq_lens[b] - 1). */
struct StepArgs {
    const uint16_t *qkv;        /* [B][(Hq + 2 Hkv) 128] bf16 at token_stride */
    long long token_stride;
    const float *q_gain, *k_gain;
    const float *cos, *sin;     /* [rope_len][64] */
    uint16_t *q_out;            /* NULL, or [B][Hq][128]: the normed, rotated queries */
    const uint16_t *ve_h, *ve;  /* NULL ve: no value embeddings; else h [B][C], table [vocab][C] */
    const float *ve_gate;       /* [Hkv][C] */
    const int32_t *ve_tokens;   /* [B]; a token outside [0, ve_rows) mixes nothing */
    int C, ve_rows;
    uint8_t *k_pages, *v_pages; /* the cache the step appends to (the launch's pools) */
    float *kv_scale;
};

/* attention.hip: nc_decode_step_fp8 for the decoder runtime (rope_len >= max_seq_len, workers = 0); the workspace
 * as nc_decode_attn_fp8's (its size checked here). */
int decode_step(const StepArgs &step, const void *k_pages, const void *v_pages, const float *kv_scale,
                const int32_t *block_table, int max_pages, int num_pages, const int32_t *seq_lens, int max_seq_len,
                int B, int Hq, int Hkv, int window, float sm_scale, void *out, void *workspace, size_t workspace_bytes,
                hipStream_t stream);

/* attention.hip: chunked prefill over runs of rows. */
int prefill_runs(const uint16_t *q, const uint8_t *k_pages, const uint8_t *v_pages, const float *kv_scale,
                 const int32_t *block_table, int max_pages, int num_pages, const int32_t *start_pos,
                 const int32_t *run_row0, const int32_t *run_count, const int32_t *run_slot, int runs, int max_count,
                 int Hq, int Hkv, int window, float sm_scale, uint16_t *out, hipStream_t stream);

/* The decode step's GEMM operands: out[n][r] = epilogue(sum_k x[n][k] w[r][k]), bf16 operands, fp32 sums,
 * N <= SG_MAX_N rows. */
constexpr int SG_MAX_N = 128;
enum { SG_STORE, SG_RESID2, SG_RELU2, SG_RESID, SG_F32 };
struct SkinnyGemm {
    const uint16_t *w;                 /* [R][K] bf16 */
    const uint16_t *x;                 /* [N][K] bf16 */
    int R, K, N;
    uint16_t *out;                     /* [N][R] bf16 (STORE, RESID2, RELU2, RESID) */
    float *out_f32;                    /* [N][R] fp32 (RESID2: the sum before rounding; F32) */
    const uint16_t *res;               /* [N][R] bf16 residual (RESID2, RESID) */
    const float *rstd;                 /* [N] (RELU2 without ssq) */
    const unsigned long long *active;  /* NULL, or the slots whose outputs are stored */
    float *ssq;                        /* NULL, or [N][ceil(R / 16)] (RESID2: written) / [N][ceil(K / 16)] (RELU2:
                                          read): each 16-row tile's sum of squares of the residual sum x; RELU2 then
                                          takes rstd = 1 / sqrt((sum over tiles in order) / K + FLT_EPSILON) from it
                                          (one slice only) */
};

/* slot_gemm.hip: the decode step's GEMM with every global access range-checked by buffer instructions. */
bool slot_gemm_fits(int R, int K, int N);
/* K-slices for (R, K): 1, or enough that each covers at most 2048 of K (fixed per shape, never per slot count). */
int slot_gemm_slices(int R, int K);
/* The workgroup tile a launch of (R, K, N, S) uses: 100 RT + CT (RT 16-row weight tiles, CT 16-slot tiles). */
int slot_gemm_tile(int R, int K, int N, int S);
/* Bytes of the partial sums of S slices (0 for S = 1). */
long long slot_gemm_part_bytes(int R, int N, int S);
/* S = 1: the epilogue in the GEMM. S > 1: fp32 partials to part [S][N][R] (part_bytes: its allocation, which must
 * hold them), summed by slot_gemm_reduce. Returns 0, a hipError_t, or -2 when the shape, S, the partial buffer or an
 * operand the epilogue needs does not fit. */
int slot_gemm(const SkinnyGemm &g, int epi, float *part, long long part_bytes, int S, hipStream_t stream);
int slot_gemm_reduce(const SkinnyGemm &g, int epi, const float *part, long long part_bytes, int S,
                     hipStream_t stream);
/* The fp32 partial sums of S >= 1 slices to part [S][N][R] (part_bytes must hold S N R floats), for a caller that
 * finishes the sum itself. */
int slot_gemm_partials(const SkinnyGemm &g, float *part, long long part_bytes, int S, hipStream_t stream);

/* prefill_gemm.hip: out[m][n] = epilogue(sum_k a[m][k] w[n][k]) for the rows of a prefill call, every output's sum in
 * one fixed order over K whatever M is. Epilogues SG_STORE, SG_RESID, SG_F32, SG_RELU2. Returns 0, a hipError_t, or -2
 * when the shape (K a multiple of 128, N of 4, every array under 2 GiB) or an operand the epilogue needs does not fit. */
struct PfGemm {
    const uint16_t *a;     /* [M][K] bf16 */
    const uint16_t *w;     /* [N][K] bf16 */
    int M, N, K;
    uint16_t *out;         /* [M][N] bf16 (SG_STORE, SG_RESID, SG_RELU2) */
    float *out_f32;        /* [M][N] fp32 (SG_F32) */
    const uint16_t *res;   /* [M][N] bf16 (SG_RESID) */
    const float *rstd;     /* [M] fp32 (SG_RELU2) */
};
int prefill_gemm(const PfGemm &g, int epi, hipStream_t stream);

}  // namespace nc
