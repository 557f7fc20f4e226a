/*
 * Launchers shared between the kernel files and the decoder runtime (decoder.hip), not part of the C ABI.
 * Arguments are checked by the caller.
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nc {

/* kv_append.hip: the fused QK-norm/RoPE fp8 append of n sequences of one token each; ve non-NULL adds the
 * value embedding 2 sigmoid(ve_gate[head] . ve_h[b]) ve[tokens[b]] to v before it is quantized (C: ve_h's width). */
int append_rows(const uint16_t *qkv, long long token_stride, int n, int Hq, int Hkv, const int32_t *pos,
                const int32_t *num_new, const int32_t *seq_slot, const float *q_gain, const float *k_gain,
                const float *cos, const float *sin, int rope_len, uint16_t *q_out, const int32_t *block_table,
                int max_pages, uint8_t *k_pages, uint8_t *v_pages, float *kv_scale, int num_pages,
                const uint16_t *ve_h, const uint16_t *ve, const float *ve_gate, const int32_t *tokens, int C,
                hipStream_t stream);

/* attention.hip: chunked prefill over runs of rows. */
int prefill_runs(const uint16_t *q, const uint8_t *k_pages, const uint8_t *v_pages, const float *kv_scale,
                 const int32_t *block_table, int max_pages, int num_pages, const int32_t *start_pos,
                 const int32_t *run_row0, const int32_t *run_count, const int32_t *run_slot, int runs, int max_count,
                 int Hq, int Hkv, int window, float sm_scale, uint16_t *out, hipStream_t stream);

}  // namespace nc
