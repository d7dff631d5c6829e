/*
 * pcp_sample.h — the rollout sampler on the GPU.
 *
 * Reference: Sampler.sample (src/core/math.zig:21-58), called once per generated
 * token by GenerationEngine.generateRolloutStreaming
 * (src/nodes/workers/generation_engine.zig:255-268) after a device-to-host copy of
 * the full logits row. Here the logits stay in HBM and only the token id comes back.
 *
 * The random stream stays the caller's: uniforms[r] is the value the reference draws
 * with self.prng.random().float(f32) for row r, so a Zig caller keeps its Sampler's
 * PRNG and passes the draws. Status codes and the context are those of pcp_grpo.h.
 */
#ifndef PCP_SAMPLE_H
#define PCP_SAMPLE_H

#include <stdint.h>

#include "pcp_grpo.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Largest vocabulary and batch per call. */
#define PCP_SAMPLE_MAX_VOCAB (1 << 20)
#define PCP_SAMPLE_MAX_ROWS 65535

/* For each row r < n_rows of logits (dtype PCP_F32 or PCP_BF16, row r at element
 * offset r * row_stride, device memory):
 *  - temperature < 1e-6: the index of the first maximum (math.zig:22-25, argmax
 *    :61-73; NaN never wins; a row with no value above -inf gives 0);
 *  - otherwise the first index i with sum_{j<=i} e_j >= uniforms[r] * sum_j e_j,
 *    e_j = exp((logit_j - max) / temperature) (:27-53); a NaN or +Inf logit, or a row
 *    of -Inf, makes the sum NaN and gives vocab - 1, the reference's fallback (:56).
 *    A NaN temperature is not below 1e-6, so it samples too, and every row gives
 *    vocab - 1 for the same reason; +Inf makes every finite term 1 (uniform draw).
 * 1 <= n_rows <= PCP_SAMPLE_MAX_ROWS. ids[r] receives the token (int64, device). uniforms (device, n_rows floats in
 * [0, 1)) may be NULL when temperature < 1e-6. The kernel sums in a fixed parallel
 * order, not the reference's sequential f32 loop, so a draw whose threshold lies
 * within f32 rounding of a cumulative boundary can pick the neighbouring token. */
int pcp_sample_tokens(pcp_ctx* ctx, const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                      int64_t row_stride, float temperature, const float* uniforms, int64_t* ids,
                      void* stream);
/* The same, enqueued only: one kernel launch on `stream` behind the work that produced
 * the logits (a decode step's forward), the token ids left in device memory, no host
 * synchronisation (as PCP_FLAG_ASYNC; pcp_sync waits for it). For the reference's one
 * sampled row per generated token (generation_engine.zig:255-268) without its
 * device-to-host copy of the row. Calls on one context use its per-row tickets: calls
 * that may overlap on different streams need separate contexts. */
int pcp_sample_tokens_async(pcp_ctx* ctx, const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                            int64_t row_stride, float temperature, const float* uniforms, int64_t* ids,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PCP_SAMPLE_H */
