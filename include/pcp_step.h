/*
 * pcp_step.h — the device-resident work around the GRPO loss head in one training
 * step: rollout packing, gradient statistics and the Nesterov parameter update.
 *
 * Reference: RLShepherd.trainStep (src/nodes/controllers/rl_shepherd.zig:460-687)
 * packs ids/mask on the host (:487-515), logs gradient statistics (:600-641) and
 * applies the host Nesterov optimizer (src/optimizers/nesterov.zig) to the master
 * weights, which are slices of one flat f32 weight file in tensor order
 * (loadWeightsFromFile, :141-229). Here the same data stays in HBM: master weights,
 * velocities and gradients are flat device buffers in that order.
 *
 * Status codes and the context are those of pcp_grpo.h. Pointers named dev_* or
 * documented as device pointers are HBM; `stream` is a hipStream_t (NULL: the
 * default stream). Calls are synchronous unless stated otherwise.
 */
#ifndef PCP_STEP_H
#define PCP_STEP_H

#include <stddef.h>
#include <stdint.h>

#include "pcp_grpo.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- rollout packing (rl_shepherd.zig:487-515) ------------------------------------
 * Row r < n_rollouts: prompt tokens then completion tokens of rollout r, truncated at
 * seq_len, into ids[r, :] (int64, zero-padded) with mask[r, :] = 1 over the filled
 * positions and 0 elsewhere. Rows n_rollouts <= r < n_rows are all zero (the
 * reference leaves missing rollouts of a group empty). Token arrays are
 * concatenated; rollout r's prompt is prompt_tokens[prompt_offsets[r] ..
 * prompt_offsets[r+1]) (device pointers; offsets are int64[n_rollouts + 1], token
 * arrays hold n_prompt_tokens / n_completion_tokens). Offsets that decrease or run
 * past their token array are reported as PCP_ERR_INVALID_ARG after the call (those
 * rollouts read nothing out of range and pack as empty). */
int pcp_pack_rollouts(pcp_ctx* ctx, const int64_t* prompt_tokens, int64_t n_prompt_tokens,
                      const int64_t* prompt_offsets, const int64_t* completion_tokens,
                      int64_t n_completion_tokens, const int64_t* completion_offsets, int64_t n_rollouts,
                      int64_t n_rows, int64_t seq_len, int64_t* ids, float* mask, void* stream);

/* ---- gradient statistics (rl_shepherd.zig:600-641) --------------------------------
 * Over n f32 gradients: NaN and Inf counts; over the finite ones the f64 sum of
 * squares and max |g| (starting at 0); l2_norm = sqrt(sumsq); elements counts all.
 * With accumulate != 0 the call adds to *stats (statistics over several tensors, as
 * the reference's loop over gradients), else it overwrites it. The f64 sum runs in a
 * fixed order (deterministic), not the reference's sequential one. */
typedef struct {
  double sumsq;
  double l2_norm;
  float max_abs;
  int64_t nan_count;
  int64_t inf_count;
  int64_t elements;
} pcp_grad_stats;

int pcp_grad_stats_compute(pcp_ctx* ctx, const float* grad, int64_t n, int accumulate, pcp_grad_stats* stats,
                           void* stream);

/* ---- Nesterov optimizer on HBM (src/optimizers/nesterov.zig) ---------------------- */
typedef enum {
  /* Host Nesterov used by RLShepherd (nesterov.zig:86-97), strict f32 rounding:
   *   v <- mu*v + g;   p <- p - lr*(g + mu*v)                                      */
  PCP_NESTEROV_SUTSKEVER = 0,
  /* NesterovMLIR.update (src/optimizers/nesterov_mlir.zig:93-99):
   *   v <- mu*v + lr*g;  p <- p - v                                                */
  PCP_NESTEROV_MLIR = 1
} pcp_nesterov_mode;

typedef struct pcp_nesterov pcp_nesterov;

/* ~ Nesterov.init + initParameters (nesterov.zig:21-54): zeroed velocities for
 * n_tensors tensors of counts[i] f32 elements, in one flat device allocation (tensor
 * i starts at counts[0] + ... + counts[i-1], the layout of the flat weight file). */
int pcp_nesterov_create(pcp_ctx* ctx, float learning_rate, float momentum, int mode, int n_tensors,
                        const int64_t* counts, pcp_nesterov** out);
/* ~ Nesterov.deinit (:31-38). NULL is a no-op. */
void pcp_nesterov_destroy(pcp_nesterov* opt);
/* ~ resetVelocity (:57-63). */
int pcp_nesterov_reset(pcp_nesterov* opt, void* stream);
/* ~ update(index, master_param, outer_gradient) (:70-98): param and grad are device
 * pointers to `count` f32 each. PCP_ERR_OUT_OF_BOUNDS when index >= n_tensors,
 * PCP_ERR_DIMENSION_MISMATCH when count differs from the tensor's. */
int pcp_nesterov_update(pcp_nesterov* opt, int index, float* param, const float* grad, int64_t count,
                        void* stream);
/* Every tensor in one launch: params and grads are flat device buffers laid out like
 * the velocities (total elements). param_bf16 (may be NULL) receives the updated
 * weights rounded to bf16 (nearest even) for the next bf16 forward, in the same pass.
 * No reference counterpart: the reference loops update() over the tensors. */
int pcp_nesterov_update_flat(pcp_nesterov* opt, float* params, const float* grads, void* param_bf16,
                             void* stream);
/* Total velocity elements and the serialized size in bytes (4 per element). */
int64_t pcp_nesterov_total(const pcp_nesterov* opt);
/* ~ serialize (:101-115): the velocities, tensor after tensor, into host memory of
 * at least pcp_nesterov_total(opt) * 4 bytes. */
int pcp_nesterov_serialize(pcp_nesterov* opt, void* host, size_t bytes);
/* ~ deserialize (:117-131): PCP_ERR_CORRUPT_STATE when bytes is too short; extra
 * bytes are ignored. */
int pcp_nesterov_deserialize(pcp_nesterov* opt, const void* host, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* PCP_STEP_H */
