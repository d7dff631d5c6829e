// Host-side launch interface of the GRPO kernels (implemented in grpo_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pcp {

struct RowArgs;

// Which row kernel serves a request.
struct RowPlan {
  enum Kind { kResident = 0, kStreamVec = 1, kStreamScalar = 2, kForward = 3 };
  int kind;
  int cfg;    // resident configuration index
  int block;  // lanes per workgroup
  int nch;    // resident 16-byte chunks per lane
  int edge;   // resident rows off 16 bytes (head / tail element-wise)
  int exact;  // bf16 -> bf16 resident rows without the f16 softmax cache (PCP_FLAG_EXACT_BF16)
};

// in_bytes: logits element size; aligned16: every row base is 16-byte aligned;
// edge_ok: dlogits (if any) have the logits' element type and the same address mod 16,
// so rows off 16 bytes split alike; forward_only: no dlogits are written.
RowPlan plan_rows(int in_bytes, int64_t vocab, bool aligned16, bool edge_ok, bool forward_only, bool force_stream);

hipError_t launch_rows(const RowPlan& p, int in_dtype, int out_dtype, const RowArgs& a,
                       int64_t nrows, hipStream_t st);
hipError_t launch_seq_prep(const void* mask, int mask_u8, int64_t n_seq, int64_t rows,
                           int64_t tok_stride, int64_t tok_offset, float loss_norm,
                           float* seq_len, float* seq_scale, hipStream_t st);
hipError_t launch_advantages(const float* r, int64_t n, int64_t group, float eps, float* adv,
                             hipStream_t st);
hipError_t launch_loss_reduce(const float* token_loss, int64_t n_seq, int64_t rows,
                              int64_t tok_stride, int64_t tok_offset, const float* seq_len,
                              const float* adv, int reinforce, float loss_norm, float* seq_val,
                              float* loss, hipStream_t st);

// One launch before the row kernel: per-sequence lengths and loss scales (as
// launch_seq_prep), the group advantages (as launch_advantages, when rewards is set)
// or a copy of the given ones into adv_out, and up to three counters zeroed.
struct StepPrepArgs {
  const void* mask;       // nullptr: all ones
  int32_t mask_u8;
  int64_t n_seq, rows, tok_stride, tok_offset;
  float loss_norm;
  float* seq_len;
  float* seq_scale;
  const float* rewards;   // nullptr: the advantages are given (adv_in)
  const float* adv_in;
  int64_t group;
  float std_eps;
  float* adv;             // the computed advantages (rewards set)
  float* adv_out;         // optional copy of the advantages used
  int* zero[3];           // optional counters set to 0
};
hipError_t launch_step_prep(const StepPrepArgs& a, hipStream_t st);

// The loss in one launch (seq_loss_kernel + loss_final_kernel, the same summation
// order): done must be 0 at the launch (step_prep_kernel zeroes it) and is left 0.
struct LossReduceArgs {
  const float* token_loss;
  int64_t rows, tok_stride, tok_offset;
  const float* seq_len;
  const float* adv;
  int32_t reinforce;
  float* seq_val;         // [n_seq] work
  int64_t n_seq;
  float loss_norm;
  int* done;
  float* loss;
};
hipError_t launch_loss_reduce_fused(const LossReduceArgs& a, hipStream_t st);

}  // namespace pcp
