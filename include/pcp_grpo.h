/*
 * pcp_grpo.h — C ABI of the MI355X (gfx950) GRPO loss-head library.
 *
 * This library replaces, for the GRPO training step of PCP, the IREE-compiled
 * loss head that the RL shepherd reaches through the worker backend:
 *
 *   RLShepherd.trainStep            src/nodes/controllers/rl_shepherd.zig:460-687
 *     -> IreeBackend.execute        src/backends/iree.zig:336-442
 *        (WorkerBackend vtable      src/backends/worker_backend.zig:7-62)
 *     -> VMFB "main": Qwen forward + loss (tools/export_qwen_forward.py:146-163)
 *        differentiated by src/compiler/graph_builder.zig:302-426.
 *
 * Two ways in:
 *   1. Host-bytes path (pcp_execute / pcp_free): mirrors WorkerBackend.executeFunction
 *      — borrowed host byte slices + i64 shapes + DType codes in, caller-owned
 *      output byte slices out. Synchronous.
 *   2. Device-pointer path (pcp_grpo_* with pcp_grpo_args): the caller owns HBM
 *      buffers (mirrors IreeBackend.executeWithDeviceBuffers, iree.zig:256-311).
 *      Synchronous on return unless PCP_FLAG_ASYNC is set.
 *
 * Every function returns PCP_OK (0) or a negative pcp_status; none aborts.
 * pcp_last_error() returns the message of the most recent failure on a context.
 * A context is not thread-safe (same contract as iree.zig:7). Calls on one context
 * run in stream order; calls that may overlap on different streams need separate
 * contexts (they share the context's work buffers and row counter).
 */
#ifndef PCP_GRPO_H
#define PCP_GRPO_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types, in the order of DType (src/core/tensor.zig:9-16); byte sizes as
 * DType.sizeInBytes (tensor.zig:50-60). */
typedef enum pcp_dtype {
  PCP_F16 = 0,
  PCP_BF16 = 1,
  PCP_F32 = 2,
  PCP_F64 = 3,
  PCP_I32 = 4,
  PCP_I64 = 5,
  PCP_BOOL = 6
} pcp_dtype;

/* Backend kinds, in the order of Backend (src/backends/selection.zig:32-38).
 * This library implements PCP_BACKEND_ROCM only. */
typedef enum pcp_backend {
  PCP_BACKEND_METAL = 0,
  PCP_BACKEND_CUDA = 1,
  PCP_BACKEND_VULKAN = 2,
  PCP_BACKEND_ROCM = 3,
  PCP_BACKEND_CPU = 4
} pcp_backend;

typedef enum pcp_status {
  PCP_OK = 0,
  PCP_ERR_INVALID_ARG = -1,      /* null pointer, bad rank/shape, bad enum value      */
  PCP_ERR_DTYPE = -2,            /* dtype not supported for that operand              */
  PCP_ERR_TOKEN_RANGE = -3,      /* a live token id outside [0, V) and != -100         */
  PCP_ERR_NONFINITE = -4,        /* a live row has a non-finite log-sum-exp            */
  PCP_ERR_OOM = -5,              /* device or host allocation failed                  */
  PCP_ERR_DEVICE = -6,           /* HIP runtime error (iree.zig:26-36 analogue)        */
  PCP_ERR_UNKNOWN_FUNCTION = -7, /* pcp_execute: no such function name                */
  PCP_ERR_COUNT_MISMATCH = -8,   /* pcp_execute: wrong number of inputs
                                    (rl_shepherd.zig:601-604 analogue)                */
  PCP_ERR_OVERFLOW = -9,         /* size computation overflows int64 / byte counts     */
  PCP_ERR_UNSUPPORTED = -10,     /* valid request this build does not implement        */
  PCP_ERR_OUT_OF_BOUNDS = -11,   /* tensor index past the optimizer's tensors (nesterov.zig:72)  */
  PCP_ERR_DIMENSION_MISMATCH = -12, /* element counts differ (nesterov.zig:73-76)        */
  PCP_ERR_CORRUPT_STATE = -13,   /* serialized state or file too short (nesterov.zig:124,
                                    rl_shepherd.zig:199 WeightFileTooSmall, EndOfStream)  */
  PCP_ERR_IO = -14               /* a file could not be opened, read or written        */
} pcp_status;

/* Loss definitions for the per-token term l_t (aggregation is identical):
 *   loss = (1/loss_norm) * sum_s [ sum_t m_{s,t} * l_{s,t} ] / max(sum_t m_{s,t}, 1)
 *
 * PCP_LOSS_REINFORCE: the reference graph, tools/export_qwen_forward.py:150-163:
 *     l_t = -A_s * logp_t   (token_losses = cross_entropy * mask; seq mean; * adv; mean)
 * PCP_LOSS_GRPO_CLIP_KL: clipped-ratio surrogate + k3 KL (no reference counterpart):
 *     rho = exp(logp - old_logp)
 *     l_t = -min(rho*A, clip(rho, 1-eps, 1+eps)*A) + beta*(exp(ref-logp) - (ref-logp) - 1)
 * dlogits[row, v] = c_t * (onehot(id_t)[v] - softmax(row)[v]),  c_t = d loss / d logp_t.
 */
typedef enum pcp_loss_mode {
  PCP_LOSS_REINFORCE = 0,
  PCP_LOSS_GRPO_CLIP_KL = 1
} pcp_loss_mode;

/* pcp_grpo_args.flags */
#define PCP_FLAG_ASYNC 0x1u            /* return after enqueueing; errors surface in pcp_sync */
#define PCP_FLAG_NO_ZERO_FILL 0x2u     /* leave dlogits rows of masked / pad tokens untouched
                                          (ids and mask must not change while the call runs:
                                          a row first listed live and then found dead fails
                                          the call with PCP_ERR_INVALID_ARG)                  */
#define PCP_FLAG_FORCE_STREAMING 0x4u  /* use the two-read streaming kernel even when the
                                          register-resident one fits (testing / comparison);
                                          on pcp_grpo_lmhead_fwd_bwd with a vocab_chunk: the
                                          chunked backward's low-memory form (K-major
                                          operands, no transposed copies)                    */
/* bf16 logits -> bf16 dlogits: every output is the f32 result rounded once to nearest
 * even. By default the resident kernel keeps the softmax terms of the sum pass as f16
 * (unit roundoff 2^-11) and scales them into dlogits, which saves one exponential per
 * element (3-5% of the step at configs 2-4) and adds, before the bf16 rounding, up to
 * 2^-11 of |dlogit| plus 2^-25 * |c| (terms below f16's normal range). On
 * pcp_grpo_lmhead_fwd_bwd the forward keeps its softmax terms as f32 instead of f16,
 * so the bf16 dlogits operand of the backward is likewise the f32 value rounded once
 * (about twice the backward workspace). */
#define PCP_FLAG_EXACT_BF16 0x8u

/* The token id that contributes nothing (F.cross_entropy ignore_index; the
 * "compare NE -100" select in models/tests/qwen_test.mlir:267-280). */
#define PCP_IGNORE_INDEX (-100)
/* Largest vocab of the logits entry points: 2^31 - 2^20, so every per-row index, one
 * batch past the row end, stays a 32-bit integer. */
#define PCP_GRPO_MAX_VOCAB ((int64_t)2147483648 - 1048576)

typedef struct pcp_ctx pcp_ctx;

/*
 * Device-pointer arguments. All pointers are device (HBM) addresses.
 *
 * Row layout. There are n_seq sequences. Sequence s owns logits rows
 *   [s*logit_seq_stride, (s+1)*logit_seq_stride)  of the [*, vocab] matrices.
 * The first `rows` of them carry a token: row (s, t), t < rows, scores token
 *   ids[s*tok_seq_stride + tok_offset + t]
 * with weight mask[same index] and old_logp[same index]. Rows t >= rows are pad
 * rows: their dlogits are zero-filled. The reference's shifted view
 * (logits[:, :-1] vs input_ids[:, 1:], export_qwen_forward.py:150-152) is
 *   rows = T-1, logit_seq_stride = T, tok_seq_stride = T, tok_offset = 1.
 * The aligned layout is rows = T, strides 0 (meaning "= rows"), tok_offset = 0.
 *
 * Per-token outputs (logp, ref_logp, token_loss) use the token indexing of ids;
 * entries that no row addresses are not written.
 */
typedef struct pcp_grpo_args {
  int64_t n_seq;            /* S = prompts * group_size                                 */
  int64_t rows;             /* token-carrying rows per sequence                          */
  int64_t vocab;            /* V, 1 .. PCP_GRPO_MAX_VOCAB                                */
  int64_t group_size;       /* consecutive sequences per group (advantages); >= 1        */
  int64_t logit_seq_stride; /* rows between sequences in logits/dlogits; 0 => rows       */
  int64_t tok_seq_stride;   /* elements between sequences in ids/mask/...; 0 => rows     */
  int64_t tok_offset;       /* token index of row t is tok_offset + t                    */

  int32_t logits_dtype;     /* PCP_BF16 | PCP_F16 | PCP_F32 (ref_logits: same)            */
  int32_t dlogits_dtype;    /* PCP_BF16 | PCP_F16 | PCP_F32; must be logits_dtype or F32  */
  int32_t ids_dtype;        /* PCP_I64 | PCP_I32                                          */
  int32_t mask_dtype;       /* PCP_F32 | PCP_BOOL (u8); ignored when mask == NULL         */

  const void* logits;       /* [n_seq*logit_seq_stride, V] policy logits                 */
  const void* ref_logits;   /* same shape; required for PCP_LOSS_GRPO_CLIP_KL, optional
                               for logprob_fwd, unused by PCP_LOSS_REINFORCE              */
  const void* ids;          /* token ids                                                  */
  const void* mask;         /* token weights (0/1); NULL => all ones                      */
  const float* old_logp;    /* behaviour-policy log-probs; NULL => on-policy (rho = 1)    */
  const float* advantages;  /* [n_seq]; NULL => computed from rewards                     */
  const float* rewards;     /* [n_seq]; used only when advantages == NULL                 */

  void* dlogits;            /* [n_seq*logit_seq_stride, V]; NULL => forward only          */
  float* logp;              /* optional per-token outputs                                 */
  float* ref_logp;
  float* token_loss;        /* m_t * l'_t (l' = -logp in REINFORCE, l_t in CLIP_KL)      */
  float* advantages_out;    /* optional [n_seq]: the advantages used                      */
  float* loss;              /* optional device scalar                                     */

  int32_t loss_mode;        /* pcp_loss_mode                                              */
  float clip_eps;           /* e.g. 0.2                                                   */
  float kl_beta;            /* e.g. 0.04                                                  */
  float std_eps;            /* added to the group std (rl_shepherd.zig:474): 1e-8        */
  float loss_norm;          /* divisor of the sequence sum; 0 => n_seq (.mean())          */
  uint32_t flags;           /* PCP_FLAG_*                                                 */
  void* stream;             /* hipStream_t; NULL => the default stream                    */
} pcp_grpo_args;

/* Fill *a with defaults: strides 0, offset 0, dtypes bf16/bf16/i64/f32, eps 0.2,
 * beta 0.04, std_eps 1e-8, loss_norm 0, REINFORCE, flags 0. */
void pcp_grpo_args_init(pcp_grpo_args* a);

/* ~ IreeBackend.init(allocator, .rocm, device_id)  (src/backends/iree.zig:84).
 * backend must be PCP_BACKEND_ROCM. */
int pcp_init(int backend, int device_ordinal, pcp_ctx** out);
/* ~ IreeBackend.deinit / WorkerBackend.deinit (worker_backend.zig:37). NULL is a no-op. */
void pcp_destroy(pcp_ctx* ctx);
/* ~ WorkerBackend.getBackendType (worker_backend.zig:34). */
int pcp_get_backend_type(const pcp_ctx* ctx);
/* Message of the last failure on ctx (iree_status_fprint analogue, iree.zig:26-36). */
const char* pcp_last_error(const pcp_ctx* ctx);
/* Wait for work enqueued with PCP_FLAG_ASYNC; returns the first device-side error. */
int pcp_sync(pcp_ctx* ctx);
/* Free the context's grow-only device work buffers: the per-call scratch and the
 * LM-head backward workspace (the softmax cache: 11.3 GB at 16,384 tokens, V =
 * 151,936, H = 4,096; 21.4 GB with PCP_FLAG_EXACT_BF16), which otherwise stay held
 * until pcp_destroy. Synchronises the device first (every stream: calls enqueued with
 * PCP_FLAG_ASYNC may still use the buffers). The next call allocates again. No
 * counterpart in the reference (IREE holds its own device pools). */
int pcp_release_workspace(pcp_ctx* ctx);
/* Bytes of device work buffers the context holds now (0 for NULL). */
size_t pcp_workspace_bytes(const pcp_ctx* ctx);

/*
 * Host-bytes path. ~ WorkerBackend.executeFunction (worker_backend.zig:27-33),
 * IreeBackend.execute (iree.zig:336-442). `fn` names one of:
 *
 *  "grpo_loss_fwd_bwd"
 *     the reference loss head: in  (logits[G,T,V] bf16|f16|f32, input_ids[G,T] i64|i32,
 *                                   attention_mask[G,T] f32|bool, advantages[G] f32)
 *                              out (loss f32[], dlogits[G,T,V] logits dtype)
 *  "main" (executeTrainingStep's name, iree.zig:463-486) is the training VMFB's whole
 *     step, [params..., buffers..., ids, mask, adv] -> parameter gradients
 *     (graph_builder.zig:302-426, rl_shepherd.zig:529-604). This library holds only its
 *     loss head, so "main" returns PCP_ERR_UNSUPPORTED with a message naming the split:
 *     the model forward to logits, "grpo_loss_fwd_bwd", the model backward from dlogits.
 *  "grpo_clip_kl_fwd_bwd"
 *     in  (logits[S,T,V], ref_logits[S,T,V], input_ids[S,T], attention_mask[S,T],
 *          old_logp f32[S,T], rewards f32[S], hyper f32[4] = {group_size, clip_eps,
 *          kl_beta, loss_norm (0 => S)})
 *     out (loss f32[], dlogits[S,T,V], logp f32[S,T], ref_logp f32[S,T], advantages f32[S])
 *  "grpo_logprob_fwd"
 *     in  (logits[S,T,V], input_ids[S,T])  or  (logits, ref_logits, input_ids)
 *     out (logp f32[S,T]) or (logp, ref_logp)
 *  "grpo_advantages"
 *     in  (rewards f32[n], group_size i64[])   out (advantages f32[n])
 *  "grpo_lmhead_fwd_bwd"  (the LM head + loss of export_qwen_forward.py:146-163)
 *     in  (hidden bf16[S,T,H], weight bf16[V,H], ref_weight bf16[V,H], input_ids[S,T],
 *          attention_mask[S,T], old_logp f32[S,T], rewards f32[S], hyper f32[5] =
 *          {group_size, clip_eps, kl_beta, loss_norm (0 => S), loss_mode (0|1)})
 *     out (loss f32[], dhidden f32[S,T,H], dweight f32[V,H], logp f32[S,T],
 *          ref_logp f32[S,T], advantages f32[S]); ref_weight is read in mode 1 only.
 *     A ninth input norm_weight f32[H] fuses the decoder's final RMSNorm
 *     (pcp_lmhead_args.norm_weight; hyper may then be f32[6] with norm_eps last,
 *     1e-6 otherwise): hidden is the last layer's output, dhidden the gradient there,
 *     and a seventh output is dnorm_weight f32[H].
 *
 * All [.,T,V] and [.,T,H] functions use the reference's shift: row t scores token t+1,
 * per-token outputs are indexed by token position (position 0 is 0).
 * dtypes == NULL selects each function's default dtypes (f32 floats, i64 ids).
 * On success *out_data[i] (*out_nbytes[i] bytes of host memory) belong to the caller
 * until pcp_free, which releases everything: outputs of 4 MiB and more are pinned
 * buffers that pcp_free returns to a process-wide pool for later calls (up to 64 GiB
 * kept), smaller ones are malloc'd. Inputs of 4 MiB and more are staged to the device
 * through a pinned ring of the context, filled by up to 8 host threads. The loss
 * functions on logits of two groups or more (PCP_EXECUTE_GROUP_MIB of policy logits
 * per group, default 1024) run group by group, with the upload of later groups, the
 * kernels and the download of earlier groups' dlogits overlapping; the results are
 * those of one call.
 */
int pcp_execute(pcp_ctx* ctx, const char* fn, int n_in, const void* const* data,
                const size_t* nbytes, const int64_t* const* shapes, const int* ranks,
                const int* dtypes, int* n_out, void*** out_data, size_t** out_nbytes);
/* ~ rl_shepherd.zig:595,680 freeing every output slice and the outer slice. */
void pcp_free(pcp_ctx* ctx, int n_out, void** out_data, size_t* out_nbytes);

/*
 * Device-pointer path.
 */
/* a1: per-token log-softmax + sampled-token gather for policy (and ref if given).
 * export_qwen_forward.py:154-156 / qwen_test.mlir:257-277 (returns logp, not -logp). */
int pcp_grpo_logprob_fwd(pcp_ctx* ctx, const pcp_grpo_args* a);
/* a3: group-relative advantages, bit-exact with rl_shepherd.zig:462-479.
 * rewards, adv: device f32 [n]; groups are consecutive blocks of group_size (the
 * last may be partial, as @min(i+group_size, len) there). */
int pcp_grpo_advantages(pcp_ctx* ctx, const float* rewards, int64_t n, int64_t group_size,
                        float std_eps, float* adv, void* stream);
/* a2+a4+a5 fused: logprobs, loss and (if dlogits != NULL) the dlogits backward in one
 * streaming pass per row; replaces the loss head + its AD backward inside the VMFB
 * (graph_builder.zig:302-426). */
int pcp_grpo_loss_fwd_bwd(pcp_ctx* ctx, const pcp_grpo_args* a);

/* Allocation-free variant of pcp_grpo_loss_fwd_bwd. It has no counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Same arguments, results and
 * error codes as pcp_grpo_loss_fwd_bwd, but it calls no hipMalloc / hipFree and makes
 * no host allocation. Its work buffers (advantages, per-sequence lengths and sums, the
 * loss, the row kernel's counter and, when a->token_loss is NULL, the per-token
 * losses) live in one static device array of PCP_NOALLOC_SCRATCH_BYTES per GPU, which
 * that GPU holds until the process ends. A request needing more than the array,
 *   4*round256(4*n_seq) + 512 + (token_loss ? 0 : round256(4*n_seq*tok_seq_stride))
 *     + (PCP_FLAG_NO_ZERO_FILL and dlogits ? round256(4*n_seq*logit_seq_stride) : 0),
 * fails with PCP_ERR_OVERFLOW before any device work; passing token_loss removes the
 * per-token part. Every call on one GPU shares that GPU's array, which keeps the last
 * call's contents: calls that may overlap on one GPU (other streams or contexts) race
 * and must be ordered by the caller. */
#define PCP_NOALLOC_SCRATCH_BYTES (4u << 20)
int pcp_grpo_loss_fwd_bwd_noalloc(pcp_ctx* ctx, const pcp_grpo_args* a);

/*
 * a6: fused LM-head + GRPO loss (the LM head of tools/export_qwen_forward.py:146-147
 * and its VJP, src/autodiff/vjp_rules.zig:426-497). Tokens use the aligned layout:
 * token t of sequence s is row s*rows + t of hidden_states and scores ids[s*rows+t].
 * logits = hidden_states * weight^T are computed in 256 x 256 tiles on bf16 MFMA and
 * reduced in-tile (per-token log-sum-exp and target logit); full f32 logits are never
 * stored. By default (vocab_chunk 0) the policy forward also keeps its softmax terms
 * as f16 (one 2-byte term per live token and vocab entry), the backward turns them into
 * bf16 dlogits and runs dhidden = dlogits * weight and dweight = dlogits^T *
 * hidden_states (fp32) over the whole vocabulary. The f16 term adds to an off-target
 * dlogit, before its bf16 rounding, at most 2^-11 of |c * softmax| (terms in f16's
 * normal range) plus 2^-25 * |c| * 2^(m_b - lse) (terms below it; m_b = the largest
 * logit of the entry's 128-entry block): PCP_FLAG_EXACT_BF16 keeps the terms as f32
 * (4 bytes per live token and vocab entry), so each dlogit is the f32 value rounded
 * once. The backward workspace (softmax cache, dlogits^T, weight^T; 11.3 GB at 16,384
 * tokens, V = 151,936, H = 4,096) is allocated when it fits the budget: at most 64 GiB
 * and at most half of the device memory free at the call plus what the context holds.
 * It stays held until pcp_release_workspace or pcp_destroy; growing it synchronises
 * the device (PCP_FLAG_ASYNC calls included) before freeing the smaller buffer. With an
 * explicit vocab_chunk, or a workspace above the budget, the backward recomputes the
 * logit tiles per vocab chunk instead (dlogits = the f32 value rounded once): with a
 * transposed copy of the chunk and of the weight (2 * (2 * tokens * chunk + hidden *
 * vocab) bytes, within the same budget), or, when that does not fit, in memory
 * bounded by the chunk alone (2 * tokens * chunk bytes).
 * The live-token count never leaves the device: with PCP_FLAG_ASYNC the call only
 * enqueues work, and it can be captured in a HIP graph. A captured graph uses the
 * context's work buffers as they were at capture: make one uncaptured call of the same
 * (or larger) sizes first, and re-capture after any call on the context that needed
 * larger buffers (growing them frees the old ones).
 */
typedef struct pcp_lmhead_args {
  int64_t n_seq;              /* sequences                                                */
  int64_t rows;               /* tokens per sequence                                      */
  int64_t hidden;             /* H; multiple of 64                                        */
  int64_t vocab;              /* V                                                        */
  int64_t group_size;         /* sequences per advantage group                            */
  int64_t vocab_chunk;        /* 0: softmax cache (see above); else the recomputing
                                 backward's chunk width (a multiple of 256)               */
  int32_t ids_dtype;          /* PCP_I64 | PCP_I32                                        */
  int32_t mask_dtype;         /* PCP_F32 | PCP_BOOL                                       */
  const void* hidden_states;  /* [n_seq*rows, H] bf16                                     */
  const void* weight;         /* [V, H] bf16 (policy LM head)                             */
  const void* ref_weight;     /* [V, H] bf16; required for PCP_LOSS_GRPO_CLIP_KL          */
  const void* ids;            /* [n_seq*rows]                                             */
  const void* mask;           /* [n_seq*rows] or NULL (all ones)                          */
  const float* old_logp;      /* [n_seq*rows] or NULL (on-policy)                         */
  const float* advantages;    /* [n_seq] or NULL (from rewards)                           */
  const float* rewards;       /* [n_seq]                                                  */
  float* logp;                /* optional [n_seq*rows] outputs                            */
  float* ref_logp;
  float* token_loss;
  float* advantages_out;      /* optional [n_seq]                                         */
  float* loss;                /* optional device scalar                                   */
  float* dhidden;             /* [n_seq*rows, H] f32, or NULL                             */
  float* dweight;             /* [V, H] f32, or NULL                                      */
  int32_t loss_mode;
  float clip_eps;
  float kl_beta;
  float std_eps;
  float loss_norm;            /* 0 => n_seq                                               */
  uint32_t flags;             /* PCP_FLAG_ASYNC | PCP_FLAG_EXACT_BF16                     */
  void* stream;
  /* The decoder's final RMSNorm (Qwen2RMSNorm: the model.norm that
   * tools/export_qwen_forward.py:112 applies before lm_head), fused at both ends. With
   * norm_weight set, hidden_states are the last decoder layer's output h (bf16), the
   * LM head's operand is bf16(norm_weight * bf16(h * rsqrt(mean(h^2) + norm_eps))) and
   * dhidden receives dL/dh, the gradient the last block's VJP takes. hidden <= 8192;
   * norm_weight and dhidden 16-byte aligned. */
  const float* norm_weight;   /* [H] f32, or NULL (hidden_states are the LM-head input)   */
  float* dnorm_weight;        /* [H] f32 gradient of norm_weight, or NULL                 */
  float norm_eps;             /* Qwen2: 1e-6                                              */
} pcp_lmhead_args;

/* Defaults as pcp_grpo_args_init (ids i64, mask f32, eps 0.2, beta 0.04, std_eps 1e-8;
 * norm_eps 1e-6). */
void pcp_lmhead_args_init(pcp_lmhead_args* a);
/* Forward loss (+ logp / ref logp / token losses) and, when dhidden / dweight are
 * given, their gradients. */
int pcp_grpo_lmhead_fwd_bwd(pcp_ctx* ctx, const pcp_lmhead_args* a);

/*
 * Kernel timing (no reference counterpart: the reference never times its step).
 * Between pcp_profile_start and pcp_profile_stop, every row-kernel launch of
 * pcp_grpo_loss_fwd_bwd / pcp_grpo_logprob_fwd, the policy forward-tile launch of
 * pcp_grpo_lmhead_fwd_bwd, the kernels of pcp_sample_tokens and the launch of
 * pcp_nesterov_update_flat are bracketed by HIP events recorded on the launch stream
 * (at most max_launches launches are recorded). Stop
 * synchronises those events and returns the count and the summed kernel time.
 */
int pcp_profile_start(pcp_ctx* ctx, int max_launches);
int pcp_profile_stop(pcp_ctx* ctx, int* n_launches, double* total_ms);

/* Library version string. */
const char* pcp_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PCP_GRPO_H */
