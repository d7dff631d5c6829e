// Device-pointer entry points of the C ABI: context lifetime, argument
// validation and the launch sequence of the GRPO loss head.
//
// Mirrors the device-resident half of IreeBackend (src/backends/iree.zig:84,
// :166-333): the caller owns HBM buffers; the library owns only small scratch
// (advantages, per-sequence lengths and sums, per-token losses, error word).

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <mutex>

#include "context.hpp"
#include "host_transfer.hpp"
#include "grpo_device.hpp"
#include "grpo_launch.hpp"
#include "pcp_grpo.h"

namespace pcp {

char* thread_error() {
  static thread_local char msg[kErrLen];
  return msg;
}

int add_pending(pcp_ctx* ctx, hipStream_t st) {
  for (int i = 0; i < ctx->n_pending; ++i)
    if (ctx->pending[i] == st) return PCP_OK;
  if (ctx->n_pending < pcp_ctx::kMaxPending) {
    ctx->pending[ctx->n_pending++] = st;
    return PCP_OK;
  }
  hipError_t e = hipStreamSynchronize(st);
  return e == hipSuccess ? PCP_OK : hip_fail(ctx, e, "hipStreamSynchronize");
}

int ensure_scratch(pcp_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->scratch_bytes) return PCP_OK;
  if (ctx->scratch) {
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_fail(ctx, e, "hipDeviceSynchronize");
    (void)hipFree(ctx->scratch);
    ctx->scratch = nullptr;
    ctx->scratch_bytes = 0;
  }
  const size_t want = (bytes + 0xFFFFF) & ~static_cast<size_t>(0xFFFFF);
  hipError_t e = hipMalloc(&ctx->scratch, want);
  if (e != hipSuccess) {
    ctx->scratch = nullptr;
    (void)hipGetLastError();
    return fail(ctx, PCP_ERR_OOM, "hipMalloc(%zu bytes of scratch) failed: %s", want,
                hipGetErrorString(e));
  }
  ctx->scratch_bytes = want;
  return PCP_OK;
}

int collect_device_errors(pcp_ctx* ctx) {
  int h = 0;
  hipError_t e = hipMemcpy(&h, ctx->d_err, sizeof(int), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(ctx, e, "reading the device error word");
  if (h == 0) return PCP_OK;
  const int zero = 0;
  e = hipMemcpy(ctx->d_err, &zero, sizeof(int), hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(ctx, e, "clearing the device error word");
  if (h & kErrTokenRange)
    return fail(ctx, PCP_ERR_TOKEN_RANGE, "a live token id is outside [0, vocab) and is not -100");
  if (h & kErrBadRagged)
    return fail(ctx, PCP_ERR_INVALID_ARG, "rollout offsets decrease or run past the token array");
  if (h & kErrListedRow)
    return fail(ctx, PCP_ERR_INVALID_ARG, "a row listed as live was not live in the row kernel (ids or mask "
                                          "changed during the call)");
  if (h & kErrBadBase64)
    return fail(ctx, PCP_ERR_INVALID_ARG, "base64 text has a character outside the alphabet or misplaced padding "
                                          "(InvalidCharacter / InvalidPadding)");
  return fail(ctx, PCP_ERR_NONFINITE, "a live row has a non-finite log-sum-exp (NaN/Inf logits)");
}

// Work buffers of pcp_grpo_loss_fwd_bwd_noalloc: one array per GPU, which holds it
// until the process ends. Host code never passes this name to a kernel (on the host it
// is only a stand-in for the symbol): pcp_init resolves the device address of each
// GPU's copy with hipGetSymbolAddress and the entry point uses that address.
static __device__ __align__(256) unsigned char scratch[PCP_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this GPU's scratch array; the caller has made `device` current.
int resolve_noalloc_scratch(int device, void** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices)
    return fail(nullptr, PCP_ERR_UNSUPPORTED, "device ordinal %d: the allocation-free path serves ordinals < %d",
                device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      return fail(nullptr, PCP_ERR_DEVICE, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    }
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return PCP_OK;
}

// Resolved geometry of a request.
struct Geo {
  int64_t n_seq, rows, vocab, group, lstride, tstride, toff, nrows;
  float loss_norm;
};

enum Op { kLogprob = 0, kLoss = 1 };

int validate(const pcp_grpo_args* a, Op op, Geo* g) {
  if (!a) return fail(nullptr, PCP_ERR_INVALID_ARG, "args is NULL");
  if (a->n_seq < 1) return fail(nullptr, PCP_ERR_INVALID_ARG, "n_seq must be >= 1 (got %lld)", (long long)a->n_seq);
  if (a->rows < 0) return fail(nullptr, PCP_ERR_INVALID_ARG, "rows must be >= 0");
  if (a->vocab < 1 || a->vocab > PCP_GRPO_MAX_VOCAB)
    return fail(nullptr, PCP_ERR_INVALID_ARG, "vocab must be in [1, 2^31 - 2^20] (got %lld)", (long long)a->vocab);
  if (a->group_size < 1) return fail(nullptr, PCP_ERR_INVALID_ARG, "group_size must be >= 1");
  g->n_seq = a->n_seq;
  g->rows = a->rows;
  g->vocab = a->vocab;
  g->group = a->group_size;
  g->lstride = a->logit_seq_stride ? a->logit_seq_stride : a->rows;
  g->tstride = a->tok_seq_stride ? a->tok_seq_stride : a->rows;
  g->toff = a->tok_offset;
  if (g->lstride < g->rows || g->lstride < 1)
    return fail(nullptr, PCP_ERR_INVALID_ARG, "logit_seq_stride (%lld) must be >= max(rows, 1)", (long long)g->lstride);
  if (g->toff < 0 || g->toff + g->rows > g->tstride)
    return fail(nullptr, PCP_ERR_INVALID_ARG, "tok_offset + rows must fit in tok_seq_stride");
  int64_t tmp;
  if (mul_overflows(g->n_seq, g->lstride, &g->nrows) || g->nrows > INT32_MAX)
    return fail(nullptr, PCP_ERR_OVERFLOW, "n_seq * logit_seq_stride exceeds 2^31-1 rows");
  if (mul_overflows(g->nrows, g->vocab, &tmp) || mul_overflows(tmp, 4, &tmp))
    return fail(nullptr, PCP_ERR_OVERFLOW, "logits byte size overflows int64");
  if (mul_overflows(g->n_seq, g->tstride, &tmp))
    return fail(nullptr, PCP_ERR_OVERFLOW, "token array size overflows int64");
  if (a->logits_dtype != PCP_BF16 && a->logits_dtype != PCP_F16 && a->logits_dtype != PCP_F32)
    return fail(nullptr, PCP_ERR_DTYPE, "logits dtype must be bf16, f16 or f32 (got %d)", a->logits_dtype);
  if (a->ids_dtype != PCP_I64 && a->ids_dtype != PCP_I32)
    return fail(nullptr, PCP_ERR_DTYPE, "ids dtype must be i64 or i32 (got %d)", a->ids_dtype);
  if (a->mask && a->mask_dtype != PCP_F32 && a->mask_dtype != PCP_BOOL)
    return fail(nullptr, PCP_ERR_DTYPE, "mask dtype must be f32 or bool (got %d)", a->mask_dtype);
  if (!a->logits) return fail(nullptr, PCP_ERR_INVALID_ARG, "logits is NULL");
  if (!a->ids && g->rows > 0) return fail(nullptr, PCP_ERR_INVALID_ARG, "ids is NULL");
  {
    // Rows may start anywhere, but each element on its own size.
    const uintptr_t m = static_cast<uintptr_t>(dtype_bytes(a->logits_dtype)) - 1;
    const uintptr_t md = a->dlogits && op == kLoss ? static_cast<uintptr_t>(dtype_bytes(a->dlogits_dtype)) - 1 : 0;
    if ((reinterpret_cast<uintptr_t>(a->logits) & m) || (reinterpret_cast<uintptr_t>(a->ref_logits) & m) ||
        (op == kLoss && (reinterpret_cast<uintptr_t>(a->dlogits) & md)))
      return fail(nullptr, PCP_ERR_INVALID_ARG, "logits / ref_logits / dlogits must be aligned to their element size");
  }
  if (op == kLoss) {
    if (a->dlogits) {
      if (a->dlogits_dtype != a->logits_dtype && a->dlogits_dtype != PCP_F32)
        return fail(nullptr, PCP_ERR_DTYPE, "dlogits dtype must equal the logits dtype or be f32");
    }
    if (a->loss_mode != PCP_LOSS_REINFORCE && a->loss_mode != PCP_LOSS_GRPO_CLIP_KL)
      return fail(nullptr, PCP_ERR_INVALID_ARG, "unknown loss_mode %d", a->loss_mode);
    if (a->loss_mode == PCP_LOSS_GRPO_CLIP_KL && !a->ref_logits)
      return fail(nullptr, PCP_ERR_INVALID_ARG, "GRPO_CLIP_KL needs ref_logits");
    if (!a->advantages && !a->rewards)
      return fail(nullptr, PCP_ERR_INVALID_ARG, "advantages and rewards are both NULL");
    if (!(a->clip_eps >= 0.f && a->clip_eps < 1.f))
      return fail(nullptr, PCP_ERR_INVALID_ARG, "clip_eps must be in [0, 1)");
    if (!(a->loss_norm >= 0.f)) return fail(nullptr, PCP_ERR_INVALID_ARG, "loss_norm must be >= 0");
  }
  g->loss_norm = a->loss_norm > 0.f ? a->loss_norm : static_cast<float>(g->n_seq);
  return PCP_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline size_t round256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

int finish(pcp_ctx* ctx, const pcp_grpo_args* a, hipStream_t st) {
  if (a->flags & PCP_FLAG_ASYNC) {
    return add_pending(ctx, st);
  }
  hipError_t e = hipStreamSynchronize(st);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  return collect_device_errors(ctx);
}

// noalloc: take the work buffers from the device's static scratch array instead of
// the context's grow-only buffer (no allocation of any kind on this path).
int run(pcp_ctx* ctx, const pcp_grpo_args* a, Op op, bool noalloc = false) {
  Geo g;
  int rc = validate(a, op, &g);
  if (rc != PCP_OK) {
    if (ctx) copy_thread_error(ctx);
    return rc;
  }

  // Scratch: adv | seq_len | seq_scale | seq_val | loss | row counter, live-row count,
  // loss ticket | token_loss | live-row list (without zero-fill).
  const size_t sv = round256(sizeof(float) * g.n_seq);
  const bool need_tl = (op == kLoss) && a->token_loss == nullptr;
  const size_t tl_bytes = need_tl ? round256(sizeof(float) * g.n_seq * g.tstride) : 0;
  const bool need_list = (op == kLoss) && a->dlogits != nullptr && (a->flags & PCP_FLAG_NO_ZERO_FILL);
  const size_t list_bytes = need_list ? round256(sizeof(int) * static_cast<size_t>(g.nrows)) : 0;
  const size_t need = 4 * sv + 512 + tl_bytes + list_bytes;
  if (noalloc && need > PCP_NOALLOC_SCRATCH_BYTES)
    return fail(ctx, PCP_ERR_OVERFLOW,
                "the allocation-free call needs %zu bytes of work space, more than its %u-byte array: pass "
                "token_loss (n_seq*tok_seq_stride floats) or use pcp_grpo_loss_fwd_bwd",
                need, static_cast<unsigned>(PCP_NOALLOC_SCRATCH_BYTES));
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  if (noalloc && !ctx->noalloc_scratch)
    return fail(ctx, PCP_ERR_DEVICE, "the scratch array of device %d was not resolved at pcp_init", ctx->device);
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  hipStream_t st = static_cast<hipStream_t>(a->stream);

  if (!noalloc && (rc = ensure_scratch(ctx, need)) != PCP_OK) return rc;
  char* sp = static_cast<char*>(noalloc ? ctx->noalloc_scratch : ctx->scratch);
  float* s_adv = reinterpret_cast<float*>(sp);
  float* s_len = reinterpret_cast<float*>(sp + sv);
  float* s_scale = reinterpret_cast<float*>(sp + 2 * sv);
  float* s_val = reinterpret_cast<float*>(sp + 3 * sv);
  float* s_loss = reinterpret_cast<float*>(sp + 4 * sv);
  // The persistent row kernel's counter, zeroed before each launch (by step_prep_kernel
  // on the loss path). The allocation-free path keeps it in the shared array, the other
  // path in the context's own allocation. The loss ticket of loss_reduce_kernel and the
  // live-row count sit in the scratch.
  int* s_next = noalloc ? reinterpret_cast<int*>(sp + 4 * sv + 256) : ctx->d_next_row;
  int* s_count = reinterpret_cast<int*>(sp + 4 * sv + 256 + 64);
  int* s_done = reinterpret_cast<int*>(sp + 4 * sv + 256 + 128);
  float* s_tl = need_tl ? reinterpret_cast<float*>(sp + 4 * sv + 512) : a->token_loss;
  int* s_list = need_list ? reinterpret_cast<int*>(sp + 4 * sv + 512 + tl_bytes) : nullptr;

  RowArgs ra;
  std::memset(&ra, 0, sizeof(ra));
  ra.logits = a->logits;
  ra.ids = a->ids;
  ra.mask = a->mask;
  ra.err = ctx->d_err;
  ra.next_row = s_next;
  ra.row_list = s_list;
  ra.row_count = s_list ? s_count : nullptr;
  ra.nrows = g.nrows;
  ra.vocab = g.vocab;
  ra.rows = g.rows;
  ra.logit_stride = g.lstride;
  ra.tok_stride = g.tstride;
  ra.tok_offset = g.toff;
  ra.ids_i64 = a->ids_dtype == PCP_I64;
  ra.mask_u8 = a->mask_dtype == PCP_BOOL;
  ra.zero_fill = (a->flags & PCP_FLAG_NO_ZERO_FILL) ? 0 : 1;
  ra.logp = a->logp;
  ra.ref_logp = a->ref_logp;

  if (op == kLoss) {
    // One launch: advantages (or the copy of the given ones), per-sequence lengths, and
    // the row kernel's and the loss ticket's counters zeroed.
    const float* adv = a->advantages ? a->advantages : s_adv;
    StepPrepArgs pa;
    std::memset(&pa, 0, sizeof(pa));
    pa.mask = a->mask;
    pa.mask_u8 = ra.mask_u8;
    pa.n_seq = g.n_seq;
    pa.rows = g.rows;
    pa.tok_stride = g.tstride;
    pa.tok_offset = g.toff;
    pa.loss_norm = g.loss_norm;
    pa.seq_len = s_len;
    pa.seq_scale = s_scale;
    pa.rewards = a->advantages ? nullptr : a->rewards;
    pa.adv_in = a->advantages;
    pa.group = g.group;
    pa.std_eps = a->std_eps;
    pa.adv = s_adv;
    pa.adv_out = a->advantages_out != adv ? a->advantages_out : nullptr;
    pa.zero[0] = s_next;
    pa.zero[1] = s_list ? s_count : nullptr;
    pa.zero[2] = s_done;
    e = launch_step_prep(pa, st);
    if (e != hipSuccess) return hip_fail(ctx, e, "step prep launch");
    ra.counters_zeroed = 1;
    ra.ref_logits = (a->loss_mode == PCP_LOSS_GRPO_CLIP_KL) ? a->ref_logits : nullptr;
    ra.old_logp = a->old_logp;
    ra.adv = adv;
    ra.seq_scale = s_scale;
    ra.dlogits = a->dlogits;
    ra.token_loss = s_tl;
    ra.loss_mode = a->loss_mode;
    ra.clip_eps = a->clip_eps;
    ra.kl_beta = a->kl_beta;
  } else {
    ra.ref_logits = a->ref_logits;
  }

  const int in_bytes = dtype_bytes(a->logits_dtype);
  const bool al = aligned16(a->logits) && (!ra.ref_logits || aligned16(ra.ref_logits)) &&
                  (!ra.dlogits || aligned16(ra.dlogits));
  const bool edge_ok = !ra.dlogits || (a->dlogits_dtype == a->logits_dtype &&
                                       ((reinterpret_cast<uintptr_t>(a->logits) ^
                                         reinterpret_cast<uintptr_t>(ra.dlogits)) & 15u) == 0);
  RowPlan plan = plan_rows(in_bytes, g.vocab, al, edge_ok, ra.dlogits == nullptr,
                           (a->flags & PCP_FLAG_FORCE_STREAMING) != 0);
  plan.exact = (a->flags & PCP_FLAG_EXACT_BF16) ? 1 : 0;
  const int out_dt = ra.dlogits ? a->dlogits_dtype : a->logits_dtype;
  const bool timed = ctx->prof_on && ctx->prof_used < static_cast<int>(ctx->prof_start.size());
  if (timed) {
    e = hipEventRecord(ctx->prof_start[ctx->prof_used], st);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipEventRecord");
  }
  e = launch_rows(plan, a->logits_dtype, out_dt == PCP_F32 ? PCP_F32 : a->logits_dtype, ra, g.nrows, st);
  if (e != hipSuccess) return hip_fail(ctx, e, "row kernel launch");
  if (timed) {
    e = hipEventRecord(ctx->prof_stop[ctx->prof_used++], st);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipEventRecord");
  }

  if (op == kLoss) {
    const LossReduceArgs la{s_tl, g.rows, g.tstride, g.toff, s_len, ra.adv, a->loss_mode == PCP_LOSS_REINFORCE,
                            s_val, g.n_seq, g.loss_norm, s_done, a->loss ? a->loss : s_loss};
    e = launch_loss_reduce_fused(la, st);
    if (e != hipSuccess) return hip_fail(ctx, e, "loss reduction launch");
  }
  return finish(ctx, a, st);
}

}  // namespace
}  // namespace pcp

using namespace pcp;

extern "C" {

void pcp_grpo_args_init(pcp_grpo_args* a) {
  if (!a) return;
  std::memset(a, 0, sizeof(*a));
  a->group_size = 1;
  a->logits_dtype = PCP_BF16;
  a->dlogits_dtype = PCP_BF16;
  a->ids_dtype = PCP_I64;
  a->mask_dtype = PCP_F32;
  a->loss_mode = PCP_LOSS_REINFORCE;
  a->clip_eps = 0.2f;
  a->kl_beta = 0.04f;
  a->std_eps = 1e-8f;
}

int pcp_init(int backend, int device_ordinal, pcp_ctx** out) {
  if (!out) return fail(nullptr, PCP_ERR_INVALID_ARG, "out is NULL");
  *out = nullptr;
  if (backend != PCP_BACKEND_ROCM)
    return fail(nullptr, PCP_ERR_UNSUPPORTED, "backend %d: this library implements PCP_BACKEND_ROCM only", backend);
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) {
    (void)hipGetLastError();
    return fail(nullptr, PCP_ERR_DEVICE, "no HIP device available (%s)", hipGetErrorString(e));
  }
  if (device_ordinal < 0 || device_ordinal >= n)
    return fail(nullptr, PCP_ERR_INVALID_ARG, "device ordinal %d out of range [0, %d)", device_ordinal, n);
  e = hipSetDevice(device_ordinal);
  if (e != hipSuccess) return hip_fail(nullptr, e, "hipSetDevice");
  pcp_ctx* c = new (std::nothrow) pcp_ctx();
  if (!c) return fail(nullptr, PCP_ERR_OOM, "allocating the context");
  c->device = device_ordinal;
  // Error word at 0, the row kernel's counter 64 bytes on (its own cache line).
  e = hipMalloc(&c->d_err, 128);
  if (e != hipSuccess) {
    delete c;
    return fail(nullptr, PCP_ERR_OOM, "hipMalloc(error word): %s", hipGetErrorString(e));
  }
  c->d_next_row = c->d_err + 16;
  e = hipMemset(c->d_err, 0, 128);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    (void)hipFree(c->d_err);
    delete c;
    return hip_fail(nullptr, e, "initialising the error word");
  }
  // Resolve this device's copy of the allocation-free path's scratch array (once per
  // device, with the device current). A failure here only disables that entry point,
  // which then reports it.
  if (resolve_noalloc_scratch(device_ordinal, &c->noalloc_scratch) != PCP_OK) copy_thread_error(c);
  *out = c;
  return PCP_OK;
}

static void release_profile_events(pcp_ctx* ctx) {
  for (hipEvent_t ev : ctx->prof_start) (void)hipEventDestroy(ev);
  for (hipEvent_t ev : ctx->prof_stop) (void)hipEventDestroy(ev);
  ctx->prof_start.clear();
  ctx->prof_stop.clear();
  ctx->prof_used = 0;
  ctx->prof_on = false;
}

int pcp_profile_start(pcp_ctx* ctx, int max_launches) {
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  if (max_launches < 1 || max_launches > 1 << 20) return fail(ctx, PCP_ERR_INVALID_ARG, "max_launches out of range");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  release_profile_events(ctx);
  for (int i = 0; i < max_launches; ++i) {
    hipEvent_t a, b;
    if ((e = hipEventCreate(&a)) != hipSuccess) return hip_fail(ctx, e, "hipEventCreate");
    if ((e = hipEventCreate(&b)) != hipSuccess) {
      (void)hipEventDestroy(a);
      return hip_fail(ctx, e, "hipEventCreate");
    }
    ctx->prof_start.push_back(a);
    ctx->prof_stop.push_back(b);
  }
  ctx->prof_on = true;
  return PCP_OK;
}

int pcp_profile_stop(pcp_ctx* ctx, int* n_launches, double* total_ms) {
  if (!ctx || !n_launches || !total_ms) return fail(ctx, PCP_ERR_INVALID_ARG, "NULL argument");
  *n_launches = 0;
  *total_ms = 0.0;
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  double tot = 0.0;
  for (int i = 0; i < ctx->prof_used; ++i) {
    if ((e = hipEventSynchronize(ctx->prof_stop[i])) != hipSuccess) return hip_fail(ctx, e, "hipEventSynchronize");
    float ms = 0.f;
    if ((e = hipEventElapsedTime(&ms, ctx->prof_start[i], ctx->prof_stop[i])) != hipSuccess)
      return hip_fail(ctx, e, "hipEventElapsedTime");
    tot += ms;
  }
  *n_launches = ctx->prof_used;
  *total_ms = tot;
  release_profile_events(ctx);
  return PCP_OK;
}

void pcp_destroy(pcp_ctx* ctx) {
  if (!ctx) return;
  if (hipSetDevice(ctx->device) == hipSuccess) {
    (void)hipDeviceSynchronize();
    release_profile_events(ctx);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->lm_dbuf) (void)hipFree(ctx->lm_dbuf);
    if (ctx->sample_ticket) (void)hipFree(ctx->sample_ticket);
    destroy_stager(ctx);
    for (hipStream_t x : ctx->xs)
      if (x) (void)hipStreamDestroy(x);
    if (ctx->d_err) (void)hipFree(ctx->d_err);
  }
  delete ctx;
}

int pcp_release_workspace(pcp_ctx* ctx) {
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  if (!ctx->scratch && !ctx->lm_dbuf) return PCP_OK;
  // Earlier calls (PCP_FLAG_ASYNC ones included) may still use the buffers.
  if ((e = hipDeviceSynchronize()) != hipSuccess) return hip_fail(ctx, e, "hipDeviceSynchronize");
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  if (ctx->lm_dbuf) (void)hipFree(ctx->lm_dbuf);
  ctx->scratch = ctx->lm_dbuf = nullptr;
  ctx->scratch_bytes = ctx->lm_dbuf_bytes = 0;
  return PCP_OK;
}

size_t pcp_workspace_bytes(const pcp_ctx* ctx) { return ctx ? ctx->scratch_bytes + ctx->lm_dbuf_bytes : 0; }

int pcp_get_backend_type(const pcp_ctx* ctx) { return ctx ? ctx->backend : PCP_ERR_INVALID_ARG; }

const char* pcp_last_error(const pcp_ctx* ctx) {
  return ctx ? ctx->last_error : thread_error();
}

int pcp_sync(pcp_ctx* ctx) {
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  const int n = ctx->n_pending;
  ctx->n_pending = 0;
  for (int i = 0; i < n; ++i) {
    e = hipStreamSynchronize(ctx->pending[i]);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  }
  return collect_device_errors(ctx);
}

int pcp_grpo_logprob_fwd(pcp_ctx* ctx, const pcp_grpo_args* a) { return run(ctx, a, kLogprob); }

int pcp_grpo_loss_fwd_bwd(pcp_ctx* ctx, const pcp_grpo_args* a) { return run(ctx, a, kLoss); }

int pcp_grpo_loss_fwd_bwd_noalloc(pcp_ctx* ctx, const pcp_grpo_args* a) { return run(ctx, a, kLoss, true); }

int pcp_grpo_advantages(pcp_ctx* ctx, const float* rewards, int64_t n, int64_t group_size,
                        float std_eps, float* adv, void* stream) {
  if (n < 1) return fail(ctx, PCP_ERR_INVALID_ARG, "n must be >= 1");
  if (group_size < 1) return fail(ctx, PCP_ERR_INVALID_ARG, "group_size must be >= 1");
  if (!rewards || !adv) return fail(ctx, PCP_ERR_INVALID_ARG, "rewards / adv is NULL");
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  hipStream_t st = static_cast<hipStream_t>(stream);
  e = launch_advantages(rewards, n, group_size, std_eps, adv, st);
  if (e != hipSuccess) return hip_fail(ctx, e, "advantages launch");
  e = hipStreamSynchronize(st);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  return PCP_OK;
}

const char* pcp_version(void) { return "pcp_grpo 0.1.0 gfx950"; }

}  // extern "C"
