// Host-bytes entry point of the C ABI: pcp_execute / pcp_free.
//
// Mirrors WorkerBackend.executeFunction (src/backends/worker_backend.zig:27-33)
// as implemented by IreeBackend.execute (src/backends/iree.zig:336-442): borrowed
// host byte slices with i64 shapes and DType codes in, every input copied to the
// device, the function run synchronously, every output copied back into a
// caller-owned host buffer. Argument checks run before any device call.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "context.hpp"
#include "grpo_launch.hpp"
#include "host_transfer.hpp"
#include "pcp_grpo.h"

namespace pcp {
namespace {

struct In {
  const void* data;
  size_t nbytes;
  std::vector<int64_t> shape;
  int dtype;
  int64_t numel;
};

struct OutSpec {
  size_t nbytes;
};

int check_inputs(int n_in, const void* const* data, const size_t* nbytes,
                 const int64_t* const* shapes, const int* ranks, const int* dtypes,
                 const int* defaults, std::vector<In>* ins) {
  ins->resize(n_in);
  for (int i = 0; i < n_in; ++i) {
    In& t = (*ins)[i];
    t.data = data[i];
    t.nbytes = nbytes[i];
    t.dtype = dtypes ? dtypes[i] : defaults[i];
    if (dtype_bytes(t.dtype) == 0) return fail(nullptr, PCP_ERR_DTYPE, "input %d: unknown dtype %d", i, t.dtype);
    if (ranks[i] < 0 || ranks[i] > 8) return fail(nullptr, PCP_ERR_INVALID_ARG, "input %d: bad rank %d", i, ranks[i]);
    if (ranks[i] > 0 && !shapes[i]) return fail(nullptr, PCP_ERR_INVALID_ARG, "input %d: shape is NULL", i);
    t.shape.assign(shapes[i], shapes[i] + ranks[i]);
    int64_t n = 1;
    for (int64_t d : t.shape) {
      if (d < 0) return fail(nullptr, PCP_ERR_INVALID_ARG, "input %d: negative dimension", i);
      if (mul_overflows(n, d, &n)) return fail(nullptr, PCP_ERR_OVERFLOW, "input %d: element count overflows", i);
    }
    t.numel = n;
    int64_t b;
    if (mul_overflows(n, dtype_bytes(t.dtype), &b)) return fail(nullptr, PCP_ERR_OVERFLOW, "input %d: byte size overflows", i);
    if (static_cast<size_t>(b) != t.nbytes)
      return fail(nullptr, PCP_ERR_INVALID_ARG, "input %d: %zu bytes given, shape x dtype needs %lld", i, t.nbytes, (long long)b);
    if (b > 0 && !t.data) return fail(nullptr, PCP_ERR_INVALID_ARG, "input %d: data is NULL", i);
  }
  return PCP_OK;
}

int expect_dtype(const In& t, int i, std::initializer_list<int> ok, const char* what) {
  for (int d : ok)
    if (t.dtype == d) return PCP_OK;
  return fail(nullptr, PCP_ERR_DTYPE, "input %d (%s): dtype %d not supported", i, what, t.dtype);
}

int expect_shape(const In& t, int i, std::initializer_list<int64_t> dims, const char* what) {
  if (t.shape.size() != dims.size())
    return fail(nullptr, PCP_ERR_INVALID_ARG, "input %d (%s): rank %zu, expected %zu", i, what, t.shape.size(), dims.size());
  size_t k = 0;
  for (int64_t d : dims) {
    if (d >= 0 && t.shape[k] != d)
      return fail(nullptr, PCP_ERR_INVALID_ARG, "input %d (%s): dim %zu is %lld, expected %lld", i, what, k,
                  (long long)t.shape[k], (long long)d);
    ++k;
  }
  return PCP_OK;
}

int64_t id_at(const In& ids, int64_t i) {
  return ids.dtype == PCP_I64 ? static_cast<const int64_t*>(ids.data)[i]
                              : static_cast<const int32_t*>(ids.data)[i];
}
bool mask_at(const In* m, int64_t i) {
  if (!m) return true;
  return m->dtype == PCP_BOOL ? static_cast<const uint8_t*>(m->data)[i] != 0
                              : static_cast<const float*>(m->data)[i] != 0.f;
}

// Host check of the targets the kernels will gather (shifted: positions 1..T-1).
int check_ids(const In& ids, const In* mask, int64_t S, int64_t T, int64_t V) {
  for (int64_t s = 0; s < S; ++s)
    for (int64_t t = 1; t < T; ++t) {
      const int64_t i = s * T + t;
      const int64_t id = id_at(ids, i);
      if (mask_at(mask, i) && id != PCP_IGNORE_INDEX && (id < 0 || id >= V))
        return fail(nullptr, PCP_ERR_TOKEN_RANGE, "token id %lld at [%lld, %lld] outside [0, %lld)", (long long)id,
                    (long long)s, (long long)t, (long long)V);
    }
  return PCP_OK;
}

// Device allocations of one call, released on every exit path.
struct DevArena {
  std::vector<void*> ptrs;
  ~DevArena() {
    for (void* p : ptrs) (void)hipFree(p);
  }
  int alloc(pcp_ctx* ctx, size_t bytes, void** out) {
    *out = nullptr;
    if (bytes == 0) bytes = 16;
    hipError_t e = hipMalloc(out, bytes);
    if (e != hipSuccess) {
      *out = nullptr;
      (void)hipGetLastError();
      return fail(ctx, PCP_ERR_OOM, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    }
    ptrs.push_back(*out);
    return PCP_OK;
  }
  int upload(pcp_ctx* ctx, const In& t, void** out) {
    int rc = alloc(ctx, t.nbytes, out);
    if (rc != PCP_OK) return rc;
    if (t.nbytes == 0) return PCP_OK;
    hipError_t e = upload_pageable(ctx, *out, t.data, t.nbytes, nullptr);
    return e == hipSuccess ? PCP_OK : hip_fail(ctx, e, "host-to-device copy");
  }
  int zeroed(pcp_ctx* ctx, size_t bytes, void** out) {
    int rc = alloc(ctx, bytes, out);
    if (rc != PCP_OK) return rc;
    hipError_t e = hipMemset(*out, 0, bytes ? bytes : 16);
    return e == hipSuccess ? PCP_OK : hip_fail(ctx, e, "hipMemset");
  }
};

struct Outputs {
  std::vector<void*> dev;
  std::vector<size_t> bytes;
  std::vector<void*> host;   // optional: outputs already copied into their host buffer
  ~Outputs() {
    for (void* h : host) host_out_free(h);   // still owned here: not handed to the caller
  }
};

int download(pcp_ctx* ctx, Outputs& o, int* n_out, void*** out_data, size_t** out_nbytes) {
  const int n = static_cast<int>(o.dev.size());
  void** od = static_cast<void**>(std::calloc(n, sizeof(void*)));
  size_t* ob = static_cast<size_t*>(std::calloc(n, sizeof(size_t)));
  if (!od || !ob) {
    std::free(od);
    std::free(ob);
    return fail(ctx, PCP_ERR_OOM, "allocating the output list");
  }
  for (int i = 0; i < n; ++i) {
    void* pre = i < static_cast<int>(o.host.size()) ? o.host[i] : nullptr;
    od[i] = pre ? pre : host_out_alloc(o.bytes[i]);
    ob[i] = o.bytes[i];
    hipError_t e = pre ? hipSuccess
                 : od[i] ? hipMemcpy(od[i], o.dev[i], o.bytes[i], hipMemcpyDeviceToHost)
                         : hipErrorOutOfMemory;
    if (e != hipSuccess) {
      for (int k = 0; k <= i; ++k)
        if (!(k < static_cast<int>(o.host.size()) && o.host[k])) host_out_free(od[k]);   // others: o's
      std::free(od);
      std::free(ob);
      return e == hipErrorOutOfMemory ? fail(ctx, PCP_ERR_OOM, "allocating output %d", i)
                                      : hip_fail(ctx, e, "device-to-host copy");
    }
  }
  *n_out = n;
  *out_data = od;
  *out_nbytes = ob;
  o.host.clear();   // the caller owns them now
  return PCP_OK;
}

// ---- the loss functions over sequence groups ---------------------------------
// A host-bytes loss call on large logits is moved and computed in groups of whole
// sequences: the upload stream stages group k's policy (and reference) rows while the
// compute stream runs the loss head on earlier groups and the download stream copies
// their dlogits into the pinned output, so both PCIe directions carry data at once.
// The advantages are computed once over all sequences before the groups, and the
// sequence lengths and the loss reduction once over all token losses after them, with
// the same kernels and arguments as one call over every sequence: every output is
// bit-identical to it.
// Policy-logit bytes per group: PCP_EXECUTE_GROUP_MIB (MiB, default 1024). Calls with
// fewer than two groups' worth of logits run as one call.
size_t group_bytes() {
  const char* v = std::getenv("PCP_EXECUTE_GROUP_MIB");
  const long long mib = v ? std::atoll(v) : 0;
  return (mib > 0 && mib < (1LL << 30) ? static_cast<size_t>(mib) : size_t{1024}) << 20;
}

int64_t seqs_per_group(size_t seq_bytes, size_t gbytes) {
  return std::max<int64_t>(1, static_cast<int64_t>(gbytes / std::max<size_t>(seq_bytes, 1)));
}

int ensure_xs(pcp_ctx* ctx) {
  for (hipStream_t& x : ctx->xs) {
    if (x) continue;
    const hipError_t e = hipStreamCreateWithFlags(&x, hipStreamNonBlocking);
    if (e != hipSuccess) {
      x = nullptr;
      return hip_fail(ctx, e, "hipStreamCreateWithFlags");
    }
  }
  return PCP_OK;
}

// Waits for the call's streams and releases its events on every exit path, before
// the device buffers they use are freed.
struct GroupDrain {
  pcp_ctx* ctx;
  std::vector<hipEvent_t> ev;
  ~GroupDrain() {
    for (hipStream_t x : ctx->xs)
      if (x) (void)hipStreamSynchronize(x);
    for (hipEvent_t e : ev) (void)hipEventDestroy(e);
  }
  hipError_t mark(hipStream_t after, hipStream_t waiter) {
    hipEvent_t e = nullptr;
    hipError_t r = hipEventCreateWithFlags(&e, hipEventDisableTiming);
    if (r != hipSuccess) return r;
    ev.push_back(e);
    if ((r = hipEventRecord(e, after)) != hipSuccess) return r;
    return hipStreamWaitEvent(waiter, e, 0);
  }
};

// full: the call over all S sequences with every device buffer allocated and the
// small inputs uploaded; its logits / ref_logits / dlogits are filled or drained here.
// tl, slen, sscale, sval: device f32 [S*T], [S], [S], [S]. host_dl: the dlogits output.
int run_loss_groups(pcp_ctx* ctx, const pcp_grpo_args& full, const In& L, const In* R, int64_t S, int64_t T,
                    int64_t gs, float* tl, float* slen, float* sscale, float* sval, void* host_dl) {
  int rc = ensure_xs(ctx);
  if (rc != PCP_OK) return rc;
  hipError_t e = hipDeviceSynchronize();   // allocations, clears and small uploads of the call
  if (e != hipSuccess) return hip_fail(ctx, e, "hipDeviceSynchronize");
  const hipStream_t up = ctx->xs[0], run = ctx->xs[1], down = ctx->xs[2];
  GroupDrain drain{ctx, {}};
  const size_t seq_bytes = L.nbytes / static_cast<size_t>(S);
  const float gtot = full.loss_norm > 0.f ? full.loss_norm : static_cast<float>(S);
  const size_t id_b = dtype_bytes(full.ids_dtype), m_b = full.mask_dtype == PCP_BOOL ? 1 : 4;
  const float* adv = full.advantages ? full.advantages : full.advantages_out;
  if (!full.advantages) {
    e = launch_advantages(full.rewards, S, full.group_size, full.std_eps, full.advantages_out, run);
    if (e != hipSuccess) return hip_fail(ctx, e, "advantages launch");
  }
  for (int64_t s0 = 0; s0 < S; s0 += gs) {
    const int64_t n = std::min(gs, S - s0);
    const size_t off = static_cast<size_t>(s0) * seq_bytes, len = static_cast<size_t>(n) * seq_bytes;
    e = upload_pageable(ctx, static_cast<char*>(const_cast<void*>(full.logits)) + off,
                        static_cast<const char*>(L.data) + off, len, up);
    if (e == hipSuccess && R)
      e = upload_pageable(ctx, static_cast<char*>(const_cast<void*>(full.ref_logits)) + off,
                          static_cast<const char*>(R->data) + off, len, up);
    if (e == hipSuccess) e = drain.mark(up, run);
    if (e != hipSuccess) return hip_fail(ctx, e, "host-to-device copy");
    pcp_grpo_args g = full;
    const int64_t t0 = s0 * T;
    g.n_seq = n;
    g.logits = static_cast<const char*>(full.logits) + off;
    g.ref_logits = full.ref_logits ? static_cast<const char*>(full.ref_logits) + off : nullptr;
    g.dlogits = static_cast<char*>(full.dlogits) + off;
    g.ids = static_cast<const char*>(full.ids) + t0 * id_b;
    g.mask = static_cast<const char*>(full.mask) + t0 * m_b;
    g.old_logp = full.old_logp ? full.old_logp + t0 : nullptr;
    g.advantages = adv + s0;
    g.rewards = nullptr;
    g.logp = full.logp ? full.logp + t0 : nullptr;
    g.ref_logp = full.ref_logp ? full.ref_logp + t0 : nullptr;
    g.token_loss = tl + t0;
    g.advantages_out = nullptr;
    g.loss = nullptr;
    g.loss_norm = gtot;
    g.flags = PCP_FLAG_ASYNC;
    g.stream = run;
    if ((rc = pcp_grpo_loss_fwd_bwd(ctx, &g)) != PCP_OK) return rc;
    e = drain.mark(run, down);
    if (e == hipSuccess)
      e = hipMemcpyAsync(static_cast<char*>(host_dl) + off, static_cast<char*>(full.dlogits) + off, len,
                         hipMemcpyDeviceToHost, down);
    if (e != hipSuccess) return hip_fail(ctx, e, "device-to-host copy");
  }
  e = launch_seq_prep(full.mask, full.mask_dtype == PCP_BOOL, S, full.rows, T, full.tok_offset, gtot, slen, sscale,
                      run);
  if (e == hipSuccess)
    e = launch_loss_reduce(tl, S, full.rows, T, full.tok_offset, slen, adv, full.loss_mode == PCP_LOSS_REINFORCE,
                           gtot, sval, full.loss, run);
  if (e != hipSuccess) return hip_fail(ctx, e, "loss reduction launch");
  if ((rc = pcp_sync(ctx)) != PCP_OK) return rc;   // the compute stream and the device error word
  e = hipStreamSynchronize(down);
  return e == hipSuccess ? PCP_OK : hip_fail(ctx, e, "device-to-host copy");
}

// ---- functions ------------------------------------------------------------

enum Fn { kLossFwdBwd, kClipKl, kLogprob, kAdvantages, kLmhead, kMain, kUnknown };

Fn lookup(const char* fn) {
  if (!std::strcmp(fn, "grpo_loss_fwd_bwd")) return kLossFwdBwd;
  if (!std::strcmp(fn, "main")) return kMain;
  if (!std::strcmp(fn, "grpo_clip_kl_fwd_bwd")) return kClipKl;
  if (!std::strcmp(fn, "grpo_logprob_fwd")) return kLogprob;
  if (!std::strcmp(fn, "grpo_advantages")) return kAdvantages;
  if (!std::strcmp(fn, "grpo_lmhead_fwd_bwd")) return kLmhead;
  return kUnknown;
}

// Shifted layout of the reference graph over [S, T] token arrays.
void shifted_layout(pcp_grpo_args* a, int64_t S, int64_t T, int64_t V) {
  a->n_seq = S;
  a->rows = T > 0 ? T - 1 : 0;
  a->vocab = V;
  a->logit_seq_stride = T;
  a->tok_seq_stride = T;
  a->tok_offset = T > 0 ? 1 : 0;
}

// Per-token outputs of the shifted layout: aligned value t belongs to position t+1.
void shift_to_positions(float* v, int64_t S, int64_t T) {
  for (int64_t s = 0; s < S; ++s) {
    float* r = v + s * T;
    if (T > 1) std::memmove(r + 1, r, sizeof(float) * (T - 1));
    r[0] = 0.f;
  }
}

// "grpo_lmhead_fwd_bwd": the LM head and loss of export_qwen_forward.py:146-163 on
// hidden states, with the reference's shift (hidden row t scores token t+1). The
// shift is applied to ids / mask / old_logp on the host; the last row of each
// sequence has no target (mask 0), so its dhidden row is 0. An optional ninth input,
// norm_weight f32[H], fuses the decoder's final RMSNorm (hyper[5], when given, is its
// eps; 1e-6 otherwise): hidden is then the last layer's output and a seventh output
// carries dnorm_weight.
int execute_lmhead(pcp_ctx* ctx, const std::vector<In>& in, int* n_out, void*** out_data, size_t** out_nbytes) {
  int rc;
  const In& Hs = in[0];
  if ((rc = expect_dtype(Hs, 0, {PCP_BF16}, "hidden")) || (rc = expect_shape(Hs, 0, {-1, -1, -1}, "hidden")))
    return rc;
  const int64_t S = Hs.shape[0], T = Hs.shape[1], H = Hs.shape[2];
  if (S < 1 || T < 2 || H < 1) return fail(nullptr, PCP_ERR_INVALID_ARG, "hidden dims must be S >= 1, T >= 2, H >= 1");
  if ((rc = expect_dtype(in[1], 1, {PCP_BF16}, "weight")) || (rc = expect_shape(in[1], 1, {-1, H}, "weight")))
    return rc;
  const int64_t V = in[1].shape[0];
  if (V < 1) return fail(nullptr, PCP_ERR_INVALID_ARG, "weight must have >= 1 rows");
  if ((rc = expect_dtype(in[2], 2, {PCP_BF16}, "ref_weight")) || (rc = expect_shape(in[2], 2, {V, H}, "ref_weight")) ||
      (rc = expect_dtype(in[3], 3, {PCP_I64, PCP_I32}, "input_ids")) || (rc = expect_shape(in[3], 3, {S, T}, "input_ids")) ||
      (rc = expect_dtype(in[4], 4, {PCP_F32, PCP_BOOL}, "attention_mask")) ||
      (rc = expect_shape(in[4], 4, {S, T}, "attention_mask")) ||
      (rc = expect_dtype(in[5], 5, {PCP_F32}, "old_logp")) || (rc = expect_shape(in[5], 5, {S, T}, "old_logp")) ||
      (rc = expect_dtype(in[6], 6, {PCP_F32}, "rewards")) || (rc = expect_shape(in[6], 6, {S}, "rewards")) ||
      (rc = expect_dtype(in[7], 7, {PCP_F32}, "hyper")))
    return rc;
  const bool norm = in.size() == 9;
  if ((rc = expect_shape(in[7], 7, {norm && in[7].numel == 6 ? 6 : 5}, "hyper"))) return rc;
  if (norm && ((rc = expect_dtype(in[8], 8, {PCP_F32}, "norm_weight")) || (rc = expect_shape(in[8], 8, {H}, "norm_weight"))))
    return rc;
  float hyper[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 1e-6f};
  std::memcpy(hyper, in[7].data, sizeof(float) * static_cast<size_t>(in[7].numel));
  if (!(hyper[0] >= 1.f) || hyper[0] != static_cast<float>(static_cast<int64_t>(hyper[0])))
    return fail(nullptr, PCP_ERR_INVALID_ARG, "hyper[0] (group_size) must be a positive integer");
  if (hyper[4] != 0.f && hyper[4] != 1.f)
    return fail(nullptr, PCP_ERR_INVALID_ARG, "hyper[4] (loss_mode) must be 0 (REINFORCE) or 1 (GRPO_CLIP_KL)");
  if ((rc = check_ids(in[3], &in[4], S, T, V))) return rc;
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");

  // Shifted token arrays (aligned: row t carries position t+1; row T-1 is dead).
  const int64_t N = S * T;
  std::vector<int64_t> ids(N, 0);
  std::vector<float> mask(N, 0.f), old(N, 0.f);
  const float* old_in = static_cast<const float*>(in[5].data);
  for (int64_t s = 0; s < S; ++s)
    for (int64_t t = 0; t + 1 < T; ++t) {
      const int64_t src = s * T + t + 1, dst = s * T + t;
      ids[dst] = id_at(in[3], src);
      mask[dst] = in[4].dtype == PCP_F32 ? static_cast<const float*>(in[4].data)[src] : (mask_at(&in[4], src) ? 1.f : 0.f);
      old[dst] = old_in[src];
    }
  DevArena arena;
  pcp_lmhead_args a;
  pcp_lmhead_args_init(&a);
  a.n_seq = S;
  a.rows = T;
  a.hidden = H;
  a.vocab = V;
  a.group_size = static_cast<int64_t>(hyper[0]);
  a.clip_eps = hyper[1];
  a.kl_beta = hyper[2];
  a.loss_norm = hyper[3];
  a.loss_mode = hyper[4] == 1.f ? PCP_LOSS_GRPO_CLIP_KL : PCP_LOSS_REINFORCE;
  a.ids_dtype = PCP_I64;
  a.mask_dtype = PCP_F32;
  void* p;
  if ((rc = arena.upload(ctx, in[0], &p))) return rc;
  a.hidden_states = p;
  if ((rc = arena.upload(ctx, in[1], &p))) return rc;
  a.weight = p;
  if (a.loss_mode == PCP_LOSS_GRPO_CLIP_KL) {
    if ((rc = arena.upload(ctx, in[2], &p))) return rc;
    a.ref_weight = p;
  }
  auto put = [&](const void* src, size_t bytes, void** dst) {
    int r = arena.alloc(ctx, bytes, dst);
    if (r != PCP_OK) return r;
    hipError_t e = hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice);
    return e == hipSuccess ? PCP_OK : hip_fail(ctx, e, "host-to-device copy");
  };
  if ((rc = put(ids.data(), 8 * N, &p))) return rc;
  a.ids = p;
  if ((rc = put(mask.data(), 4 * N, &p))) return rc;
  a.mask = p;
  if ((rc = put(old.data(), 4 * N, &p))) return rc;
  a.old_logp = static_cast<float*>(p);
  if ((rc = arena.upload(ctx, in[6], &p))) return rc;
  a.rewards = static_cast<float*>(p);
  if (norm) {
    if ((rc = arena.upload(ctx, in[8], &p))) return rc;
    a.norm_weight = static_cast<float*>(p);
    a.norm_eps = hyper[5];
  }

  Outputs outs;
  auto out = [&](size_t bytes, bool zero, void** dst) {
    int r = zero ? arena.zeroed(ctx, bytes, dst) : arena.alloc(ctx, bytes, dst);
    if (r == PCP_OK) {
      outs.dev.push_back(*dst);
      outs.bytes.push_back(bytes);
    }
    return r;
  };
  if ((rc = out(4, false, &p))) return rc;
  a.loss = static_cast<float*>(p);
  if ((rc = out(4 * static_cast<size_t>(N) * H, false, &p))) return rc;
  a.dhidden = static_cast<float*>(p);
  if ((rc = out(4 * static_cast<size_t>(V) * H, false, &p))) return rc;
  a.dweight = static_cast<float*>(p);
  if ((rc = out(4 * N, true, &p))) return rc;
  a.logp = static_cast<float*>(p);
  if ((rc = out(4 * N, true, &p))) return rc;
  a.ref_logp = static_cast<float*>(p);
  if ((rc = out(4 * S, false, &p))) return rc;
  a.advantages_out = static_cast<float*>(p);
  if (norm) {
    if ((rc = out(4 * static_cast<size_t>(H), false, &p))) return rc;
    a.dnorm_weight = static_cast<float*>(p);
  }
  if ((rc = pcp_grpo_lmhead_fwd_bwd(ctx, &a))) return rc;
  if ((rc = download(ctx, outs, n_out, out_data, out_nbytes))) return rc;
  shift_to_positions(static_cast<float*>((*out_data)[3]), S, T);
  shift_to_positions(static_cast<float*>((*out_data)[4]), S, T);
  return PCP_OK;
}

}  // namespace

int execute(pcp_ctx* ctx, const char* fn, int n_in, const void* const* data, const size_t* nbytes,
            const int64_t* const* shapes, const int* ranks, const int* dtypes, int* n_out,
            void*** out_data, size_t** out_nbytes) {
  if (!fn || !n_out || !out_data || !out_nbytes || n_in < 0 || (n_in > 0 && (!data || !nbytes || !shapes || !ranks)))
    return fail(ctx, PCP_ERR_INVALID_ARG, "pcp_execute: NULL argument");
  *n_out = 0;
  *out_data = nullptr;
  *out_nbytes = nullptr;
  const Fn f = lookup(fn);
  if (f == kUnknown) return fail(ctx, PCP_ERR_UNKNOWN_FUNCTION, "no function named '%s'", fn);
  if (f == kMain)
    return fail(ctx, PCP_ERR_UNSUPPORTED,
                "'main' is the training VMFB's whole step ([params..., buffers..., input_ids, attention_mask, "
                "advantages] -> parameter gradients); this library is its loss head only: run the model "
                "forward to logits, call 'grpo_loss_fwd_bwd' (logits, input_ids, attention_mask, advantages) "
                "-> (loss, dlogits), then the model backward seeded with dlogits");

  static const int kDefLoss[] = {PCP_F32, PCP_I64, PCP_F32, PCP_F32};
  static const int kDefClip[] = {PCP_F32, PCP_F32, PCP_I64, PCP_F32, PCP_F32, PCP_F32, PCP_F32};
  static const int kDefLp2[] = {PCP_F32, PCP_I64};
  static const int kDefLp3[] = {PCP_F32, PCP_F32, PCP_I64};
  static const int kDefAdv[] = {PCP_F32, PCP_I64};
  static const int kDefLm[] = {PCP_BF16, PCP_BF16, PCP_BF16, PCP_I64, PCP_F32, PCP_F32, PCP_F32, PCP_F32, PCP_F32};
  const int* defaults = nullptr;
  int want = 0;
  switch (f) {
    case kLossFwdBwd: want = 4; defaults = kDefLoss; break;
    case kClipKl: want = 7; defaults = kDefClip; break;
    case kLogprob: want = (n_in == 3) ? 3 : 2; defaults = (n_in == 3) ? kDefLp3 : kDefLp2; break;
    case kAdvantages: want = 2; defaults = kDefAdv; break;
    case kLmhead: want = (n_in == 9) ? 9 : 8; defaults = kDefLm; break;
    default: break;
  }
  if (n_in != want) return fail(ctx, PCP_ERR_COUNT_MISMATCH, "'%s' takes %d inputs, got %d", fn, want, n_in);

  std::vector<In> in;
  int rc = check_inputs(n_in, data, nbytes, shapes, ranks, dtypes, defaults, &in);
  if (rc != PCP_OK) goto arg_error;
  if (f == kLmhead) {
    rc = execute_lmhead(ctx, in, n_out, out_data, out_nbytes);
    if (rc != PCP_OK && ctx) copy_thread_error(ctx);
    return rc;
  }

  {
    pcp_grpo_args a;
    pcp_grpo_args_init(&a);
    Outputs outs;
    DevArena arena;

    if (f == kAdvantages) {
      if ((rc = expect_dtype(in[0], 0, {PCP_F32}, "rewards")) || (rc = expect_shape(in[0], 0, {-1}, "rewards")) ||
          (rc = expect_dtype(in[1], 1, {PCP_I64, PCP_I32}, "group_size")) ||
          (rc = expect_shape(in[1], 1, {}, "group_size")))
        goto arg_error;
      const int64_t n = in[0].numel;
      const int64_t G = id_at(in[1], 0);
      if (n < 1 || G < 1) {
        rc = fail(nullptr, PCP_ERR_INVALID_ARG, "grpo_advantages: need n >= 1 and group_size >= 1");
        goto arg_error;
      }
      if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
      void *dr, *da;
      if ((rc = arena.upload(ctx, in[0], &dr)) || (rc = arena.alloc(ctx, n * sizeof(float), &da))) return rc;
      if ((rc = pcp_grpo_advantages(ctx, static_cast<float*>(dr), n, G, 1e-8f, static_cast<float*>(da), nullptr)))
        return rc;
      outs.dev.push_back(da);
      outs.bytes.push_back(n * sizeof(float));
      return download(ctx, outs, n_out, out_data, out_nbytes);
    }

    // [S, T, V] functions.
    const int ix_ids = (f == kLossFwdBwd || f == kLogprob) ? (f == kLogprob && n_in == 3 ? 2 : 1) : 2;
    const In& L = in[0];
    if ((rc = expect_dtype(L, 0, {PCP_BF16, PCP_F16, PCP_F32}, "logits")) || (rc = expect_shape(L, 0, {-1, -1, -1}, "logits")))
      goto arg_error;
    const int64_t S = L.shape[0], T = L.shape[1], V = L.shape[2];
    if (S < 1 || T < 1 || V < 1) {
      rc = fail(nullptr, PCP_ERR_INVALID_ARG, "logits dims must be >= 1");
      goto arg_error;
    }
    const In& ids = in[ix_ids];
    if ((rc = expect_dtype(ids, ix_ids, {PCP_I64, PCP_I32}, "input_ids")) || (rc = expect_shape(ids, ix_ids, {S, T}, "input_ids")))
      goto arg_error;
    const bool has_ref = (f == kClipKl) || (f == kLogprob && n_in == 3);
    if (has_ref) {
      if ((rc = expect_dtype(in[1], 1, {L.dtype}, "ref_logits")) || (rc = expect_shape(in[1], 1, {S, T, V}, "ref_logits")))
        goto arg_error;
    }
    const In* mask = nullptr;
    if (f == kLossFwdBwd || f == kClipKl) {
      const int im = ix_ids + 1;
      mask = &in[im];
      if ((rc = expect_dtype(*mask, im, {PCP_F32, PCP_BOOL}, "attention_mask")) ||
          (rc = expect_shape(*mask, im, {S, T}, "attention_mask")))
        goto arg_error;
    }
    if (f == kLossFwdBwd) {
      if ((rc = expect_dtype(in[3], 3, {PCP_F32}, "advantages")) || (rc = expect_shape(in[3], 3, {S}, "advantages")))
        goto arg_error;
    }
    float hyper[4] = {1.f, 0.2f, 0.04f, 0.f};
    if (f == kClipKl) {
      if ((rc = expect_dtype(in[4], 4, {PCP_F32}, "old_logp")) || (rc = expect_shape(in[4], 4, {S, T}, "old_logp")) ||
          (rc = expect_dtype(in[5], 5, {PCP_F32}, "rewards")) || (rc = expect_shape(in[5], 5, {S}, "rewards")) ||
          (rc = expect_dtype(in[6], 6, {PCP_F32}, "hyper")) || (rc = expect_shape(in[6], 6, {4}, "hyper")))
        goto arg_error;
      std::memcpy(hyper, in[6].data, sizeof(hyper));
      const float G = hyper[0];
      if (!(G >= 1.f) || G != static_cast<float>(static_cast<int64_t>(G))) {
        rc = fail(nullptr, PCP_ERR_INVALID_ARG, "hyper[0] (group_size) must be a positive integer");
        goto arg_error;
      }
    }
    if ((rc = check_ids(ids, mask, S, T, V))) goto arg_error;
    if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");

    shifted_layout(&a, S, T, V);
    a.logits_dtype = L.dtype;
    a.dlogits_dtype = L.dtype;
    a.ids_dtype = ids.dtype;
    void* p;
    const size_t gbytes = group_bytes();
    const int64_t gs = seqs_per_group(L.nbytes / S, gbytes);
    const bool grouped = f != kLogprob && L.nbytes >= 2 * gbytes && gs < S;
    if ((rc = grouped ? arena.alloc(ctx, L.nbytes, &p) : arena.upload(ctx, L, &p))) return rc;
    a.logits = p;
    if (has_ref) {
      if ((rc = grouped ? arena.alloc(ctx, in[1].nbytes, &p) : arena.upload(ctx, in[1], &p))) return rc;
      a.ref_logits = p;
    }
    if ((rc = arena.upload(ctx, ids, &p))) return rc;
    a.ids = p;
    if (mask) {
      if ((rc = arena.upload(ctx, *mask, &p))) return rc;
      a.mask = p;
      a.mask_dtype = mask->dtype;
    }
    const size_t tok_bytes = sizeof(float) * S * T;
    if (f == kLogprob) {
      if ((rc = arena.zeroed(ctx, tok_bytes, &p))) return rc;
      a.logp = static_cast<float*>(p);
      outs.dev.push_back(p);
      outs.bytes.push_back(tok_bytes);
      if (has_ref) {
        if ((rc = arena.zeroed(ctx, tok_bytes, &p))) return rc;
        a.ref_logp = static_cast<float*>(p);
        outs.dev.push_back(p);
        outs.bytes.push_back(tok_bytes);
      }
      if ((rc = pcp_grpo_logprob_fwd(ctx, &a))) return rc;
      return download(ctx, outs, n_out, out_data, out_nbytes);
    }

    if ((rc = arena.alloc(ctx, sizeof(float), &p))) return rc;
    a.loss = static_cast<float*>(p);
    outs.dev.push_back(p);
    outs.bytes.push_back(sizeof(float));
    if ((rc = arena.alloc(ctx, L.nbytes, &p))) return rc;
    a.dlogits = p;
    outs.dev.push_back(p);
    outs.bytes.push_back(L.nbytes);
    if (f == kLossFwdBwd) {
      if ((rc = arena.upload(ctx, in[3], &p))) return rc;
      a.advantages = static_cast<float*>(p);
      a.group_size = S;
      a.loss_mode = PCP_LOSS_REINFORCE;
    } else {
      if ((rc = arena.upload(ctx, in[4], &p))) return rc;
      a.old_logp = static_cast<float*>(p);
      if ((rc = arena.upload(ctx, in[5], &p))) return rc;
      a.rewards = static_cast<float*>(p);
      a.group_size = static_cast<int64_t>(hyper[0]);
      a.clip_eps = hyper[1];
      a.kl_beta = hyper[2];
      a.loss_norm = hyper[3];
      a.loss_mode = PCP_LOSS_GRPO_CLIP_KL;
      for (int k = 0; k < 2; ++k) {
        if ((rc = arena.zeroed(ctx, tok_bytes, &p))) return rc;
        (k == 0 ? a.logp : a.ref_logp) = static_cast<float*>(p);
        outs.dev.push_back(p);
        outs.bytes.push_back(tok_bytes);
      }
      if ((rc = arena.alloc(ctx, sizeof(float) * S, &p))) return rc;
      a.advantages_out = static_cast<float*>(p);
      outs.dev.push_back(p);
      outs.bytes.push_back(sizeof(float) * S);
    }
    if (grouped) {
      void *tl, *slen, *sscale, *sval;
      if ((rc = arena.alloc(ctx, tok_bytes, &tl)) || (rc = arena.alloc(ctx, sizeof(float) * S, &slen)) ||
          (rc = arena.alloc(ctx, sizeof(float) * S, &sscale)) || (rc = arena.alloc(ctx, sizeof(float) * S, &sval)))
        return rc;
      outs.host.assign(outs.dev.size(), nullptr);
      outs.host[1] = host_out_alloc(L.nbytes);   // dlogits, filled group by group
      if (!outs.host[1]) return fail(ctx, PCP_ERR_OOM, "allocating the dlogits output");
      if ((rc = run_loss_groups(ctx, a, L, has_ref ? &in[1] : nullptr, S, T, gs, static_cast<float*>(tl),
                                static_cast<float*>(slen), static_cast<float*>(sscale), static_cast<float*>(sval),
                                outs.host[1])))
        return rc;
    } else if ((rc = pcp_grpo_loss_fwd_bwd(ctx, &a))) {
      return rc;
    }
    return download(ctx, outs, n_out, out_data, out_nbytes);
  }

arg_error:
  if (ctx) copy_thread_error(ctx);
  return rc;
}

}  // namespace pcp

extern "C" {

int pcp_execute(pcp_ctx* ctx, const char* fn, int n_in, const void* const* data, const size_t* nbytes,
                const int64_t* const* shapes, const int* ranks, const int* dtypes, int* n_out,
                void*** out_data, size_t** out_nbytes) {
  if (ctx) {
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return pcp::hip_fail(ctx, e, "hipSetDevice");
  }
  return pcp::execute(ctx, fn, n_in, data, nbytes, shapes, ranks, dtypes, n_out, out_data, out_nbytes);
}

void pcp_free(pcp_ctx* ctx, int n_out, void** out_data, size_t* out_nbytes) {
  (void)ctx;
  if (out_data) {
    for (int i = 0; i < n_out; ++i) pcp::host_out_free(out_data[i]);
    std::free(out_data);
  }
  std::free(out_nbytes);
}

}  // extern "C"
