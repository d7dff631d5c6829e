// Device-resident work around the loss head in one training step (pcp_step.h):
// rollout packing, gradient statistics and the Nesterov parameter update.
//
// References: RLShepherd.trainStep (src/nodes/controllers/rl_shepherd.zig:487-515
// packing, :600-641 statistics, :643-682 update loop), the host Nesterov optimizer
// (src/optimizers/nesterov.zig:70-98) and NesterovMLIR.update
// (src/optimizers/nesterov_mlir.zig:93-99). All three are HBM-bound streams; the
// update moves 20 bytes per parameter (read p, v, g; write p, v), +2 with the bf16
// shadow copy.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <new>
#include <vector>

#include "context.hpp"
#include "grpo_device.hpp"
#include "pcp_step.h"

// The reference rounds every product and sum in f32 (Zig's strict float mode); a
// contracted FMA would round once and differ in the last bit.
#pragma clang fp contract(off)

struct pcp_nesterov {
  pcp_ctx* ctx = nullptr;
  float lr = 0.f, mu = 0.f;
  int mode = PCP_NESTEROV_SUTSKEVER;
  std::vector<int64_t> counts, offsets;
  int64_t total = 0;
  float* vel = nullptr;
};

namespace pcp {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// The optimizer step's streaming stores, nontemporal at system scope (store_nt_sys):
// 1.900 -> 1.859 ms for the 494M-parameter update (four interleaved runs each) against
// device-scope nontemporal stores.
__device__ __forceinline__ void st_stream(f32x4 v, f32x4* p) { store_nt_sys(__builtin_bit_cast(u32x4, v), p); }
__device__ __forceinline__ void st_stream(u32x2 v, u32x2* p) { store_nt_sys(v, p); }

// ---- packing ------------------------------------------------------------------------

struct PackArgs {
  const int64_t* pt;
  const int64_t* po;
  const int64_t* ct;
  const int64_t* co;
  int64_t npt, nct, R, T;
  int64_t* ids;
  float* mask;
  int* err;
};

// One workgroup per output row. Rollout r: prompt then completion, truncated at T.
__global__ void __launch_bounds__(256) pack_kernel(PackArgs a) {
  const int64_t r = blockIdx.x;
  int64_t p0 = 0, lp = 0, c0 = 0, lc = 0;
  if (r < a.R) {
    p0 = a.po[r];
    lp = a.po[r + 1] - p0;
    c0 = a.co[r];
    lc = a.co[r + 1] - c0;
    const bool ok = p0 >= 0 && lp >= 0 && p0 + lp <= a.npt && c0 >= 0 && lc >= 0 && c0 + lc <= a.nct;
    if (!ok) {
      if (threadIdx.x == 0) atomicOr(a.err, kErrBadRagged);
      lp = 0;
      lc = 0;
    }
  }
  int64_t* ids = a.ids + r * a.T;
  float* mask = a.mask + r * a.T;
  for (int64_t t = threadIdx.x; t < a.T; t += 256) {
    int64_t id = 0;
    float m = 0.f;
    if (t < lp) {
      id = a.pt[p0 + t];
      m = 1.f;
    } else if (t - lp < lc) {
      id = a.ct[c0 + (t - lp)];
      m = 1.f;
    }
    ids[t] = id;
    mask[t] = m;
  }
}

// ---- gradient statistics --------------------------------------------------------------

struct StatsPart {
  double sumsq;
  float max_abs;
  int pad;
  int64_t nan_count;
  int64_t inf_count;
};

constexpr int kStatsBlocks = 2048;

__device__ __forceinline__ void stats_add(StatsPart& s, float g) {
  if (__builtin_isnan(g)) {
    s.nan_count += 1;
  } else if (__builtin_isinf(g)) {
    s.inf_count += 1;
  } else {
    s.sumsq += static_cast<double>(g) * static_cast<double>(g);
    s.max_abs = fmaxf(s.max_abs, fabsf(g));
  }
}

__device__ __forceinline__ void stats_merge(StatsPart& a, const StatsPart& b) {
  a.sumsq += b.sumsq;
  a.max_abs = fmaxf(a.max_abs, b.max_abs);
  a.nan_count += b.nan_count;
  a.inf_count += b.inf_count;
}

// Fixed-order tree over the 256 threads of a block (deterministic).
__device__ __forceinline__ StatsPart stats_block(StatsPart s, StatsPart* lds) {
  lds[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < static_cast<unsigned>(w)) {
      StatsPart o = lds[threadIdx.x + w];
      StatsPart m = lds[threadIdx.x];
      stats_merge(m, o);
      lds[threadIdx.x] = m;
    }
    __syncthreads();
  }
  return lds[0];
}

// Thread i of the grid reads vectors i, i + stride, ... (16-byte loads when the
// pointer allows, else elements); one partial per block.
__global__ void __launch_bounds__(256) stats_kernel(const float* g, int64_t n, int vec, StatsPart* parts) {
  __shared__ StatsPart lds[256];
  StatsPart s{0.0, 0.f, 0, 0, 0};
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  if (vec) {
    const int64_t n4 = n / 4;
    const f32x4* g4 = reinterpret_cast<const f32x4*>(g);
    for (int64_t i = tid; i < n4; i += stride) {
      const f32x4 x = __builtin_nontemporal_load(g4 + i);
      stats_add(s, x.x);
      stats_add(s, x.y);
      stats_add(s, x.z);
      stats_add(s, x.w);
    }
    for (int64_t i = n4 * 4 + tid; i < n; i += stride) stats_add(s, g[i]);
  } else {
    for (int64_t i = tid; i < n; i += stride) stats_add(s, g[i]);
  }
  s = stats_block(s, lds);
  if (threadIdx.x == 0) parts[blockIdx.x] = s;
}

__global__ void __launch_bounds__(256) stats_final_kernel(const StatsPart* parts, int nparts, StatsPart* out) {
  __shared__ StatsPart lds[256];
  StatsPart s{0.0, 0.f, 0, 0, 0};
  for (int i = threadIdx.x; i < nparts; i += 256) stats_merge(s, parts[i]);
  s = stats_block(s, lds);
  if (threadIdx.x == 0) *out = s;
}

// ---- Nesterov ---------------------------------------------------------------------------

template <int MODE>
__device__ __forceinline__ void nesterov_one(float& p, float& v, float g, float lr, float mu) {
  if constexpr (MODE == PCP_NESTEROV_SUTSKEVER) {
    // nesterov.zig:86-97: v_new = mu*v + g;  p = p - lr*(g + mu*v_new)
    const float vn = mu * v + g;
    v = vn;
    p = p - lr * (g + mu * vn);
  } else {
    // nesterov_mlir.zig:93-99: v_new = mu*v + lr*g;  p = p - v_new
    const float vn = mu * v + lr * g;
    v = vn;
    p = p - vn;
  }
}

// Elements [head, head + 4*n4) as 16-byte vectors (all three pointers share their
// alignment there), [0, head) and [head + 4*n4, n) one by one; both grid-stride.
// Every element is read and written exactly once.
template <int MODE, bool SHADOW>
__global__ void __launch_bounds__(256) nesterov_kernel(float* p, float* v, const float* g, uint16_t* shadow, int64_t n,
                                                       int64_t head, int64_t n4, float lr, float mu) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  f32x4* p4 = reinterpret_cast<f32x4*>(p + head);
  f32x4* v4 = reinterpret_cast<f32x4*>(v + head);
  const f32x4* g4 = reinterpret_cast<const f32x4*>(g + head);
  // kUnroll vectors per thread per iteration, all loads first (memory-level parallelism).
  constexpr int kUnroll = 8;
  int64_t i = tid;
  for (; i + (kUnroll - 1) * stride < n4; i += kUnroll * stride) {
    f32x4 pp[kUnroll], vv[kUnroll], gg[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      pp[u] = __builtin_nontemporal_load(p4 + i + u * stride);
      vv[u] = __builtin_nontemporal_load(v4 + i + u * stride);
      gg[u] = __builtin_nontemporal_load(g4 + i + u * stride);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float pc = pp[u][c], vc = vv[u][c];
        nesterov_one<MODE>(pc, vc, gg[u][c], lr, mu);
        pp[u][c] = pc;
        vv[u][c] = vc;
      }
      st_stream(pp[u], p4 + i + u * stride);
      st_stream(vv[u], v4 + i + u * stride);
      if constexpr (SHADOW) {
        const u32x2 b = {pack2<BF16T>(pp[u].x, pp[u].y), pack2<BF16T>(pp[u].z, pp[u].w)};
        st_stream(b, reinterpret_cast<u32x2*>(shadow + head) + i + u * stride);
      }
    }
  }
  for (; i < n4; i += stride) {
    f32x4 pp = __builtin_nontemporal_load(p4 + i);
    f32x4 vv = __builtin_nontemporal_load(v4 + i);
    const f32x4 gg = __builtin_nontemporal_load(g4 + i);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float pc = pp[c], vc = vv[c];
      nesterov_one<MODE>(pc, vc, gg[c], lr, mu);
      pp[c] = pc;
      vv[c] = vc;
    }
    st_stream(pp, p4 + i);
    st_stream(vv, v4 + i);
    if constexpr (SHADOW) {
      const u32x2 b = {pack2<BF16T>(pp.x, pp.y), pack2<BF16T>(pp.z, pp.w)};
      st_stream(b, reinterpret_cast<u32x2*>(shadow + head) + i);
    }
  }
  const int64_t tail0 = head + 4 * n4;
  const int64_t nscalar = head + (n - tail0);
  for (int64_t j = tid; j < nscalar; j += stride) {
    const int64_t e = j < head ? j : tail0 + (j - head);
    float pp = p[e], vv = v[e];
    nesterov_one<MODE>(pp, vv, g[e], lr, mu);
    p[e] = pp;
    v[e] = vv;
    if constexpr (SHADOW) shadow[e] = static_cast<uint16_t>(pack2<BF16T>(pp, 0.f) & 0xFFFFu);
  }
}

__global__ void __launch_bounds__(256) zero_kernel(float* x, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    x[i] = 0.f;
}

unsigned grid_for(int64_t work, int64_t per_block) {
  int64_t b = (work + per_block - 1) / per_block;
  if (b < 1) b = 1;
  if (b > 65536) b = 65536;
  return static_cast<unsigned>(b);
}

hipError_t launch_nesterov(const pcp_nesterov* o, float* p, float* v, const float* g, uint16_t* shadow, int64_t n,
                           hipStream_t st) {
  // Vector body when p, v, g (and the shadow, at half the offset) share 16-byte
  // alignment after a common head of 0-3 elements.
  const uintptr_t ap = reinterpret_cast<uintptr_t>(p) & 15u, av = reinterpret_cast<uintptr_t>(v) & 15u,
                  ag = reinterpret_cast<uintptr_t>(g) & 15u;
  int64_t head = n, n4 = 0;
  if (ap == av && av == ag && (ap & 3u) == 0) {
    head = static_cast<int64_t>(((16u - ap) & 15u) / 4u);
    if (head > n) head = n;
    const bool shadow_ok = !shadow || ((reinterpret_cast<uintptr_t>(shadow + head) & 7u) == 0);
    if (shadow_ok) n4 = (n - head) / 4;
    else head = n;
  }
  // One vector per thread over an uncapped grid: waves that issue few stores each
  // write faster than a capped grid-stride loop (measured 5.84 vs 5.62 TB/s at 494M
  // parameters for two vectors per thread; one vector measured 0.5% faster again,
  // interleaved). n <= 2^40 keeps the block count below 2^31.
  const unsigned grid = static_cast<unsigned>((n4 > 0 ? n4 + 255 : 256) / 256);
  const unsigned grid_s = grid_for(head + (n - head - 4 * n4), 256);
  const unsigned g2 = grid > grid_s ? grid : grid_s;
  const bool sh = shadow != nullptr;
  if (o->mode == PCP_NESTEROV_SUTSKEVER) {
    if (sh) nesterov_kernel<PCP_NESTEROV_SUTSKEVER, true><<<g2, 256, 0, st>>>(p, v, g, shadow, n, head, n4, o->lr, o->mu);
    else nesterov_kernel<PCP_NESTEROV_SUTSKEVER, false><<<g2, 256, 0, st>>>(p, v, g, shadow, n, head, n4, o->lr, o->mu);
  } else {
    if (sh) nesterov_kernel<PCP_NESTEROV_MLIR, true><<<g2, 256, 0, st>>>(p, v, g, shadow, n, head, n4, o->lr, o->mu);
    else nesterov_kernel<PCP_NESTEROV_MLIR, false><<<g2, 256, 0, st>>>(p, v, g, shadow, n, head, n4, o->lr, o->mu);
  }
  return hipGetLastError();
}

// The update and reset raise no device-side conditions: waiting is enough.
int sync_only(pcp_ctx* ctx, hipStream_t st) {
  hipError_t e = hipStreamSynchronize(st);
  return e == hipSuccess ? PCP_OK : hip_fail(ctx, e, "hipStreamSynchronize");
}

int finish(pcp_ctx* ctx, hipStream_t st) {
  hipError_t e = hipStreamSynchronize(st);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  return collect_device_errors(ctx);
}

}  // namespace
}  // namespace pcp

using namespace pcp;

extern "C" {

int pcp_pack_rollouts(pcp_ctx* ctx, const int64_t* prompt_tokens, int64_t n_prompt_tokens,
                      const int64_t* prompt_offsets, const int64_t* completion_tokens,
                      int64_t n_completion_tokens, const int64_t* completion_offsets, int64_t n_rollouts,
                      int64_t n_rows, int64_t seq_len, int64_t* ids, float* mask, void* stream) {
  if (n_rollouts < 0 || n_rows < n_rollouts || n_rows < 1 || seq_len < 1 || n_prompt_tokens < 0 ||
      n_completion_tokens < 0)
    return fail(ctx, PCP_ERR_INVALID_ARG, "need 0 <= n_rollouts <= n_rows, n_rows >= 1, seq_len >= 1");
  if (n_rows > (int64_t(1) << 31) - 1) return fail(ctx, PCP_ERR_OVERFLOW, "n_rows exceeds 2^31 - 1");
  int64_t cells;
  if (mul_overflows(n_rows, seq_len, &cells)) return fail(ctx, PCP_ERR_OVERFLOW, "n_rows * seq_len overflows");
  if (!ids || !mask || (n_rollouts > 0 && (!prompt_offsets || !completion_offsets)) ||
      (n_prompt_tokens > 0 && !prompt_tokens) || (n_completion_tokens > 0 && !completion_tokens))
    return fail(ctx, PCP_ERR_INVALID_ARG, "a required pointer is NULL");
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  hipStream_t st = static_cast<hipStream_t>(stream);
  PackArgs a{prompt_tokens, prompt_offsets, completion_tokens, completion_offsets, n_prompt_tokens,
             n_completion_tokens, n_rollouts, seq_len, ids, mask, ctx->d_err};
  pack_kernel<<<dim3(static_cast<unsigned>(n_rows)), dim3(256), 0, st>>>(a);
  if ((e = hipGetLastError()) != hipSuccess) return hip_fail(ctx, e, "pack launch");
  return finish(ctx, st);
}

int pcp_grad_stats_compute(pcp_ctx* ctx, const float* grad, int64_t n, int accumulate, pcp_grad_stats* stats,
                           void* stream) {
  if (!stats || n < 0 || (n > 0 && !grad)) return fail(ctx, PCP_ERR_INVALID_ARG, "grad / stats is NULL or n < 0");
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t parts_bytes = sizeof(StatsPart) * (kStatsBlocks + 1);
  int rc = ensure_scratch(ctx, parts_bytes);
  if (rc != PCP_OK) return rc;
  StatsPart* parts = static_cast<StatsPart*>(ctx->scratch);
  StatsPart h{0.0, 0.f, 0, 0, 0};
  if (n > 0) {
    const int vec = (reinterpret_cast<uintptr_t>(grad) & 15u) == 0;
    const unsigned grid = grid_for(n, 256 * 16) < kStatsBlocks ? grid_for(n, 256 * 16) : kStatsBlocks;
    stats_kernel<<<grid, 256, 0, st>>>(grad, n, vec, parts);
    stats_final_kernel<<<1, 256, 0, st>>>(parts, static_cast<int>(grid), parts + kStatsBlocks);
    if ((e = hipGetLastError()) != hipSuccess) return hip_fail(ctx, e, "statistics launch");
    if ((e = hipMemcpyAsync(&h, parts + kStatsBlocks, sizeof(h), hipMemcpyDeviceToHost, st)) != hipSuccess)
      return hip_fail(ctx, e, "reading statistics");
    if ((e = hipStreamSynchronize(st)) != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  }
  if (!accumulate) *stats = pcp_grad_stats{0.0, 0.0, 0.f, 0, 0, 0};
  stats->sumsq += h.sumsq;
  stats->max_abs = std::fmax(stats->max_abs, h.max_abs);
  stats->nan_count += h.nan_count;
  stats->inf_count += h.inf_count;
  stats->elements += n;
  stats->l2_norm = std::sqrt(stats->sumsq);
  return PCP_OK;
}

int pcp_nesterov_create(pcp_ctx* ctx, float learning_rate, float momentum, int mode, int n_tensors,
                        const int64_t* counts, pcp_nesterov** out) {
  if (!out) return fail(ctx, PCP_ERR_INVALID_ARG, "out is NULL");
  *out = nullptr;
  if (mode != PCP_NESTEROV_SUTSKEVER && mode != PCP_NESTEROV_MLIR)
    return fail(ctx, PCP_ERR_INVALID_ARG, "unknown Nesterov mode %d", mode);
  if (n_tensors < 1 || !counts) return fail(ctx, PCP_ERR_INVALID_ARG, "need n_tensors >= 1 and counts");
  if (!std::isfinite(learning_rate) || !std::isfinite(momentum))
    return fail(ctx, PCP_ERR_INVALID_ARG, "learning_rate and momentum must be finite");
  pcp_nesterov* o = new (std::nothrow) pcp_nesterov;
  if (!o) return fail(ctx, PCP_ERR_OOM, "allocating the optimizer");
  o->ctx = ctx;
  o->lr = learning_rate;
  o->mu = momentum;
  o->mode = mode;
  for (int i = 0; i < n_tensors; ++i) {
    if (counts[i] < 0) {
      delete o;
      return fail(ctx, PCP_ERR_INVALID_ARG, "counts[%d] < 0", i);
    }
    o->offsets.push_back(o->total);
    o->counts.push_back(counts[i]);
    if (o->total > (int64_t(1) << 40) - counts[i]) {
      delete o;
      return fail(ctx, PCP_ERR_OVERFLOW, "more than 2^40 parameters");
    }
    o->total += counts[i];
  }
  if (!ctx) {
    delete o;
    return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  }
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&o->vel), sizeof(float) * (o->total > 0 ? o->total : 1));
  if (e != hipSuccess) {
    (void)hipGetLastError();
    delete o;
    return fail(ctx, PCP_ERR_OOM, "allocating velocities: %s", hipGetErrorString(e));
  }
  *out = o;
  return pcp_nesterov_reset(o, nullptr);
}

void pcp_nesterov_destroy(pcp_nesterov* opt) {
  if (!opt) return;
  if (opt->ctx && hipSetDevice(opt->ctx->device) == hipSuccess) {
    (void)hipDeviceSynchronize();
    if (opt->vel) (void)hipFree(opt->vel);
  }
  delete opt;
}

int pcp_nesterov_reset(pcp_nesterov* opt, void* stream) {
  if (!opt) return fail(nullptr, PCP_ERR_INVALID_ARG, "optimizer is NULL");
  pcp_ctx* ctx = opt->ctx;
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  hipStream_t st = static_cast<hipStream_t>(stream);
  zero_kernel<<<grid_for(opt->total, 256 * 8), 256, 0, st>>>(opt->vel, opt->total);
  if ((e = hipGetLastError()) != hipSuccess) return hip_fail(ctx, e, "zeroing velocities");
  return sync_only(ctx, st);
}

int pcp_nesterov_update(pcp_nesterov* opt, int index, float* param, const float* grad, int64_t count, void* stream) {
  if (!opt) return fail(nullptr, PCP_ERR_INVALID_ARG, "optimizer is NULL");
  pcp_ctx* ctx = opt->ctx;
  if (index < 0 || index >= static_cast<int>(opt->counts.size()))
    return fail(ctx, PCP_ERR_OUT_OF_BOUNDS, "tensor index %d outside [0, %zu)", index, opt->counts.size());
  if (count != opt->counts[index])
    return fail(ctx, PCP_ERR_DIMENSION_MISMATCH, "tensor %d has %lld elements, got %lld", index,
                (long long)opt->counts[index], (long long)count);
  if (count > 0 && (!param || !grad)) return fail(ctx, PCP_ERR_INVALID_ARG, "param / grad is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (count == 0) return PCP_OK;
  if ((e = launch_nesterov(opt, param, opt->vel + opt->offsets[index], grad, nullptr, count, st)) != hipSuccess)
    return hip_fail(ctx, e, "Nesterov launch");
  return sync_only(ctx, st);
}

int pcp_nesterov_update_flat(pcp_nesterov* opt, float* params, const float* grads, void* param_bf16, void* stream) {
  if (!opt) return fail(nullptr, PCP_ERR_INVALID_ARG, "optimizer is NULL");
  pcp_ctx* ctx = opt->ctx;
  if (opt->total > 0 && (!params || !grads)) return fail(ctx, PCP_ERR_INVALID_ARG, "params / grads is NULL");
  if (reinterpret_cast<uintptr_t>(param_bf16) & 1u) return fail(ctx, PCP_ERR_INVALID_ARG, "param_bf16 is misaligned");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (opt->total == 0) return PCP_OK;
  const bool timed = prof_begin(ctx, st);
  e = launch_nesterov(opt, params, opt->vel, grads, static_cast<uint16_t*>(param_bf16), opt->total, st);
  prof_end(ctx, st, timed);
  if (e != hipSuccess) return hip_fail(ctx, e, "Nesterov launch");
  return sync_only(ctx, st);
}

int64_t pcp_nesterov_total(const pcp_nesterov* opt) { return opt ? opt->total : PCP_ERR_INVALID_ARG; }

int pcp_nesterov_serialize(pcp_nesterov* opt, void* host, size_t bytes) {
  if (!opt) return fail(nullptr, PCP_ERR_INVALID_ARG, "optimizer is NULL");
  pcp_ctx* ctx = opt->ctx;
  const size_t need = sizeof(float) * static_cast<size_t>(opt->total);
  if (!host || bytes < need) return fail(ctx, PCP_ERR_INVALID_ARG, "host buffer needs %zu bytes", need);
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess && need) e = hipMemcpy(host, opt->vel, need, hipMemcpyDeviceToHost);
  return e == hipSuccess ? PCP_OK : hip_fail(ctx, e, "copying velocities");
}

int pcp_nesterov_deserialize(pcp_nesterov* opt, const void* host, size_t bytes) {
  if (!opt) return fail(nullptr, PCP_ERR_INVALID_ARG, "optimizer is NULL");
  pcp_ctx* ctx = opt->ctx;
  const size_t need = sizeof(float) * static_cast<size_t>(opt->total);
  if (bytes < need) return fail(ctx, PCP_ERR_CORRUPT_STATE, "state holds %zu bytes, the velocities need %zu", bytes, need);
  if (!host && need) return fail(ctx, PCP_ERR_INVALID_ARG, "host is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess && need) e = hipMemcpy(opt->vel, host, need, hipMemcpyHostToDevice);
  return e == hipSuccess ? PCP_OK : hip_fail(ctx, e, "copying velocities");
}

}  // extern "C"
