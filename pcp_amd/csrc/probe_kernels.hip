// HBM stream probes (pcp_hbm_stream): the bandwidth that plain streaming kernels reach
// on this device for the access mixes of the library's kernels, so their roofline
// fractions can be read against a measured practical roof as well as the 8 TB/s spec.
//
//   read   a -> (nothing kept)          bytes moved: n
//   write  pattern -> c                 n
//   copy   a -> c                       2 n
//   mix    a, b -> c = a ^ b            3 n  (two reads per write: the row kernel's policy
//                                             + reference logits in, dlogits out)
//
// Each kind comes plain or with nontemporal loads and stores (the streaming hint the
// row kernel uses), over a flat grid: each 256-lane workgroup moves 256 x VPT 16-byte
// vectors, VPT = 1, 2, 4 or 8 per lane. One vector per lane writes fastest (6.8 TB/s
// against 5.6-5.8 TB/s for a grid of 32 workgroups per CU striding 8 per lane), so the
// benchmark reports the best shape of each kind.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "context.hpp"
#include "grpo_device.hpp"
#include "pcp_grpo.h"
#include "pcp_probe.h"

namespace pcp {
namespace {

constexpr int kThreads = 256;

template <bool NT>
__device__ __forceinline__ u32x4 ld(const u32x4* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  return *p;
}
template <bool NT>
__device__ __forceinline__ void st(u32x4* p, u32x4 v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// KIND: 0 read, 1 write, 2 copy, 3 mix. Workgroup w moves vectors [w * 256 * VPT, ...),
// lane t the ones at t + 256 k (coalesced per instruction).
template <int KIND, bool NT, int VPT>
__global__ void __launch_bounds__(kThreads) hbm_stream_kernel(const u32x4* a, const u32x4* b, u32x4* c, int64_t n16,
                                                              u32x4* sink) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * VPT + threadIdx.x;
  u32x4 x[VPT], y[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int64_t i = base + k * kThreads;
    if (i < n16) {
      if constexpr (KIND == 0 || KIND == 2 || KIND == 3) x[k] = ld<NT>(a + i);
      if constexpr (KIND == 3) y[k] = ld<NT>(b + i);
    }
  }
  u32x4 acc = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int64_t i = base + k * kThreads;
    if (i < n16) {
      if constexpr (KIND == 0) acc ^= x[k];
      if constexpr (KIND == 1) st<NT>(c + i, u32x4{static_cast<uint32_t>(i), 1u, 2u, 3u});
      if constexpr (KIND == 2) st<NT>(c + i, x[k]);
      if constexpr (KIND == 3) st<NT>(c + i, x[k] ^ y[k]);
    }
  }
  // The read kernel keeps its loads by a store that only an all-ones XOR would make.
  if constexpr (KIND == 0)
    if (acc[0] == 0xFFFFFFFFu && acc[1] == 0xFFFFFFFFu && acc[2] == 0xFFFFFFFFu && acc[3] == 0xFFFFFFFFu) *sink = acc;
}

template <int KIND, bool NT, int VPT>
hipError_t launch(const void* a, const void* b, void* c, int64_t n16, hipStream_t st) {
  const int64_t grid = (n16 + kThreads * VPT - 1) / (kThreads * VPT);
  hbm_stream_kernel<KIND, NT, VPT><<<dim3(static_cast<unsigned>(grid)), kThreads, 0, st>>>(
      static_cast<const u32x4*>(a), static_cast<const u32x4*>(b), static_cast<u32x4*>(c), n16, static_cast<u32x4*>(c));
  return hipGetLastError();
}

template <int KIND, bool NT>
hipError_t launch_vpt(int vpt, const void* a, const void* b, void* c, int64_t n16, hipStream_t st) {
  switch (vpt) {
    case 1: return launch<KIND, NT, 1>(a, b, c, n16, st);
    case 2: return launch<KIND, NT, 2>(a, b, c, n16, st);
    case 4: return launch<KIND, NT, 4>(a, b, c, n16, st);
    default: return launch<KIND, NT, 8>(a, b, c, n16, st);
  }
}

}  // namespace
}  // namespace pcp

extern "C" int pcp_hbm_stream(pcp_ctx* ctx, int kind, int nontemporal, int vectors_per_lane, const void* a,
                              const void* b, void* c, int64_t bytes, void* stream) {
  using namespace pcp;
  if (kind < 0 || kind > 3 || bytes < 16 || bytes % 16 != 0 || bytes / 16 > (int64_t{1} << 38))
    return fail(ctx, PCP_ERR_INVALID_ARG, "pcp_hbm_stream: kind must be 0..3 and bytes a positive multiple of 16");
  const int vpt = vectors_per_lane;
  if (vpt != 1 && vpt != 2 && vpt != 4 && vpt != 8)
    return fail(ctx, PCP_ERR_INVALID_ARG, "pcp_hbm_stream: vectors_per_lane must be 1, 2, 4 or 8");
  const bool need_a = kind != 1, need_b = kind == 3, need_c = kind != 0;
  if ((need_a && !a) || (need_b && !b) || (need_c && !c) || (kind == 0 && !c) ||
      ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(c)) & 15u))
    return fail(ctx, PCP_ERR_INVALID_ARG, "pcp_hbm_stream: a buffer is NULL or not 16-byte aligned");
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  const int64_t n16 = bytes / 16;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool timed = prof_begin(ctx, st);
  switch (kind * 2 + (nontemporal ? 1 : 0)) {
    case 0: e = launch_vpt<0, false>(vpt, a, b, c, n16, st); break;
    case 1: e = launch_vpt<0, true>(vpt, a, b, c, n16, st); break;
    case 2: e = launch_vpt<1, false>(vpt, a, b, c, n16, st); break;
    case 3: e = launch_vpt<1, true>(vpt, a, b, c, n16, st); break;
    case 4: e = launch_vpt<2, false>(vpt, a, b, c, n16, st); break;
    case 5: e = launch_vpt<2, true>(vpt, a, b, c, n16, st); break;
    case 6: e = launch_vpt<3, false>(vpt, a, b, c, n16, st); break;
    default: e = launch_vpt<3, true>(vpt, a, b, c, n16, st); break;
  }
  prof_end(ctx, st, timed);
  if (e != hipSuccess) return hip_fail(ctx, e, "pcp_hbm_stream launch");
  return PCP_OK;
}
