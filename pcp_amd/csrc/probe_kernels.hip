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
//
// MFMA probe (pcp_mfma_peak): the bf16 matrix rate that register-resident
// v_mfma_f32_32x32x16_bf16 or v_mfma_f32_16x16x32_bf16 reaches with the tile kernel's
// wave shape and occupancy (eight waves per workgroup, two per SIMD, a 128 x 64 block
// of accumulators per wave), no memory traffic at all. The spec's 2.5 PFLOP/s assumes
// 2.4 GHz; under sustained MFMA load the clock is held lower by the power limit, and
// this probe measures where the rate settles for each shape.

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
  // The read kernel keeps its loads by a store that a lane makes only when the XOR of
  // its own vectors is all ones (never for the probes' data; several lanes may store
  // then, all to the same word).
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

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMfmaWaves = 8;

// Pseudo-random bf16 in [-1, 1): element idx of the probe's operands (the same on every
// wave), a murmur3-style mix of (seed, idx) mapped to a float and truncated to bf16.
__device__ __forceinline__ __bf16 probe_bf16(uint32_t seed, uint32_t idx) {
  uint32_t x = seed ^ (idx * 0x9E3779B9u);
  x ^= x >> 16;
  x *= 0x85EBCA6Bu;
  x ^= x >> 13;
  x *= 0xC2B2AE35u;
  x ^= x >> 16;
  const float f = static_cast<float>(static_cast<int32_t>(x >> 8) - (1 << 23)) * (1.f / (1 << 23));
  return __builtin_bit_cast(__bf16, static_cast<uint16_t>(__builtin_bit_cast(uint32_t, f) >> 16));
}

// Each wave: operand sets s = 0, 1 of 4 A fragments (element idx ((s*4 + i)*64 + lane)*8
// + e) and 2 B fragments (4096 + ((s*2 + j)*64 + lane)*8 + e), then `iters` rounds of the
// 8 products acc[i][j] += A_s[i] B_s[j], s alternating (iters even).
__global__ void __launch_bounds__(64 * kMfmaWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
mfma_peak_kernel(int iters, uint32_t seed, float* out, uint64_t* clocks) {
  const int lane = threadIdx.x & 63;
  bf16x8 a[2][4], b[2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
#pragma unroll
      for (int i = 0; i < 4; ++i) a[s][i][e] = probe_bf16(seed, ((s * 4 + i) * 64 + lane) * 8 + e);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[s][j][e] = probe_bf16(seed, 4096 + ((s * 2 + j) * 64 + lane) * 8 + e);
    }
  }
  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  __builtin_amdgcn_sched_barrier(0);
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_sched_barrier(0);
  for (int it = 0; it < iters; it += 2) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s][i], b[s][j], acc[i][j], 0, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_sched_barrier(0);
  if (blockIdx.x == 0 && threadIdx.x < 64) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) out[((i * 2 + j) * 16 + r) * 64 + lane] = acc[i][j][r];
  } else {
    // Every other wave keeps its products by a store that only a NaN sum would make. None
    // occurs: the operands lie in [-1, 1), so |acc| <= 16 * iters stays far below the f32
    // range for any int iters.
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) sum += acc[i][j][r];
    if (sum != sum) out[lane] = sum;
  }
  if (clocks && threadIdx.x == 0) {
    uint64_t* c = clocks + 4 * static_cast<int64_t>(blockIdx.x);
    c[0] = t0;
    c[1] = t1;
    c[2] = r0;
    c[3] = r1;
  }
}

// The same with v_mfma_f32_16x16x32_bf16 (16384 flops each): operand sets s = 0, 1 of 8 A
// fragments (element ((s*8 + i)*64 + lane)*8 + e) and 4 B fragments (8192 + ((s*4 + j)*64
// + lane)*8 + e), 32 products acc[i][j] += A_s[i] B_s[j] per round (twice the flops of a
// 32x32x16 round).
__global__ void __launch_bounds__(64 * kMfmaWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
mfma_peak16_kernel(int iters, uint32_t seed, float* out, uint64_t* clocks) {
  const int lane = threadIdx.x & 63;
  bf16x8 a[2][8], b[2][4];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
#pragma unroll
      for (int i = 0; i < 8; ++i) a[s][i][e] = probe_bf16(seed, ((s * 8 + i) * 64 + lane) * 8 + e);
#pragma unroll
      for (int j = 0; j < 4; ++j) b[s][j][e] = probe_bf16(seed, 8192 + ((s * 4 + j) * 64 + lane) * 8 + e);
    }
  }
  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.f;
  __builtin_amdgcn_sched_barrier(0);
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_sched_barrier(0);
  for (int it = 0; it < iters; it += 2) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[s][i], b[s][j], acc[i][j], 0, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_sched_barrier(0);
  if (blockIdx.x == 0 && threadIdx.x < 64) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) out[((i * 4 + j) * 4 + r) * 64 + lane] = acc[i][j][r];
  } else {
    // As in mfma_peak_kernel: |acc| <= 32 * iters, so the NaN store never happens.
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) sum += acc[i][j][r];
    if (sum != sum) out[lane] = sum;
  }
  if (clocks && threadIdx.x == 0) {
    uint64_t* c = clocks + 4 * static_cast<int64_t>(blockIdx.x);
    c[0] = t0;
    c[1] = t1;
    c[2] = r0;
    c[3] = r1;
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
  // The flat grid launches one lane per vpt vectors: at most 2^32 - 1 lanes.
  if ((bytes / 16 + kThreads * vpt - 1) / (kThreads * vpt) * kThreads >= (int64_t{1} << 32))
    return fail(ctx, PCP_ERR_INVALID_ARG,
                "pcp_hbm_stream: %lld bytes at vectors_per_lane %d need 2^32 lanes or more: raise vectors_per_lane",
                (long long)bytes, vpt);
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

extern "C" int pcp_mfma_peak(pcp_ctx* ctx, int shape, int workgroups, int iters, uint32_t seed, float* out,
                             uint64_t* clocks, void* stream) {
  using namespace pcp;
  if (shape != 0 && shape != 1)
    return fail(ctx, PCP_ERR_INVALID_ARG, "pcp_mfma_peak: shape must be 0 (32x32x16) or 1 (16x16x32)");
  if (workgroups < 1 || workgroups > (1 << 20) || iters < 2 || iters % 2 != 0)
    return fail(ctx, PCP_ERR_INVALID_ARG, "pcp_mfma_peak: workgroups must be in [1, 2^20] and iters even and >= 2");
  if (!out || (reinterpret_cast<uintptr_t>(out) & 3u) || (reinterpret_cast<uintptr_t>(clocks) & 7u))
    return fail(ctx, PCP_ERR_INVALID_ARG, "pcp_mfma_peak: out is NULL or a buffer is misaligned");
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool timed = prof_begin(ctx, st);
  if (shape == 0)
    mfma_peak_kernel<<<dim3(static_cast<unsigned>(workgroups)), dim3(64 * kMfmaWaves), 0, st>>>(iters, seed, out,
                                                                                               clocks);
  else
    mfma_peak16_kernel<<<dim3(static_cast<unsigned>(workgroups)), dim3(64 * kMfmaWaves), 0, st>>>(iters, seed, out,
                                                                                                 clocks);
  e = hipGetLastError();
  prof_end(ctx, st, timed);
  if (e != hipSuccess) return hip_fail(ctx, e, "pcp_mfma_peak launch");
  return PCP_OK;
}
