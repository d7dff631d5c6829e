// Seeded synthetic GRPO inputs generated in HBM (see include/pcp_synth.h).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "context.hpp"
#include "pcp_grpo.h"
#include "pcp_synth.h"

namespace pcp {
namespace {

// Philox4x32-10, Salmon et al. SC'11: 10 rounds of two 32x32->64 multiplies with
// the published multipliers and Weyl key increments.
__host__ __device__ inline void philox(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                       uint32_t k1, uint32_t out[4]) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = static_cast<uint64_t>(M0) * c0;
    const uint64_t p1 = static_cast<uint64_t>(M1) * c2;
    const uint32_t hi0 = static_cast<uint32_t>(p0 >> 32), lo0 = static_cast<uint32_t>(p0);
    const uint32_t hi1 = static_cast<uint32_t>(p1 >> 32), lo1 = static_cast<uint32_t>(p1);
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
    k0 += W0;
    k1 += W1;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

// Uniform in (0, 1): (x + 0.5) * 2^-32.
__device__ inline float u01(uint32_t x) { return (static_cast<float>(x) + 0.5f) * 2.3283064365386963e-10f; }

// Four standard normals for elements [4q, 4q+4) of tensor `tag`.
__device__ inline void normals4(uint64_t q, uint32_t tag, uint64_t seed, float z[4]) {
  uint32_t u[4];
  philox(static_cast<uint32_t>(q), static_cast<uint32_t>(q >> 32), tag, 0u, static_cast<uint32_t>(seed),
         static_cast<uint32_t>(seed >> 32), u);
  const float two_pi = 6.283185307179586f;
  const float r0 = sqrtf(-2.f * logf(u01(u[0])));
  const float r1 = sqrtf(-2.f * logf(u01(u[2])));
  float s0, c0, s1, c1;
  sincosf(two_pi * u01(u[1]), &s0, &c0);
  sincosf(two_pi * u01(u[3]), &s1, &c1);
  z[0] = r0 * c0;
  z[1] = r0 * s0;
  z[2] = r1 * c1;
  z[3] = r1 * s1;
}

template <typename T>
__device__ inline T cvt(float x);
template <>
__device__ inline float cvt<float>(float x) { return x; }
template <>
__device__ inline __bf16 cvt<__bf16>(float x) { return static_cast<__bf16>(x); }
template <>
__device__ inline _Float16 cvt<_Float16>(float x) { return static_cast<_Float16>(x); }

template <typename T>
__global__ void __launch_bounds__(256) synth_logits_kernel(T* policy, T* ref, int64_t n, float std_p, float std_r,
                                                           uint64_t seed) {
  const int64_t nq = (n + 3) / 4;
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; q < nq;
       q += static_cast<int64_t>(gridDim.x) * 256) {
    float zp[4], zr[4];
    normals4(q, 1u, seed, zp);
    if (ref) normals4(q, 2u, seed, zr);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t i = 4 * q + j;
      if (i < n) {
        const T p = cvt<T>(std_p * zp[j]);
        policy[i] = p;
        if (ref) ref[i] = cvt<T>(static_cast<float>(p) + std_r * zr[j]);
      }
    }
  }
}

template <typename T>
__global__ void __launch_bounds__(256) sample_tokens_kernel(const T* logits, int64_t vocab, uint64_t seed,
                                                            int64_t* ids) {
  __shared__ float sv[4];
  __shared__ int64_t si[4];
  const int64_t row = blockIdx.x;
  const T* x = logits + row * vocab;
  float best = -__builtin_inff();
  int64_t bi = vocab;  // sentinel: larger than every index
  const int64_t base = row * vocab;
  // Elements are visited in groups of 4 consecutive flat indices sharing one Philox call.
  const int64_t q0 = base / 4, q1 = (base + vocab + 3) / 4;
  for (int64_t q = q0 + threadIdx.x; q < q1; q += 256) {
    uint32_t u[4];
    philox(static_cast<uint32_t>(q), static_cast<uint32_t>(q >> 32), 3u, 0u, static_cast<uint32_t>(seed),
           static_cast<uint32_t>(seed >> 32), u);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t flat = 4 * q + j;
      const int64_t v = flat - base;
      if (v >= 0 && v < vocab) {
        const float g = -logf(-logf(u01(u[j])));
        const float val = static_cast<float>(x[v]) + g;
        if (val > best || (val == best && v < bi)) {
          best = val;
          bi = v;
        }
      }
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int64_t oi = __shfl_xor(bi, off);
    if (ov > best || (ov == best && oi < bi)) {
      best = ov;
      bi = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = best;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    best = sv[0];
    bi = si[0];
    for (int w = 1; w < 4; ++w)
      if (sv[w] > best || (sv[w] == best && si[w] < bi)) {
        best = sv[w];
        bi = si[w];
      }
    ids[row] = bi < vocab ? bi : 0;
  }
}

int launch_status(hipError_t e, const char* what) {
  return e == hipSuccess ? PCP_OK : hip_fail(nullptr, e, what);
}

}  // namespace
}  // namespace pcp

using namespace pcp;

extern "C" {

void pcp_synth_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  philox(ctr[0], ctr[1], ctr[2], ctr[3], key[0], key[1], out);
}

int pcp_synth_logits(void* policy, void* ref, int64_t n, int dtype, float std_p, float std_r, uint64_t seed,
                     void* stream) {
  if (!policy || n < 0) return fail(nullptr, PCP_ERR_INVALID_ARG, "pcp_synth_logits: bad arguments");
  if (n == 0) return PCP_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nq = (n + 3) / 4;
  const unsigned grid = static_cast<unsigned>(nq / 256 + 1 < 65536 ? nq / 256 + 1 : 65536);
  switch (dtype) {
    case PCP_BF16:
      synth_logits_kernel<__bf16><<<grid, 256, 0, st>>>(static_cast<__bf16*>(policy), static_cast<__bf16*>(ref), n,
                                                        std_p, std_r, seed);
      break;
    case PCP_F16:
      synth_logits_kernel<_Float16><<<grid, 256, 0, st>>>(static_cast<_Float16*>(policy),
                                                          static_cast<_Float16*>(ref), n, std_p, std_r, seed);
      break;
    case PCP_F32:
      synth_logits_kernel<float><<<grid, 256, 0, st>>>(static_cast<float*>(policy), static_cast<float*>(ref), n,
                                                       std_p, std_r, seed);
      break;
    default:
      return fail(nullptr, PCP_ERR_DTYPE, "pcp_synth_logits: dtype %d", dtype);
  }
  return launch_status(hipGetLastError(), "pcp_synth_logits launch");
}

int pcp_synth_sample_tokens(const void* logits, int dtype, int64_t nrows, int64_t vocab, uint64_t seed, int64_t* ids,
                            void* stream) {
  if (!logits || !ids || nrows < 0 || vocab < 1 || nrows > INT32_MAX)
    return fail(nullptr, PCP_ERR_INVALID_ARG, "pcp_synth_sample_tokens: bad arguments");
  if (nrows == 0) return PCP_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>(nrows);
  switch (dtype) {
    case PCP_BF16:
      sample_tokens_kernel<__bf16><<<grid, 256, 0, st>>>(static_cast<const __bf16*>(logits), vocab, seed, ids);
      break;
    case PCP_F16:
      sample_tokens_kernel<_Float16><<<grid, 256, 0, st>>>(static_cast<const _Float16*>(logits), vocab, seed, ids);
      break;
    case PCP_F32:
      sample_tokens_kernel<float><<<grid, 256, 0, st>>>(static_cast<const float*>(logits), vocab, seed, ids);
      break;
    default:
      return fail(nullptr, PCP_ERR_DTYPE, "pcp_synth_sample_tokens: dtype %d", dtype);
  }
  return launch_status(hipGetLastError(), "pcp_synth_sample_tokens launch");
}

}  // extern "C"
