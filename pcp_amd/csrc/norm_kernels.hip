// The decoder's final RMSNorm fused around the LM head (pcp_lmhead_args.norm_weight).
//
// Qwen2RMSNorm (transformers' modeling_qwen2), the model.norm that
// tools/export_qwen_forward.py:112 applies to the last decoder layer's output before
// lm_head (:147):
//   r = 1 / sqrt(mean(h^2) + eps)     (f32)
//   y = gamma * bf16(h * r)           (the input dtype is bf16), rounded to bf16 as the
//                                     LM head's MFMA operand
// Backward (roundings pass gradients through, as a dtype cast does under autograd):
//   g = dy * gamma,  dh = r g - h (r^3 / H) sum_k g_k h_k,  dgamma = sum_rows dy * bf16(h r)
// so the gradient that leaves the LM head is the one the last block's VJP takes. dh is
// one block per token (dead tokens: zero rows); dgamma is column-parallel over slices of
// the live rows, then the slices are summed in a fixed order.
//
// The forward's sum of squares has a fixed order (each thread adds its columns
// tid, tid + 256, ... in turn; an xor butterfly over the wave; waves 0..3 in turn) and
// the square root and division are correctly rounded, so the bf16 operand is a
// function of the inputs that a CPU restatement reproduces bit for bit.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "lmhead_launch.hpp"

#pragma clang fp contract(off)

namespace pcp {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));   // round to nearest even
}
__device__ __forceinline__ float bf16_round(float x) { return static_cast<float>(static_cast<__bf16>(x)); }

// Sum over the 256 threads of the block in a fixed order: inside each wave an xor
// butterfly (lane i adds lane i ^ 32, then i ^ 16, ..., i ^ 1; every lane ends with
// the same value), then (w0 + w1) + w2 + w3.
__device__ __forceinline__ float block_sum_fixed(float v, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float s = ((red[0] + red[1]) + red[2]) + red[3];
  __syncthreads();   // red is rewritten by the next call
  return s;
}

// One block per live row c < *count (token live[c]): y[c] = bf16(gamma * bf16(h * r)),
// rstd[c] = r. The grid covers every token; blocks past the live count return.
template <int PER>
__global__ void __launch_bounds__(256) lm_norm_rows_kernel(const uint16_t* __restrict__ h,
                                                           const float* __restrict__ gamma, float eps,
                                                           const int* __restrict__ live,
                                                           const int* __restrict__ count, int H,
                                                           uint16_t* __restrict__ y, float* __restrict__ rstd) {
  __shared__ float red[4];
  const int c = blockIdx.x;
  if (c >= *count) return;
  const uint16_t* hr = h + static_cast<int64_t>(live[c]) * H;
  float v[PER];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int k = threadIdx.x + 256 * i;
    v[i] = k < H ? bf16_to_f32(hr[k]) : 0.f;
    ss += v[i] * v[i];
  }
  const float r = 1.f / sqrtf(block_sum_fixed(ss, red) / static_cast<float>(H) + eps);
  uint16_t* yr = y + static_cast<int64_t>(c) * H;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int k = threadIdx.x + 256 * i;
    if (k < H) yr[k] = f32_to_bf16(gamma[k] * bf16_round(v[i] * r));
  }
  if (threadIdx.x == 0) rstd[c] = r;
}

// One block per token t: a dead token's dh row is zero; a live token's is formed from
// its compact dy row. Lanes take four adjacent columns (16-byte dy loads and dh stores,
// 8-byte h loads), PER4 groups of 1024 columns apart.
template <int PER4>
__global__ void __launch_bounds__(256) lm_norm_dx_kernel(LmNormBwdArgs a) {
  __shared__ float red[4];
  const int H = a.H, nv = H / 4;
  const int64_t t = blockIdx.x;
  const int c = a.cidx[t];
  f32x4* dhr = reinterpret_cast<f32x4*>(a.dh + t * H);
  if (c < 0) {
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < PER4; ++i) {
      const int j = threadIdx.x + 256 * i;
      if (j < nv) dhr[j] = z;
    }
    return;
  }
  const float r = a.rstd[c];
  const f32x4* dyr = reinterpret_cast<const f32x4*>(a.dyc + static_cast<int64_t>(c) * H);
  const u16x4* hr = reinterpret_cast<const u16x4*>(a.h + t * H);
  const f32x4* gm = reinterpret_cast<const f32x4*>(a.gamma);
  f32x4 gy[PER4], hv[PER4];
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < PER4; ++i) {
    const int j = threadIdx.x + 256 * i;
    gy[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    hv[i] = gy[i];
    if (j < nv) {
      const f32x4 dy = dyr[j], g = gm[j];
      const u16x4 hb = hr[j];
      hv[i] = f32x4{bf16_to_f32(hb.x), bf16_to_f32(hb.y), bf16_to_f32(hb.z), bf16_to_f32(hb.w)};
      gy[i] = f32x4{dy.x * g.x, dy.y * g.y, dy.z * g.z, dy.w * g.w};
      dot += gy[i].x * hv[i].x + gy[i].y * hv[i].y + gy[i].z * hv[i].z + gy[i].w * hv[i].w;
    }
  }
  const float s = r * r * r * (block_sum_fixed(dot, red) / static_cast<float>(H));
#pragma unroll
  for (int i = 0; i < PER4; ++i) {
    const int j = threadIdx.x + 256 * i;
    if (j < nv)
      dhr[j] = f32x4{r * gy[i].x - hv[i].x * s, r * gy[i].y - hv[i].y * s, r * gy[i].z - hv[i].z * s,
                     r * gy[i].w - hv[i].w * s};
  }
}

// dgamma partials: block (x, y) sums column k = 256 x + lane over live rows
// c = y, y + kLmNormSlices, ... : dy[c, k] * bf16(h[live[c], k] * r[c]) (the forward's
// rounded normalised value), written to gpart[y, k] (0 for slices past the live count).
// Lanes read consecutive columns.
__global__ void __launch_bounds__(256) lm_norm_dgamma_part_kernel(LmNormBwdArgs a) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  if (k >= a.H) return;
  const int H = a.H;
  const int n_live = *a.count;
  float acc = 0.f;
  for (int c = blockIdx.y; c < n_live; c += kLmNormSlices) {
    const float x = bf16_round(bf16_to_f32(a.h[static_cast<int64_t>(a.live[c]) * H + k]) * a.rstd[c]);
    acc += a.dyc[static_cast<int64_t>(c) * H + k] * x;
  }
  a.gpart[static_cast<int64_t>(blockIdx.y) * H + k] = acc;
}

__global__ void __launch_bounds__(256) lm_norm_dgamma_kernel(const float* __restrict__ gpart, int H,
                                                             float* __restrict__ dgamma) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  if (k >= H) return;
  float s = 0.f;
  for (int b = 0; b < kLmNormSlices; ++b) s += gpart[static_cast<int64_t>(b) * H + k];
  dgamma[k] = s;
}

template <int PER>
hipError_t norm_rows(const void* h, const float* gamma, float eps, const int* live, const int* count, int n, int H,
                     void* y, float* rstd, hipStream_t st) {
  lm_norm_rows_kernel<PER><<<dim3(n), dim3(256), 0, st>>>(static_cast<const uint16_t*>(h), gamma, eps, live, count,
                                                          H, static_cast<uint16_t*>(y), rstd);
  return hipGetLastError();
}

template <int PER4>
hipError_t norm_dx(const LmNormBwdArgs& a, hipStream_t st) {
  lm_norm_dx_kernel<PER4><<<dim3(static_cast<unsigned>(a.N)), dim3(256), 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_lm_norm_rows(const void* h, const float* gamma, float eps, const int* live, const int* count,
                               int n, int H, void* y, float* rstd, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  if (H <= 256) return norm_rows<1>(h, gamma, eps, live, count, n, H, y, rstd, st);
  if (H <= 512) return norm_rows<2>(h, gamma, eps, live, count, n, H, y, rstd, st);
  if (H <= 1024) return norm_rows<4>(h, gamma, eps, live, count, n, H, y, rstd, st);
  if (H <= 2048) return norm_rows<8>(h, gamma, eps, live, count, n, H, y, rstd, st);
  if (H <= 4096) return norm_rows<16>(h, gamma, eps, live, count, n, H, y, rstd, st);
  if (H <= kLmNormMaxHidden) return norm_rows<32>(h, gamma, eps, live, count, n, H, y, rstd, st);
  return hipErrorInvalidValue;
}

hipError_t launch_lm_norm_bwd(const LmNormBwdArgs& a, hipStream_t st) {
  hipError_t e = hipSuccess;
  if (a.dh) {
    if (a.H <= 1024) e = norm_dx<1>(a, st);
    else if (a.H <= 2048) e = norm_dx<2>(a, st);
    else if (a.H <= 4096) e = norm_dx<4>(a, st);
    else if (a.H <= kLmNormMaxHidden) e = norm_dx<8>(a, st);
    else return hipErrorInvalidValue;
    if (e != hipSuccess) return e;
  }
  if (!a.dgamma) return e;
  lm_norm_dgamma_part_kernel<<<dim3((a.H + 255) / 256, kLmNormSlices), dim3(256), 0, st>>>(a);
  lm_norm_dgamma_kernel<<<dim3((a.H + 255) / 256), dim3(256), 0, st>>>(a.gpart, a.H, a.dgamma);
  return hipGetLastError();
}

}  // namespace pcp
