// The rollout sampler on the GPU (pcp_sample.h): Sampler.sample
// (src/core/math.zig:21-58) over rows of logits in HBM.
//
// A row is cut into blocks of 64 lanes x 16 bytes (256 f32 or 512 bf16 logits).
// Partials (kBlocksPerWg blocks per workgroup, so a batch of rows fills the chip): per
// block (max, sum 2^((x - max) * k)), k = log2(e) / T, or for greedy rows the first
// maximum of each workgroup's span, into scratch. Selection (one wave per row): rescale
// the block sums to the row max, find the block where the running sum reaches
// u * total, re-read that block alone and scan it. HBM traffic: one read of the row +
// one block. Up to kOneLaunchMaxRows rows run both in one launch (`sample_kernel`: the
// workgroup that finishes a row last, by a per-row ticket, selects); larger batches in
// two (`sample_part_kernel`, `sample_select_kernel`).

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "context.hpp"
#include "grpo_device.hpp"
#include "pcp_sample.h"

namespace pcp {
namespace {

// Pass 1 runs 512-lane workgroups: at 64 rows of 151,936 f32 the two passes take
// 16.1-16.3 us against 17.4-17.9 us with 1024 lanes (256 lanes: 16.2-16.4 us).
constexpr int kWaves = 8;
constexpr int kBlocksPerWave = 4;          // loaded together: 4 KB in flight per wave
constexpr int kBlocksPerWg = kWaves * kBlocksPerWave;

struct SampleArgs {
  const void* logits;
  int64_t n_rows, vocab, row_stride;      // row_stride in elements
  float k;                                // log2(e) / temperature
  int greedy;
  const float* uniforms;
  int64_t* ids;
  float2* part;                           // [n_rows, nb] block (max, sum); greedy: [n_rows, nwg]
  int64_t* part_idx;                      // greedy: [n_rows, nwg] first-maximum index
  int* ticket;                            // [n_rows] workgroups done per row; 0 between launches
  int nb, nwg;
};

template <typename TI>
__device__ __forceinline__ const void* row_ptr(const SampleArgs& a, int64_t row) {
  return static_cast<const char*>(a.logits) + row * a.row_stride * TI::kBytes;
}

// The row's descriptor covers its whole dwords only (the range check is per dword), so
// no load reaches past the row: the last element of an odd bf16 row shares its dword
// with the bytes after the row and is read on its own (load_block).
template <typename TI>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_buffer(const SampleArgs& a, int64_t row) {
  return row_rsrc(row_ptr<TI>(a, row), static_cast<uint32_t>(a.vocab * TI::kBytes) & ~3u);
}

// A partial handed to the row's last workgroup (see store_coherent): one 8-byte
// coherent store.
__device__ __forceinline__ void put_part(float2* p, float2 v) {
  store_coherent(reinterpret_cast<uint64_t*>(p), __builtin_bit_cast(uint64_t, v));
}

// Lane `lane`'s EPL elements of 64-lane block b of a row (-inf past `vocab`).
template <typename TI>
__device__ __forceinline__ void load_block(__amdgpu_buffer_rsrc_t r, const void* row, int64_t vocab, int64_t b,
                                           int lane, float (&x)[16 / TI::kBytes]) {
  constexpr int EPL = 16 / TI::kBytes;
  const int64_t e0 = b * (64 * EPL) + static_cast<int64_t>(lane) * EPL;
  const u32x4 w = buf_ld16<true>(r, static_cast<uint32_t>(e0 * TI::kBytes));
  const uint32_t ws[4] = {w[0], w[1], w[2], w[3]};
#pragma unroll
  for (int j = 0; j < EPL; ++j) x[j] = (e0 + j < vocab) ? TI::unpack(ws, j) : kNegInf;
  if constexpr (TI::kBytes == 2) {
    if (vocab & 1) {
#pragma unroll
      for (int j = 0; j < EPL; ++j)
        if (e0 + j == vocab - 1) x[j] = TI::load1(row, vocab - 1);
    }
  }
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Greedy: (value, index), larger value wins, equal values the smaller index (the
// reference's strict '>' scan keeps the first maximum; NaN never compares greater,
// and -inf never beats the initial -inf, so such rows keep index 0).
__device__ __forceinline__ void better(float& v, int64_t& i, float v2, int64_t i2) {
  if (v2 > v || (v2 == v && v2 > kNegInf && i2 < i)) {
    v = v2;
    i = i2;
  }
}

__device__ __forceinline__ void wave_better(float& v, int64_t& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(v, o);
    const int64_t i2 = __shfl_xor(i, o);
    better(v, i, v2, i2);
  }
}

// Partials of workgroup (g, row): blocks [g*kBlocksPerWg, (g+1)*kBlocksPerWg).
template <typename TI>
__device__ __forceinline__ void sample_part(const SampleArgs& a, int64_t row, int g) {
  constexpr int EPL = 16 / TI::kBytes;
  constexpr int BLK = 64 * EPL;
  __shared__ float wv_max[kWaves];
  __shared__ int64_t wv_idx[kWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t V = a.vocab;
  const __amdgpu_buffer_rsrc_t r = row_buffer<TI>(a, row);
  const int64_t b0 = static_cast<int64_t>(g) * kBlocksPerWg + wave * kBlocksPerWave;
  float x[kBlocksPerWave][EPL];
#pragma unroll
  for (int u = 0; u < kBlocksPerWave; ++u)
    load_block<TI>(r, row_ptr<TI>(a, row), b0 + u < a.nb ? V : 0, b0 + u, lane, x[u]);
  if (a.greedy) {
    float best = kNegInf;
    int64_t bi = V;                                  // no value above -inf yet
#pragma unroll
    for (int u = 0; u < kBlocksPerWave; ++u)
#pragma unroll
      for (int j = 0; j < EPL; ++j) better(best, bi, x[u][j], (b0 + u) * BLK + static_cast<int64_t>(lane) * EPL + j);
    wave_better(best, bi);
    if (lane == 0) {
      wv_max[wave] = best;
      wv_idx[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float v = kNegInf;
      int64_t i = V;
      for (int w = 0; w < kWaves; ++w) better(v, i, wv_max[w], wv_idx[w]);
      put_part(a.part + row * a.nwg + g, make_float2(v, 0.f));
      store_coherent(a.part_idx + row * a.nwg + g, i);
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < kBlocksPerWave; ++u) {
    float m = kNegInf;
#pragma unroll
    for (int j = 0; j < EPL; ++j) m = fmaxf(m, x[u][j]);
    m = wave_max(m);
    const float ref = ms_ref(m);                     // a block of -inf keeps sum 0
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) s += hw_exp2((x[u][j] - ref) * a.k);
    s = wave_sum(s);
    if (lane == 0 && b0 + u < a.nb) put_part(a.part + row * a.nb + b0 + u, make_float2(m, s));
  }
}

// The selection of one row, by one wave, from every workgroup's partials.
template <typename TI>
__device__ __forceinline__ void sample_select(const SampleArgs& a, int64_t row, int lane) {
  constexpr int EPL = 16 / TI::kBytes;
  constexpr int BLK = 64 * EPL;
  const int64_t V = a.vocab;
  if (a.greedy) {
    float v = kNegInf;
    int64_t i = V;
    for (int g = lane; g < a.nwg; g += 64)
      better(v, i, a.part[row * a.nwg + g].x, a.part_idx[row * a.nwg + g]);
    wave_better(v, i);
    if (lane == 0) a.ids[row] = (i == V) ? 0 : i;
    return;
  }
  const float2* p = a.part + row * a.nb;
  const int nb = a.nb;

  // Lane l owns a contiguous run of blocks [l0, l1). Runs of up to kRun blocks are
  // held in registers (loaded once, all in flight; static indices); longer runs
  // (vocabularies past 64 * kRun blocks) are read again from memory.
  constexpr int kRun = 16;
  const int per = (nb + 63) / 64, l0 = min(lane * per, nb), l1 = min(l0 + per, nb);
  const bool cached = per <= kRun;
  float2 q[kRun];
#pragma unroll
  for (int i = 0; i < kRun; ++i) q[i] = (cached && l0 + i < l1) ? p[l0 + i] : make_float2(kNegInf, 0.f);
  // Row max; block sums rescaled to it (f64).
  float M = kNegInf;
  if (cached) {
#pragma unroll
    for (int i = 0; i < kRun; ++i) M = fmaxf(M, q[i].x);
  } else {
    for (int b = l0; b < l1; ++b) M = fmaxf(M, p[b].x);
  }
  M = wave_max(M);
  auto scaled = [&](float2 v) {
    return v.y > 0.f ? static_cast<double>(v.y) * static_cast<double>(hw_exp2((v.x - M) * a.k)) : 0.0;
  };
  double mine = 0.0;
  bool bad = false;                                  // NaN logit in a block
  if (cached) {
#pragma unroll
    for (int i = 0; i < kRun; ++i) {
      bad |= !(q[i].y == q[i].y);
      mine += scaled(q[i]);
    }
  } else {
    for (int b = l0; b < l1; ++b) {
      const float2 v = p[b];
      bad |= !(v.y == v.y);
      mine += scaled(v);
    }
  }
  // The reference's sum is NaN for a NaN logit, a +Inf logit (inf - inf) or a row
  // of -Inf (-inf - -inf): it then falls through to vocab - 1 (math.zig:56).
  const bool nan_sum = __any(bad) || M == kNegInf || M == __builtin_inff();
  double before = mine;                              // inclusive scan over lanes
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double t = __shfl_up(before, o);
    if (lane >= o) before += t;
  }
  const double total = __shfl(before, 63);
  before -= mine;                                    // exclusive
  if (nan_sum || !(total > 0.0)) {
    if (lane == 0) a.ids[row] = V - 1;
    return;
  }
  const double t = static_cast<double>(a.uniforms[row]) * total;

  // The block where the running sum first reaches t.
  int hit = -1;
  double pre = before;
  if (cached) {
#pragma unroll
    for (int i = 0; i < kRun; ++i) {
      const double sb = scaled(q[i]);
      if (hit < 0 && l0 + i < l1) {
        if (pre + sb >= t) hit = l0 + i;
        else pre += sb;
      }
    }
  } else {
    for (int b = l0; b < l1; ++b) {
      const double sb = scaled(p[b]);
      if (pre + sb >= t) {
        hit = b;
        break;
      }
      pre += sb;
    }
  }
  const uint64_t found = __ballot(hit >= 0);
  if (!found) {
    if (lane == 0) a.ids[row] = V - 1;               // rounding past the last block
    return;
  }
  const int src = __builtin_ctzll(found);
  const int hb = __shfl(hit, src);
  const double hpre = __shfl(pre, src);

  // Re-read that block and scan it in element order.
  float x[EPL];
  load_block<TI>(row_buffer<TI>(a, row), row_ptr<TI>(a, row), V, hb, lane, x);
  double e[EPL], lane_sum = 0.0;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    e[j] = static_cast<double>(hw_exp2((x[j] - M) * a.k));
    lane_sum += e[j];
  }
  double incl = lane_sum;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double v = __shfl_up(incl, o);
    if (lane >= o) incl += v;
  }
  double c = hpre + (incl - lane_sum);
  int jhit = -1;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    c += e[j];
    if (jhit < 0 && c >= t) jhit = j;
  }
  const uint64_t lanes = __ballot(jhit >= 0);
  const int l = lanes ? __builtin_ctzll(lanes) : 0;
  const int jsel = __shfl(jhit, l);
  if (lane == 0)
    a.ids[row] = lanes ? static_cast<int64_t>(hb) * BLK + static_cast<int64_t>(l) * EPL + jsel
                       : min<int64_t>(V, static_cast<int64_t>(hb + 1) * BLK) - 1;   // rounding: the block's last
}

// One launch: workgroup (g, row) writes its partials (coherent stores, complete before
// its ticket), takes a ticket of its row, and the row's last workgroup selects with its
// first wave (after an acquire fence) and returns the ticket to 0 for the next launch.
// A single-row call (the reference's one row per generated token) thus costs one
// launch.
template <typename TI>
__global__ void __launch_bounds__(64 * kWaves) sample_kernel(SampleArgs a) {
  __shared__ int last;
  const int64_t row = blockIdx.y;
  sample_part<TI>(a, row, blockIdx.x);
  wait_stores();     // this wave's partials at the coherent level
  __syncthreads();   // ... every wave's, before the ticket
  if (threadIdx.x == 0) last = atomicAdd(a.ticket + row, 1) == a.nwg - 1;
  __syncthreads();
  if (!last || threadIdx.x >= 64) return;
  acquire_coherent();
  sample_select<TI>(a, row, threadIdx.x);
  if (threadIdx.x == 0) a.ticket[row] = 0;
}

// Larger batches in two launches: the partials of every row, then one wave per row
// selects. At 64 rows of 151,936 f32 that measured 16.1-16.3 us against 20.2 us for the
// one-launch form, whose per-workgroup tickets cost more than the second launch saves
// once the grid is that large; at one row the one-launch form runs 7.9 us against
// 4.5 + 3.9 us of kernels and the gap between them.
constexpr int kOneLaunchMaxRows = 4;

template <typename TI>
__global__ void __launch_bounds__(64 * kWaves) sample_part_kernel(SampleArgs a) {
  sample_part<TI>(a, blockIdx.y, blockIdx.x);
}

template <typename TI>
__global__ void __launch_bounds__(64) sample_select_kernel(SampleArgs a) {
  sample_select<TI>(a, blockIdx.x, threadIdx.x);
}

template <typename TI>
hipError_t launch_sample(const SampleArgs& a, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(a.nwg), static_cast<unsigned>(a.n_rows));
  if (a.n_rows <= kOneLaunchMaxRows) {
    sample_kernel<TI><<<grid, dim3(64 * kWaves), 0, st>>>(a);
    return hipGetLastError();
  }
  sample_part_kernel<TI><<<grid, dim3(64 * kWaves), 0, st>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  sample_select_kernel<TI><<<dim3(static_cast<unsigned>(a.n_rows)), dim3(64), 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace
}  // namespace pcp

using namespace pcp;

namespace {

int sample_tokens(pcp_ctx* ctx, const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                  float temperature, const float* uniforms, int64_t* ids, void* stream, bool async) {
  if (dtype != PCP_F32 && dtype != PCP_BF16) return fail(ctx, PCP_ERR_DTYPE, "logits must be f32 or bf16");
  if (n_rows < 1 || n_rows > 65535 || vocab < 1 || vocab > PCP_SAMPLE_MAX_VOCAB || row_stride < vocab)
    return fail(ctx, PCP_ERR_INVALID_ARG, "need 1 <= n_rows <= 65535, 1 <= vocab <= %d, row_stride >= vocab",
                PCP_SAMPLE_MAX_VOCAB);
  const int esize = dtype == PCP_F32 ? 4 : 2;
  if (!logits || !ids) return fail(ctx, PCP_ERR_INVALID_ARG, "logits / ids is NULL");
  if ((reinterpret_cast<uintptr_t>(logits) & 15u) || ((row_stride * esize) & 15))
    return fail(ctx, PCP_ERR_INVALID_ARG, "logits rows must start on 16-byte boundaries");
  // math.zig:23: greedy only when temperature < 1e-6. A NaN temperature takes the
  // sampling path there: every term is NaN, no cumulative sum reaches the threshold and
  // the row gives len - 1, as it does here (the scale log2(e)/T is NaN).
  const bool greedy = temperature < 1e-6f;
  if (!greedy && !uniforms)
    return fail(ctx, PCP_ERR_INVALID_ARG, "uniforms is NULL and temperature is not below 1e-6");
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t blk = dtype == PCP_F32 ? 256 : 512;
  const int nb = static_cast<int>((vocab + blk - 1) / blk);
  const int nwg = (nb + kBlocksPerWg - 1) / kBlocksPerWg;
  const size_t o_idx = (sizeof(float2) * static_cast<size_t>(n_rows) * nb + 255) & ~static_cast<size_t>(255);
  int rc = ensure_scratch(ctx, o_idx + sizeof(int64_t) * static_cast<size_t>(n_rows) * nwg);
  if (rc != PCP_OK) return rc;
  char* sp = static_cast<char*>(ctx->scratch);
  // The per-row tickets: allocated and zeroed on the context's first sampler call, then
  // left at zero by every launch.
  if (!ctx->sample_ticket) {
    if ((e = hipMalloc(&ctx->sample_ticket, sizeof(int) * (PCP_SAMPLE_MAX_ROWS + 1))) != hipSuccess) {
      ctx->sample_ticket = nullptr;
      (void)hipGetLastError();
      return fail(ctx, PCP_ERR_OOM, "hipMalloc of the sampler's row tickets failed");
    }
    if ((e = hipMemsetAsync(ctx->sample_ticket, 0, sizeof(int) * (PCP_SAMPLE_MAX_ROWS + 1), st)) != hipSuccess)
      return hip_fail(ctx, e, "zeroing the sampler's row tickets");
  }
  SampleArgs a{logits, n_rows, vocab, row_stride, greedy ? 0.f : kLog2e / temperature, greedy ? 1 : 0, uniforms, ids,
               reinterpret_cast<float2*>(sp), reinterpret_cast<int64_t*>(sp + o_idx), ctx->sample_ticket, nb, nwg};
  const bool timed = prof_begin(ctx, st);
  e = dtype == PCP_F32 ? launch_sample<F32T>(a, st) : launch_sample<BF16T>(a, st);
  prof_end(ctx, st, timed);
  if (e != hipSuccess) return hip_fail(ctx, e, "sampler launch");
  if (async) return add_pending(ctx, st);
  if ((e = hipStreamSynchronize(st)) != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  return PCP_OK;
}

}  // namespace

extern "C" int pcp_sample_tokens(pcp_ctx* ctx, const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                                 int64_t row_stride, float temperature, const float* uniforms, int64_t* ids,
                                 void* stream) {
  return sample_tokens(ctx, logits, dtype, n_rows, vocab, row_stride, temperature, uniforms, ids, stream, false);
}

extern "C" int pcp_sample_tokens_async(pcp_ctx* ctx, const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                                       int64_t row_stride, float temperature, const float* uniforms, int64_t* ids,
                                       void* stream) {
  return sample_tokens(ctx, logits, dtype, n_rows, vocab, row_stride, temperature, uniforms, ids, stream, true);
}
