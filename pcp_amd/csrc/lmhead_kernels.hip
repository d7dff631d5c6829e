// Fused LM-head + GRPO log-prob kernels (gfx950, bf16 MFMA).
//
// logits[n, v] = sum_h hidden[n, h] * W[v, h] is a dense contraction; the loss
// head only needs, per token, the log-sum-exp over v and the logit of its target
// (forward), and dlogits = c_n * (onehot - softmax) (backward). The tile kernel
// computes a 128 x 128 logits tile on v_mfma_f32_32x32x16_bf16 and reduces it in
// its epilogue, so full logits never exist in HBM:
//   kFwd  -> per (token, vocab tile) partial (max, sum 2^(x*log2e - max)) and the
//            target logit when the target falls in the tile;
//   kBwd  -> dlogits for one vocab chunk in bf16, for the dhidden / dW GEMMs.
//
// Reference: the LM head and loss of tools/export_qwen_forward.py:146-163
// (self.model.lm_head(hidden) then F.cross_entropy), and matmulVJP
// (src/autodiff/vjp_rules.zig:426-497) for dhidden = dlogits*W, dW = dlogits^T*hidden.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "grpo_device.hpp"
#include "lmhead_launch.hpp"

namespace pcp {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace lm {

constexpr int BM = 128;           // tokens per tile
constexpr int BN = 128;           // vocab entries per tile
constexpr int BK = 64;            // hidden (K) per LDS stage
constexpr int LDK = BK + 8;       // padded LDS row (bf16): conflict-free 16-byte fragment reads
constexpr int NTHR = 256;         // 4 waves: 2 (tokens) x 2 (vocab), 64 x 64 each
constexpr int LDC = BN + 4;       // padded fp32 tile row in the epilogue
constexpr int kStageElems = BM * LDK + BN * LDK;
constexpr size_t kSmemGemm = 2 * kStageElems * sizeof(__bf16);
constexpr size_t kSmemEpi = BM * LDC * sizeof(float);
constexpr size_t kSmem = kSmemGemm > kSmemEpi ? kSmemGemm : kSmemEpi;
constexpr int kGroupM = 8;        // token tiles per group in the tile order

}  // namespace lm

// Tile order: work item p -> (token tile, vocab tile). Consecutive workgroup ids
// are dealt round-robin to the 8 XCDs, so ids are first regrouped per XCD; within
// an XCD, groups of kGroupM token tiles sweep the vocab tiles together, so the
// workgroups resident on one XCD read the same operand K-slabs from its L2.
__device__ __forceinline__ bool lm_tile_coords(int pid, int ntt, int nvt, int& tm, int& tn) {
  const int total = ntt * nvt;
  const int per_xcd = (total + 7) / 8;
  const int p = (pid % 8) * per_xcd + pid / 8;
  if (p >= total) return false;
  const int group = lm::kGroupM * nvt;
  const int g = p / group;
  const int first_m = g * lm::kGroupM;
  const int gm = min(ntt - first_m, lm::kGroupM);
  const int q = p - g * group;
  tm = first_m + q % gm;
  tn = q / gm;
  return true;
}

template <int MODE>
__global__ void __launch_bounds__(lm::NTHR) lm_tile_kernel(LmTileArgs a) {
  using namespace lm;
  extern __shared__ __align__(16) char smem[];
  __bf16* sA = reinterpret_cast<__bf16*>(smem);             // [2][BM][LDK]
  __bf16* sB = sA + 2 * BM * LDK;                            // [2][BN][LDK]
  float* sC = reinterpret_cast<float*>(smem);                // [BM][LDC] after the K loop

  int tm, tn;
  if (!lm_tile_coords(blockIdx.x, a.ntt, a.nvt, tm, tn)) return;
  const int m0 = tm * BM;
  const int n0 = (a.vt0 + tn) * BN;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Operand row buffers: rows past N / V read 0 (range-checked lane offsets).
  const uint32_t rowbytes = static_cast<uint32_t>(a.H) * 2u;
  const int rows_a = min(BM, a.N - m0), rows_b = min(BN, a.V - n0);
  const __amdgpu_buffer_rsrc_t ra =
      row_rsrc(reinterpret_cast<const char*>(a.A) + static_cast<int64_t>(m0) * rowbytes, rows_a * rowbytes);
  const __amdgpu_buffer_rsrc_t rb =
      row_rsrc(reinterpret_cast<const char*>(a.B) + static_cast<int64_t>(n0) * rowbytes, rows_b * rowbytes);

  // Global -> LDS staging: thread t moves 16 bytes of rows t/8 + 32*i, k = (t%8)*8.
  const int lr = tid >> 3, lk = (tid & 7) * 8;
  u32x4 ga[4], gb[4];
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t off = static_cast<uint32_t>((lr + 32 * i)) * rowbytes + (kb * BK + lk) * 2u;
      ga[i] = buf_ld16<false>(ra, off);
      gb[i] = buf_ld16<false>(rb, off);
    }
  };
  auto lstore = [&](int buf) {
    __bf16* A = sA + buf * BM * LDK;
    __bf16* B = sB + buf * BN * LDK;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<u32x4*>(A + (lr + 32 * i) * LDK + lk) = ga[i];
      *reinterpret_cast<u32x4*>(B + (lr + 32 * i) * LDK + lk) = gb[i];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = a.H / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kb = 0; kb < nk; ++kb) {
    const int buf = kb & 1;
    if (kb + 1 < nk) gload(kb + 1);
    const __bf16* A = sA + buf * BM * LDK;
    const __bf16* B = sB + buf * BN * LDK;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int ko = kk * 16 + (lane >> 5) * 8;
      bf16x8 af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(A + (wm * 64 + i * 32 + (lane & 31)) * LDK + ko);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(B + (wn * 64 + j * 32 + (lane & 31)) * LDK + ko);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kb + 1 < nk) lstore(buf ^ 1);
    __syncthreads();
  }

  // Accumulators -> LDS tile [BM][LDC]. MFMA 32x32 result layout: lane l holds
  // column l%32 and rows 8*(r/4) + 4*(l/32) + r%4 of its 32 x 32 block.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wm * 64 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        const int col = wn * 64 + j * 32 + (lane & 31);
        sC[row * LDC + col] = acc[i][j][r];
      }
  __syncthreads();

  // Epilogue: two lanes per token row, 64 vocab columns each.
  const int row = tid >> 1, half = tid & 1;
  const int n = m0 + row;
  const int c0 = half * 64;
  const int ncols = min(max(a.V - n0 - c0, 0), 64);   // valid columns of this half
  const float* crow = sC + row * LDC + c0;
  if constexpr (MODE == kLmFwd) {
    float mx = kNegInf;
    for (int c = 0; c < ncols; ++c) mx = fmaxf(mx, crow[c]);
    float m2 = mx * kLog2e;
    const float ref = ms_ref(m2);
    float s = 0.f;
    for (int c = 0; c < ncols; ++c) s += hw_exp2(fmaf(crow[c], kLog2e, -ref));
    const float om = __shfl_xor(m2, 1), os = __shfl_xor(s, 1);
    ms_merge(m2, s, om, os);
    if (n < a.N) {
      if (half == 0) a.part[static_cast<int64_t>(n) * a.ldp + a.vt0 + tn] = make_float2(m2, s);
      const int64_t id = a.ids_i64 ? static_cast<const int64_t*>(a.ids)[n]
                                   : static_cast<int64_t>(static_cast<const int32_t*>(a.ids)[n]);
      const int64_t c = id - n0 - c0;
      if (c >= 0 && c < ncols) a.tgt[n] = crow[c];
    }
  } else {
    // dlogits[n, v] = coef_n * (onehot - 2^(x*log2e - lse2_n)), bf16, columns
    // relative to the chunk start; columns past V are written as 0 (chunk padding).
    if (n < a.N) {
      const float cf = a.coef[n], l2 = a.lse2[n];
      const int64_t id = a.ids_i64 ? static_cast<const int64_t*>(a.ids)[n]
                                   : static_cast<int64_t>(static_cast<const int32_t*>(a.ids)[n]);
      const int64_t rel = id - n0 - c0;
      uint16_t* out = reinterpret_cast<uint16_t*>(a.dchunk) + static_cast<int64_t>(n) * a.ldd + (n0 - a.vc0) + c0;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int c = q * 8 + e;
          float d = 0.f;
          if (c < ncols && cf != 0.f) {
            d = -cf * hw_exp2(fmaf(crow[c], kLog2e, -l2));
            if (c == rel) d += cf;
          }
          v[e] = d;
        }
        u32x4 w = {pack2<BF16T>(v[0], v[1]), pack2<BF16T>(v[2], v[3]), pack2<BF16T>(v[4], v[5]),
                   pack2<BF16T>(v[6], v[7])};
        if (n0 - a.vc0 + c0 + q * 8 < a.ldd) *reinterpret_cast<u32x4*>(out + q * 8) = w;
      }
    }
  }
}

// Per token: merge the vocab-tile partials into the base-2 log-sum-exp. One wave
// per token; the merge is commutative, so the xor butterfly is deterministic.
__global__ void __launch_bounds__(256) lm_reduce_kernel(LmReduceArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  if (n >= a.N) return;
  float m = kNegInf, s = 0.f;
  const float2* p = a.part + n * a.ldp;
  for (int t = lane; t < a.nvt; t += 64) {
    const float2 v = p[t];
    ms_merge(m, s, v.x, v.y);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float om = __shfl_xor(m, off), os = __shfl_xor(s, off);
    ms_merge(m, s, om, os);
  }
  if (lane == 0) a.lse2[n] = m + log2f(s);
}

// GRPO terms per token from logp / ref logp (token_terms); also masks logp for
// dead tokens and keeps the policy lse (base 2) and the coefficient for the backward.
__global__ void __launch_bounds__(256) lm_terms_kernel(RowArgs ra, LmTermsArgs a) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (n >= a.N) return;
  // row_meta reads ids / mask at the token's index (aligned layout) and validates the id.
  RowMeta r;
  {
    const int64_t s = n / ra.logit_stride;
    const int64_t t = n - s * ra.logit_stride;
    r.row = n;
    r.seq = static_cast<int32_t>(s);
    r.tok = t < ra.rows;
    r.tix = s * ra.tok_stride + ra.tok_offset + t;
    r.id = ra.ids_i64 ? static_cast<const int64_t*>(ra.ids)[r.tix]
                      : static_cast<int64_t>(static_cast<const int32_t*>(ra.ids)[r.tix]);
    if (ra.mask == nullptr) r.w = 1.f;
    else if (ra.mask_u8) r.w = static_cast<const uint8_t*>(ra.mask)[r.tix] ? 1.f : 0.f;
    else r.w = static_cast<const float*>(ra.mask)[r.tix];
    const bool in_range = r.id >= 0 && r.id < ra.vocab;
    if (r.w != 0.f && r.id != PCP_IGNORE_INDEX && !in_range) atomicOr(ra.err, kErrTokenRange);
    r.live = r.tok && r.w != 0.f && in_range;
  }
  float lp = 0.f, lr = 0.f;
  TokenTerms tt{0.f, 0.f};
  // Live tokens are exactly those the compaction kept (same predicate).
  const int c = a.cidx[n];
  if (r.live && c >= 0) {
    // Non-finite logits of a live token poison its log-sum-exp (NaN propagates
    // through the partial merges); flag it like the logits-input path does.
    const float l2 = a.lse2[c], rl2 = a.ref_tgt ? a.ref_lse2[c] : 0.f;
    if (!(__builtin_isfinite(l2) && __builtin_isfinite(rl2))) atomicOr(ra.err, kErrNonFinite);
    lp = a.tgt[c] - l2 * kLn2;
    lr = a.ref_tgt ? a.ref_tgt[c] - rl2 * kLn2 : 0.f;
    tt = token_terms(ra, r, lp, lr);
    a.coef[c] = tt.coef;
  }
  if (ra.logp) ra.logp[r.tix] = lp;
  if (ra.ref_logp) ra.ref_logp[r.tix] = lr;
  if (ra.token_loss) ra.token_loss[r.tix] = tt.loss;
}

// Live-token compaction in one workgroup: each pass ranks 1024 tokens with a
// ballot prefix per wave and a 16-entry wave scan in LDS, so the compact order is
// the token order (deterministic).
__global__ void __launch_bounds__(1024) lm_compact_kernel(LmCompactArgs a) {
  __shared__ int wsum[16];
  __shared__ int base_s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) base_s = 0;
  __syncthreads();
  for (int n0 = 0; n0 < a.N; n0 += 1024) {
    const int n = n0 + tid;
    bool live = false;
    int64_t id = -1;
    if (n < a.N) {
      id = a.ids_i64 ? static_cast<const int64_t*>(a.ids)[n] : static_cast<int64_t>(static_cast<const int32_t*>(a.ids)[n]);
      float w = 1.f;
      if (a.mask) w = a.mask_u8 ? (static_cast<const uint8_t*>(a.mask)[n] ? 1.f : 0.f) : static_cast<const float*>(a.mask)[n];
      live = w != 0.f && id >= 0 && id < a.V;
    }
    const uint64_t bal = __ballot(live);
    const int before = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0));
    if (lane == 0) wsum[wave] = __popcll(bal);
    __syncthreads();
    int off = base_s;
    for (int w = 0; w < wave; ++w) off += wsum[w];
    int total = 0;
    for (int w = 0; w < 16; ++w) total += wsum[w];
    if (n < a.N) {
      const int c = live ? off + before : -1;
      a.cidx[n] = c;
      if (live) {
        a.live[c] = n;
        a.ids_c[c] = static_cast<int>(id);
      }
    }
    __syncthreads();
    if (tid == 0) base_s += total;
    __syncthreads();
  }
  if (tid == 0) a.count[0] = base_s;
}

__global__ void __launch_bounds__(256) lm_gather_rows_kernel(const u32x4* src, u32x4* dst, const int* live, int H) {
  const int c = blockIdx.x;
  const int nv = H / 8;  // 16-byte vectors per bf16 row
  const u32x4* s = src + static_cast<int64_t>(live[c]) * nv;
  u32x4* d = dst + static_cast<int64_t>(c) * nv;
  for (int i = threadIdx.x; i < nv; i += 256) d[i] = s[i];
}

__global__ void __launch_bounds__(256) lm_scatter_rows_kernel(const u32x4* src, u32x4* dst, const int* cidx, int H) {
  const int t = blockIdx.x;
  const int nv = H / 4;  // 16-byte vectors per f32 row
  const int c = cidx[t];
  u32x4* d = dst + static_cast<int64_t>(t) * nv;
  if (c >= 0) {
    const u32x4* s = src + static_cast<int64_t>(c) * nv;
    for (int i = threadIdx.x; i < nv; i += 256) d[i] = s[i];
  } else {
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (int i = threadIdx.x; i < nv; i += 256) d[i] = z;
  }
}

__global__ void __launch_bounds__(256) lm_zero_kernel(float* dst, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    dst[i] = 0.f;
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
size_t lm_tile_smem_bytes() { return lm::kSmem; }

hipError_t launch_lm_tiles(int mode, const LmTileArgs& a, hipStream_t st) {
  const int total = a.ntt * a.nvt;
  const int grid = ((total + 7) / 8) * 8;
  if (mode == kLmFwd) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&lm_tile_kernel<kLmFwd>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lm::kSmem));
    if (e != hipSuccess) return e;
    lm_tile_kernel<kLmFwd><<<dim3(grid), dim3(lm::NTHR), lm::kSmem, st>>>(a);
  } else {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&lm_tile_kernel<kLmBwd>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lm::kSmem));
    if (e != hipSuccess) return e;
    lm_tile_kernel<kLmBwd><<<dim3(grid), dim3(lm::NTHR), lm::kSmem, st>>>(a);
  }
  return hipGetLastError();
}

hipError_t launch_lm_reduce(const LmReduceArgs& a, hipStream_t st) {
  lm_reduce_kernel<<<dim3(static_cast<unsigned>((a.N + 3) / 4)), dim3(256), 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_lm_compact(const LmCompactArgs& a, hipStream_t st) {
  lm_compact_kernel<<<dim3(1), dim3(1024), 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_lm_gather_rows(const void* src, void* dst, const int* live, int n, int H, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  lm_gather_rows_kernel<<<dim3(n), dim3(256), 0, st>>>(static_cast<const u32x4*>(src), static_cast<u32x4*>(dst),
                                                       live, H);
  return hipGetLastError();
}

hipError_t launch_lm_scatter_rows(const float* src, float* dst, const int* cidx, int N, int H, hipStream_t st) {
  lm_scatter_rows_kernel<<<dim3(N), dim3(256), 0, st>>>(reinterpret_cast<const u32x4*>(src),
                                                        reinterpret_cast<u32x4*>(dst), cidx, H);
  return hipGetLastError();
}

hipError_t launch_lm_zero(float* dst, int64_t n, hipStream_t st) {
  const int64_t blocks = (n + 255) / 256;
  lm_zero_kernel<<<dim3(static_cast<unsigned>(blocks < 65536 ? blocks : 65536)), dim3(256), 0, st>>>(dst, n);
  return hipGetLastError();
}

hipError_t launch_lm_terms(const RowArgs& ra, const LmTermsArgs& a, hipStream_t st) {
  lm_terms_kernel<<<dim3(static_cast<unsigned>((a.N + 255) / 256)), dim3(256), 0, st>>>(ra, a);
  return hipGetLastError();
}

}  // namespace pcp
