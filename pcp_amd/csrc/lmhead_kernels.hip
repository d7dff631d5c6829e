// Fused LM-head + GRPO log-prob kernels (gfx950, bf16 MFMA).
//
// logits[n, v] = sum_h hidden[n, h] * W[v, h] is a dense contraction; the loss
// head only needs, per token, the log-sum-exp over v and the logit of its target
// (forward), and dlogits = c_n * (onehot - softmax) (backward). The tile kernel
// computes a 256 x 256 logits tile on bf16 MFMAs and reduces it in its epilogue, so
// full logits never exist in HBM:
//   kLmFwd  -> per (token, kLmPart vocab entries) partial (max, sum 2^(x*log2e - max))
//              and the target logit when the target falls in the tile, for the policy
//              and (n_model = 2) the reference model in one launch; with ECACHE also
//              every policy term 2^(x*log2e - max) as f16 (the softmax cache), or as f32
//              (lm_tile_fwd32_kernel, the exact-rounding backward);
//   kLmBwd  -> dlogits for one vocab chunk in bf16, for the dhidden / dW products (the
//              backward without the cache recomputes the logits this way);
//   kLmGemm -> up to two plain products C = B * A^T on K-contiguous or K-major
//              operands (dhidden and dW from the dlogits and their transpose);
//              with FRAG the token-role operand A is stored fragment-major (written by
//              lm_transpose_frag_kernel) and read straight into registers.
// The logit tiles (kLmFwd, kLmBwd) and the FRAG products run on
// v_mfma_f32_16x16x32_bf16 (lm_tile16), the K-major and plain products on
// v_mfma_f32_32x32x16_bf16 (lm_tile).
//
// Reference: the LM head and loss of tools/export_qwen_forward.py:146-163
// (self.model.lm_head(hidden) then F.cross_entropy), and matmulVJP
// (src/autodiff/vjp_rules.zig:426-497) for dhidden = dlogits*W, dW = dlogits^T*hidden.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstring>
#include <type_traits>

#include "grpo_device.hpp"
#include "lmhead_launch.hpp"

namespace pcp {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace lm {

constexpr int BV = 256;           // vocab rows per tile (MFMA A operand: W rows)
constexpr int BT = 256;           // tokens per tile (MFMA B operand: hidden rows)
constexpr int BK = 64;            // hidden (K) per pipeline stage (one barrier each)
constexpr int NST = 2;            // LDS stages: one in flight while the other is read
constexpr int ROWB = BK * 2;      // bytes of one operand row in one stage
constexpr int kOpBytes = BV * ROWB;             // 32 KB: one operand, one stage
constexpr int kStageBytes = 2 * kOpBytes;       // 64 KB
constexpr size_t kSmemGemm = NST * kStageBytes; // 128 KB
// Waves per workgroup: 8 (two per SIMD; 2 along the vocab x 4 along the tokens, 128 x
// 64 each, 128 accumulators). The code also builds with 4 (one per SIMD; 2 x 2, 128 x
// 128 each, 256 accumulators in AGPRs, a third fewer LDS fragment bytes per flop):
// parity-green, but 10-15% slower at config 5 (step 47.3 against 42.6 ms; forward tiles
// 11.0-11.4 against 9.5-9.9 ms), as one wave per SIMD cannot cover its own waits.
constexpr int NW = 8;
static_assert(NW == 8 || NW == 4, "8 or 4 waves");
constexpr int NTHR = 64 * NW;
constexpr int WPE = NW / 4;       // waves per SIMD
constexpr int WT = NW / 2;        // waves along the tokens
constexpr int TW = 256 / WT;      // token columns per wave
constexpr int NJ = TW / 32;       // 32-column token blocks per wave
constexpr int QN = 32 / NW;       // direct-to-LDS loads per wave per operand per stage
constexpr size_t kSmem = kSmemGemm;
constexpr int kPart = 128;        // vocab entries per log-sum-exp partial (one wave's rows)

// s_waitcnt immediate for vmcnt(n), expcnt and lgkmcnt left at their maxima: vmcnt
// bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8].
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }
constexpr int kWaitVm0 = wait_vm(0);
constexpr int kWaitStage = kWaitVm0;        // the one stage in flight has landed
static_assert(wait_vm(0) == 0x0F70 && wait_vm(8) == 0x0F78 && wait_vm(16) == 0x4F70 && wait_vm(24) == 0x4F78,
              "vmcnt encoding");

}  // namespace lm

#define LM_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// Slot of 16-byte chunk c of an operand row in LDS: c ^ lm_swz(row). Rows are 128
// bytes (8 chunks) unpadded, as the direct-to-LDS loads write 1 KB per instruction
// contiguously. Two rows share one 256-byte span of the 64 banks, so XOR with bits
// 1-3 of the row spreads the 16 rows of an MFMA fragment read that share a chunk
// over 16 distinct 16-byte bank groups.
__device__ __forceinline__ int lm_swz(int row) { return (row >> 1) & 7; }

// Tile order: work item p -> (token tile, vocab tile). Each XCD works through its own
// contiguous range of work items (see lm_tile_kernel); within it, groups
// of group_m token tiles sweep the vocab tiles together, so the workgroups resident on
// one XCD read the same operand K-slabs from its L2, and W comes from HBM once per group.
__device__ __forceinline__ void lm_tile_of(int p, int ntt, int nvt, int group_m, int& tm, int& tn) {
  const int group = group_m * nvt;
  const int g = p / group;
  const int first_m = g * group_m;
  const int gm = min(ntt - first_m, group_m);
  const int q = p - g * group;
  tm = first_m + q % gm;
  tn = q / gm;
}

// The forward's order while the live hidden rows fit in half of the 256 MB MALL (the
// token tiles times 256 rows of H bf16 within 128 MiB): groups of two vocab tiles
// sweep every token tile, so the hidden slabs come back from the MALL and each W slab
// pair is shared by the XCD's resident tiles. Forward-only launches at H = 4096,
// interleaved on one box (ms, this order against lm_tile_of's): 10 / 20 / 32 token
// tiles equal; 38: 18.92-19.04 against 19.11-19.18 (the full step's forward, with the
// softmax cache and W^T stores, 18.75-18.77 against 19.12-19.16; groups of 1, 3 and
// 4: 19.04-19.06, 19.78-19.85 and 20.22-20.24 against 19.52-19.55 for 2 on a slower
// box); 48: 23.58-23.70 against 23.75-24.08; 64: 31.55-31.60 against 31.65-31.69; but
// 96: 48.50-48.56 against 47.47-48.23 and 128: 65.41-65.50 against 63.30-63.65, where
// the hidden rows no longer fit.
constexpr int kLmFwdVocabGroup = 2;
__device__ __forceinline__ bool lm_fwd_vocab_groups(int ntt, int H) {
  return static_cast<int64_t>(ntt) * kLmTileT * H * 2 <= (int64_t{128} << 20);
}
__device__ __forceinline__ void lm_tile_of_vgroups(int p, int ntt, int nvt, int group_n, int& tm, int& tn) {
  const int group = group_n * ntt;
  const int g = p / group;
  const int first_n = g * group_n;
  const int gn = min(nvt - first_n, group_n);
  const int q = p - g * group;
  tn = first_n + q % gn;
  tm = q / gn;
}

// Token tiles per group in the tile order. lm_tile_coords gives each XCD a
// contiguous eighth of the work items; the forward measured fastest with the
// smallest group (at least 8 token tiles) whose boundaries fall on those eighths:
// 8 * group a multiple of the token tiles, or the token tiles a multiple of
// 8 * group. Forward launch, H = 4096, V = 151936, all tokens live, interleaved on
// one box (ms):
//   token tiles 10:  groups of 10  2.70 | 8 (misaligned)   2.85
//   token tiles 20:  groups of 10  5.39 | 20 5.43-5.46
//   token tiles 32:  groups of 8   8.73-8.82 | 16 8.91-8.99 | 32 9.45-9.50
//   token tiles 38:  groups of 19  10.28 | 13 10.70-10.81 | 10 11.02-11.09 | 8 11.05 (config 5)
//   token tiles 64:  groups of 8   17.46-17.53 | 16 17.88-17.94 | 32 18.59-18.61 | 64 18.26-18.28
//   token tiles 128: groups of 8   34.86-34.93 | 16 36.87-36.91 | 32 38.25-38.28
// The backward's chunks (64 vocab tiles) measured best with groups of 4 at config 5
// (step 55.3 ms against 55.6 with 8; 2 matched 4, 1 and 38 were slower), and so did
// the whole-vocabulary products of the cached backward (dhidden / dW groups of 4 / 4:
// step 42.19-42.25 ms; 4 / 8 42.28, 4 / 2 42.43, 4 / 16 42.65, 8 / 16 42.75, 2 / 16
// 43.0, 16 / 16 43.1); on the 16x16x32 products, 4 again (products launch 17.13-17.15
// ms against 17.28-17.32 with 8, 17.57-17.62 with 2, 17.97-18.00 with 16). The forward
// computes its group in the kernel from the live token count.
constexpr int kLmBwdGroup = 4;

__host__ __device__ inline int lm_group_m(int mode, int ntt) {
  if (ntt < 1) return 1;
  if (mode != kLmFwd) return ntt < kLmBwdGroup ? ntt : kLmBwdGroup;
  for (int g = ntt < 8 ? ntt : 8; g < ntt; ++g)
    if ((8 * g) % ntt == 0 || ntt % (8 * g) == 0) return g;
  return ntt;
}

__device__ __forceinline__ int64_t lm_id(const LmTileArgs& a, int n) {
  return a.ids_i64 ? static_cast<const int64_t*>(a.ids)[n] : static_cast<int64_t>(static_cast<const int32_t*>(a.ids)[n]);
}

// Workgroup barrier without a memory fence: LDS data of the pipeline is ordered by
// the explicit s_waitcnt before it; the empty asm statements keep the compiler from
// moving memory operations across it.
__device__ __forceinline__ void lm_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// One 256 (vocab) x 256 (token) logits tile C[v][t] = sum_h W[v][h] * hidden[t][h].
// Eight waves, two per SIMD: wave (wv, wt) owns vocab rows wv*128 + [0,128) and token
// columns wt*64 + [0,64) as 4 x 2 blocks of v_mfma_f32_32x32x16_bf16 (128 accumulators,
// so two waves share a SIMD and one issues MFMAs while the other waits on a load, a
// fragment read or the barrier; measured 2-7% faster than four waves of 128 x 128,
// which fill the register file). Result layout of a 32 x 32 block:
// lane l holds token column l%32 and vocab rows 8*(r/4) + 4*(l/32) + r%4, r < 16.
// Operands stream global -> LDS with buffer_load_dwordx4 ... lds (no VGPR staging)
// through two stages of BK hidden columns.
// This 32x32x16 tile serves the products of the chunked backward's low-memory form
// (ATR: the token-role operand stored K-major, its fragments read with
// ds_read_b64_tr_b16, see below) and the plain products; the logit tiles and the
// other products run on lm_tile16 below.
// Tile p of product prod, called by lm_tile_kernel.
template <int MODE, bool ATR>
__device__ __forceinline__ void lm_tile(const LmTileArgs& a, int prod, int p, char* smem) {
  using namespace lm;
  static_assert(MODE == kLmGemm, "32x32x16 tiles: the K-major and plain products");

  // The product: the loss-head modes read rows of H elements of hidden (A) and W (B);
  // kLmGemm takes one of its (up to) two products.
  const void* opA = a.A;
  const void* opB = a.B;
  int N = a.N, V = a.V, K = a.H, lda = a.H, ldb = a.H, ntt = a.ntt, nvt = a.nvt, gm = 1, vt0 = a.vt0;
  float* C = nullptr;
  int ldc = 0, accumulate = 0, transpose_c = 0, krows_a = 0;
  if constexpr (MODE == kLmGemm) {
    const LmTileArgs::Gemm& g = a.gemm[prod];
    opA = g.A;
    opB = g.B;
    N = g.N;
    V = g.V;
    K = g.K;
    lda = g.lda;
    ldb = g.ldb;
    ntt = g.ntt;
    nvt = g.nvt;
    gm = g.group_m;
    vt0 = 0;
    C = g.C;
    ldc = g.ldc;
    accumulate = g.accumulate;
    transpose_c = g.transpose_c;
    krows_a = g.krows_a;
    if (g.vcount) {
      V = min(V, *g.vcount);
      nvt = (V + BV - 1) / BV;
    }
    if (g.kcount) {
      krows_a = min(K, *g.kcount);
      K = min(K, (krows_a + BK - 1) / BK * BK);
    }
  }
  int tm, tn;
  lm_tile_of(p, ntt, nvt, gm, tm, tn);
  const int m0 = tm * BT;                  // first token
  const int v0 = (vt0 + tn) * BV;          // first vocab entry
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wv = wave / WT, wt = wave % WT;

  // Operand row buffers: rows past V / N read 0 (range-checked lane offsets).
  const uint32_t wbytes = static_cast<uint32_t>(ldb) * 2u;
  const uint32_t hbytes = static_cast<uint32_t>(lda) * 2u;
  const int rows_w = min(BV, V - v0), rows_h = min(BT, N - m0);
  const __amdgpu_buffer_rsrc_t rw =
      row_rsrc(reinterpret_cast<const char*>(opB) + static_cast<int64_t>(v0) * wbytes, rows_w * wbytes);
  // K-major token operand (ATR): the tile is columns [m0, m0 + 256) of rows k; rows
  // past krows_a fall outside the descriptor and read 0. The range check drops a whole
  // 16-byte load that runs past the end, so the last row's extent is rounded up to 8
  // columns (the operand's rows are at least that wide). Columns past N belong to
  // result columns that are not stored.
  const __amdgpu_buffer_rsrc_t rh =
      ATR ? row_rsrc(reinterpret_cast<const char*>(opA) + static_cast<int64_t>(m0) * 2,
                     krows_a > 0 ? static_cast<uint32_t>(krows_a - 1) * hbytes +
                                       static_cast<uint32_t>((rows_h + 7) & ~7) * 2u
                                 : 0u)
          : row_rsrc(reinterpret_cast<const char*>(opA) + static_cast<int64_t>(m0) * hbytes, rows_h * hbytes);

  // Direct-to-LDS loads: wave w fills rows 8*(4w+q) + lane/8, q < 4, of each operand;
  // lane writes LDS slot lane%8 of its row, which holds chunk (lane%8) ^ swz(row).
  // A K-major operand's stage is 64 k-rows of 512 bytes (256 columns): instruction q
  // of wave w fills k-rows 2*(4w+q) + lane/32, and LDS slot lane%32 of a k-row holds
  // 16-byte chunk (lane%32) ^ 4*(k-row % 4), so the transpose reads below, which take
  // 64 bytes from each of 8 k-rows (k-row % 4 = 0..3, twice), hit every bank twice.
  uint32_t dofw[QN], dofh[QN];
#pragma unroll
  for (int q = 0; q < QN; ++q) {
    const int row = 8 * (QN * wave + q) + (lane >> 3);
    const uint32_t c16 = 16u * static_cast<uint32_t>((lane & 7) ^ lm_swz(row));
    dofw[q] = static_cast<uint32_t>(row) * wbytes + c16;
    if constexpr (ATR) {
      const int krow = 2 * (QN * wave + q) + (lane >> 5);
      dofh[q] = static_cast<uint32_t>(krow) * hbytes + 16u * static_cast<uint32_t>((lane & 31) ^ (4 * (krow & 3)));
    } else {
      dofh[q] = static_cast<uint32_t>(row) * hbytes + c16;
    }
  }
  auto issue = [&](int st, int buf) {
    char* base = smem + buf * kStageBytes;
    const uint32_t koff = static_cast<uint32_t>(st) * ROWB;
    const uint32_t kofh = ATR ? static_cast<uint32_t>(st) * BK * hbytes : koff;
#pragma unroll
    for (int q = 0; q < QN; ++q) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, LM_LDS(base + (QN * wave + q) * 1024), 16, dofw[q] + koff, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rh, LM_LDS(base + kOpBytes + (QN * wave + q) * 1024), 16, dofh[q] + kofh,
                                               0, 0, 0);
    }
  };

  // Fragment reads: row (lane%32) of each 32-row block, chunk 2*kk + lane/32 for
  // k-step kk < 4. The swizzle depends on lane%32 only, so one offset per k-step
  // serves every block.
  const int sw = lm_swz(lane & 31);
  int fo[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) fo[kk] = 16 * ((2 * kk + (lane >> 5)) ^ sw);
  const int offA = (wv * 128 + (lane & 31)) * ROWB, offB = kOpBytes + (wt * TW + (lane & 31)) * ROWB;
  // K-major token operand: ds_read_b64_tr_b16 hands lane i of each 16-lane block the
  // element i%4 of the 8-byte chunks addressed by source lanes i/4 + 4k (k < 4). Source
  // lane j of block b points at k-row k0 + j/4, columns 16*(b%2) + 4*(j%4) of the
  // fragment's 32, so lane l receives column l%32 at k-rows k0 .. k0 + 3: with k0 =
  // 16*kk + 8*(l/32) and a second read 4 rows on, the MFMA operand layout (column l%32,
  // k = 8*(l/32) + 0..7). offBt[j] is the part of the address fixed per lane and block.
  int offBt[NJ];
  if constexpr (ATR) {
    const int x = (lane >> 2) & 3;   // = k-row % 4 of this lane's source row
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int chunk = (wt * TW) / 8 + 4 * j + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
      offBt[j] = kOpBytes + (8 * (lane >> 5) + x) * 512 + 16 * (chunk ^ (4 * x)) + 8 * (lane & 1);
    }
  }
  bf16x8 af[2][4], bfr[2][NJ];
  auto fload = [&](int set, int st, int kk) {
    const char* base = smem + (st % NST) * kStageBytes + fo[kk];
#pragma unroll
    for (int i = 0; i < 4; ++i) af[set][i] = *reinterpret_cast<const bf16x8*>(base + offA + i * 32 * ROWB);
    if constexpr (ATR) {
      typedef short v4i16 __attribute__((ext_vector_type(4)));
      const char* tb = smem + (st % NST) * kStageBytes + kk * 16 * 512;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)LM_LDS(tb + offBt[j]));
        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)LM_LDS(tb + offBt[j] + 4 * 512));
        bfr[set][j] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    } else {
#pragma unroll
      for (int j = 0; j < NJ; ++j) bfr[set][j] = *reinterpret_cast<const bf16x8*>(base + offB + j * 32 * ROWB);
    }
  };

  f32x16 acc[4][NJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  auto mfmas = [&](int set) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[set][i], bfr[set][j], acc[i][j], 0, 0, 0);
  };

  // Pipeline: stage kb is read from LDS buffer kb % 2 while stage kb + 1 loads into
  // the other one (8 direct-to-LDS loads per wave; past the end the last stage is
  // reloaded into a buffer nobody reads, an L2 hit). Each stage ends with vmcnt(0)
  // and one barrier, which makes every wave's loads of the next stage visible and
  // frees the buffer just read. Branch-free, so the compiler's LDS waits stay exact.
  // With two waves per SIMD covering each other's waits, 64-deep stages (one barrier
  // per 64 hidden columns, 64 KB in flight) measured 6% faster on config 5 than
  // 32-deep ones with three in flight.
  // Issue order: one memory instruction per MFMA. The wave issues in order, so a
  // burst of the stage's direct-to-LDS loads right after the barrier held the MFMAs
  // behind it whenever the memory pipeline pushed back; one load (or fragment read)
  // between consecutive MFMAs measured 6% faster on config 5.
  const int nk = K / BK;
  issue(0, 0);
  __builtin_amdgcn_s_waitcnt(kWaitStage);
  lm_barrier();
  fload(0, 0, 0);
  // Per k-step and wave: kRd fragment reads (4 vocab-role, NJ token-role, or 2 NJ when
  // the token role takes two transpose reads per fragment) and 4 NJ MFMAs, one read per
  // MFMA and the rest of the MFMAs after them. The stage's loads follow the first
  // k-step's fragment reads in groups of 4 between its next MFMAs (with 8 waves, 1-2%
  // faster than one load per MFMA with these 64-deep stages).
  constexpr int kRd = 4 + (ATR ? 2 : 1) * NJ, kMf = 4 * NJ, kLdG = 2 * QN / 4;
  constexpr int kRd0 = kRd - (ATR ? kLdG : 0);   // reads before the loads in the first k-step
  static_assert(kRd <= kMf && kRd0 + kLdG <= kMf, "schedule");
  auto sched_step = [&]() {
#pragma unroll
    for (int q = 0; q < kRd; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // a fragment read of the next k-step
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // an MFMA of this one
    }
    if constexpr (kMf > kRd) __builtin_amdgcn_sched_group_barrier(0x008, kMf - kRd, 0);
  };
  for (int kb = 0; kb < nk; ++kb) {
    // Buffer (kb + 1) % 2 held stage kb - 1, whose reads all completed before the
    // last barrier; past the end the last stage is reloaded into it (nobody reads it).
    issue(min(kb + 1, nk - 1), (kb + 1) & 1);
    fload(1, kb, 1);
    mfmas(0);
#pragma unroll
    for (int q = 0; q < kRd0; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // a fragment read of k-step 1
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // an MFMA of k-step 0
    }
#pragma unroll
    for (int q = 0; q < kLdG; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x020, 4, 0);  // 4 of the stage's loads
      if constexpr (ATR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    if constexpr (kMf > kRd0 + kLdG) __builtin_amdgcn_sched_group_barrier(0x008, kMf - kRd0 - kLdG, 0);
    fload(0, kb, 2);
    mfmas(1);
    sched_step();
    fload(1, kb, 3);
    mfmas(0);
    sched_step();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kWaitStage);               // stage kb+1 landed
    lm_barrier();
    fload(0, min(kb + 1, nk - 1), 0);
    mfmas(1);
    sched_step();
  }
  // Drain the trailing loads before any LDS reuse (the backward epilogue).
  __builtin_amdgcn_s_waitcnt(kWaitVm0);

  const int vw = v0 + wv * 128;                 // first vocab row of this wave
  const int half = lane >> 5;
  // Vocab row of acc[i][*][r] relative to vw.
  auto vrow = [&](int i, int r) { return 32 * i + 8 * (r >> 2) + 4 * half + (r & 3); };

  if constexpr (MODE == kLmGemm) {
    // C[v][t] (+)= the tile; rows past V and columns past N are not stored. For fixed
    // (i, r) lanes 0-31 and 32-63 each write 32 consecutive floats of one row. With
    // transpose_c the lane's 4 consecutive rows of a column are one 16-byte store.
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = m0 + wt * TW + 32 * j + (lane & 31);
      if (n >= N) continue;
      if (transpose_c) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int vr = vw + vrow(i, 4 * q);
            if (vr < V) {
              float4* p = reinterpret_cast<float4*>(C + static_cast<int64_t>(n) * ldc + vr);
              float4 v = make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
              if (accumulate) {
                const float4 o = *p;
                v.x += o.x;
                v.y += o.y;
                v.z += o.z;
                v.w += o.w;
              }
              *p = v;
            }
          }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int vr = vw + vrow(i, r);
            if (vr < V) {
              float* p = C + static_cast<int64_t>(vr) * ldc + n;
              *p = accumulate ? *p + acc[i][j][r] : acc[i][j][r];
            }
          }
      }
    }
  }
}

// Per token: merge the vocab-tile partials into the base-2 log-sum-exp. One wave
// per token; the merge is commutative, so the xor butterfly is deterministic.
__global__ void __launch_bounds__(256) lm_reduce_kernel(LmReduceArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  if (n >= *a.count) return;
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

typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace lm {
constexpr int NI16 = 8;         // 16-row vocab blocks per wave (its 128 rows)
constexpr int NJ16 = TW / 16;   // 16-column token blocks per wave
constexpr int KS16 = BK / 32;   // 32-deep k-steps per stage
}  // namespace lm

// A tile on v_mfma_f32_16x16x32_bf16: the logit tiles (kLmFwd, kLmBwd: both operands
// through LDS) and the products (kLmGemm with a fragment-major token operand). Same tile, waves,
// stages and operand paths as lm_tile; each wave's 128 x 64 block is 8 x 4 products of
// 16 x 16 (128 accumulators), two 32-deep k-steps per stage. Under the power limit this
// shape runs the pipes at a higher clock than 32x32x16 for the same work (the
// register-resident probe: 1.93-1.98 against 1.72-1.80 GHz at the same MFMA occupancy),
// as each instruction reduces twice as deep per accumulator update.
// Fragment layouts (pinned by the MFMA probe's test): an operand lane holds row
// lane % 16 at k = 8 (lane / 16) + 0..7; the result lane holds column lane % 16 at rows
// 4 (lane / 16) + 0..3.
// E32 (with ECACHE): the softmax terms are stored as f32 (a.ecache32) in place of f16.
template <int MODE, bool ECACHE, bool E32 = false>
__device__ __forceinline__ void lm_tile16(const LmTileArgs& a, int prod, int p, char* smem) {
  using namespace lm;
  constexpr bool FWD = MODE == kLmFwd, BWD = MODE == kLmBwd;
  constexpr bool TL = FWD || BWD;   // the token operand through LDS too (the logit tiles)
  const LmTileArgs::Gemm& g = a.gemm[FWD ? 0 : prod];
  const void* opA = TL ? a.A : g.A;
  const void* opB = TL ? (prod == 1 ? a.B2 : a.B) : g.B;
  int N, V, K, nvt, ntt, gm, lda, ldb, vt0 = 0;
  if constexpr (TL) {
    // Tiles over the live tokens only (the grid covers all N).
    N = min(a.N, *a.count);
    V = a.V;
    K = lda = ldb = a.H;
    ntt = (N + BT - 1) / BT;
    nvt = a.nvt;
    gm = lm_group_m(MODE, ntt);
    vt0 = a.vt0;
  } else {
    N = g.N;
    V = g.V;
    K = g.K;
    lda = g.lda;
    ldb = g.ldb;
    nvt = g.nvt;
    ntt = g.ntt;
    gm = g.group_m;
    if (g.vcount) {
      V = min(V, *g.vcount);
      nvt = (V + BV - 1) / BV;
    }
    if (g.kcount) K = min(K, (min(K, *g.kcount) + BK - 1) / BK * BK);
  }
  int tm, tn;
  if (FWD && lm_fwd_vocab_groups(ntt, K))
    lm_tile_of_vgroups(p, ntt, nvt, kLmFwdVocabGroup, tm, tn);
  else
    lm_tile_of(p, ntt, nvt, gm, tm, tn);
  const int m0 = tm * BT, v0 = (vt0 + tn) * BV;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wv = wave / WT, wt = wave % WT;

  // Operands through LDS as in lm_tile: the vocab role (B) always, the token role (A)
  // for the forward. A stage buffer holds one operand (products) or both (forward).
  constexpr int kBuf = TL ? kStageBytes : kOpBytes;
  const uint32_t wbytes = static_cast<uint32_t>(ldb) * 2u, hbytes = static_cast<uint32_t>(lda) * 2u;
  const int rows_w = min(BV, V - v0), rows_h = min(BT, N - m0);
  // A tile-major B (the cached backward's D, D^T; lm_tile_block_off): the tile's stages
  // are consecutive 32 KB blocks. Its rows past V hold whatever was there; they only
  // reach result rows past V, which are not stored.
  const bool btile = !TL && g.b_tiled;
  const __amdgpu_buffer_rsrc_t rw =
      btile ? row_rsrc(reinterpret_cast<const char*>(opB) + static_cast<int64_t>(v0 / BV) * (ldb / BK) * kOpBytes,
                       static_cast<uint32_t>(ldb / BK) * kOpBytes)
            : row_rsrc(reinterpret_cast<const char*>(opB) + static_cast<int64_t>(v0) * wbytes, rows_w * wbytes);
  const uint32_t wrow = btile ? static_cast<uint32_t>(ROWB) : wbytes;   // bytes between B rows
  const uint32_t wstage = btile ? static_cast<uint32_t>(kOpBytes) : static_cast<uint32_t>(ROWB);
  const __amdgpu_buffer_rsrc_t rh =
      row_rsrc(reinterpret_cast<const char*>(opA) + static_cast<int64_t>(m0) * hbytes, TL ? rows_h * hbytes : 0u);
  uint32_t dofw[QN], dofh[QN];
#pragma unroll
  for (int q = 0; q < QN; ++q) {
    const int row = 8 * (QN * wave + q) + (lane >> 3);
    const uint32_t c16 = 16u * static_cast<uint32_t>((lane & 7) ^ lm_swz(row));
    dofw[q] = static_cast<uint32_t>(row) * wrow + c16;
    dofh[q] = static_cast<uint32_t>(row) * hbytes + c16;
  }
  auto issue = [&](int st, int buf) {
    char* base = smem + buf * kBuf;
    const uint32_t koff = static_cast<uint32_t>(st) * ROWB;
    const uint32_t kofw = static_cast<uint32_t>(st) * wstage;
#pragma unroll
    for (int q = 0; q < QN; ++q) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, LM_LDS(base + (QN * wave + q) * 1024), 16, dofw[q] + kofw, 0, 0,
                                               0);
      if constexpr (TL)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rh, LM_LDS(base + kOpBytes + (QN * wave + q) * 1024), 16,
                                                 dofh[q] + koff, 0, 0, 0);
    }
  };
  // Products: the token-role operand fragment-major in 16 x 32 fragments: fragment (b, s)
  // at byte 1024 (b lda/32 + s), lane l's 16 bytes at 16 l (row 16 b + l % 16, k 32 s +
  // 8 (l / 16) + 0..7). Blocks past the tile's rows fall outside the descriptor and read 0.
  const __amdgpu_buffer_rsrc_t rt =
      row_rsrc(reinterpret_cast<const char*>(opA) + static_cast<int64_t>(m0 / 16) * (lda / 32) * 1024,
               FWD ? 0u : static_cast<uint32_t>((rows_h + 15) / 16) * static_cast<uint32_t>(lda / 32) * 1024u);
  uint32_t roff[NJ16];
#pragma unroll
  for (int j = 0; j < NJ16; ++j)
    roff[j] = static_cast<uint32_t>((wt * NJ16 + j) * (lda / 32)) * 1024u + 16u * static_cast<uint32_t>(lane);

  // Fragment reads from LDS: row (wv*128 | wt*64) + 16 i + lane % 16, 16-byte chunk
  // 4 kk + lane / 16 of the row's 8; the swizzle depends on lane % 16 only.
  const int sw = lm_swz(lane & 15);
  int fo[KS16];
#pragma unroll
  for (int kk = 0; kk < KS16; ++kk) fo[kk] = 16 * ((4 * kk + (lane >> 4)) ^ sw);
  const int offA = (wv * 128 + (lane & 15)) * ROWB, offB = kOpBytes + (wt * TW + (lane & 15)) * ROWB;
  // af: vocab-role fragments; bt: token-role fragments (from LDS for the forward, the
  // register ring for the products; slot kk holds k-step kk of the current stage).
  bf16x8 af[2][NI16], bt[KS16][NJ16];
  auto fload = [&](int set, int st, int kk) {
    const char* base = smem + (st % NST) * kBuf + fo[kk];
#pragma unroll
    for (int i = 0; i < NI16; ++i) af[set][i] = *reinterpret_cast<const bf16x8*>(base + offA + i * 16 * ROWB);
    if constexpr (TL) {
#pragma unroll
      for (int j = 0; j < NJ16; ++j) bt[kk][j] = *reinterpret_cast<const bf16x8*>(base + offB + j * 16 * ROWB);
    }
  };
  auto ring_load = [&](int kk, int st) {
    if constexpr (!TL) {
#pragma unroll
      for (int j = 0; j < NJ16; ++j)
        bt[kk][j] =
            __builtin_bit_cast(bf16x8, buf_ld16<false>(rt, roff[j] + static_cast<uint32_t>(KS16 * st + kk) * 1024u));
    }
  };
  f32x4 acc[NI16][NJ16];
#pragma unroll
  for (int i = 0; i < NI16; ++i)
#pragma unroll
    for (int j = 0; j < NJ16; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.f;
  // j-major, so token slot (kk, j) is free after its 8 MFMAs.
  auto mf = [&](int set, int kk) {
#pragma unroll
    for (int j = 0; j < NJ16; ++j)
#pragma unroll
      for (int i = 0; i < NI16; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[set][i], bt[kk][j], acc[i][j], 0, 0, 0);
  };
  constexpr int kMf16 = NI16 * NJ16;
  constexpr int kRd16 = NI16 + (TL ? NJ16 : 0);     // fragment reads per k-step
  constexpr int kLd16 = TL ? 2 * QN : QN;          // direct-to-LDS loads per stage
  // Per k-step: the next k-step's fragment reads between the first MFMAs (and the
  // stage's direct-to-LDS loads after them when the k-step starts a buffer), the ring
  // reloads after the last.
  auto sched16 = [&](auto dma) {
    constexpr int nd = decltype(dma)::value ? kLd16 : 0;
#pragma unroll
    for (int q = 0; q < kRd16; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
#pragma unroll
    for (int q = 0; q < nd; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, kMf16 - kRd16 - nd, 0);
    if constexpr (!TL) __builtin_amdgcn_sched_group_barrier(0x020, NJ16, 0);
  };
  static_assert(kRd16 + kLd16 <= kMf16, "schedule");

  // Pipeline: LDS buffer kb % 2 holds stage kb; the DMA of stage kb + 2 goes into it
  // once every wave has issued its last read of stage kb (the barrier), one stage ahead
  // of its use. The products reload ring slot kk with stage kb + 1 after k-step kk's
  // MFMAs. At the barrier of iteration kb the loads issued after stage kb + 1's DMA are
  // the ring reloads of (kb, 1) and (kb + 1, 0) (none in the forward): vmcnt(2 NJ16),
  // or vmcnt(0), leaves only those in flight.
  const int nk = K / BK;
  // The forward's policy tiles also write W^T [H, ldwt] (the dhidden product's token
  // operand, fragment-major) from the W slabs they hold: stage st of vocab tile tn by
  // token tile st % ntt, so each stage is written once and every token tile writes
  // about nk / ntt of them. Wave w writes the four fragments of vocab rows v0 + 32 w +
  // [0, 32) and the stage's 64 hidden columns; lane l holds hidden column 16 bb + l % 16
  // and vocab rows 8 (l / 16) + [0, 8), read from the swizzled LDS rows as 16-bit
  // pairs. Called at the end of the iteration whose barrier landed stage st (after its
  // MFMAs are issued): the buffer is refilled only after the next barrier, whose
  // vmcnt(0) also covers these stores. Vocab rows past V hold zeros (the W
  // descriptor's range); fragments past ldwt are not written. At config 5 this costs
  // the forward 0.34 ms and saves the 0.49 ms transpose kernel that wrote W^T.
  const bool wt_on = FWD && a.wt != nullptr && prod == 0 && v0 + 32 * wave < a.ldwt;
  auto wt_write = [&](int st) {
    if constexpr (FWD) {
      if (!wt_on || st % ntt != tm) return;
      const char* wb = smem + (st % NST) * kBuf;
      // The thread index through an opaque copy: the addresses below are then formed
      // here rather than hoisted out of the main loop, where they would hold VGPRs
      // through every stage.
      int ti = tid;
      asm volatile("" : "+v"(ti));
      const int ln = ti & 63, wv8 = ti >> 6;
      const int r0 = 32 * wv8 + 8 * (ln >> 4);
      // The stage's four fragment rows of W^T: ldwt / 32 fragments of 1 KB each.
      const uint32_t frow = static_cast<uint32_t>(a.ldwt / 32) * 1024u;
      const __amdgpu_buffer_rsrc_t rw =
          row_rsrc(reinterpret_cast<const char*>(a.wt) + static_cast<int64_t>(4 * st) * frow, 4u * frow);
      const uint32_t o0 = static_cast<uint32_t>(v0 / 32 + wv8) * 1024u + 16u * ln;
      // Lane l: hidden column 16 bb + l % 16 of vocab rows r0 + [0, 8), read as 16-bit
      // pairs. (ds_read_b64_tr_b16 would read the same eight values in two instructions,
      // but hipcc waits for every direct-to-LDS load in flight before one, here the next
      // stage's; as inline assembly with its own wait it measured the same as this.)
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        const int hl = 16 * bb + (ln & 15);
        uint32_t w[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int r = r0 + 2 * jj;   // rows r and r + 1 share the swizzle (r even)
          const char* p = wb + r * ROWB + (((hl >> 3) ^ lm_swz(r)) << 4) + (hl & 7) * 2;
          w[jj] = static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(p)) |
                  (static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(p + ROWB)) << 16);
        }
        buf_st16<true>(rw, u32x4{w[0], w[1], w[2], w[3]}, o0 + static_cast<uint32_t>(bb) * frow);
      }
    }
  };
  issue(0, 0);
  ring_load(0, 0);
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  lm_barrier();
  wt_write(0);
  issue(min(1, nk - 1), 1);
  ring_load(1, 0);
  fload(0, 0, 0);
  for (int kb = 0; kb < nk; ++kb) {
    const int n1 = min(kb + 1, nk - 1);   // past the end: reloads of the last stage, unused
    fload(1, kb, 1);
    mf(0, 0);
    ring_load(0, n1);
    sched16(std::false_type{});
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(TL ? kWaitVm0 : wait_vm(2 * NJ16));   // stage kb+1's LDS loads landed
    lm_barrier();
    // The forward's 8 direct-to-LDS loads go between the k-step's MFMAs after its
    // fragment reads; the products issue their 4 first (measured faster each way).
    if constexpr (TL) {
      fload(0, n1, 0);
      issue(min(kb + 2, nk - 1), kb & 1);
    } else {
      issue(min(kb + 2, nk - 1), kb & 1);
      fload(0, n1, 0);
    }
    mf(1, 1);
    ring_load(1, n1);
    sched16(std::true_type{});
    if constexpr (FWD) {
      __builtin_amdgcn_sched_barrier(0);
      if (kb + 1 < nk) wt_write(kb + 1);
    }
  }
  __builtin_amdgcn_s_waitcnt(kWaitVm0);

  const int vw = v0 + wv * 128;   // first vocab row of this wave
  const int grp = lane >> 4;      // the lane's 4-row group of each 16-row block
  if constexpr (FWD) {
    // Per token column: (max * log2e, sum 2^(x*log2e - max*log2e)) over this wave's
    // 128 vocab rows (32 in-lane, the rest in lanes l ^ 16, l ^ 32, l ^ 48), and the
    // target logit. Vocab rows past V (last tile only) become -inf, whose term is 0.
    const bool any_v = vw < a.V;
    const int vlim = a.V - vw;
    if (vw + 128 > V) {
#pragma unroll
      for (int i = 0; i < NI16; ++i)
#pragma unroll
        for (int j = 0; j < NJ16; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][j][r] = 16 * i + 4 * grp + r < vlim ? acc[i][j][r] : kNegInf;
    }
    float ref[NJ16];
#pragma unroll
    for (int j = 0; j < NJ16; ++j) {
      float mx = kNegInf;
#pragma unroll
      for (int i = 0; i < NI16; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, acc[i][j][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      ref[j] = mx * kLog2e;   // the block's max * log2e; ms_ref maps -inf to 0 below
    }
    // Two token blocks at a time, so each pair's accumulators die before the next.
#pragma unroll
    for (int jj = 0; jj < NJ16; jj += 2) {
      float sum[2] = {0.f, 0.f};
#pragma unroll
      for (int i = 0; i < NI16; ++i) {
        float ev[2][4];
        uint32_t pk[2][2];
#pragma unroll
        for (int jo = 0; jo < 2; ++jo) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            ev[jo][r] = hw_exp2(fmaf(acc[i][jj + jo][r], kLog2e, -ms_ref(ref[jj + jo])));
            sum[jo] += ev[jo][r];
          }
          pk[jo][0] = pack2<F16T>(ev[jo][0], ev[jo][1]);
          pk[jo][1] = pack2<F16T>(ev[jo][2], ev[jo][3]);
        }
        if (ECACHE && E32 && prod == 0) {
          // f32 terms: the same exchange per register (rows 4 grp + r), after which the
          // lane holds rows 16 i + 8 (grp / 2) + 0..3 in w0 and + 4..7 in w1: two 16-byte
          // stores.
          u32x4 w0, w1;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(ev[0][r]), __float_as_uint(ev[1][r]),
                                                             false, false);
            w0[r] = sw[0];
            w1[r] = sw[1];
          }
          const int n = m0 + wt * TW + 16 * (jj + (grp & 1)) + (lane & 15);
          const int64_t c = vw + 16 * i + 8 * (grp >> 1);
          if (n < N && c < a.lde) {   // tile-major as the f16 cache (64 KB blocks of f32)
            u32x4* dst = reinterpret_cast<u32x4*>(a.ecache32 + lm_tile_block_off(n, c, a.lde));
            dst[0] = w0;
            dst[1] = w1;
          }
        } else if (ECACHE && prod == 0) {
          // Softmax cache: ecache[n][v] = f16(2^(x*log2e - ref)) in the products' tile-major
          // layout (lm_tile_block_off, K extent lde; vocab past V holds 0), which the
          // dlogits pass rewrites in place as D. The lane's terms of block (i, j) are vocab rows
          // 16 i + 4 grp + 0..3 of token column 16 j + lane % 16. One v_permlane16_swap
          // per register trades the odd groups' block-jj terms with the even groups'
          // block-(jj+1) terms, after which lanes of an even group hold 8 consecutive rows
          // (16 i + 8 (grp / 2) + 0..7) of token 16 jj + lane % 16, and of an odd group the
          // same rows of token 16 (jj + 1) + lane % 16: one 16-byte store each.
          const auto lo = __builtin_amdgcn_permlane16_swap(pk[0][0], pk[1][0], false, false);
          const auto hi = __builtin_amdgcn_permlane16_swap(pk[0][1], pk[1][1], false, false);
          const int n = m0 + wt * TW + 16 * (jj + (grp & 1)) + (lane & 15);
          const int64_t c = vw + 16 * i + 8 * (grp >> 1);
          if (n < N && c < a.lde) {
            const u32x4 w = {lo[0], hi[0], lo[1], hi[1]};
            *reinterpret_cast<u32x4*>(a.ecache + lm_tile_block_off(n, c, a.lde)) = w;
          }
        }
      }
#pragma unroll
      for (int jo = 0; jo < 2; ++jo) {
        const int j = jj + jo;
        float s = sum[jo];
        s += __shfl_xor(s, 16);
        s += __shfl_xor(s, 32);
        const int n = m0 + wt * TW + 16 * j + (lane & 15);
        if (n < N && any_v) {
          if (grp == 0)
            (prod ? a.part2 : a.part)[static_cast<int64_t>(n) * a.ldp + vw / kPart] = make_float2(ref[j], s);
          const int64_t rel = lm_id(a, n) - vw;
          if (rel >= 0 && rel < 128) {
            const int isel = static_cast<int>(rel) >> 4, gsel = (static_cast<int>(rel) >> 2) & 3;
            const int rsel = static_cast<int>(rel) & 3;
            float val = 0.f;
#pragma unroll
            for (int i = 0; i < NI16; ++i)
#pragma unroll
              for (int r = 0; r < 4; ++r) val = (i == isel && r == rsel) ? acc[i][j][r] : val;
            if (grp == gsel) (prod ? a.tgt2 : a.tgt)[n] = val;
          }
        }
      }
    }
  } else if constexpr (BWD) {
    // dlogits[t][v] = coef_t * (onehot - 2^(x*log2e - lse2_t)) in bf16 into the chunk
    // buffer (columns relative to the chunk start; vocab past V is written as 0), with
    // the forward's exchange: after one v_permlane16_swap per register pair each lane
    // holds 8 consecutive vocab rows of one token, one 16-byte store.
    const int vlim = a.V - vw;
#pragma unroll
    for (int jj = 0; jj < NJ16; jj += 2) {
      float cf[2], l2[2];
      int rel[2];
#pragma unroll
      for (int jo = 0; jo < 2; ++jo) {
        const int n = m0 + wt * TW + 16 * (jj + jo) + (lane & 15);
        cf[jo] = l2[jo] = 0.f;
        rel[jo] = -1;
        if (n < N) {
          cf[jo] = a.coef[n];
          l2[jo] = a.lse2[n];
          rel[jo] = static_cast<int>(lm_id(a, n) - vw);
        }
      }
#pragma unroll
      for (int i = 0; i < NI16; ++i) {
        uint32_t pk[2][2];
#pragma unroll
        for (int jo = 0; jo < 2; ++jo) {
          float d[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int vr = 16 * i + 4 * grp + r;
            const float x = -cf[jo] * hw_exp2(fmaf(acc[i][jj + jo][r], kLog2e, -l2[jo])) + (vr == rel[jo] ? cf[jo] : 0.f);
            d[r] = (cf[jo] != 0.f && vr < vlim) ? x : 0.f;
          }
          pk[jo][0] = pack2<BF16T>(d[0], d[1]);
          pk[jo][1] = pack2<BF16T>(d[2], d[3]);
        }
        const auto lo = __builtin_amdgcn_permlane16_swap(pk[0][0], pk[1][0], false, false);
        const auto hi = __builtin_amdgcn_permlane16_swap(pk[0][1], pk[1][1], false, false);
        const int n = m0 + wt * TW + 16 * (jj + (grp & 1)) + (lane & 15);
        const int col = vw - a.vc0 + 16 * i + 8 * (grp >> 1);
        if (n < N) {
          const u32x4 w = {lo[0], hi[0], lo[1], hi[1]};
          *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(a.dchunk) + static_cast<int64_t>(n) * a.ldd + col) = w;
        }
      }
    }
  } else {
    // C[v][t] (+)= the tile; rows past V and columns past N are not stored. For fixed
    // (i, r) each 16-lane group writes 16 consecutive floats of one row per token block,
    // and the wave's four token blocks follow each other, so each row's 256 bytes are
    // written by four consecutive stores (whole cache lines before any eviction).
    float* C = g.C;
    const int ldc = g.ldc, accumulate = g.accumulate;
    const int n0 = m0 + wt * TW + (lane & 15);
#pragma unroll
    for (int i = 0; i < NI16; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int vr = vw + 16 * i + 4 * grp + r;
        if (vr >= V) continue;
        float* row = C + static_cast<int64_t>(vr) * ldc;
#pragma unroll
        for (int j = 0; j < NJ16; ++j) {
          const int n = n0 + 16 * j;
          if (n < N) row[n] = accumulate ? row[n] + acc[i][j][r] : acc[i][j][r];
        }
      }
  }
}

// Tiles of product prod at this launch's live sizes (the kLmGemm row / K counts and
// the loss-head modes' token count are read from device memory).
template <int MODE>
__device__ __forceinline__ int lm_total_tiles(const LmTileArgs& a, int prod) {
  using namespace lm;
  if constexpr (MODE == kLmGemm) {
    const LmTileArgs::Gemm& g = a.gemm[prod];
    const int V = g.vcount ? min(g.V, *g.vcount) : g.V;
    return g.ntt * ((V + BV - 1) / BV);
  } else {
    const int N = min(a.N, *a.count);
    return ((N + BT - 1) / BT) * a.nvt;
  }
}

// One kLmFwd work item (lm_tile_kernel's order). Both models' tiles of one (token,
// vocab) pair are consecutive items, so they run side by side on one XCD and read each
// hidden slab from its L2 once.
template <bool ECACHE, bool E32>
__device__ __forceinline__ void lm_fwd_item(const LmTileArgs& a, char* smem) {
  const int xcd = blockIdx.x % 8, i = blockIdx.x / 8;
  const int nm = a.n_model > 1 ? 2 : 1;
  const int tt = lm_total_tiles<kLmFwd>(a, 0) * nm;
  const int per = (tt + 7) / 8;
  const int p = xcd * per + i;
  if (i >= per || p >= tt) return;
  lm_tile16<kLmFwd, ECACHE, E32>(a, p % nm, p / nm, smem);
}

// One workgroup per tile. Workgroup ids are dealt round-robin to the 8 XCDs, so
// workgroup b runs on XCD b % 8 and takes item b / 8 of that XCD's contiguous eighth of
// every product's tiles (products in order). The grid is sized for every token and
// the tiles for the live ones, so items past the XCD's share exit at once. Measured at
// config 5 against a persistent grid of one workgroup per CU that takes tiles from
// per-XCD atomic queues: 43.5 against 43.9 ms of kernel time per step (the queue's
// per-tile barriers and atomic cost more than these early exits), and against a
// persistent static split, 46.2 ms.
// ECACHE (kLmFwd): the policy's tiles also store the softmax terms. FRAG (kLmGemm): the
// token-role operands are fragment-major (the 16x16x32 tile, as the logit tiles);
// otherwise the products run on the 32x32x16 tile, ATR with a K-major token operand.
template <int MODE, bool ATR = false, bool ECACHE = false, bool FRAG = false>
__global__ void __launch_bounds__(lm::NTHR) __attribute__((amdgpu_waves_per_eu(lm::WPE, lm::WPE)))
lm_tile_kernel(LmTileArgs a) {
  extern __shared__ __align__(16) char smem[];
  if constexpr (MODE == kLmFwd) {
    lm_fwd_item<ECACHE, false>(a, smem);
  } else {
    const int xcd = blockIdx.x % 8, i = blockIdx.x / 8;
    const int t0 = lm_total_tiles<MODE>(a, 0);
    const int t1 = (MODE == kLmGemm && a.n_gemm > 1) ? lm_total_tiles<MODE>(a, 1) : 0;
    const int per0 = (t0 + 7) / 8, per1 = (t1 + 7) / 8;
    if (i >= per0 + per1) return;
    const int prod = i < per0 ? 0 : 1;
    const int p = prod == 0 ? xcd * per0 + i : xcd * per1 + (i - per0);
    if (p >= (prod == 0 ? t0 : t1)) return;
    if constexpr (FRAG || MODE == kLmBwd)
      lm_tile16<MODE, false>(a, prod, p, smem);
    else
      lm_tile<MODE, ATR>(a, prod, p, smem);
  }
}

// The kLmFwd launch that keeps the policy's softmax terms as f32 (a.ecache32), for
// the exact-rounding backward (PCP_FLAG_EXACT_BF16).
__global__ void __launch_bounds__(lm::NTHR) __attribute__((amdgpu_waves_per_eu(lm::WPE, lm::WPE)))
lm_tile_fwd32_kernel(LmTileArgs a) {
  extern __shared__ __align__(16) char smem[];
  lm_fwd_item<true, true>(a, smem);
}

// 64 x 64 bf16 tiles staged in LDS for a transpose: rows of 66 elements (33 words),
// so the column reads below, 8 rows apart per lane group, fall on distinct banks.
constexpr int kTilePitch = 66;

// t[r][c .. c+7] = v (c % 8 == 0), as four 32-bit writes (rows are 4-byte aligned).
__device__ __forceinline__ void tile_put8(uint16_t* t, int r, int c, u32x4 v) {
  uint32_t* w = reinterpret_cast<uint32_t*>(t + r * kTilePitch + c);
  w[0] = v[0];
  w[1] = v[1];
  w[2] = v[2];
  w[3] = v[3];
}

// Column c of rows r .. r+7, packed as 8 bf16.
__device__ __forceinline__ u32x4 tile_col8(const uint16_t* t, int r, int c) {
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    w[k] = static_cast<uint32_t>(t[(r + 2 * k) * kTilePitch + c]) |
           (static_cast<uint32_t>(t[(r + 2 * k + 1) * kTilePitch + c]) << 16);
  return u32x4{w[0], w[1], w[2], w[3]};
}

// Vocab tiles of 64 per lm_dcache_kernel block. With tile-major D and D^T, config 5
// (kernel traces, interleaved on one box): 1 tile 1.685 ms, 2 tiles 1.616-1.621 ms,
// 4 tiles 1.679, 8 tiles 1.696.
constexpr int kDcacheVocabTiles = 2;

// dlogits from the forward's softmax cache, per 64 x 64 tile (tokens x vocab): D is
// written in place over the cache (f16 terms -> bf16; the dhidden product's operand,
// tile-major with K extent ld: lm_tile_block_off) and transposed through LDS into Dt
// (the dW product's operand: vocab rows, tile-major with K extent ldt; tokens past n
// are 0). Each 64 x 64 tile is 8 KB contiguous in both. D[n][v] = -c_n * e * 2^(ref -
// lse2_n), with ref the exponent reference of v's 128-entry partial (from the
// policy's partials), except at the target, where D = c_n - c_n * 2^(tgt_n*log2e -
// lse2_n) from the f32 target logit, as the recomputing backward forms it. Columns
// past V and rows with c_n = 0 are 0. The cache is read and D, Dt written with
// nontemporal accesses: each byte is touched once here and read back only by the next
// launch, so keeping the lines in L2 only delays other traffic (config 5, kernel
// traces: 2.07 -> 1.85 ms; the same hint on the forward's cache stores cost 0.5 ms).
// D and Dt stores are nontemporal at system scope (written through to memory): 1.836 ->
// 1.801 ms at config 5 (kernel traces, three interleaved runs each).
// A block takes one 64-token tile and kDcacheVocabTiles vocab tiles in turn: the
// rows' scalars are read once, and each vocab tile's loads are issued before the
// previous tile's stores, so a wave's wait for them (vector-memory counts retire in
// issue order) does not include those stores. All accesses go through per-tile
// buffer descriptors with 32-bit offsets (the host checks ld and ldt).
// F32: the terms are f32 at a.src32 (the exact-rounding forward, tile-major as D) and D
// goes to a.d beside them, not in place.
template <bool F32>
__device__ __forceinline__ void lm_dcache_body(const LmDcacheArgs& a) {
  __shared__ uint16_t t[64 * kTilePitch];    // [token][vocab] bf16
  const int tid = threadIdx.x;
  const int64_t n = *a.count;
  const int64_t ntile = (n + 63) / 64;     // token tiles that the dW product reads
  const int cc = (tid & 7) * 8;            // the thread's 8 columns of a vocab tile
  const int rq = tid >> 3;                 // and its rows rq, rq + 32 of the token tile
  const int64_t vbase = static_cast<int64_t>(blockIdx.y) * kDcacheVocabTiles * 64;
  for (int64_t tb = blockIdx.x; tb < ntile; tb += gridDim.x) {
    const int64_t r0 = tb * 64;
    const uint32_t nr = static_cast<uint32_t>(min<int64_t>(64, n - r0));   // rows past n read 0, stores drop
    // D's 64 x 64 tile at vocab v0: 8 KB, row rr at 128 rr (rows past n: reads 0, stores drop).
    auto dtile = [&](int64_t v0) { return row_rsrc(a.d + lm_tile_block_off(r0, v0, a.ld), nr * 128u); };
    // F32: the terms' 64 x 64 tile at vocab v0, tile-major as D (rows of 256 bytes).
    auto stile = [&](int64_t v0) { return row_rsrc(a.src32 + lm_tile_block_off(r0, v0, a.ld), nr * 256u); };
    const __amdgpu_buffer_rsrc_t rp = row_rsrc(a.part + r0 * a.ldp, nr * static_cast<uint32_t>(a.ldp) * 8u);
    float cf[2], l2[2], tg[2];
    int id[2];
    {
      const __amdgpu_buffer_rsrc_t rc = row_rsrc(a.coef + r0, nr * 4u), rl = row_rsrc(a.lse2 + r0, nr * 4u),
                                   rt = row_rsrc(a.tgt + r0, nr * 4u), ri = row_rsrc(a.ids + r0, nr * 4u);
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const uint32_t off = static_cast<uint32_t>(rq + 32 * it) * 4u;
        cf[it] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rc, off, 0, 0));
        l2[it] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rl, off, 0, 0));
        tg[it] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rt, off, 0, 0));
        id[it] = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(ri, off, 0, 0));
      }
    }
    // Loads of vocab tile v0 into set q: the terms (16 or 32 bytes per row) and the
    // exponent reference of the tile's 128-entry partial. Past the row's columns they
    // read the next row's bytes (past the last row 0), never used.
    u32x4 w[2][2], w2[2][2];
    float m2[2][2];
    auto load = [&](int q, int64_t v0) {
      const uint32_t c0 = static_cast<uint32_t>(v0) + cc;
      const uint32_t pi = min(c0 / kLmPart, static_cast<uint32_t>(a.ldp - 1));
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const uint32_t rr = static_cast<uint32_t>(rq + 32 * it);
        if constexpr (F32) {
          const __amdgpu_buffer_rsrc_t rs = stile(v0);
          w[q][it] = buf_ld16<true>(rs, rr * 256u + static_cast<uint32_t>(cc) * 4u);
          w2[q][it] = buf_ld16<true>(rs, rr * 256u + static_cast<uint32_t>(cc) * 4u + 16u);
        } else {
          w[q][it] = buf_ld16<true>(dtile(v0), rr * 128u + static_cast<uint32_t>(cc) * 2u);
        }
        m2[q][it] = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(rp, (rr * static_cast<uint32_t>(a.ldp) + pi) * 8u, 0, 0));
      }
    };
    load(0, vbase);
#pragma unroll
    for (int vs = 0; vs < kDcacheVocabTiles; ++vs) {
      const int64_t v0 = vbase + vs * 64;
      if (v0 >= a.ld) break;
      const int q = vs & 1;
      if (vs + 1 < kDcacheVocabTiles) load(q ^ 1, v0 + 64);
      const int64_t c0 = v0 + cc;
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int rr = rq + 32 * it;
        u32x4 out = {0u, 0u, 0u, 0u};
        if (cf[it] != 0.f && c0 < a.V) {
          const float f = -cf[it] * hw_exp2(ms_ref(m2[q][it]) - l2[it]);
          const uint32_t ww[4] = {w[q][it][0], w[q][it][1], w[q][it][2], w[q][it][3]};
          const int64_t rel = static_cast<int64_t>(id[it]) - c0;
          float d[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const float e = F32 ? __uint_as_float(k < 4 ? w[q][it][k] : w2[q][it][k - 4]) : F16T::unpack(ww, k);
            d[k] = c0 + k < a.V ? f * e : 0.f;
          }
          if (rel >= 0 && rel < 8) {
            const float pt = hw_exp2(fmaf(tg[it], kLog2e, -l2[it]));
#pragma unroll
            for (int k = 0; k < 8; ++k) d[k] = k == rel ? -cf[it] * pt + cf[it] : d[k];
          }
          out = u32x4{pack2<BF16T>(d[0], d[1]), pack2<BF16T>(d[2], d[3]), pack2<BF16T>(d[4], d[5]),
                      pack2<BF16T>(d[6], d[7])};
        }
        buf_st16<true, kBufNTSystem>(dtile(v0), out, static_cast<uint32_t>(rr) * 128u + static_cast<uint32_t>(cc) * 2u);
        tile_put8(t, rr, cc, out);
      }
      __syncthreads();
      // Dt row v0 + c, tokens r0 + 8g .. +7: eight lanes write one row's 128 bytes, the
      // tile's 64 rows one 8 KB block piece.
      if (a.dt) {
        const __amdgpu_buffer_rsrc_t rdt = row_rsrc(a.dt + lm_tile_block_off(v0, r0, a.ldt), 64u * 128u);
#pragma unroll
        for (int it = 0; it < 2; ++it) {
          const int c = rq + 32 * it, g = tid & 7;
          buf_st16<true, kBufNTSystem>(rdt, tile_col8(t, 8 * g, c), static_cast<uint32_t>(c) * 128u + 16u * g);
        }
      }
      __syncthreads();
    }
  }
}

__global__ void __launch_bounds__(256) lm_dcache_kernel(LmDcacheArgs a) {
  lm_dcache_body<false>(a);
}
__global__ void __launch_bounds__(256) lm_dcache32_kernel(LmDcacheArgs a) { lm_dcache_body<true>(a); }

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

__global__ void __launch_bounds__(256) lm_gather_rows_kernel(const u32x4* src, u32x4* dst, const int* live,
                                                              const int* count, int H) {
  const int c = blockIdx.x;
  if (c >= *count) return;
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

// bf16 transpose through LDS, 64 x 64 tiles: 16-byte loads along source rows and
// 16-byte stores along destination rows, eight lanes per 128-byte row segment on both
// sides. Source rows past R read as 0, so the destination is zero-padded up to ld_dst.
__global__ void __launch_bounds__(256) lm_transpose_kernel(LmTransposeArgs a) {
  __shared__ uint16_t t[64 * kTilePitch];
  const int R = a.rcount ? min(a.R, *a.rcount) : a.R;
  const int64_t rend = min(a.ld_dst, (static_cast<int64_t>(R) + 63) / 64 * 64);   // destination columns written
  const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  if (r0 >= rend) return;
  const int tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int rr = it * 32 + (tid >> 3), cc = (tid & 7) * 8;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r0 + rr < R && c0 + cc < a.C)
      v = *reinterpret_cast<const u32x4*>(a.src + static_cast<int64_t>(r0 + rr) * a.ld_src + c0 + cc);
    tile_put8(t, rr, cc, v);
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int c = (tid >> 3) + 32 * it;   // source column = destination row
    const int g = tid & 7;                // source rows 8g .. 8g+7
    const int64_t r = r0 + 8 * g;
    if (c0 + c < a.C && r < rend)
      *reinterpret_cast<u32x4*>(a.dst + static_cast<int64_t>(c0 + c) * a.ld_dst + r) = tile_col8(t, 8 * g, c);
  }
}

// The same transpose into the fragment-major layout of the tile kernel's FRAG operand
// (the MFMA B fragment of destination rows FM b + [0, FM) and k FK s + [0, FK) at
// fragment b ld_dst/FK + s, lane l holding row FM b + l % FM and k FK s + 8 (l / FM) +
// 0..7; FM x FK = 16 x 32): destination rows are source columns, k runs over source
// rows. Each block's 64 x 64 tile is eight whole fragments, written as 1 KB runs; k from
// R up to R rounded to 64 is zero, and k past that is not written.
__global__ void __launch_bounds__(256) lm_transpose_frag_kernel(LmTransposeArgs a) {
  __shared__ uint16_t t[64 * kTilePitch];
  const int R = a.rcount ? min(a.R, *a.rcount) : a.R;
  const int64_t rend = min(a.ld_dst, (static_cast<int64_t>(R) + 63) / 64 * 64);
  const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  if (r0 >= rend) return;
  const int tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int rr = it * 32 + (tid >> 3), cc = (tid & 7) * 8;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r0 + rr < R && c0 + cc < a.C)
      v = *reinterpret_cast<const u32x4*>(a.src + static_cast<int64_t>(r0 + rr) * a.ld_src + c0 + cc);
    tile_put8(t, rr, cc, v);
  }
  __syncthreads();
  u32x4* dst = reinterpret_cast<u32x4*>(a.dst);
  constexpr int FM = 16, FK = 32;   // the 16x16x32 MFMA B fragment
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int idx = tid + 256 * it, f = idx >> 6, l = idx & 63;   // fragment f of the 8, lane l
    const int bl = f / (64 / FK), sl = f % (64 / FK);
    const int c = FM * bl + l % FM, r = FK * sl + 8 * (l / FM);
    if (c0 + c < a.C && r0 + r < rend)
      dst[(static_cast<int64_t>(c0 / FM + bl) * (a.ld_dst / FK) + r0 / FK + sl) * 64 + l] = tile_col8(t, r, c);
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

template <int MODE, bool EC = false, bool kAtr = MODE == kLmGemm, bool kFrag = false>
hipError_t launch_tiles_mode(const LmTileArgs& a, int max_tiles, hipStream_t st) {
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&lm_tile_kernel<MODE, kAtr, EC, kFrag>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lm::kSmem));
  if (e != hipSuccess) return e;
  // Items per XCD at the largest sizes: each product rounds its share up separately.
  const int grid = 8 * ((max_tiles + 7) / 8 + (MODE == kLmGemm && a.n_gemm > 1 ? 1 : 0));
  lm_tile_kernel<MODE, kAtr, EC, kFrag><<<dim3(grid), dim3(lm::NTHR), lm::kSmem, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_lm_tiles(int mode, const LmTileArgs& args, hipStream_t st) {
  LmTileArgs a = args;
  const int grid = a.ntt * a.nvt * (mode == kLmFwd && a.n_model > 1 ? 2 : 1);   // tiles at the largest token count
  if (grid <= 0) return hipSuccess;
  if (a.wt && (mode != kLmFwd || a.vt0 != 0 || a.ldwt % 64 != 0 || a.ldwt < a.V ||
               static_cast<int64_t>(a.nvt) * lm::BV < a.V || a.ldwt >= (int64_t{1} << 25)))
    return hipErrorInvalidValue;   // W^T from the forward: whole vocabulary, one stage's rows in 32-bit offsets
  if (mode == kLmFwd && a.ecache32) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&lm_tile_fwd32_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lm::kSmem));
    if (e != hipSuccess) return e;
    lm_tile_fwd32_kernel<<<dim3(8 * ((grid + 7) / 8)), dim3(lm::NTHR), lm::kSmem, st>>>(a);
    return hipGetLastError();
  }
  if (mode == kLmFwd)
    return a.ecache ? launch_tiles_mode<kLmFwd, true>(a, grid, st) : launch_tiles_mode<kLmFwd>(a, grid, st);
  return launch_tiles_mode<kLmBwd>(a, grid, st);
}

hipError_t launch_lm_gemms(const LmTileArgs::Gemm* g, int n_gemm, bool k_major_a, hipStream_t st) {
  LmTileArgs a;
  std::memset(&a, 0, sizeof(a));
  int grid = 0;
  a.n_gemm = n_gemm < 2 ? n_gemm : 2;
  for (int p = 0; p < a.n_gemm; ++p) {
    a.gemm[p] = g[p];
    a.gemm[p].group_m = lm_group_m(kLmGemm, g[p].ntt);
    grid += g[p].ntt * g[p].nvt;
  }
  if (grid <= 0) return hipSuccess;
  const bool frag = a.n_gemm > 0 && a.gemm[0].a_frag;
  if (a.n_gemm > 1 && (a.gemm[1].a_frag != 0) != frag) return hipErrorInvalidValue;   // one layout per launch
  if (frag && k_major_a) return hipErrorInvalidValue;
  for (int p = 0; p < a.n_gemm; ++p) {
    const LmTileArgs::Gemm& q = a.gemm[p];
    // Tile-major B: fragment-major launches only (the 16x16x32 tile reads it), whole
    // 64-deep blocks, a tile's K extent (ldb / 64 blocks of 32 KB) in 32-bit offsets.
    if (q.b_tiled && (!frag || q.ldb % 64 != 0 || q.K > q.ldb || static_cast<int64_t>(q.ldb / 64) * 32768 >= (int64_t{1} << 32)))
      return hipErrorInvalidValue;
  }
  if (frag) return launch_tiles_mode<kLmGemm, false, false, true>(a, grid, st);
  if (!k_major_a) return launch_tiles_mode<kLmGemm, false, false>(a, grid, st);
  return launch_tiles_mode<kLmGemm>(a, grid, st);
}

hipError_t launch_lm_transpose(const LmTransposeArgs& a, hipStream_t st) {
  if (a.C <= 0 || a.ld_dst <= 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((a.C + 63) / 64), static_cast<unsigned>((a.ld_dst + 63) / 64));
  lm_transpose_kernel<<<grid, dim3(256), 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_lm_transpose_frag(const LmTransposeArgs& a, hipStream_t st) {
  if (a.C <= 0 || a.ld_dst <= 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((a.C + 63) / 64), static_cast<unsigned>((a.ld_dst + 63) / 64));
  lm_transpose_frag_kernel<<<grid, dim3(256), 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_lm_reduce(const LmReduceArgs& a, hipStream_t st) {
  lm_reduce_kernel<<<dim3(static_cast<unsigned>((a.N + 3) / 4)), dim3(256), 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_lm_dcache(const LmDcacheArgs& a, hipStream_t st) {
  if (a.ldt <= 0 || a.ld <= 0) return hipSuccess;
  // 32-bit offsets within a tile's descriptors: 64 rows of f32 terms, 64 Dt rows.
  if (a.ld >= (int64_t{1} << 24) || a.ldt >= (int64_t{1} << 25) || static_cast<int64_t>(a.ldp) * 64 * 8 >= (int64_t{1} << 32))
    return hipErrorInvalidValue;
  // Token tiles are the grid's fast dimension: the blocks past the live count (the grid
  // is sized for every token) are interleaved with live ones instead of forming a tail.
  // At config 5, 1.95 ms with an exact grid (host-read count), 2.08 ms with the dead
  // blocks as a tail or with a 16-row grid looping over token tiles.
  const int64_t ntile = a.ldt / 64;
  const int64_t vblocks = (a.ld / 64 + kDcacheVocabTiles - 1) / kDcacheVocabTiles;
  const dim3 grid(static_cast<unsigned>(ntile < 65535 ? ntile : 65535), static_cast<unsigned>(vblocks));
  if (a.src32)
    lm_dcache32_kernel<<<grid, dim3(256), 0, st>>>(a);
  else
    lm_dcache_kernel<<<grid, dim3(256), 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_lm_compact(const LmCompactArgs& a, hipStream_t st) {
  lm_compact_kernel<<<dim3(1), dim3(1024), 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_lm_gather_rows(const void* src, void* dst, const int* live, const int* count, int n, int H,
                                 hipStream_t st) {
  if (n <= 0) return hipSuccess;
  lm_gather_rows_kernel<<<dim3(n), dim3(256), 0, st>>>(static_cast<const u32x4*>(src), static_cast<u32x4*>(dst),
                                                       live, count, H);
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
