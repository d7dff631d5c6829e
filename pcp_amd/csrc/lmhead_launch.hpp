// Host-side launch interface of the fused LM-head kernels (lmhead_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pcp {

struct RowArgs;

enum { kLmFwd = 0, kLmBwd = 1, kLmGemm = 2 };

constexpr int kLmTileV = 256;    // vocab entries per tile
constexpr int kLmTileT = 256;    // tokens per tile
constexpr int kLmPart = 128;     // vocab entries per log-sum-exp partial

// Tile-major bf16 operand of the products (the cached backward's D and D^T): 32 KB
// blocks of [256 rows][64 k], block (r / 256, k / 64) at element
// ((r / 256) * (ld / 64) + k / 64) * 16384, row r % 256 at 64 (r % 256) within it, so
// one product stage (256 rows x 64 k) is one contiguous block and a 64 x 64 tile of
// the dlogits pass is 8 KB contiguous. ld: the K extent, a multiple of 64.
__host__ __device__ __forceinline__ int64_t lm_tile_block_off(int64_t r, int64_t k, int64_t ld) {
  return ((r >> 8) * (ld >> 6) + (k >> 6)) * 16384 + (r & 255) * 64 + (k & 63);
}

// One launch covers token tiles [0, ntt) x vocab tiles [vt0, vt0 + nvt) of
// kLmTileT x kLmTileV. kLmGemm reuses the roles for plain products
// C[v][t] = sum_k B[v][k] * A[t][k] (both operands K-contiguous, bf16): "vocab" rows
// come from B, "token" rows from A.
struct LmTileArgs {
  const void* A;        // hidden [N, H] bf16, row-major
  const void* B;        // weight [V, H] bf16, row-major
  int N, V, H;          // H % 64 == 0; N bounds *count
  int vt0, nvt, ntt;    // ntt: token tiles of N (sizes the grid); the kernel uses *count's
  const int* count;     // [1] live tokens (device): the kLmFwd / kLmBwd tiles cover rows < *count
  int n_gemm;           // kLmGemm: products in gemm[] (1 or 2)
  const void* ids;      // [N] target ids
  int ids_i64;
  // kLmFwd (model 0: B, part, tgt, ecache; with n_model = 2 also model 1: B2, part2,
  // tgt2, in the same launch, its tiles interleaved with model 0's)
  float2* part;         // [N, ldp]: per kLmPart vocab entries (max * log2e, sum 2^(x*log2e - max*log2e))
  int ldp;              // ceil(V / kLmPart)
  float* tgt;           // [N] target logit
  int n_model;          // 1 or 2
  const void* B2;       // [V, H] bf16: model 1's weight
  float2* part2;
  float* tgt2;
  uint16_t* ecache;     // or nullptr: f16 softmax terms 2^(x*log2e - ref) of the partial's
  int64_t lde;          //   reference ref, tile-major (lm_tile_block_off: token rows, K extent
                        //   lde; lde % 64 == 0, >= V; 0 past V)
  float* ecache32;      // or nullptr: the same terms as f32, in the same layout (ecache then nullptr)
  uint16_t* wt;         // or nullptr: W^T [H, ldwt] fragment-major (launch_lm_transpose_frag's layout),
  int64_t ldwt;         //   written by model 0's tiles from their W slabs (ldwt % 64 == 0, >= V)
  // kLmBwd
  const float* lse2;    // [N] base-2 log-sum-exp
  const float* coef;    // [N] d loss / d logp
  void* dchunk;         // [N, ldd] bf16 dlogits of vocab [vc0, vc0 + ldd)
  int vc0, ldd;
  // kLmGemm: up to two independent products in one launch (each XCD takes its share of
  // gemm[0]'s tiles, then of gemm[1]'s); the fields above are unused.
  // result[v][t] = sum_k B[v][k] * A(k, t): B rows are K-contiguous; A is either
  // K-contiguous too (element (k, t) at A[t * lda + k]) or stored K-major (at
  // A[k * lda + t]) and read with LDS transpose loads (launch_lm_gemms' k_major_a).
  struct Gemm {
    const void* A;      // [krows_a, lda] K-major or [N, lda] bf16: "token" columns (result columns)
    const void* B;      // [V, ldb] bf16, K-contiguous: "vocab" rows (result rows)
    int N, V, K;        // K % 64 == 0, K <= ldb
    int lda, ldb;       // row strides in elements (lda >= N rounded up to 8)
    int krows_a;        // K-major A: rows that exist; rows [krows_a, K) read as 0
    int a_frag;         // A stored fragment-major (launch_lm_transpose_frag, K extent lda): read
                        //   straight into registers; both products of a launch alike
    int b_tiled;        // (a_frag only) B stored tile-major: 32 KB blocks of [256 rows][64 k],
                        //   block (v / 256, k / 64) at byte ((v / 256) * (ldb / 64) + k / 64) * 32768,
                        //   row v % 256 at 128 (v % 256) within it (lm_tile_block_off)
    const int* vcount;  // or nullptr: V = *vcount (<= V; tiles past it exit)
    const int* kcount;  // or nullptr: K = *kcount rounded up to 64 (<= K), krows_a = *kcount
    float* C;           // f32 result: row v, column t at C[v * ldc + t], or at
    int ldc;            //   C[t * ldc + v] with transpose_c (then V % 4 == 0)
    int transpose_c;
    int accumulate;     // 1: C += product, 0: C = product
    int ntt, nvt;       // tiles over N and over V (nvt at the largest V)
    int group_m;        // set by launch_lm_gemms
  } gemm[2];
};

// dst[c][r] = src[r][c] for r < R, c < C; dst[c][r] = 0 for R <= r < min(ld_dst, R
// rounded up to 64) (bf16). With rcount, R = *rcount (device; at most the R given).
struct LmTransposeArgs {
  const uint16_t* src;
  int64_t ld_src;
  int R, C;
  uint16_t* dst;
  int64_t ld_dst;
  const int* rcount;
};

// Over the softmax cache: d[n][v] (f16 term) -> bf16 dlogits in place for n < *count,
// and the same values transposed into dt[v][n], zero for *count <= n < *count rounded
// up to 64 (columns past that are not written).
struct LmDcacheArgs {
  uint16_t* d;            // bf16 D, tile-major (lm_tile_block_off: token rows, K extent ld),
                          //   written over the f16 terms the forward stored there (src32 nullptr)
  const float* src32;     // or the f32 terms (tile-major as d), read in place of d's
  int64_t ld;             // multiple of 64, >= V
  const int* count;       // [1] live tokens (device)
  uint16_t* dt;           // D^T, tile-major (vocab rows, K extent ldt), or nullptr
  int64_t ldt;            // multiple of 64, >= *count
  int64_t V;
  const float2* part;     // [n, ldp] the policy's forward partials
  int ldp;
  const float* lse2;      // [n]
  const float* coef;      // [n]
  const float* tgt;       // [n] target logit
  const int* ids;         // [n] compact target ids
};

struct LmReduceArgs {
  const float2* part;
  int64_t N;              // bounds *count (the grid)
  const int* count;       // [1] live tokens (device)
  int ldp, nvt;
  float* lse2;          // out
};

struct LmTermsArgs {
  int64_t N;
  const int* cidx;        // [N] token -> compact index (-1: not live)
  const float* tgt;       // per compact index
  const float* lse2;
  const float* ref_tgt;   // nullptr: no reference model
  const float* ref_lse2;
  float* coef;            // out, per compact index
};

// Live-token compaction: live = mask != 0 and 0 <= id < V, in ascending token order.
struct LmCompactArgs {
  const void* ids;
  int ids_i64;
  const void* mask;       // nullptr: all live
  int mask_u8;
  int N, V;
  int* live;              // [N] compact -> token
  int* cidx;              // [N] token -> compact, -1 when not live
  int* ids_c;             // [N] compact target ids (int32)
  int* count;             // [1] number of live tokens
};

size_t lm_tile_smem_bytes();
// Final RMSNorm around the LM head (norm_kernels.hip).
constexpr int kLmNormMaxHidden = 8192;   // the forward holds 32 columns per thread
constexpr int kLmNormSlices = 64;        // dgamma partials (slices of the live rows)

struct LmNormBwdArgs {
  const float* dyc;       // [n_live, H] f32 gradient of the normed operand, compact rows
  const uint16_t* h;      // [N, H] bf16 pre-norm hidden states (token order)
  const float* gamma;     // [H]
  const float* rstd;      // [n_live] from the forward
  const int* cidx;        // [N] token -> compact index (-1: not live)
  const int* live;        // [n_live] compact index -> token
  int64_t N;
  int H;
  const int* count;       // [1] n_live (device)
  float* dh;              // [N, H] or nullptr
  float* gpart;           // [kLmNormSlices, H] dgamma partials, or nullptr
  float* dgamma;          // [H] or nullptr
};

// y / rstd rows c < *count from live[c]; n bounds the count (the grid).
hipError_t launch_lm_norm_rows(const void* h, const float* gamma, float eps, const int* live, const int* count,
                               int n, int H, void* y, float* rstd, hipStream_t st);
hipError_t launch_lm_norm_bwd(const LmNormBwdArgs& a, hipStream_t st);

hipError_t launch_lm_compact(const LmCompactArgs& a, hipStream_t st);
// dst[c, :] = src[live[c], :] for c < *count <= n (bf16 rows of H elements, H % 64 == 0).
hipError_t launch_lm_gather_rows(const void* src, void* dst, const int* live, const int* count, int n, int H,
                                 hipStream_t st);
// dst[t, :] = cidx[t] >= 0 ? src[cidx[t], :] : 0 for t < N (f32 rows of H elements).
hipError_t launch_lm_scatter_rows(const float* src, float* dst, const int* cidx, int N, int H, hipStream_t st);
hipError_t launch_lm_zero(float* dst, int64_t n, hipStream_t st);
hipError_t launch_lm_tiles(int mode, const LmTileArgs& a, hipStream_t st);
// One launch of one or two products (n_gemm = 1 or 2; fields per LmTileArgs::Gemm,
// group_m is filled in here). The longer product should come first. k_major_a: A is
// stored K-major (read with LDS transpose loads); otherwise A is K-contiguous like B
// ([N, lda], krows_a unused).
hipError_t launch_lm_gemms(const LmTileArgs::Gemm* g, int n_gemm, bool k_major_a, hipStream_t st);
hipError_t launch_lm_transpose(const LmTransposeArgs& a, hipStream_t st);
// The same transpose written in the fragment-major layout of Gemm::a_frag operands
// (dst rows = C, padded to 32; k extent ld_dst, a multiple of 64).
hipError_t launch_lm_transpose_frag(const LmTransposeArgs& a, hipStream_t st);
hipError_t launch_lm_reduce(const LmReduceArgs& a, hipStream_t st);
hipError_t launch_lm_dcache(const LmDcacheArgs& a, hipStream_t st);
hipError_t launch_lm_terms(const RowArgs& ra, const LmTermsArgs& a, hipStream_t st);

}  // namespace pcp
