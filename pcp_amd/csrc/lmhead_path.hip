// Device-pointer entry point of the fused LM-head + GRPO loss (pcp_grpo_lmhead_fwd_bwd).
//
// Live tokens (mask != 0, id in [0, V)) are compacted first: a masked or ignored
// token has zero loss weight and zero gradient, so only live hidden rows enter the
// products. The live count stays on the device: buffers and grids are sized for all
// tokens and every kernel reads the count, so the call never waits for the device
// (PCP_FLAG_ASYNC returns after enqueueing, and the call can be captured in a graph).
// Forward, per model (reference, then policy): MFMA logits tiles reduced in-tile to
// per-(token, vocab tile) log-sum-exp partials and the target logit; one wave per
// token merges the partials. Then the GRPO terms per token and the loss reduction
// (the same kernels as the logits-input path).
// Backward, by default: the policy forward also stored its softmax terms (f16, or f32
// with PCP_FLAG_EXACT_BF16); one pass turns them into bf16 dlogits D (in place over
// f16 terms, beside f32 ones) and writes D^T, the policy forward's tiles also write W^T
// from the W slabs they hold, and one launch of the MFMA tile kernel (kLmGemm, both
// operands K-contiguous) runs
//   dhidden = D * W      over the whole vocabulary (rows: live tokens), and
//   dW      = D^T * hidden over the live tokens (rows: vocab).
// Chunked backward (an explicit vocab_chunk, or a workspace past cache_budget):
// per vocab chunk, logits tiles recomputed into bf16 D, then the same two products
// (on transposed copies of the chunk and of W when they fit the budget, else with one
// operand read K-major through LDS transpose loads), dhidden accumulating over the
// chunks.
// Either way the compact dhidden rows are scattered back (zero rows for dead tokens).
// This mirrors the LM head's VJP (src/autodiff/vjp_rules.zig:426-497, matmulVJP).

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>

#include "context.hpp"
#include "grpo_device.hpp"
#include "grpo_launch.hpp"
#include "lmhead_launch.hpp"
#include "pcp_grpo.h"
#include "pcp_synth.h"

namespace pcp {
namespace {

constexpr int64_t kDefaultChunk = 16384;
// Cap on the backward workspace (softmax cache, D^T, W^T; sized for all N tokens) the
// default path allocates: 11.3 GB at configuration 5 (16,384 tokens, V = 151,936,
// H = 4,096). 64 GiB holds it up to about 110,000 tokens at that vocabulary.
constexpr size_t kCacheBudgetCap = size_t{64} << 30;

// Bytes the backward workspace may occupy on this call: the cap, and at most half of
// the device memory that is free now plus what the context already holds, so a
// training loop sharing the GPU keeps the other half. A workspace larger than this
// budget is not allocated: the backward then runs chunked, in less memory.
size_t cache_budget(pcp_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->lm_dbuf_bytes) return ctx->lm_dbuf_bytes;   // already held
  size_t free_b = 0, total_b = 0;
  if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  const size_t avail = (free_b + ctx->lm_dbuf_bytes) / 2;
  return avail < kCacheBudgetCap ? avail : kCacheBudgetCap;
}

inline size_t r256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

// Grow ctx->lm_dbuf to at least `bytes` (grow-only; synchronises before freeing the
// old buffer, which earlier asynchronous calls may still use). A failed hipMalloc
// leaves no buffer and no sticky error.
hipError_t grow_dbuf(pcp_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->lm_dbuf_bytes) return hipSuccess;
  if (ctx->lm_dbuf) {
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return e;
    (void)hipFree(ctx->lm_dbuf);
    ctx->lm_dbuf = nullptr;
    ctx->lm_dbuf_bytes = 0;
  }
  const size_t want = (bytes + 0xFFFFF) & ~static_cast<size_t>(0xFFFFF);
  const hipError_t e = hipMalloc(&ctx->lm_dbuf, want);
  if (e != hipSuccess) {
    ctx->lm_dbuf = nullptr;
    (void)hipGetLastError();
    return e;
  }
  ctx->lm_dbuf_bytes = want;
  return hipSuccess;
}

int validate_lm(const pcp_lmhead_args* a) {
  if (!a) return fail(nullptr, PCP_ERR_INVALID_ARG, "args is NULL");
  if (a->n_seq < 1 || a->rows < 1) return fail(nullptr, PCP_ERR_INVALID_ARG, "n_seq and rows must be >= 1");
  if (a->hidden < 64 || a->hidden % 64 != 0 || a->hidden > (1 << 20))
    return fail(nullptr, PCP_ERR_INVALID_ARG, "hidden must be a positive multiple of 64 (got %lld)", (long long)a->hidden);
  if (a->vocab < 1 || a->vocab > (1 << 30)) return fail(nullptr, PCP_ERR_INVALID_ARG, "vocab out of range");
  if (a->group_size < 1) return fail(nullptr, PCP_ERR_INVALID_ARG, "group_size must be >= 1");
  int64_t n;
  if (mul_overflows(a->n_seq, a->rows, &n) || n > (1 << 28))
    return fail(nullptr, PCP_ERR_OVERFLOW, "n_seq * rows exceeds 2^28 tokens");
  // The products address a dlogits chunk [tokens, chunk] and a W chunk [chunk, H] with
  // 32-bit buffer offsets.
  {
    const int64_t ch = a->vocab_chunk ? a->vocab_chunk : kDefaultChunk;
    if ((a->dweight || a->dhidden || a->dnorm_weight) &&
        ((n + 63) / 64 * 64 * ch * 2 >= (int64_t{1} << 32) || ch * a->hidden * 2 >= (int64_t{1} << 32)))
      return fail(nullptr, PCP_ERR_OVERFLOW,
                  "tokens x vocab_chunk and vocab_chunk x hidden must stay under 2^31 elements for the "
                  "backward (%lld tokens, chunk %lld, hidden %lld): pass a smaller vocab_chunk",
                  (long long)n, (long long)ch, (long long)a->hidden);
  }
  if (a->vocab_chunk < 0 || a->vocab_chunk % kLmTileV != 0)
    return fail(nullptr, PCP_ERR_INVALID_ARG, "vocab_chunk must be a multiple of %d", kLmTileV);
  if (!a->hidden_states || !a->weight || !a->ids) return fail(nullptr, PCP_ERR_INVALID_ARG, "hidden_states / weight / ids is NULL");
  if (a->ids_dtype != PCP_I64 && a->ids_dtype != PCP_I32) return fail(nullptr, PCP_ERR_DTYPE, "ids dtype must be i64 or i32");
  if (a->mask && a->mask_dtype != PCP_F32 && a->mask_dtype != PCP_BOOL)
    return fail(nullptr, PCP_ERR_DTYPE, "mask dtype must be f32 or bool");
  if (a->loss_mode != PCP_LOSS_REINFORCE && a->loss_mode != PCP_LOSS_GRPO_CLIP_KL)
    return fail(nullptr, PCP_ERR_INVALID_ARG, "unknown loss_mode %d", a->loss_mode);
  if (a->loss_mode == PCP_LOSS_GRPO_CLIP_KL && !a->ref_weight)
    return fail(nullptr, PCP_ERR_INVALID_ARG, "GRPO_CLIP_KL needs ref_weight");
  if (!a->advantages && !a->rewards) return fail(nullptr, PCP_ERR_INVALID_ARG, "advantages and rewards are both NULL");
  if (!(a->clip_eps >= 0.f && a->clip_eps < 1.f)) return fail(nullptr, PCP_ERR_INVALID_ARG, "clip_eps must be in [0, 1)");
  if (!(a->loss_norm >= 0.f)) return fail(nullptr, PCP_ERR_INVALID_ARG, "loss_norm must be >= 0");
  if (a->dnorm_weight && !a->norm_weight) return fail(nullptr, PCP_ERR_INVALID_ARG, "dnorm_weight needs norm_weight");
  if (a->norm_weight && a->hidden > kLmNormMaxHidden)
    return fail(nullptr, PCP_ERR_INVALID_ARG, "the fused final norm takes hidden <= %d (got %lld)", kLmNormMaxHidden,
                (long long)a->hidden);
  if (a->norm_weight && !(a->norm_eps >= 0.f && a->norm_eps < 1e30f))
    return fail(nullptr, PCP_ERR_INVALID_ARG, "norm_eps must be finite and >= 0");
  if (a->norm_weight && ((reinterpret_cast<uintptr_t>(a->norm_weight) | reinterpret_cast<uintptr_t>(a->dhidden)) & 15u))
    return fail(nullptr, PCP_ERR_INVALID_ARG, "norm_weight / dhidden must be 16-byte aligned");
  const uintptr_t al = reinterpret_cast<uintptr_t>(a->hidden_states) | reinterpret_cast<uintptr_t>(a->weight) |
                       reinterpret_cast<uintptr_t>(a->ref_weight);
  if (al & 15u) return fail(nullptr, PCP_ERR_INVALID_ARG, "hidden_states / weights must be 16-byte aligned");
  return PCP_OK;
}

int run_lm(pcp_ctx* ctx, const pcp_lmhead_args* a) {
  int rc = validate_lm(a);
  if (rc != PCP_OK) {
    if (ctx) copy_thread_error(ctx);
    return rc;
  }
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  hipStream_t st = static_cast<hipStream_t>(a->stream);

  const int64_t S = a->n_seq, T = a->rows, N = S * T, H = a->hidden, V = a->vocab;
  const int nvt = static_cast<int>((V + kLmTileV - 1) / kLmTileV);     // vocab tiles
  const int npart = static_cast<int>((V + kLmPart - 1) / kLmPart);    // log-sum-exp partials per token
  const bool ref = a->loss_mode == PCP_LOSS_GRPO_CLIP_KL;
  const bool norm = a->norm_weight != nullptr;
  const bool bwd = a->dhidden || a->dweight || a->dnorm_weight;
  const bool want_dy = a->dhidden || a->dnorm_weight;   // compact gradient of the LM head's operand
  const int64_t chunk = a->vocab_chunk ? a->vocab_chunk : kDefaultChunk;
  const float loss_norm = a->loss_norm > 0.f ? a->loss_norm : static_cast<float>(S);

  // Scratch layout (token arrays sized for N; the live prefix is used).
  size_t off = 0;
  auto take = [&](size_t bytes) { const size_t o = off; off += r256(bytes); return o; };
  const size_t o_adv = take(4 * S), o_len = take(4 * S), o_scale = take(4 * S), o_val = take(4 * S), o_loss = take(4);
  const size_t o_done = take(4);
  const size_t o_tl = a->token_loss ? 0 : take(4 * N);
  const size_t o_live = take(4 * N), o_cidx = take(4 * N), o_idsc = take(4 * N), o_cnt = take(4);
  const size_t o_hid = take(2 * static_cast<size_t>(N) * H);
  const size_t o_part = take(8 * static_cast<size_t>(N) * npart);
  const size_t o_part2 = ref ? take(8 * static_cast<size_t>(N) * npart) : 0;
  const size_t o_tgt = take(4 * N), o_l2 = take(4 * N), o_rtgt = take(4 * N), o_rl2 = take(4 * N), o_coef = take(4 * N);
  // Row stride, in tokens, of the transposed operands (hidden^T, D^T): a multiple of the
  // 64-deep pipeline stage, and off multiples of 256 (a 2^k-byte stride puts the rows
  // that one block writes or one tile reads on the same HBM channels).
  const int64_t ldt_max = (N + 63) / 64 * 64 + ((N + 63) / 64 * 64 % 256 == 0 ? 64 : 0);
  const size_t o_ht = a->dweight ? take(2 * static_cast<size_t>(H) * ldt_max) : 0;
  const size_t o_dhc = want_dy ? take(4 * static_cast<size_t>(N) * H) : 0;
  const size_t o_rstd = norm ? take(4 * N) : 0;
  const size_t o_gpart = a->dnorm_weight ? take(4 * static_cast<size_t>(kLmNormSlices) * H) : 0;
  rc = ensure_scratch(ctx, off);
  if (rc != PCP_OK) return rc;
  char* sp = static_cast<char*>(ctx->scratch);
  auto F = [&](size_t o) { return reinterpret_cast<float*>(sp + o); };
  auto I = [&](size_t o) { return reinterpret_cast<int*>(sp + o); };
  float* tl = a->token_loss ? a->token_loss : F(o_tl);
  float2* part = reinterpret_cast<float2*>(sp + o_part);
  const int mask_u8 = a->mask_dtype == PCP_BOOL;

  // The backward's bf16 operands, sized for all N tokens (the live count stays on the
  // device). By default: the whole-vocabulary softmax cache (the policy forward stores
  // its f16 terms there, tile-major over token rows with K extent ldv; a pass rewrites
  // them in place as dlogits D and writes D^T, tile-major over vocab rows with K extent
  // ldt, beside it) and W^T [H, ldv], so both products read K-contiguous operands.
  // With PCP_FLAG_EXACT_BF16 the terms are f32, in the same layout, and D follows them
  // (D is then the f32 value rounded once). With an explicit vocab_chunk, more than
  // cache_budget bytes, or no memory for them: one dlogits chunk [N, chunk] that the
  // backward refills by recomputing the logits.
  // D and D^T are tile-major (lm_tile_block_off: 32 KB blocks of 256 rows x 64 k), so
  // their rows round up to 256: D's token rows ldr, D^T's vocab rows ldv256.
  const bool exact = (a->flags & PCP_FLAG_EXACT_BF16) != 0;
  const int64_t ldv = (V + 63) / 64 * 64;
  const int64_t ldt = ldt_max;
  const int64_t ldr = (ldt + 255) / 256 * 256, ldv256 = (ldv + 255) / 256 * 256;
  const size_t o_d = exact ? 4 * static_cast<size_t>(ldr) * ldv : 0;
  const size_t o_dt = o_d + 2 * static_cast<size_t>(ldr) * ldv;
  const size_t o_wt = o_dt + (a->dweight ? 2 * static_cast<size_t>(ldv256) * ldt : 0);
  const size_t cache_bytes = o_wt + (want_dy ? 2 * static_cast<size_t>(H) * ldv : 0);
  const size_t o_cdt = 2 * static_cast<size_t>(ldt) * chunk;
  const size_t o_cwt = o_cdt + (a->dweight ? 2 * static_cast<size_t>(chunk) * ldt : 0);
  const size_t chunk_frag_bytes = o_cwt + (want_dy ? 2 * static_cast<size_t>(H) * ldv : 0);
  bool cached = false, chunk_frag = false;
  // 32-bit offsets: a 64-token tile of f32 terms in the dlogits pass (launch_lm_dcache)
  // and a product tile's K extent of tile-major D or D^T (ld / 64 blocks of 32 KB,
  // launch_lm_gemms): larger shapes take the chunked backward.
  const bool cache_fits = ldv < (int64_t{1} << 23) && ldt < (int64_t{1} << 23);
  // W^T comes out of the forward while one stage's four fragment rows fit 32-bit offsets.
  const bool wt_fwd = ldv < (int64_t{1} << 25);
  if (bwd) {
    if (a->vocab_chunk == 0 && cache_fits && cache_bytes <= cache_budget(ctx, cache_bytes)) {
      e = grow_dbuf(ctx, cache_bytes);
      if (e == hipSuccess) cached = true;
      else if (e != hipErrorOutOfMemory) return hip_fail(ctx, e, "allocating the softmax cache");
    }
    // Chunked: the dlogits chunk [ldt, chunk], with room for its transpose [chunk, ldt] and
    // W^T [H, ldv] (fragment-major, once per call) the products run as on the cached
    // path; past the budget, in less memory, or with PCP_FLAG_FORCE_STREAMING, with
    // K-major operands and no transposed copies.
    if (!cached && !(a->flags & PCP_FLAG_FORCE_STREAMING) &&
        chunk_frag_bytes <= cache_budget(ctx, chunk_frag_bytes)) {
      e = grow_dbuf(ctx, chunk_frag_bytes);
      if (e == hipSuccess) chunk_frag = true;
      else if (e != hipErrorOutOfMemory) return hip_fail(ctx, e, "allocating the dlogits chunk");
    }
    if (!cached && !chunk_frag && (e = grow_dbuf(ctx, 2 * static_cast<size_t>(N) * chunk)) != hipSuccess) {
      if (e == hipErrorOutOfMemory)
        return fail(ctx, PCP_ERR_OOM, "hipMalloc of the %lld x %lld dlogits chunk failed", (long long)N,
                    (long long)chunk);
      return hip_fail(ctx, e, "allocating the dlogits chunk");
    }
  }

  // Live-token compaction. The count stays on the device: every kernel below reads it
  // (grids cover all N tokens; work past the count exits or is zero), so the call never
  // waits for the device.
  const int* cnt = I(o_cnt);
  LmCompactArgs ca{a->ids, a->ids_dtype == PCP_I64, a->mask, mask_u8, static_cast<int>(N), static_cast<int>(V),
                   I(o_live), I(o_cidx), I(o_idsc), I(o_cnt)};
  if ((e = launch_lm_compact(ca, st)) != hipSuccess) return hip_fail(ctx, e, "compaction launch");
  const int ntl = static_cast<int>((N + kLmTileT - 1) / kLmTileT);
  if (norm) {
    if ((e = launch_lm_norm_rows(a->hidden_states, a->norm_weight, a->norm_eps, I(o_live), cnt, static_cast<int>(N),
                                 static_cast<int>(H), sp + o_hid, F(o_rstd), st)) != hipSuccess)
      return hip_fail(ctx, e, "final norm of live hidden rows");
  } else if ((e = launch_lm_gather_rows(a->hidden_states, sp + o_hid, I(o_live), cnt, static_cast<int>(N),
                                        static_cast<int>(H), st)) != hipSuccess) {
    return hip_fail(ctx, e, "gathering live hidden rows");
  }

  // Advantages (or the copy of the given ones), per-sequence lengths and the loss
  // ticket's counter, in one launch.
  const float* adv = a->advantages ? a->advantages : F(o_adv);
  {
    StepPrepArgs pa;
    std::memset(&pa, 0, sizeof(pa));
    pa.mask = a->mask;
    pa.mask_u8 = mask_u8;
    pa.n_seq = S;
    pa.rows = T;
    pa.tok_stride = T;
    pa.tok_offset = 0;
    pa.loss_norm = loss_norm;
    pa.seq_len = F(o_len);
    pa.seq_scale = F(o_scale);
    pa.rewards = a->advantages ? nullptr : a->rewards;
    pa.adv_in = a->advantages;
    pa.group = a->group_size;
    pa.std_eps = a->std_eps;
    pa.adv = F(o_adv);
    pa.adv_out = a->advantages_out != adv ? a->advantages_out : nullptr;
    pa.zero[0] = I(o_done);
    if ((e = launch_step_prep(pa, st)) != hipSuccess) return hip_fail(ctx, e, "step prep launch");
  }

  // Forward, per model: tiles -> partials + target logit; merge -> lse2.
  LmTileArgs ta;
  std::memset(&ta, 0, sizeof(ta));
  ta.A = sp + o_hid;
  ta.N = static_cast<int>(N);
  ta.count = cnt;
  ta.V = static_cast<int>(V);
  ta.H = static_cast<int>(H);
  ta.vt0 = 0;
  ta.nvt = nvt;
  ta.ntt = ntl;
  ta.ids = I(o_idsc);
  ta.ids_i64 = 0;
  ta.part = part;
  ta.ldp = npart;
  // Both models in one launch (their tiles interleaved, so each hidden slab is read once
  // for both), then one merge per model.
  ta.B = a->weight;
  ta.tgt = F(o_tgt);
  ta.ecache = cached && !exact ? static_cast<uint16_t*>(ctx->lm_dbuf) : nullptr;
  ta.ecache32 = cached && exact ? static_cast<float*>(ctx->lm_dbuf) : nullptr;
  ta.lde = ldv;
  // W^T [H, ldv] fragment-major (the dhidden product's token operand) comes out of the
  // forward: the policy's tiles write it from the W slabs they hold.
  if (want_dy && wt_fwd && (cached || chunk_frag)) {
    ta.wt = reinterpret_cast<uint16_t*>(static_cast<char*>(ctx->lm_dbuf) + (cached ? o_wt : o_cwt));
    ta.ldwt = ldv;
  }
  ta.n_model = ref ? 2 : 1;
  if (ref) {
    ta.B2 = a->ref_weight;
    ta.tgt2 = F(o_rtgt);
    ta.part2 = reinterpret_cast<float2*>(sp + o_part2);
  }
  {
    // pcp_profile_start timing: the forward launch when the backward is chunked, the
    // products launch (below) when it reads the softmax cache.
    const bool timed = !cached && ctx->prof_on && ctx->prof_used < static_cast<int>(ctx->prof_start.size());
    if (timed && (e = hipEventRecord(ctx->prof_start[ctx->prof_used], st)) != hipSuccess)
      return hip_fail(ctx, e, "hipEventRecord");
    if ((e = launch_lm_tiles(kLmFwd, ta, st)) != hipSuccess) return hip_fail(ctx, e, "LM-head forward tiles");
    ta.wt = nullptr;   // the backward's recompute tiles reuse ta
    if (timed && (e = hipEventRecord(ctx->prof_stop[ctx->prof_used++], st)) != hipSuccess)
      return hip_fail(ctx, e, "hipEventRecord");
  }
  for (int m = 0; m < (ref ? 2 : 1); ++m) {
    const LmReduceArgs rd{m == 0 ? part : reinterpret_cast<float2*>(sp + o_part2), N, cnt, npart, npart,
                          F(m == 0 ? o_l2 : o_rl2)};
    if ((e = launch_lm_reduce(rd, st)) != hipSuccess) return hip_fail(ctx, e, "LM-head reduce");
  }

  // GRPO terms and the loss.
  RowArgs ra;
  std::memset(&ra, 0, sizeof(ra));
  ra.ids = a->ids;
  ra.mask = a->mask;
  ra.old_logp = a->old_logp;
  ra.adv = adv;
  ra.seq_scale = F(o_scale);
  ra.logp = a->logp;
  ra.ref_logp = a->ref_logp;
  ra.token_loss = tl;
  ra.err = ctx->d_err;
  ra.vocab = V;
  ra.rows = T;
  ra.logit_stride = T;
  ra.tok_stride = T;
  ra.tok_offset = 0;
  ra.ids_i64 = a->ids_dtype == PCP_I64;
  ra.mask_u8 = mask_u8;
  ra.loss_mode = a->loss_mode;
  ra.clip_eps = a->clip_eps;
  ra.kl_beta = a->kl_beta;
  LmTermsArgs tma{N, I(o_cidx), F(o_tgt), F(o_l2), ref ? F(o_rtgt) : nullptr, ref ? F(o_rl2) : nullptr, F(o_coef)};
  if ((e = launch_lm_terms(ra, tma, st)) != hipSuccess) return hip_fail(ctx, e, "LM-head terms");
  {
    const LossReduceArgs la{tl, T, T, 0, F(o_len), adv, a->loss_mode == PCP_LOSS_REINFORCE, F(o_val), S, loss_norm,
                            I(o_done), a->loss ? a->loss : F(o_loss)};
    if ((e = launch_loss_reduce_fused(la, st)) != hipSuccess) return hip_fail(ctx, e, "loss reduction");
  }

  // Backward over the live tokens. With none, the products have no tiles (dhidden) or
  // an empty K (dW: zero), and dead rows are written as zero, so every gradient is 0.
  if (bwd) {
    char* dbuf = static_cast<char*>(ctx->lm_dbuf);
    float* dhc = want_dy ? F(o_dhc) : nullptr;
    // hidden^T [H, ldt], zero past the live tokens: an operand of dW (fragment-major
    // when it is the products' token operand on the cached path).
    const LmTransposeArgs tr{reinterpret_cast<const uint16_t*>(sp + o_hid), H, static_cast<int>(N),
                             static_cast<int>(H), reinterpret_cast<uint16_t*>(sp + o_ht), ldt, cnt};
    // Chunked backward: the products of one vocab range [vc0, vc0 + w) of D
    // (token-major rows of ldd columns at dbuf), in one launch (they are independent):
    // the longer one (dhidden, K = the range, over fewer tiles) first, so the shorter
    // dW tiles fill the CUs its last round leaves idle. D is read K-major for dW and W
    // K-major for dhidden, with LDS transpose loads, so no chunk is transposed.
    auto products = [&](int64_t vc0, int64_t w, int64_t ldd) -> hipError_t {
      LmTileArgs::Gemm g[2];
      int ng = 0;
      std::memset(g, 0, sizeof(g));
      if (want_dy) {
        // dhidden_c[t][h] (+)= sum_v D[t][v] * W[vc0 + v][h]: rows = live tokens, columns
        // = H; W rows past the range read as 0 (as D's columns there are 0).
        LmTileArgs::Gemm& d = g[ng++];
        d.B = dbuf;
        d.ldb = static_cast<int>(ldd);
        d.V = static_cast<int>(N);
        d.vcount = cnt;
        d.A = static_cast<const uint16_t*>(a->weight) + vc0 * H;
        d.lda = static_cast<int>(H);
        d.krows_a = static_cast<int>(w);
        d.N = static_cast<int>(H);
        d.K = static_cast<int>((w + 63) / 64 * 64);
        d.nvt = ntl;
        d.ntt = static_cast<int>((H + kLmTileT - 1) / kLmTileT);
        d.C = dhc;
        d.ldc = static_cast<int>(H);
        d.accumulate = vc0 > 0;
      }
      if (a->dweight) {
        // dW[vc0 + v][h] = sum_t hidden^T[h][t] * D[t][v]: result rows = H, columns = the
        // range's vocab, stored transposed; D rows past the live tokens read as 0.
        LmTileArgs::Gemm& d = g[ng++];
        d.B = sp + o_ht;
        d.ldb = static_cast<int>(ldt);
        d.V = static_cast<int>(H);
        d.A = dbuf;
        d.lda = static_cast<int>(ldd);
        d.krows_a = static_cast<int>(N);
        d.kcount = cnt;
        d.N = static_cast<int>(w);
        d.K = static_cast<int>(ldt);
        d.nvt = static_cast<int>((H + kLmTileV - 1) / kLmTileV);
        d.ntt = static_cast<int>((w + kLmTileT - 1) / kLmTileT);
        d.C = a->dweight + vc0 * H;
        d.ldc = static_cast<int>(H);
        d.transpose_c = 1;
        d.accumulate = 0;
      }
      return launch_lm_gemms(g, ng, true, st);
    };
    if (cached) {
      // D and D^T over the whole vocabulary from the cache, W^T, then both products in
      // one launch on K-contiguous operands (K = the vocabulary for dhidden, the live
      // tokens for dW; dhidden's 608 long tiles at configuration 5 go first). The token
      // operands (W^T, hidden^T) are written fragment-major and loaded straight into
      // registers; D and D^T go through LDS.
      uint16_t* dt = a->dweight ? reinterpret_cast<uint16_t*>(dbuf + o_dt) : nullptr;
      uint16_t* wt = want_dy ? reinterpret_cast<uint16_t*>(dbuf + o_wt) : nullptr;
      uint16_t* dd = reinterpret_cast<uint16_t*>(dbuf + o_d);
      const LmDcacheArgs dc{dd, exact ? reinterpret_cast<const float*>(dbuf) : nullptr, ldv, cnt, dt, ldt, V,
                            part, npart, F(o_l2), F(o_coef), F(o_tgt), I(o_idsc)};
      if ((e = launch_lm_dcache(dc, st)) != hipSuccess) return hip_fail(ctx, e, "dlogits from the softmax cache");
      if (a->dweight && (e = launch_lm_transpose_frag(tr, st)) != hipSuccess)
        return hip_fail(ctx, e, "transposing hidden rows");
      LmTileArgs::Gemm g[2];
      int ng = 0;
      std::memset(g, 0, sizeof(g));
      if (want_dy) {
        // W^T [H, ldv] (fragment-major, zero past V), written by the forward.
        if (!wt_fwd) {
          const LmTransposeArgs tw{static_cast<const uint16_t*>(a->weight), H, static_cast<int>(V),
                                   static_cast<int>(H), wt, ldv, nullptr};
          if ((e = launch_lm_transpose_frag(tw, st)) != hipSuccess) return hip_fail(ctx, e, "transposing the LM head");
        }
        // dhidden_c[t][h] = sum_v D[t][v] * W^T[h][v].
        LmTileArgs::Gemm& d = g[ng++];
        d.B = dd;
        d.b_tiled = 1;
        d.ldb = static_cast<int>(ldv);
        d.V = static_cast<int>(N);
        d.vcount = cnt;
        d.A = wt;
        d.a_frag = 1;
        d.lda = static_cast<int>(ldv);
        d.N = static_cast<int>(H);
        d.K = static_cast<int>(ldv);
        d.nvt = ntl;
        d.ntt = static_cast<int>((H + kLmTileT - 1) / kLmTileT);
        d.C = dhc;
        d.ldc = static_cast<int>(H);
      }
      if (a->dweight) {
        // dW[v][h] = sum_t D^T[v][t] * hidden^T[h][t].
        LmTileArgs::Gemm& d = g[ng++];
        d.B = dt;
        d.b_tiled = 1;
        d.ldb = static_cast<int>(ldt);
        d.V = static_cast<int>(V);
        d.A = sp + o_ht;
        d.a_frag = 1;
        d.lda = static_cast<int>(ldt);
        d.N = static_cast<int>(H);
        d.K = static_cast<int>(ldt);
        d.kcount = cnt;
        d.nvt = static_cast<int>((V + kLmTileV - 1) / kLmTileV);
        d.ntt = static_cast<int>((H + kLmTileT - 1) / kLmTileT);
        d.C = a->dweight;
        d.ldc = static_cast<int>(H);
      }
      const bool timed = ctx->prof_on && ctx->prof_used < static_cast<int>(ctx->prof_start.size());
      if (timed && (e = hipEventRecord(ctx->prof_start[ctx->prof_used], st)) != hipSuccess)
        return hip_fail(ctx, e, "hipEventRecord");
      if ((e = launch_lm_gemms(g, ng, false, st)) != hipSuccess)
        return hip_fail(ctx, e, "dhidden / dweight products");
      if (timed && (e = hipEventRecord(ctx->prof_stop[ctx->prof_used++], st)) != hipSuccess)
        return hip_fail(ctx, e, "hipEventRecord");
    } else {
      if (a->dweight && (e = chunk_frag ? launch_lm_transpose_frag(tr, st) : launch_lm_transpose(tr, st)) != hipSuccess)
        return hip_fail(ctx, e, "transposing hidden rows");
      uint16_t* cdt = chunk_frag && a->dweight ? reinterpret_cast<uint16_t*>(dbuf + o_cdt) : nullptr;
      uint16_t* cwt = chunk_frag && want_dy ? reinterpret_cast<uint16_t*>(dbuf + o_cwt) : nullptr;
      if (cwt && !wt_fwd) {   // otherwise written by the forward
        const LmTransposeArgs tw{static_cast<const uint16_t*>(a->weight), H, static_cast<int>(V), static_cast<int>(H),
                                 cwt, ldv, nullptr};
        if ((e = launch_lm_transpose_frag(tw, st)) != hipSuccess) return hip_fail(ctx, e, "transposing the LM head");
      }
      // The cached path's products over one chunk [vc0, vc0 + w): D_c token-major (rows of
      // chunk entries) with W^T's fragments of that range, and D_c^T with hidden^T.
      auto products_frag = [&](int64_t vc0, int64_t w) -> hipError_t {
        LmTileArgs::Gemm g[2];
        int ng = 0;
        std::memset(g, 0, sizeof(g));
        if (want_dy) {
          LmTileArgs::Gemm& d = g[ng++];
          d.B = dbuf;
          d.ldb = static_cast<int>(chunk);
          d.V = static_cast<int>(N);
          d.vcount = cnt;
          d.A = cwt + 16 * vc0;   // fragment column vc0 / 32 (1 KB = 512 elements each)
          d.a_frag = 1;
          d.lda = static_cast<int>(ldv);
          d.N = static_cast<int>(H);
          d.K = static_cast<int>((w + 63) / 64 * 64);
          d.nvt = ntl;
          d.ntt = static_cast<int>((H + kLmTileT - 1) / kLmTileT);
          d.C = dhc;
          d.ldc = static_cast<int>(H);
          d.accumulate = vc0 > 0;
        }
        if (a->dweight) {
          LmTileArgs::Gemm& d = g[ng++];
          d.B = cdt;
          d.ldb = static_cast<int>(ldt);
          d.V = static_cast<int>(w);
          d.A = sp + o_ht;
          d.a_frag = 1;
          d.lda = static_cast<int>(ldt);
          d.N = static_cast<int>(H);
          d.K = static_cast<int>(ldt);
          d.kcount = cnt;
          d.nvt = static_cast<int>((w + kLmTileV - 1) / kLmTileV);
          d.ntt = static_cast<int>((H + kLmTileT - 1) / kLmTileT);
          d.C = a->dweight + vc0 * H;
          d.ldc = static_cast<int>(H);
        }
        return launch_lm_gemms(g, ng, false, st);
      };
      ta.B = a->weight;
      ta.lse2 = F(o_l2);
      ta.coef = F(o_coef);
      ta.dchunk = dbuf;
      ta.ldd = static_cast<int>(chunk);
      ta.ecache = nullptr;
      for (int64_t vc0 = 0; vc0 < V; vc0 += chunk) {
        const int64_t w = (V - vc0 < chunk) ? V - vc0 : chunk;
        ta.vc0 = static_cast<int>(vc0);
        ta.vt0 = static_cast<int>(vc0 / kLmTileV);
        ta.nvt = static_cast<int>((w + kLmTileV - 1) / kLmTileV);
        if ((e = launch_lm_tiles(kLmBwd, ta, st)) != hipSuccess) return hip_fail(ctx, e, "LM-head backward tiles");
        if (cdt) {
          // D_c^T [w, ldt], zero past the live tokens.
          const LmTransposeArgs td{reinterpret_cast<const uint16_t*>(dbuf), chunk, static_cast<int>(N),
                                   static_cast<int>(w), cdt, ldt, cnt};
          if ((e = launch_lm_transpose(td, st)) != hipSuccess) return hip_fail(ctx, e, "transposing dlogits");
        }
        if ((e = chunk_frag ? products_frag(vc0, w) : products(vc0, w, chunk)) != hipSuccess)
          return hip_fail(ctx, e, "dhidden / dweight products");
      }
    }
    if (norm && want_dy) {
      const LmNormBwdArgs nb{dhc, static_cast<const uint16_t*>(a->hidden_states), a->norm_weight, F(o_rstd),
                             I(o_cidx), I(o_live), N, static_cast<int>(H), cnt, a->dhidden,
                             a->dnorm_weight ? F(o_gpart) : nullptr, a->dnorm_weight};
      if ((e = launch_lm_norm_bwd(nb, st)) != hipSuccess) return hip_fail(ctx, e, "final norm backward");
    } else if (!norm && a->dhidden && (e = launch_lm_scatter_rows(dhc, a->dhidden, I(o_cidx), static_cast<int>(N),
                                                         static_cast<int>(H), st)) != hipSuccess) {
      return hip_fail(ctx, e, "scattering dhidden rows");
    }
  }

  if (a->flags & PCP_FLAG_ASYNC) {
    return add_pending(ctx, st);
  }
  if ((e = hipStreamSynchronize(st)) != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  return collect_device_errors(ctx);
}

}  // namespace

}  // namespace pcp

using namespace pcp;

extern "C" {

int pcp_synth_lmhead_tokens(pcp_ctx* ctx, const void* hidden, const void* weight, int64_t n, int64_t hidden_dim,
                            int64_t vocab, int64_t chunk, uint64_t seed, int64_t* ids, void* stream) {
  using namespace pcp;
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  if (!hidden || !weight || !ids || n < 0 || n > (int64_t{1} << 28) || vocab < 1 || vocab > (1 << 30) ||
      hidden_dim < 64 || hidden_dim % 64 != 0 || hidden_dim > (1 << 20) || chunk < 0 ||
      ((reinterpret_cast<uintptr_t>(hidden) | reinterpret_cast<uintptr_t>(weight)) & 15u))
    return fail(ctx, PCP_ERR_INVALID_ARG, "pcp_synth_lmhead_tokens: bad arguments");
  if (n == 0) return PCP_OK;
  const int64_t rows = chunk > 0 ? (chunk < n ? chunk : n) : (n < 1024 ? n : 1024);
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  int rc = ensure_scratch(ctx, 4 * static_cast<size_t>(rows) * vocab);
  if (rc != PCP_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* logits = static_cast<float*>(ctx->scratch);
  for (int64_t n0 = 0, k = 0; n0 < n; n0 += rows, ++k) {
    const int64_t m = n - n0 < rows ? n - n0 : rows;
    // logits[t][v] = sum_h hidden[n0 + t][h] * weight[v][h]: token rows in the product's
    // row role, vocabulary in its column role, both operands K-contiguous.
    LmTileArgs::Gemm g;
    std::memset(&g, 0, sizeof(g));
    g.B = static_cast<const uint16_t*>(hidden) + n0 * hidden_dim;
    g.ldb = static_cast<int>(hidden_dim);
    g.V = static_cast<int>(m);
    g.A = weight;
    g.lda = static_cast<int>(hidden_dim);
    g.N = static_cast<int>(vocab);
    g.K = static_cast<int>(hidden_dim);
    g.nvt = static_cast<int>((m + kLmTileV - 1) / kLmTileV);
    g.ntt = static_cast<int>((vocab + kLmTileT - 1) / kLmTileT);
    g.C = logits;
    g.ldc = static_cast<int>(vocab);
    if ((e = launch_lm_gemms(&g, 1, false, st)) != hipSuccess) return hip_fail(ctx, e, "logits tiles");
    rc = pcp_synth_sample_tokens(logits, PCP_F32, m, vocab, seed + static_cast<uint64_t>(k), ids + n0, stream);
    if (rc != PCP_OK) return rc;
  }
  return PCP_OK;
}


void pcp_lmhead_args_init(pcp_lmhead_args* a) {
  if (!a) return;
  std::memset(a, 0, sizeof(*a));
  a->group_size = 1;
  a->ids_dtype = PCP_I64;
  a->mask_dtype = PCP_F32;
  a->loss_mode = PCP_LOSS_REINFORCE;
  a->clip_eps = 0.2f;
  a->kl_beta = 0.04f;
  a->std_eps = 1e-8f;
  a->norm_eps = 1e-6f;
}

int pcp_grpo_lmhead_fwd_bwd(pcp_ctx* ctx, const pcp_lmhead_args* a) { return run_lm(ctx, a); }

}  // extern "C"
