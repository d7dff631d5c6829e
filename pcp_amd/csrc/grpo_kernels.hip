// GRPO loss-head kernels for MI355X (gfx950).
//
// One workgroup owns one logits row at a time. The hot kernel (grpo_resident_kernel)
// is persistent: one workgroup per CU takes rows from a counter. It keeps the policy
// row in VGPRs as packed 16-bit words (V=151936 bf16 = 19 x 16 B per lane at 1024
// lanes), so a live row costs exactly one read of the policy row, one read of the
// reference row and one write of dlogits:
//   1. issue every 16-byte load of the policy row (coalesced, 1 KiB per wave per
//      chunk), then stream the reference row in batches;
//   2. per-lane max and sum of 2^(x*log2e - m) over the resident values, online
//      (max, sum) over the reference batches;
//   3. one workgroup merge of both (m, s) pairs: xor-butterfly in the wave, then a
//      fixed-order combine of the 16 wave results through LDS;
//   4. token math (logp, ref logp, ratio, clip, k3-KL, coefficient c);
//   5. dlogits = c * (onehot - softmax) straight from the registers, packed to
//      bf16 with v_cvt_pk_bf16_f32, stored 16 B per lane. For bf16 -> bf16 the
//      softmax terms come from the sum pass, cached as f16 in place of the row.
// Rows whose token is masked, ignored or a pad row only zero-fill dlogits.
// Forward-only calls (no dlogits) take grpo_fwd_kernel instead: one online pass per
// row at 256 lanes, several workgroups per CU.
//
// Reference semantics: tools/export_qwen_forward.py:150-163 (loss),
// models/tests/qwen_test.mlir:257-286 (cross-entropy lowering),
// src/nodes/controllers/rl_shepherd.zig:462-479 (advantages).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "grpo_device.hpp"
#include "grpo_launch.hpp"

#ifndef PCP_RES_PREFETCH
#define PCP_RES_PREFETCH 1
#endif

namespace pcp {

// ---------------------------------------------------------------------------
// Row helpers
// ---------------------------------------------------------------------------
template <typename TO, int EPV, int BLOCK>
__device__ __forceinline__ void zero_row_vec(void* dl, int64_t row_elem, int nv) {
  float z[EPV];
#pragma unroll
  for (int j = 0; j < EPV; ++j) z[j] = 0.f;
  for (int vi = threadIdx.x; vi < nv; vi += BLOCK)
    store_vals<TO, EPV, true>(dl, row_elem + static_cast<int64_t>(vi) * EPV, z);
}

template <typename TO, int BLOCK>
__device__ __forceinline__ void zero_row_scalar(void* dl, int64_t row_elem, int64_t v) {
  for (int64_t i = threadIdx.x; i < v; i += BLOCK) store1<TO>(dl, row_elem + i, 0.f);
}

__device__ __forceinline__ void flag_nonfinite(const RowArgs& a, float lse, float lr_lse) {
  if (threadIdx.x == 0 && !(__builtin_isfinite(lse) && __builtin_isfinite(lr_lse)))
    atomicOr(a.err, kErrNonFinite);
}

// A row that may start off 16 bytes: its 16-byte-aligned interior of nv vectors, and
// the head (before it) and tail (after it) of fewer than EPV elements each.
struct RowSpan {
  const void* vec;
  int head, nv, tail;
};

template <typename TI>
__device__ __forceinline__ RowSpan row_span(const void* p, int64_t vocab) {
  constexpr int EPV = 16 / TI::kBytes;
  RowSpan s;
  const int mis = static_cast<int>(reinterpret_cast<uintptr_t>(p) & 15u);
  s.head = static_cast<int>(min<int64_t>(((16 - mis) & 15) / TI::kBytes, vocab));
  s.nv = static_cast<int>((vocab - s.head) / EPV);
  s.tail = static_cast<int>(vocab - s.head - static_cast<int64_t>(s.nv) * EPV);
  s.vec = static_cast<const char*>(p) + s.head * TI::kBytes;
  return s;
}

// The head or tail element that thread tid handles: threads [0, head) take the head,
// [head, head + tail) the tail; -1 for the rest.
template <typename TI>
__device__ __forceinline__ int edge_index(const RowSpan& sp, int tid) {
  constexpr int EPV = 16 / TI::kBytes;
  return tid < sp.head ? tid : (tid - sp.head < sp.tail ? sp.head + sp.nv * EPV + (tid - sp.head) : -1);
}

// Thread tid's head or tail element of the row as a one-element online state (m, s).
template <typename TI>
__device__ __forceinline__ void edge_state(const void* p, const RowSpan& sp, int tid, float& m, float& s) {
  const int k = edge_index<TI>(sp, tid);
  m = kNegInf;
  s = 0.f;
  if (k < 0) return;
  const float x = TI::load1(p, k) * kLog2e;
  m = fmaxf(m, x);
  s = hw_exp2(x - ms_ref(m));
}

// ---------------------------------------------------------------------------
// Register-resident fused forward+backward.
//   TI/TO: input / output codecs; BLOCK lanes; NCH 16-byte chunks per lane
//   (row capacity BLOCK*NCH*16 bytes); RB reference chunks per batch; CACHE: bf16 ->
//   bf16 rows keep the sum pass's softmax terms as f16 for the dlogits pass (false:
//   that pass recomputes them, so each output is the f32 result rounded once).
// Requirements (checked on the host): V <= BLOCK*NCH*EPV; without EDGE, V % EPV == 0
// and 16-byte aligned rows. EDGE: rows may start off 16 bytes, and dlogits rows have
// the logits rows' element type and offset mod 16: the aligned interior is held and
// stored as vectors, the head and tail (under EPV elements each) by threads 0..13 one
// element each. dlogits == nullptr: forward only (log-probs).
// ---------------------------------------------------------------------------
// Chunk k of a row through its descriptor: 16 bytes at lane offset voff, or for kSplit
// (16-bit logits, f32 dlogits) the two 8-byte halves of 4-element group sgrp, 512 bytes
// apart (see resident_row).
template <typename TI, typename TO, int BLOCK>
__device__ __forceinline__ u32x4 load_chunk(const __amdgpu_buffer_rsrc_t buf, int k, uint32_t voff, uint32_t sgrp) {
  constexpr uint32_t kChunkBytes = BLOCK * 16;
  if constexpr (TI::kBytes == 2 && TO::kBytes == 4) {
    const u32x2 lo = buf_ld8<true>(buf, fresh_off(sgrp * 8u, k * kChunkBytes));
    const u32x2 hi = buf_ld8<true>(buf, fresh_off(sgrp * 8u, k * kChunkBytes + 512u));
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  } else {
    return buf_ld16<true>(buf, fresh_off(voff, k * kChunkBytes));
  }
}

template <typename TI, typename TO, int BLOCK>
__device__ __forceinline__ uint32_t split_group(int tid) {
  return (TI::kBytes == 2 && TO::kBytes == 4) ? static_cast<uint32_t>(128 * (tid >> 6) + (tid & 63)) : 0u;
}

// The policy row's descriptor for rows without EDGE handling (aligned, V % EPV == 0);
// row < 0 gives an empty descriptor, whose loads return 0 without a memory access.
template <typename TI>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t policy_rsrc(const RowArgs& a, int64_t row) {
  constexpr int EPV = 16 / TI::kBytes;
  const bool ok = row >= 0;
  const char* base = static_cast<const char*>(a.logits) + (ok ? row * a.vocab * TI::kBytes : 0);
  return row_rsrc(base, ok ? static_cast<uint32_t>(a.vocab / EPV) * 16u : 0u);
}

// PF (listed live rows without EDGE handling): the policy row arrives in xv already
// loaded (by the caller for the first row, by the previous row's dlogits pass after
// that). Thread 0 passes the list entry of the row after this one (next_listed, valid
// when next_ok), which reaches every thread through s_pub under the merge's barrier
// (the select sits there too, so no wave waits for the entry's load before then); the
// dlogits pass then loads that row's chunks into xv as it frees them, so the next
// row's policy loads are in flight under this row's stores. Returns the next row (PF,
// -1 for none) or -1.
template <typename TI, typename TO, int BLOCK, int NCH, int RB, bool EDGE, bool CACHE, bool PF = false,
          int SP = kBufNT>
__device__ __forceinline__ int64_t resident_row(const RowArgs& a, const int64_t row, float* lds, u32x4 (&xv)[NCH],
                                                int next_listed = -1, bool next_ok = false, int* s_pub = nullptr) {
  static_assert(!(PF && EDGE), "prefetching rows are aligned rows");
  constexpr int EPV = 16 / TI::kBytes;
  constexpr uint32_t kChunkBytes = BLOCK * 16;          // one chunk: 16 bytes per lane
  constexpr uint32_t kOutVec = EPV * TO::kBytes;        // output bytes per input vector
  // bf16 logits -> bf16 dlogits: the sum pass's softmax terms are cached (f16) and
  // scaled into dlogits, one exponential per element fewer. Other pairs recompute.
  constexpr bool kBf16Pair = __is_same(TI, BF16T) && __is_same(TO, BF16T);
  constexpr bool kCache = kBf16Pair && CACHE;
  // 16-bit logits with f32 dlogits: a lane's chunk is two 8-byte halves 512 bytes apart
  // in its wave's 1 KB of the chunk (elements 4 l + 0..3 and 256 + 4 l + 0..3 of the
  // wave's 512), so each half's f32 output is one 16-byte store and each store
  // instruction writes 1 KB contiguously (16-byte halves of 32-byte outputs, stride 32,
  // leave every instruction writing half lines). Rows of this pair are never EDGE rows.
  constexpr bool kSplit = TI::kBytes == 2 && TO::kBytes == 4;
  static_assert(!(kSplit && EDGE), "16-bit -> f32 rows are not EDGE rows");

  constexpr int kPrefetch = PCP_RES_PREFETCH;   // reference batches in flight ahead of the math
  const int tid = threadIdx.x;
  // kSplit: half h of chunk k of this lane is 4-element group
  //   k * 2 * BLOCK + 128 * wave + 64 * h + lane,
  // valid when below 2 * nv; its input at 8 bytes, its output at 16 bytes per group.
  const uint32_t sgrp = split_group<TI, TO, BLOCK>(tid);
  const RowMeta r = row_meta(a, row);
  const int64_t row_elem = row * a.vocab;
  const void* xrow = static_cast<const char*>(a.logits) + row_elem * TI::kBytes;
  const RowSpan xsp = EDGE ? row_span<TI>(xrow, a.vocab) : RowSpan{xrow, 0, static_cast<int>(a.vocab / EPV), 0};
  const int nv = xsp.nv;
  const int ek = EDGE ? edge_index<TI>(xsp, tid) : -1;   // this thread's head / tail element
  const uint32_t in_bytes = static_cast<uint32_t>(nv) * 16u;
  const uint32_t out_bytes = static_cast<uint32_t>(nv) * kOutVec;
  const __amdgpu_buffer_rsrc_t drow =
      row_rsrc(static_cast<char*>(a.dlogits) + (row_elem + xsp.head) * TO::kBytes, out_bytes);

  const uint32_t voff = tid * 16u;

  if (!r.live) {
    write_token_outputs(a, r, 0.f, 0.f, 0.f);
    if (a.dlogits && a.zero_fill) {
      const u32x4 z = {0u, 0u, 0u, 0u};   // 0 bits are 0 in every output type
      if constexpr (kSplit) {
#pragma unroll
        for (int k = 0; k < NCH; ++k)
#pragma unroll
          for (int h = 0; h < 2; ++h) buf_st16<true, SP>(drow, z, (k * 2 * BLOCK + 64 * h + sgrp) * 16u);
      } else {
#pragma unroll
        for (int k = 0; k < NCH; ++k)
#pragma unroll
          for (uint32_t q = 0; q < kOutVec; q += 16) buf_st16<true, SP>(drow, z, (k * BLOCK + tid) * kOutVec + q);
      }
      if (EDGE && ek >= 0) store1<TO>(a.dlogits, row_elem + ek, 0.f);
    }
    if constexpr (PF) {
      // live_rows_kernel listed this row as live from the same ids and mask, so the
      // inputs changed under the launch. Fail loudly (PCP_ERR_INVALID_ARG); this
      // workgroup's claimed rows stay unprocessed. (Loading the next row here as well
      // as in the live path's dlogits pass made hipcc spill 75-110 VGPRs.)
      if (tid == 0) atomicOr(a.err, kErrListedRow);
    }
    return -1;
  }

  const bool has_ref = a.ref_logits != nullptr;
  const void* rrow =
      has_ref ? static_cast<const char*>(a.ref_logits) + row_elem * TI::kBytes : nullptr;

  // Target logits: one broadcast load each, completing under the row stream.
  const float xy = TI::load1(xrow, r.id);
  const float ry = has_ref ? TI::load1(rrow, r.id) : 0.f;

  // 1. Policy row -> registers: all NCH loads back to back through one row
  //    descriptor (lanes past the row end read 0 and are skipped below).
  const __amdgpu_buffer_rsrc_t xbuf = row_rsrc(xsp.vec, in_bytes);
  if constexpr (!PF) {
#pragma unroll
    for (int k = 0; k < NCH; ++k) xv[k] = load_chunk<TI, TO, BLOCK>(xbuf, k, voff, sgrp);
  }
  // kSplit: half h of chunk k of this lane holds row values (past the row end it read 0).
  auto half_ok = [&](int k, int h) {
    return static_cast<int64_t>(k) * 2 * BLOCK + 64 * h + sgrp < 2 * static_cast<int64_t>(nv);
  };
  const float xe = (EDGE && ek >= 0) ? TI::load1(xrow, ek) : kNegInf;

  // 2. Per-lane (max, sum) of the resident policy values and online (max, sum) of
  //    the reference row, streamed in batches of RB chunks PD batches ahead. The
  //    policy sum for chunks [kb, kb + RB) runs in the same step as reference batch
  //    kb, so its exponentials overlap reference loads in flight instead of leaving
  //    the CU's memory idle. For bf16 -> bf16 the policy terms e = 2^(x*log2e - m2)
  //    are also kept, as f16 in place of the row (e <= 1: 2^-11 relative, 2^-25
  //    absolute below the f16 normal range), and dlogits become a multiple of them.
  constexpr int NB = (NCH + RB - 1) / RB;
  constexpr int PD = kPrefetch;
  // The reference row's own split (its offset may differ from the policy row's).
  const RowSpan rsp = (EDGE && has_ref) ? row_span<TI>(rrow, a.vocab) : RowSpan{rrow, 0, nv, 0};
  const int nvr = rsp.nv;
  const __amdgpu_buffer_rsrc_t rbuf = has_ref ? row_rsrc(rsp.vec, static_cast<uint32_t>(nvr) * 16u) : xbuf;
  u32x4 rv[PD + 1][RB];
  if (has_ref) {
#pragma unroll
    for (int b = 0; b < PD; ++b)
#pragma unroll
      for (int q = 0; q < RB; ++q)
        if (b < NB && b * RB + q < NCH) rv[b][q] = buf_ld16<true>(rbuf, fresh_off(voff, (b * RB + q) * kChunkBytes));
  }
  float pm;
  {
    float mx = kNegInf;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      if constexpr (kSplit) {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(&xv[k]);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (!half_ok(k, h)) continue;
          if constexpr (__is_same(TI, BF16T)) {
            // bf16 halves by byte permutes, as for the bf16 pair below.
#pragma unroll
            for (int q = 2 * h; q < 2 * h + 2; ++q)
              mx = fmaxf(fmaxf(mx, __uint_as_float(__builtin_amdgcn_perm(w[q], 0u, 0x05040c0cu))),
                         __uint_as_float(__builtin_amdgcn_perm(w[q], 0u, 0x07060c0cu)));
          } else {
#pragma unroll
            for (int j = 4 * h; j < 4 * h + 4; ++j) mx = fmaxf(mx, TI::unpack(w, j));
          }
        }
      } else if (k * BLOCK + tid < nv) {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(&xv[k]);
        if constexpr (kBf16Pair) {
          // bf16 halves by byte permutes: the same values as unpack(), but not
          // merged with the sum pass's unpacks, which would keep 152 f32 values
          // live from here to the sum of the last chunk.
#pragma unroll
          for (int h = 0; h < 4; ++h)
            mx = fmaxf(fmaxf(mx, __uint_as_float(__builtin_amdgcn_perm(w[h], 0u, 0x05040c0cu))),
                       __uint_as_float(__builtin_amdgcn_perm(w[h], 0u, 0x07060c0cu)));
        } else {
#pragma unroll
          for (int j = 0; j < EPV; ++j) mx = fmaxf(mx, TI::unpack(w, j));
        }
      }
    }
    if constexpr (EDGE) mx = fmaxf(mx, xe);
    pm = mx * kLog2e;
  }
  const float m2 = ms_ref(pm);   // this lane's shift (kept for the cached terms)
  float ps = 0.f, rm = kNegInf, rs = 0.f;
  if (EDGE && has_ref) edge_state<TI>(rrow, rsp, tid, rm, rs);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int kb = b * RB;
    if (has_ref) {
#pragma unroll
      for (int q = 0; q < RB; ++q)
        if (b + PD < NB && kb + PD * RB + q < NCH)
          rv[(b + PD) % (PD + 1)][q] = buf_ld16<true>(rbuf, fresh_off(voff, (kb + PD * RB + q) * kChunkBytes));
    }
    // policy sum over chunks [kb, kb + RB)
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      const int k = kb + q;
      if (k >= NCH || (!kSplit && k * BLOCK + tid >= nv)) continue;
      uint32_t* w = reinterpret_cast<uint32_t*>(&xv[k]);
      if constexpr (kCache) {
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const float e0 = hw_exp2(fmaf(TI::unpack(w, 2 * h), kLog2e, -m2));
          const float e1 = hw_exp2(fmaf(TI::unpack(w, 2 * h + 1), kLog2e, -m2));
          ps += e0;
          ps += e1;
          w[h] = pack2<F16T>(e0, e1);
          // Pin the pack here: left to itself the compiler sinks the packs into the
          // dlogits loop and keeps 152 f32 terms live across the merge.
          asm volatile("" ::"v"(w[h]));
        }
      } else if constexpr (kSplit) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (!half_ok(k, h)) continue;
#pragma unroll
          for (int j = 4 * h; j < 4 * h + 4; ++j) ps += hw_exp2(fmaf(TI::unpack(w, j), kLog2e, -m2));
        }
      } else {
#pragma unroll
        for (int j = 0; j < EPV; ++j) ps += hw_exp2(fmaf(TI::unpack(w, j), kLog2e, -m2));
      }
    }
    // reference batch b
    if (has_ref) {
      u32x4* cur = rv[b % (PD + 1)];
      float bm = kNegInf;
#pragma unroll
      for (int q = 0; q < RB; ++q) {
        if (kb + q < NCH && (kb + q) * BLOCK + tid < nvr) {
          const uint32_t* w = reinterpret_cast<const uint32_t*>(&cur[q]);
#pragma unroll
          for (int j = 0; j < EPV; ++j) bm = fmaxf(bm, TI::unpack(w, j));
        }
      }
      const float nm = fmaxf(rm, bm * kLog2e);
      const float ref = ms_ref(nm);
      float acc = ms_rescale(rs, rm, nm);
#pragma unroll
      for (int q = 0; q < RB; ++q) {
        if (kb + q < NCH && (kb + q) * BLOCK + tid < nvr) {
          const uint32_t* w = reinterpret_cast<const uint32_t*>(&cur[q]);
#pragma unroll
          for (int j = 0; j < EPV; ++j) acc += hw_exp2(fmaf(TI::unpack(w, j), kLog2e, -ref));
        }
      }
      rm = nm;
      rs = acc;
    }
  }

  if constexpr (EDGE) ps += hw_exp2(fmaf(xe, kLog2e, -m2));   // 0 for threads without one

  // 3. Workgroup merge.
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (PF) {
    if (tid == 0) s_pub[0] = next_ok ? next_listed : -1;
  }
  block_merge2<BLOCK>(pm, ps, rm, rs, lds);
  const float lse2 = pm + log2f(ps);
  const float lse = lse2 * kLn2;
  const float rlse = has_ref ? ms_lse(rm, rs) : 0.f;
  flag_nonfinite(a, lse, rlse);

  // 4. Token math.
  const float lp = xy - lse;
  const float lr = ry - rlse;
  const TokenTerms tt = token_terms(a, r, lp, lr);
  write_token_outputs(a, r, lp, lr, tt.loss);
  if constexpr (!PF) {   // PF launches always write dlogits
    if (a.dlogits == nullptr) return -1;   // forward only (log-probs)
  }
  const int64_t nxt = PF ? s_pub[0] : -1;   // PF: the next row
  const __amdgpu_buffer_rsrc_t nbuf = policy_rsrc<TI>(a, nxt);

  // 5. dlogits = c * (onehot - softmax) from the resident row; stores past the
  //    row end are dropped by the buffer range check. The target element,
  //    c * (1 - p_y) from the target logit itself, is then rewritten by the lane
  //    that stored it (one store; a lane's stores to one address land in order).
  const float c = tt.coef, nc = -tt.coef;
  const float f = nc * hw_exp2(m2 - lse2);   // softmax = e * 2^(m2 - lse2)
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(&xv[k]);
    float o[EPV];
    if constexpr (kCache) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f16x2 h = __builtin_bit_cast(f16x2, w[q]);
        o[2 * q] = f * static_cast<float>(h[0]);
        o[2 * q + 1] = f * static_cast<float>(h[1]);
      }
    } else if constexpr (kBf16Pair || kSplit) {
      // The words pass through an opaque copy: otherwise the compiler reuses the sum
      // pass's unpacked values here and keeps all of them live across the merge.
      uint32_t u[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        u[q] = w[q];
        asm volatile("" : "+v"(u[q]));
      }
#pragma unroll
      for (int j = 0; j < EPV; ++j) o[j] = nc * hw_exp2(fmaf(TI::unpack(u, j), kLog2e, -lse2));
    } else {
#pragma unroll
      for (int j = 0; j < EPV; ++j) o[j] = nc * hw_exp2(fmaf(TI::unpack(w, j), kLog2e, -lse2));
    }
    if constexpr (kSplit) {
      // Groups past the row end sit past the descriptor: their stores are dropped.
      const float (&o0)[4] = reinterpret_cast<const float (&)[4]>(o[0]);
      const float (&o1)[4] = reinterpret_cast<const float (&)[4]>(o[4]);
      buf_store_vals<TO, 4, true, SP>(drow, fresh_off(sgrp * 16u, k * 2 * BLOCK * 16u), o0);
      buf_store_vals<TO, 4, true, SP>(drow, fresh_off(sgrp * 16u, k * 2 * BLOCK * 16u + 1024u), o1);
    } else {
      buf_store_vals<TO, EPV, true, SP>(drow, fresh_off(tid * kOutVec, k * BLOCK * kOutVec), o);
    }
    if constexpr (PF) xv[k] = load_chunk<TI, TO, BLOCK>(nbuf, k, voff, sgrp);
  }
  const int64_t it = r.id - xsp.head;   // the target's index in the interior
  // The lane that stored the target's group (kSplit: group it / 4 at lane
  // 64 (r / 128) + r % 64, r = (it / 4) % (2 BLOCK); else vector it / EPV at lane
  // (it / EPV) % BLOCK).
  const int t_lane = kSplit ? static_cast<int>(64 * (((it >> 2) % (2 * BLOCK)) >> 7) + ((it >> 2) & 63))
                            : static_cast<int>((it / EPV) % BLOCK);
  if (it >= 0 && it < static_cast<int64_t>(nv) * EPV && tid == t_lane) {
    const float dy = c - c * hw_exp2(fmaf(xy, kLog2e, -lse2));
    buf_store1<TO, true, SP>(drow, static_cast<uint32_t>(it) * TO::kBytes, dy);
  }
  if constexpr (EDGE) {
    if (ek >= 0) {
      const float o = (ek == r.id) ? c - c * hw_exp2(fmaf(xy, kLog2e, -lse2))
                                   : nc * hw_exp2(fmaf(xe, kLog2e, -lse2));
      store1<TO>(a.dlogits, row_elem + ek, o);
    }
  }
  return nxt;
}

// Persistent: a workgroup takes row blockIdx.x, then rows from the launch's counter
// (zeroed before the launch) until none are left, so the CU starts its next row
// without a workgroup launch and the counter's latency hides under the current row.
// Every wave reads the same row index from LDS, so all of them leave the loop
// together. The index is double-buffered: thread 0 writes slot i & 1 at the top of
// step i, while slot (i - 1) & 1 may still be read; the barrier at the end of step i
// orders the reads of slot i & 1 before its next write, in step i + 2.

// LIST: the instance for launches without zero-fill, which visit the live rows listed
// by live_rows_kernel (a separate instance, so the zero-fill loop is compiled as before).
template <typename TI, typename TO, int BLOCK, int NCH, int RB, bool EDGE, bool CACHE, bool LIST>
__global__ void __launch_bounds__(BLOCK) grpo_resident_kernel(RowArgs a) {
  __shared__ float lds[4 * (BLOCK / 64)];
  __shared__ int s_next[2];
  if constexpr (LIST) {
    // Without zero-fill: live_rows_kernel listed the live rows and counted them earlier
    // on the stream. When fewer than half the rows are live the launch visits the listed
    // rows only; otherwise every row in order (dead rows return at once), which measured
    // faster there (config 2, 57% live: 3.01-3.04 ms against 3.14-3.16 ms listed with the
    // next-row prefetch below; config 4, 21% live: 2.25-2.28 ms listed without it against
    // 2.62-2.66 ms).
    const int n = *a.row_count;
    if (2 * static_cast<int64_t>(n) < a.nrows) {
      if (!EDGE && a.dlogits != nullptr) {
        // Every listed row is live, so each row's dlogits pass loads the next row's
        // policy chunks (resident_row, PF). List indices: blockIdx.x, then
        // blockIdx.x + gridDim.x, then from the counter (+ 2 gridDim.x). At the top of
        // each row thread 0 reads the list entry of the row after it (claim) and claims
        // the index of the one after that; the entry goes to every thread at the
        // row's merge, and the claimed index is used at the next row's top, so both
        // loads complete under the current row. Rows are claimed dynamically: dealt
        // statically (entries blockIdx.x + i gridDim.x, each row's successor known at
        // its start) the same launch was 1.5-3% slower and varied more from run to run.
        int idx = blockIdx.x;
        if (idx >= n) return;
        int64_t row = a.row_list[idx];
        const uint32_t sgrp = split_group<TI, TO, BLOCK>(threadIdx.x);
        u32x4 xv[NCH];
        {
          const __amdgpu_buffer_rsrc_t buf = policy_rsrc<TI>(a, row);
#pragma unroll
          for (int k = 0; k < NCH; ++k) xv[k] = load_chunk<TI, TO, BLOCK>(buf, k, threadIdx.x * 16u, sgrp);
        }
        int claim = idx + static_cast<int>(gridDim.x);
        for (;;) {
          int listed = -1, taken = 0;
          if (threadIdx.x == 0) {
            taken = atomicAdd(a.next_row, 1);
            listed = a.row_list[min(claim, n - 1)];
          }
          row = resident_row<TI, TO, BLOCK, NCH, RB, false, CACHE, true>(a, row, lds, xv, listed, claim < n, s_next);
          claim = taken + 2 * static_cast<int>(gridDim.x);
          __syncthreads();   // every thread has read s_next before thread 0 writes it again
          if (row < 0) return;
        }
      } else {
        int64_t idx = blockIdx.x;
        for (int i = 0; idx < n; ++i) {
          if (threadIdx.x == 0) s_next[i & 1] = atomicAdd(a.next_row, 1) + static_cast<int>(gridDim.x);
          u32x4 xv[NCH];
          resident_row<TI, TO, BLOCK, NCH, RB, EDGE, CACHE>(a, a.row_list[idx], lds, xv);
          __syncthreads();   // s_next visible; this row's LDS reads done before the next row writes
          idx = s_next[i & 1];
        }
        return;
      }
    }
  }
  {
    // Zero-fill launches store nontemporal at system scope (written through to memory):
    // interleaved on one box, 8 / 4 / 4 runs, config 2 3.579 -> 3.546 ms, config 3
    // 7.007 -> 6.949, config 4 4.718 -> 4.684, exact rounding 3.687 -> 3.631, f32
    // dlogits 5.470 -> 5.387. Launches without zero-fill keep device-scope nontemporal
    // stores, which measured 1-1.6% faster there (config 2 3.009 against 3.059 ms,
    // config 4 2.131 against 2.150).
    constexpr int kSP = LIST ? kBufNT : kBufNTSystem;
    int64_t row = blockIdx.x;
    for (int i = 0; row < a.nrows; ++i) {
      if (threadIdx.x == 0) s_next[i & 1] = atomicAdd(a.next_row, 1) + static_cast<int>(gridDim.x);
      u32x4 xv[NCH];
      resident_row<TI, TO, BLOCK, NCH, RB, EDGE, CACHE, false, kSP>(a, row, lds, xv);
      __syncthreads();   // s_next visible; this row's LDS reads done before the next row writes
      row = s_next[i & 1];
    }
  }
}

__global__ void reset_counter_kernel(int* c, int* c2) {
  *c = 0;
  if (c2) *c2 = 0;
}

// Without zero-fill: one thread per logits row lists the live rows (wave-aggregated
// appends, so the list order is not fixed; every row's result depends on its own data
// only) and writes the per-token outputs of dead token rows (0, as the row kernel's dead
// path does). A live token id outside [0, V) raises the error flag, as in row_meta.
__global__ void __launch_bounds__(256) live_rows_kernel(RowArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  bool live = false;
  if (row < a.nrows) {
    const int64_t s = row / a.logit_stride;
    const int64_t t = row - s * a.logit_stride;
    if (t < a.rows) {
      const int64_t tix = s * a.tok_stride + a.tok_offset + t;
      const int64_t id = a.ids_i64 ? static_cast<const int64_t*>(a.ids)[tix]
                                   : static_cast<int64_t>(static_cast<const int32_t*>(a.ids)[tix]);
      float w = 1.f;
      if (a.mask) w = a.mask_u8 ? (static_cast<const uint8_t*>(a.mask)[tix] ? 1.f : 0.f)
                                : static_cast<const float*>(a.mask)[tix];
      const bool in_range = id >= 0 && id < a.vocab;
      if (w != 0.f && id != PCP_IGNORE_INDEX && !in_range) atomicOr(a.err, kErrTokenRange);
      live = w != 0.f && in_range;
      if (!live) {
        if (a.logp) a.logp[tix] = 0.f;
        if (a.ref_logp) a.ref_logp[tix] = 0.f;
        if (a.token_loss) a.token_loss[tix] = 0.f;
      }
    }
  }
  const uint64_t bal = __ballot(live);
  if (bal == 0) return;
  const int before = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                               __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0));
  int base = 0;
  if (before == 0 && live) base = atomicAdd(a.row_count, __popcll(bal));
  base = __shfl(base, __builtin_ctzll(bal));
  if (live) a.row_list[base + before] = static_cast<int>(row);
}

// ---------------------------------------------------------------------------
// Forward-only rows (dlogits == nullptr: log-probs, or the loss without its
// gradient). One online (max, sum) pass over the row in batches of U 16-byte vectors
// per lane, through the row's buffer descriptor (lanes past the row end read 0 and
// are skipped). REF adds the reference row in the same batches. The small register
// footprint lets several workgroups share a CU, so one workgroup's exponentials run
// while the others' loads are in flight; the resident kernel holds one row per CU and
// leaves the CU's memory idle while it sums.
// Requirements (checked on the host): V % EPV == 0, 16-byte aligned rows.
// ---------------------------------------------------------------------------
#ifndef PCP_FWD_BLOCK
#define PCP_FWD_BLOCK 256
#endif
#ifndef PCP_FWD_U
#define PCP_FWD_U 8
#endif

// max(m, the EPV values of one 16-byte vector). bf16 halves come from byte permutes:
// the same values as unpack(), but the compiler does not merge them with the sum
// pass's unpacks, which would keep every unpacked value of the batch live.
template <typename TI>
__device__ __forceinline__ float vec_max(float m, const u32x4& v) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(&v);
  if constexpr (__is_same(TI, BF16T)) {
#pragma unroll
    for (int h = 0; h < 4; ++h)
      m = fmaxf(fmaxf(m, __uint_as_float(__builtin_amdgcn_perm(w[h], 0u, 0x05040c0cu))),
                __uint_as_float(__builtin_amdgcn_perm(w[h], 0u, 0x07060c0cu)));
  } else {
#pragma unroll
    for (int j = 0; j < 16 / TI::kBytes; ++j) m = fmaxf(m, TI::unpack(w, j));
  }
  return m;
}

template <typename TI, int BLOCK, int U, bool REF>
__global__ void __launch_bounds__(BLOCK) grpo_fwd_kernel(RowArgs a) {
  constexpr int EPV = 16 / TI::kBytes;
  constexpr uint32_t kStep = BLOCK * 16u;   // bytes between a lane's vectors in one batch
  __shared__ float lds[4 * (BLOCK / 64)];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const RowMeta r = row_meta(a, row);
  if (!r.live) {
    write_token_outputs(a, r, 0.f, 0.f, 0.f);
    return;
  }
  const int64_t row_elem = row * a.vocab;
  const void* xrow = static_cast<const char*>(a.logits) + row_elem * TI::kBytes;
  const void* rrow = REF ? static_cast<const char*>(a.ref_logits) + row_elem * TI::kBytes : nullptr;
  const float xy = TI::load1(xrow, r.id);
  const float ry = REF ? TI::load1(rrow, r.id) : 0.f;
  // Rows may start off 16 bytes (V * element size not a multiple of 16, or an offset
  // view): the aligned interior goes through the descriptor as 16-byte vectors, the
  // head and tail element by element, so no load leaves the row.
  const RowSpan xsp = row_span<TI>(xrow, a.vocab);
  const RowSpan rsp = REF ? row_span<TI>(rrow, a.vocab) : xsp;
  const __amdgpu_buffer_rsrc_t xbuf = row_rsrc(xsp.vec, static_cast<uint32_t>(xsp.nv) * 16u);
  const __amdgpu_buffer_rsrc_t rbuf = REF ? row_rsrc(rsp.vec, static_cast<uint32_t>(rsp.nv) * 16u) : xbuf;
  const int nv = REF ? max(xsp.nv, rsp.nv) : xsp.nv;

  float pm, ps, rm = kNegInf, rs = 0.f;
  edge_state<TI>(xrow, xsp, tid, pm, ps);
  if constexpr (REF) edge_state<TI>(rrow, rsp, tid, rm, rs);
  for (int base = 0; base < nv; base += BLOCK * U) {
    const uint32_t off = static_cast<uint32_t>(base + tid) * 16u;
    u32x4 xb[U], rb[U];
#pragma unroll
    for (int q = 0; q < U; ++q) xb[q] = buf_ld16<true>(xbuf, off + q * kStep);
    if constexpr (REF) {
#pragma unroll
      for (int q = 0; q < U; ++q) rb[q] = buf_ld16<true>(rbuf, off + q * kStep);
    }
    float bx = kNegInf, br = kNegInf;
#pragma unroll
    for (int q = 0; q < U; ++q) {
      if (base + q * BLOCK + tid < xsp.nv) bx = vec_max<TI>(bx, xb[q]);
      if constexpr (REF)
        if (base + q * BLOCK + tid < rsp.nv) br = vec_max<TI>(br, rb[q]);
    }
    {
      const float nm = fmaxf(pm, bx * kLog2e);
      const float ref = ms_ref(nm);
      float acc = ms_rescale(ps, pm, nm);
#pragma unroll
      for (int q = 0; q < U; ++q)
        if (base + q * BLOCK + tid < xsp.nv) {
          const uint32_t* w = reinterpret_cast<const uint32_t*>(&xb[q]);
#pragma unroll
          for (int j = 0; j < EPV; ++j) acc += hw_exp2(fmaf(TI::unpack(w, j), kLog2e, -ref));
        }
      pm = nm;
      ps = acc;
    }
    if constexpr (REF) {
      const float nm = fmaxf(rm, br * kLog2e);
      const float ref = ms_ref(nm);
      float acc = ms_rescale(rs, rm, nm);
#pragma unroll
      for (int q = 0; q < U; ++q)
        if (base + q * BLOCK + tid < rsp.nv) {
          const uint32_t* w = reinterpret_cast<const uint32_t*>(&rb[q]);
#pragma unroll
          for (int j = 0; j < EPV; ++j) acc += hw_exp2(fmaf(TI::unpack(w, j), kLog2e, -ref));
        }
      rm = nm;
      rs = acc;
    }
  }

  block_merge2<BLOCK>(pm, ps, rm, rs, lds);
  const float lse2 = pm + log2f(ps);
  const float lse = lse2 * kLn2;
  const float rlse = REF ? ms_lse(rm, rs) : 0.f;
  flag_nonfinite(a, lse, rlse);
  const float lp = xy - lse;
  const float lr = ry - rlse;
  const TokenTerms tt = token_terms(a, r, lp, lr);
  write_token_outputs(a, r, lp, lr, tt.loss);
}

// ---------------------------------------------------------------------------
// Streaming kernel: any V, any alignment (VEC = false uses element loads).
// Forward only when dlogits == nullptr; otherwise a second read of the policy
// row produces dlogits (3 row reads + 1 write per live row).
// ---------------------------------------------------------------------------
template <typename TI, bool VEC>
struct StreamIO {
  static constexpr int EPV = VEC ? 16 / TI::kBytes : 1;
  struct Raw {
    u32x4 v;
    float f;
  };
  // NT: non-temporal (streaming) policy; a temporal load leaves the line in the
  // caches for a re-read.
  template <bool NT = true>
  __device__ static __forceinline__ Raw load(const void* row, int vi) {
    Raw r;
    if constexpr (VEC) r.v = ld16<NT>(row, vi);
    else r.f = TI::load1(row, vi);
    return r;
  }
  __device__ static __forceinline__ float get(const Raw& r, int j) {
    if constexpr (VEC) return TI::unpack(reinterpret_cast<const uint32_t*>(&r.v), j);
    else return r.f;
  }
};

// NT1: cache policy of the first policy read. When the row is re-read for
// dlogits, a temporal first read lets the re-read hit the caches.
template <typename TI, typename TO, int BLOCK, int U, bool VEC, bool NT1>
__global__ void __launch_bounds__(BLOCK) grpo_stream_kernel(RowArgs a) {
  using IO = StreamIO<TI, VEC>;
  constexpr int EPV = IO::EPV;
  __shared__ float lds[4 * (BLOCK / 64)];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const RowMeta r = row_meta(a, row);
  const int nv = static_cast<int>(a.vocab / EPV);
  const int64_t row_elem = row * a.vocab;

  if (!r.live) {
    write_token_outputs(a, r, 0.f, 0.f, 0.f);
    if (a.dlogits && a.zero_fill) {
      if constexpr (VEC) zero_row_vec<TO, EPV, BLOCK>(a.dlogits, row_elem, nv);
      else zero_row_scalar<TO, BLOCK>(a.dlogits, row_elem, a.vocab);
    }
    return;
  }

  const void* xrow = static_cast<const char*>(a.logits) + row_elem * TI::kBytes;
  const bool has_ref = a.ref_logits != nullptr;
  const void* rrow =
      has_ref ? static_cast<const char*>(a.ref_logits) + row_elem * TI::kBytes : nullptr;
  const float xy = TI::load1(xrow, r.id);
  const float ry = has_ref ? TI::load1(rrow, r.id) : 0.f;

  float pm = kNegInf, ps = 0.f, rm = kNegInf, rs = 0.f;
  for (int base = 0; base < nv; base += BLOCK * U) {
    typename IO::Raw xb[U], rb[U];
#pragma unroll
    for (int q = 0; q < U; ++q) {
      const int vi = base + q * BLOCK + tid;
      if (vi < nv) {
        xb[q] = IO::template load<NT1>(xrow, vi);
        if (has_ref) rb[q] = IO::load(rrow, vi);
      }
    }
    float bx = kNegInf, br = kNegInf;
#pragma unroll
    for (int q = 0; q < U; ++q) {
      if (base + q * BLOCK + tid < nv) {
#pragma unroll
        for (int j = 0; j < EPV; ++j) {
          bx = fmaxf(bx, IO::get(xb[q], j));
          if (has_ref) br = fmaxf(br, IO::get(rb[q], j));
        }
      }
    }
    {
      const float nm = fmaxf(pm, bx * kLog2e);
      const float ref = ms_ref(nm);
      float acc = ms_rescale(ps, pm, nm);
#pragma unroll
      for (int q = 0; q < U; ++q)
        if (base + q * BLOCK + tid < nv)
#pragma unroll
          for (int j = 0; j < EPV; ++j) acc += hw_exp2(fmaf(IO::get(xb[q], j), kLog2e, -ref));
      pm = nm;
      ps = acc;
    }
    if (has_ref) {
      const float nm = fmaxf(rm, br * kLog2e);
      const float ref = ms_ref(nm);
      float acc = ms_rescale(rs, rm, nm);
#pragma unroll
      for (int q = 0; q < U; ++q)
        if (base + q * BLOCK + tid < nv)
#pragma unroll
          for (int j = 0; j < EPV; ++j) acc += hw_exp2(fmaf(IO::get(rb[q], j), kLog2e, -ref));
      rm = nm;
      rs = acc;
    }
  }

  block_merge2<BLOCK>(pm, ps, rm, rs, lds);
  const float lse2 = pm + log2f(ps);
  const float lse = lse2 * kLn2;
  const float rlse = has_ref ? ms_lse(rm, rs) : 0.f;
  flag_nonfinite(a, lse, rlse);
  const float lp = xy - lse;
  const float lr = ry - rlse;
  const TokenTerms tt = token_terms(a, r, lp, lr);
  write_token_outputs(a, r, lp, lr, tt.loss);
  if (a.dlogits == nullptr) return;

  const float c = tt.coef, nc = -tt.coef;
  const int vid = static_cast<int>(r.id / EPV);
  const int jid = static_cast<int>(r.id) - vid * EPV;
  for (int base = 0; base < nv; base += BLOCK * U) {
    typename IO::Raw xb[U];
#pragma unroll
    for (int q = 0; q < U; ++q) {
      const int vi = base + q * BLOCK + tid;
      if (vi < nv) xb[q] = IO::load(xrow, vi);
    }
#pragma unroll
    for (int q = 0; q < U; ++q) {
      const int vi = base + q * BLOCK + tid;
      if (vi < nv) {
        float o[EPV];
#pragma unroll
        for (int j = 0; j < EPV; ++j) o[j] = nc * hw_exp2(fmaf(IO::get(xb[q], j), kLog2e, -lse2));
        if (vi == vid) {
#pragma unroll
          for (int j = 0; j < EPV; ++j)
            if (j == jid) o[j] += c;
        }
        if constexpr (VEC) store_vals<TO, EPV, true>(a.dlogits, row_elem + static_cast<int64_t>(vi) * EPV, o);
        else store1<TO>(a.dlogits, row_elem + vi, o[0]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Small kernels: sequence lengths, advantages, loss reduction.
// ---------------------------------------------------------------------------

// Deterministic workgroup sum: fixed per-lane order, xor butterfly (commutative,
// so every lane agrees), fixed cross-wave order. Result on every thread.
template <int BLOCK>
__device__ __forceinline__ float block_sum(float v, float* lds) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  constexpr int NW = BLOCK / 64;
  if constexpr (NW > 1) {
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    v = lds[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += lds[w];
    __syncthreads();
  }
  return v;
}

// seq_len[s] = max(sum_t mask, 1)  (torch.clamp(shift_mask.sum(1), min=1.0),
// export_qwen_forward.py:160); seq_scale[s] = 1 / (loss_norm * seq_len[s]).
constexpr int kSmallBlock = 256;
__global__ void __launch_bounds__(kSmallBlock)
seq_prep_kernel(const void* mask, int32_t mask_u8, int64_t rows, int64_t tok_stride,
                int64_t tok_offset, float loss_norm, float* seq_len, float* seq_scale) {
  __shared__ float lds[kSmallBlock / 64];
  const int64_t s = blockIdx.x;
  float acc = 0.f;
  const int64_t base = s * tok_stride + tok_offset;
  for (int64_t t = threadIdx.x; t < rows; t += kSmallBlock) {
    float m;
    if (mask == nullptr) m = 1.f;
    else if (mask_u8) m = static_cast<const uint8_t*>(mask)[base + t] ? 1.f : 0.f;
    else m = static_cast<const float*>(mask)[base + t];
    acc += m;
  }
  const float tot = block_sum<kSmallBlock>(acc, lds);
  if (threadIdx.x == 0) {
    const float L = fmaxf(tot, 1.f);
    seq_len[s] = L;
    seq_scale[s] = 1.f / (loss_norm * L);
  }
}

// Group-relative advantages, restating rl_shepherd.zig:466-478 operation by
// operation in IEEE fp32: sequential sum, mean = sum / n, sequential sum of
// (r-mean)*(r-mean), std = sqrt(ssd / n) + eps, (r-mean)/std. hipcc contracts
// a*b+c into an FMA by default (also inside the __fmul_rn/__fadd_rn helpers,
// which are compiled outside this scope), so the arithmetic is written with
// plain operators under contract(off); fp32 '/' and sqrtf are correctly rounded
// (hipcc's default -fhip-fp32-correctly-rounded-divide-sqrt).
// The group of rewards [i, e): adv[k] (and adv2[k] when adv2 is not null).
__device__ __forceinline__ void group_advantages(const float* r, int64_t i, int64_t e, float eps, float* adv,
                                                 float* adv2) {
#pragma clang fp contract(off)
  const float cnt = static_cast<float>(e - i);
  float sum = 0.f;
  for (int64_t k = i; k < e; ++k) sum = sum + r[k];
  const float mean = sum / cnt;
  float ssd = 0.f;
  for (int64_t k = i; k < e; ++k) {
    const float d = r[k] - mean;
    const float d2 = d * d;
    ssd = ssd + d2;
  }
  const float sd = sqrtf(ssd / cnt) + eps;
  for (int64_t k = i; k < e; ++k) {
    const float v = (r[k] - mean) / sd;
    adv[k] = v;
    if (adv2) adv2[k] = v;
  }
}

// group_advantages with the group's rewards loaded by the 64 lanes of one wave at once
// (chunks of 64), so the sequential sums run on registers instead of one dependent
// load per reward: every lane forms the same sums from the same values in the same
// order (readlane copies bits), hence the same bits as group_advantages. Called by all
// 64 lanes of a wave.
__device__ __forceinline__ void group_advantages_wave(const float* r, int64_t i, int64_t e, float eps, float* adv,
                                                      float* adv2) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const float cnt = static_cast<float>(e - i);
  // Chunk c of 64 rewards: lane l holds r[i + 64 c + l]; the first chunk is kept.
  const int n0 = static_cast<int>(min<int64_t>(64, e - i));
  const float v0 = lane < n0 ? r[i + lane] : 0.f;
  auto chunk = [&](int64_t c0) { return c0 == i ? v0 : (c0 + lane < e ? r[c0 + lane] : 0.f); };
  float sum = 0.f;
  for (int64_t c0 = i; c0 < e; c0 += 64) {
    const int n = static_cast<int>(min<int64_t>(64, e - c0));
    const float v = chunk(c0);
    for (int k = 0; k < n; ++k) sum = sum + __shfl(v, k);
  }
  const float mean = sum / cnt;
  float ssd = 0.f;
  for (int64_t c0 = i; c0 < e; c0 += 64) {
    const int n = static_cast<int>(min<int64_t>(64, e - c0));
    const float v = chunk(c0);
    for (int k = 0; k < n; ++k) {
      const float d = __shfl(v, k) - mean;
      const float d2 = d * d;
      ssd = ssd + d2;
    }
  }
  const float sd = sqrtf(ssd / cnt) + eps;
  for (int64_t c0 = i; c0 < e; c0 += 64) {
    if (c0 + lane >= e) break;
    const float x = (chunk(c0) - mean) / sd;
    adv[c0 + lane] = x;
    if (adv2) adv2[c0 + lane] = x;
  }
}

__global__ void __launch_bounds__(64)
advantages_kernel(const float* r, int64_t n, int64_t group, float eps, float* adv) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
  const int64_t i = g * group;
  if (i >= n) return;
  group_advantages(r, i, (i + group < n) ? i + group : n, eps, adv, nullptr);
}

// seq_val[s] = (sum_t token_loss) / seq_len[s] (* adv[s] in REINFORCE mode):
// token_losses.sum(1) / seq_lengths; seq_nll * advantages (export_qwen_forward.py:161-162).
__global__ void __launch_bounds__(kSmallBlock)
seq_loss_kernel(const float* token_loss, int64_t rows, int64_t tok_stride, int64_t tok_offset,
                const float* seq_len, const float* adv, int32_t reinforce, float* seq_val) {
  __shared__ float lds[kSmallBlock / 64];
  const int64_t s = blockIdx.x;
  const int64_t base = s * tok_stride + tok_offset;
  float acc = 0.f;
  for (int64_t t = threadIdx.x; t < rows; t += kSmallBlock) acc += token_loss[base + t];
  const float tot = block_sum<kSmallBlock>(acc, lds);
  if (threadIdx.x == 0) {
    const float v = tot / seq_len[s];
    seq_val[s] = reinforce ? v * adv[s] : v;
  }
}

// loss = sum_s seq_val[s] / loss_norm  (weighted_losses.mean(), export_qwen_forward.py:163).
constexpr int kFinalBlock = 1024;
__global__ void __launch_bounds__(kFinalBlock)
loss_final_kernel(const float* seq_val, int64_t n_seq, float loss_norm, float* loss) {
  __shared__ float lds[kFinalBlock / 64];
  float acc = 0.f;
  for (int64_t s = threadIdx.x; s < n_seq; s += kFinalBlock) acc += seq_val[s];
  const float tot = block_sum<kFinalBlock>(acc, lds);
  if (threadIdx.x == 0) *loss = tot / loss_norm;
}

// The work before the row kernel in one launch, one workgroup per sequence s:
//  * seq_len[s], seq_scale[s] as seq_prep_kernel (the same per-lane order and reduction);
//  * with rewards: thread 0 of the first workgroup of each group computes the group's
//    advantages as advantages_kernel (the same function, so the same bits), also into
//    adv_out; without: adv_out[s] = adv_in[s] (when adv_out is set);
//  * workgroup 0 zeroes the counters the row kernel and loss_reduce_kernel start from.
__global__ void __launch_bounds__(kSmallBlock) step_prep_kernel(StepPrepArgs a) {
  const int64_t s = blockIdx.x;
  __shared__ float lds[kSmallBlock / 64];
  // The mask terms first, in batches of four per lane with every load of a batch in
  // flight before its additions (each lane still adds its terms in row order).
  float acc = 0.f;
  const int64_t base = s * a.tok_stride + a.tok_offset;
  constexpr int kB = 4;
  for (int64_t t0 = threadIdx.x; t0 < a.rows; t0 += kB * kSmallBlock) {
    float m[kB];
#pragma unroll
    for (int q = 0; q < kB; ++q) {
      const int64_t t = t0 + q * kSmallBlock;
      m[q] = 1.f;
      if (a.mask != nullptr && t < a.rows)
        m[q] = a.mask_u8 ? (static_cast<const uint8_t*>(a.mask)[base + t] ? 1.f : 0.f)
                         : static_cast<const float*>(a.mask)[base + t];
    }
#pragma unroll
    for (int q = 0; q < kB; ++q)
      if (t0 + q * kSmallBlock < a.rows) acc += m[q];
  }
  if (threadIdx.x == 0 && s == 0) {
#pragma unroll
    for (int k = 0; k < 3; ++k)
      if (a.zero[k]) *a.zero[k] = 0;
  }
  if (a.rewards) {
    if (s % a.group == 0 && threadIdx.x < 64)
      group_advantages_wave(a.rewards, s, min(s + a.group, a.n_seq), a.std_eps, a.adv, a.adv_out);
  } else if (a.adv_out && threadIdx.x == 0) {
    a.adv_out[s] = a.adv_in[s];
  }
  const float tot = block_sum<kSmallBlock>(acc, lds);
  if (threadIdx.x == 0) {
    const float L = fmaxf(tot, 1.f);
    a.seq_len[s] = L;
    a.seq_scale[s] = 1.f / (a.loss_norm * L);
  }
}

// The loss in one launch, one workgroup per sequence: seq_val[s] as seq_loss_kernel;
// the workgroup that finishes last (a ticket from *done, which step_prep_kernel zeroed)
// then forms the loss in loss_final_kernel's order, lane for lane: the 16 waves of
// that 1024-lane sum are taken four at a time by this workgroup's waves (lane l of
// wave w adds seq_val[64 w + l], [64 w + l + 1024], ... and reduces by the same xor
// butterfly), and the wave sums add in wave order. It leaves *done at 0.
__global__ void __launch_bounds__(kSmallBlock) loss_reduce_kernel(LossReduceArgs a) {
  __shared__ float lds[kFinalBlock / 64];
  __shared__ int last;
  const int64_t s = blockIdx.x;
  const int64_t base = s * a.tok_stride + a.tok_offset;
  // The sequence's scalars and token losses all in flight before any addition (each
  // lane still adds its terms in row order, batches of four).
  const float len = a.seq_len[s];
  const float av = a.reinforce ? a.adv[s] : 1.f;
  float acc = 0.f;
  constexpr int kB = 4;
  for (int64_t t0 = threadIdx.x; t0 < a.rows; t0 += kB * kSmallBlock) {
    float m[kB];
#pragma unroll
    for (int q = 0; q < kB; ++q) {
      const int64_t t = t0 + q * kSmallBlock;
      m[q] = t < a.rows ? a.token_loss[base + t] : 0.f;
    }
#pragma unroll
    for (int q = 0; q < kB; ++q)
      if (t0 + q * kSmallBlock < a.rows) acc += m[q];
  }
  const float tot = block_sum<kSmallBlock>(acc, lds);
  if (threadIdx.x == 0) {
    const float v = tot / len;
    store_coherent(a.seq_val + s, a.reinforce ? v * av : v);
    wait_stores();     // seq_val[s] at the coherent level before the ticket
    last = atomicAdd(a.done, 1) == static_cast<int>(a.n_seq - 1);
  }
  __syncthreads();
  if (!last) return;
  acquire_coherent();
  const int lane = threadIdx.x & 63, w0 = threadIdx.x >> 6;
  constexpr int kPer = kFinalBlock / kSmallBlock;   // the final sum's waves per wave here
  float v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {   // first terms of all of them in flight together
    const int64_t k = 64 * (w0 + 4 * i) + lane;
    v[i] = 0.f;
    if (k < a.n_seq) v[i] += a.seq_val[k];   // 0 + x, as loss_final_kernel's first addition
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    for (int64_t k = 64 * (w0 + 4 * i) + lane + kFinalBlock; k < a.n_seq; k += kFinalBlock) v[i] += a.seq_val[k];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v[i] += __shfl_xor(v[i], off);
    if (lane == 0) lds[w0 + 4 * i] = v[i];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = lds[0];
#pragma unroll
    for (int w = 1; w < kFinalBlock / 64; ++w) v += lds[w];
    *a.loss = v / a.loss_norm;
    *a.done = 0;
  }
}

// ---------------------------------------------------------------------------
// Host-side launchers
// ---------------------------------------------------------------------------
namespace {

template <typename TI, typename TO, int BLOCK, int NCH, bool EDGE, bool CACHE>
hipError_t launch_resident(const RowArgs& a, int64_t nrows, hipStream_t st) {
  // RB = 2: reference batches of two chunks next to a 19-chunk resident row at 128
  // VGPRs. The headline instance (bf16 -> bf16, cache) then spills 2 VGPRs and 42
  // SGPRs (12 bytes of scratch per lane); RB = 4 spills 9 VGPRs and measured ~1%
  // slower.
  constexpr int RB = 2;
  // One workgroup per resident slot of the device (the kernel's occupancy times the
  // CU count), at most one per row. Only a successful query is cached.
  static std::atomic<int> cached{0};
  int slots = cached.load(std::memory_order_relaxed);
  if (slots <= 0) {
    int dev = 0, cus = 0, occ = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess)
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &occ, reinterpret_cast<const void*>(&grpo_resident_kernel<TI, TO, BLOCK, NCH, RB, EDGE, CACHE, false>), BLOCK,
          0);
    if (e != hipSuccess) return e;
    slots = cus * (occ > 0 ? occ : 1);
    cached.store(slots, std::memory_order_relaxed);
  }
  const int64_t grid = nrows < slots ? nrows : slots;
  if (grid <= 0) return hipSuccess;
  const dim3 g(static_cast<unsigned>(grid)), b(BLOCK);
  if (!a.counters_zeroed) reset_counter_kernel<<<1, 1, 0, st>>>(a.next_row, a.row_list ? a.row_count : nullptr);
  if (a.row_list) {
    live_rows_kernel<<<dim3(static_cast<unsigned>((nrows + 255) / 256)), dim3(256), 0, st>>>(a);
    grpo_resident_kernel<TI, TO, BLOCK, NCH, RB, EDGE, CACHE, true><<<g, b, 0, st>>>(a);
  } else {
    grpo_resident_kernel<TI, TO, BLOCK, NCH, RB, EDGE, CACHE, false><<<g, b, 0, st>>>(a);
  }
  return hipGetLastError();
}

template <typename TI, typename TO, bool VEC>
hipError_t launch_stream(const RowArgs& a, int64_t nrows, hipStream_t st) {
  constexpr int BLOCK = 1024, U = 4;
  // Forward only: every byte is read once, so stream it past the caches. With a
  // backward pass the first policy read stays cacheable for the re-read.
  if (a.dlogits)
    grpo_stream_kernel<TI, TO, BLOCK, U, VEC, false>
        <<<dim3(static_cast<unsigned>(nrows)), dim3(BLOCK), 0, st>>>(a);
  else
    grpo_stream_kernel<TI, TO, BLOCK, U, VEC, true>
        <<<dim3(static_cast<unsigned>(nrows)), dim3(BLOCK), 0, st>>>(a);
  return hipGetLastError();
}

template <typename TI>
hipError_t launch_fwd(const RowArgs& a, int64_t nrows, hipStream_t st) {
  constexpr int BLOCK = PCP_FWD_BLOCK, U = PCP_FWD_U;
  if (nrows <= 0) return hipSuccess;
  if (a.ref_logits)
    grpo_fwd_kernel<TI, BLOCK, U, true><<<dim3(static_cast<unsigned>(nrows)), dim3(BLOCK), 0, st>>>(a);
  else
    grpo_fwd_kernel<TI, BLOCK, U, false><<<dim3(static_cast<unsigned>(nrows)), dim3(BLOCK), 0, st>>>(a);
  return hipGetLastError();
}

// Resident configurations: (BLOCK, NCH). A row of NV 16-byte vectors fits the
// first configuration with BLOCK*NCH >= NV.
struct ResCfg {
  int block, nch;
};
// (1024, 24) would spill at the 128-VGPR budget of a 1024-lane workgroup, so rows
// wider than 20480 16-byte vectors (V > 163840 for 16-bit logits) stream instead.
constexpr ResCfg kResCfgs[] = {{256, 1},   {256, 2},   {256, 4},   {1024, 2}, {1024, 4},
                               {1024, 8},  {1024, 12}, {1024, 16}, {1024, 19}, {1024, 20}};

// Rows off 16 bytes (EDGE) need dlogits of the logits' element type. Only bf16 -> bf16
// rows have the f16 softmax cache, so only they have instances without it (exact).
template <typename TI, typename TO, int BLOCK, int NCH>
hipError_t launch_resident_cfg(bool edge, bool exact, const RowArgs& a, int64_t nrows, hipStream_t st) {
  if constexpr (__is_same(TI, BF16T) && __is_same(TO, BF16T)) {
    if (exact)
      return edge ? launch_resident<TI, TO, BLOCK, NCH, true, false>(a, nrows, st)
                  : launch_resident<TI, TO, BLOCK, NCH, false, false>(a, nrows, st);
  }
  if constexpr (__is_same(TI, TO)) {
    if (edge) return launch_resident<TI, TO, BLOCK, NCH, true, true>(a, nrows, st);
  } else {
    if (edge) return hipErrorInvalidValue;
  }
  return launch_resident<TI, TO, BLOCK, NCH, false, true>(a, nrows, st);
}

template <typename TI, typename TO>
hipError_t dispatch_resident(int cfg, bool edge, bool exact, const RowArgs& a, int64_t nrows, hipStream_t st) {
  switch (cfg) {
    case 0: return launch_resident_cfg<TI, TO, 256, 1>(edge, exact, a, nrows, st);
    case 1: return launch_resident_cfg<TI, TO, 256, 2>(edge, exact, a, nrows, st);
    case 2: return launch_resident_cfg<TI, TO, 256, 4>(edge, exact, a, nrows, st);
    case 3: return launch_resident_cfg<TI, TO, 1024, 2>(edge, exact, a, nrows, st);
    case 4: return launch_resident_cfg<TI, TO, 1024, 4>(edge, exact, a, nrows, st);
    case 5: return launch_resident_cfg<TI, TO, 1024, 8>(edge, exact, a, nrows, st);
    case 6: return launch_resident_cfg<TI, TO, 1024, 12>(edge, exact, a, nrows, st);
    case 7: return launch_resident_cfg<TI, TO, 1024, 16>(edge, exact, a, nrows, st);
    case 8: return launch_resident_cfg<TI, TO, 1024, 19>(edge, exact, a, nrows, st);
    case 9: return launch_resident_cfg<TI, TO, 1024, 20>(edge, exact, a, nrows, st);
  }
  return hipErrorInvalidValue;
}

template <typename TI, typename TO>
hipError_t dispatch_rows(const RowPlan& p, const RowArgs& a, int64_t nrows, hipStream_t st) {
  if (p.kind == RowPlan::kResident) return dispatch_resident<TI, TO>(p.cfg, p.edge != 0, p.exact != 0, a, nrows, st);
  if (p.kind == RowPlan::kForward) return launch_fwd<TI>(a, nrows, st);
  if (p.kind == RowPlan::kStreamVec) return launch_stream<TI, TO, true>(a, nrows, st);
  return launch_stream<TI, TO, false>(a, nrows, st);
}

}  // namespace

RowPlan plan_rows(int in_bytes, int64_t vocab, bool aligned16, bool edge_ok, bool forward_only, bool force_stream) {
  RowPlan p;
  const int epv = 16 / in_bytes;
  const bool vec = aligned16 && (vocab % epv == 0);
  p.kind = vec ? RowPlan::kStreamVec : RowPlan::kStreamScalar;
  p.cfg = -1;
  p.block = 1024;
  p.nch = 0;
  p.edge = 0;
  p.exact = 0;
  if (force_stream) return p;
  // The forward kernel takes rows of any alignment. It addresses a row through a
  // 32-bit buffer offset that runs up to one batch past the row end: rows up to 2 GiB
  // take it, longer rows stream (64-bit addressing).
  if (forward_only && vocab * in_bytes <= (int64_t{1} << 31)) {
    p.kind = RowPlan::kForward;
    p.block = PCP_FWD_BLOCK;
    return p;
  }
  // Rows off 16 bytes stay resident when dlogits rows share the logits rows' element
  // type and offset (the head and tail then line up); otherwise they stream.
  if (!vec && !edge_ok) return p;

  const int64_t nv = vocab / epv;   // the interior of a row off 16 bytes has at most as many
  for (int i = 0; i < static_cast<int>(sizeof(kResCfgs) / sizeof(kResCfgs[0])); ++i) {
    if (static_cast<int64_t>(kResCfgs[i].block) * kResCfgs[i].nch >= nv) {
      p.kind = RowPlan::kResident;
      p.cfg = i;
      p.block = kResCfgs[i].block;
      p.nch = kResCfgs[i].nch;
      p.edge = vec ? 0 : 1;
      return p;
    }
  }
  return p;
}

hipError_t launch_rows(const RowPlan& p, int in_dtype, int out_dtype, const RowArgs& a,
                       int64_t nrows, hipStream_t st) {
  if (in_dtype == PCP_BF16 && out_dtype == PCP_BF16) return dispatch_rows<BF16T, BF16T>(p, a, nrows, st);
  if (in_dtype == PCP_BF16 && out_dtype == PCP_F32) return dispatch_rows<BF16T, F32T>(p, a, nrows, st);
  if (in_dtype == PCP_F16 && out_dtype == PCP_F16) return dispatch_rows<F16T, F16T>(p, a, nrows, st);
  if (in_dtype == PCP_F16 && out_dtype == PCP_F32) return dispatch_rows<F16T, F32T>(p, a, nrows, st);
  if (in_dtype == PCP_F32 && out_dtype == PCP_F32) return dispatch_rows<F32T, F32T>(p, a, nrows, st);
  return hipErrorInvalidValue;
}

hipError_t launch_seq_prep(const void* mask, int mask_u8, int64_t n_seq, int64_t rows,
                           int64_t tok_stride, int64_t tok_offset, float loss_norm,
                           float* seq_len, float* seq_scale, hipStream_t st) {
  seq_prep_kernel<<<dim3(static_cast<unsigned>(n_seq)), dim3(kSmallBlock), 0, st>>>(
      mask, mask_u8, rows, tok_stride, tok_offset, loss_norm, seq_len, seq_scale);
  return hipGetLastError();
}

hipError_t launch_advantages(const float* r, int64_t n, int64_t group, float eps, float* adv,
                             hipStream_t st) {
  const int64_t ngroups = (n + group - 1) / group;
  const unsigned nb = static_cast<unsigned>((ngroups + 63) / 64);
  advantages_kernel<<<dim3(nb), dim3(64), 0, st>>>(r, n, group, eps, adv);
  return hipGetLastError();
}

hipError_t launch_step_prep(const StepPrepArgs& a, hipStream_t st) {
  step_prep_kernel<<<dim3(static_cast<unsigned>(a.n_seq)), dim3(kSmallBlock), 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_loss_reduce_fused(const LossReduceArgs& a, hipStream_t st) {
  loss_reduce_kernel<<<dim3(static_cast<unsigned>(a.n_seq)), dim3(kSmallBlock), 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_loss_reduce(const float* token_loss, int64_t n_seq, int64_t rows,
                              int64_t tok_stride, int64_t tok_offset, const float* seq_len,
                              const float* adv, int reinforce, float loss_norm, float* seq_val,
                              float* loss, hipStream_t st) {
  seq_loss_kernel<<<dim3(static_cast<unsigned>(n_seq)), dim3(kSmallBlock), 0, st>>>(
      token_loss, rows, tok_stride, tok_offset, seq_len, adv, reinforce, seq_val);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  loss_final_kernel<<<dim3(1), dim3(kFinalBlock), 0, st>>>(seq_val, n_seq, loss_norm, loss);
  return hipGetLastError();
}

}  // namespace pcp
