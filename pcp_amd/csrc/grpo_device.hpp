// Device-side building blocks of the GRPO loss-head kernels (gfx950, wave64).
//
// Element codecs, vector row I/O, the online (max, sum-exp) pair and its wave /
// workgroup merge, and the per-token GRPO math shared by every kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pcp_grpo.h"

namespace pcp {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kNegInf = -__builtin_inff();

// Device error bits, OR-ed into the context's flag word; the host maps them to
// pcp_status codes after the stream is synchronised.
constexpr int kErrTokenRange = 1;
constexpr int kErrNonFinite = 2;
constexpr int kErrBadRagged = 4;   // rollout packing: offsets decrease or run past the token array
constexpr int kErrBadBase64 = 8;   // base64: a character outside the alphabet or misplaced padding
constexpr int kErrListedRow = 16;  // a row listed live by live_rows_kernel was not live in the row kernel

// v_exp_f32: 2^x. Used only for the per-element softmax terms, where results
// below the fp32 normal range are irrelevant (they multiply a coefficient < 1).
__device__ __forceinline__ float hw_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------
// Element codecs. `unpack(w, j)` reads element j of a packed little-endian word
// array; `load1` reads one element of a row.
// ---------------------------------------------------------------------------
struct F32T {
  static constexpr int kBytes = 4;
  __device__ static __forceinline__ float unpack(const uint32_t* w, int j) {
    return __uint_as_float(w[j]);
  }
  __device__ static __forceinline__ float load1(const void* p, int64_t i) {
    return static_cast<const float*>(p)[i];
  }
};

struct BF16T {
  static constexpr int kBytes = 2;
  __device__ static __forceinline__ float unpack(const uint32_t* w, int j) {
    const uint32_t x = w[j >> 1];
    return __uint_as_float((j & 1) ? (x & 0xffff0000u) : (x << 16));
  }
  __device__ static __forceinline__ float load1(const void* p, int64_t i) {
    return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]) << 16);
  }
};

struct F16T {
  static constexpr int kBytes = 2;
  __device__ static __forceinline__ float unpack(const uint32_t* w, int j) {
    const uint32_t x = w[j >> 1];
    const uint16_t h = (j & 1) ? static_cast<uint16_t>(x >> 16) : static_cast<uint16_t>(x & 0xffffu);
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
  }
  __device__ static __forceinline__ float load1(const void* p, int64_t i) {
    return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  }
};

// Pack two floats into one 32-bit word of the output element type (RNE).
template <typename TO>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<BF16T>(float lo, float hi) {
  f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));  // v_cvt_pk_bf16_f32
}
template <>
__device__ __forceinline__ uint32_t pack2<F16T>(float lo, float hi) {
  f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2));
}

template <typename TO>
__device__ __forceinline__ void store1(void* p, int64_t i, float v);
template <>
__device__ __forceinline__ void store1<F32T>(void* p, int64_t i, float v) {
  static_cast<float*>(p)[i] = v;
}
template <>
__device__ __forceinline__ void store1<BF16T>(void* p, int64_t i, float v) {
  static_cast<__bf16*>(p)[i] = static_cast<__bf16>(v);
}
template <>
__device__ __forceinline__ void store1<F16T>(void* p, int64_t i, float v) {
  static_cast<_Float16*>(p)[i] = static_cast<_Float16>(v);
}

// Load one 16-byte vector (kBytes*EPV == 16) of a row; `nt` selects the
// non-temporal (streaming) cache policy.
template <bool NT>
__device__ __forceinline__ u32x4 ld16(const void* base, int64_t vec_idx) {
  const u32x4* p = static_cast<const u32x4*>(base) + vec_idx;
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

// Raw buffer resource over one row (base, size in bytes). The hardware range check
// of a raw buffer access compares the lane (VGPR) offset with num_records (the
// SGPR offset is not checked), so every access passes its full byte offset in the
// VGPR: reads past the row end return 0 and writes past it are dropped. No lane
// then needs a branch around its access (a branch around a load makes the
// compiler wait for the pending load before the other path writes the same
// registers, serialising the row), and the descriptor stays in SGPRs.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* p, uint32_t nbytes) {
  // dword3 0x00020000: untyped 32-bit data format, as for any raw buffer access on gfx9.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), static_cast<short>(0),
                                           static_cast<int>(nbytes), 0x00020000);
}

// Byte offset base + add, formed at the point of use by an opaque v_add_u32. Left to
// itself the compiler computes the NCH chunk offsets of a row once and keeps them
// live from the first load to the last store (19 VGPRs at V = 151936), which pushes
// the resident kernel past its 128-VGPR budget.
__device__ __forceinline__ uint32_t fresh_off(uint32_t base, uint32_t add) {
  uint32_t r;
  asm volatile("v_add_u32 %0, %1, %2" : "=v"(r) : "s"(add), "v"(base));
  return r;
}

// Cache-policy bits of buffer accesses: 2 = NT (streaming, not retained).
constexpr int kBufNT = 2;
// sc0 | sc1 | nt: nontemporal at system scope (stores written through to memory).
constexpr int kBufNTSystem = 19;

// 16-byte load / store at byte offset `off` of a row buffer (range-checked).
template <bool NT>
__device__ __forceinline__ u32x4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, NT ? kBufNT : 0));
}

template <bool NT>
__device__ __forceinline__ u32x2 buf_ld8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, NT ? kBufNT : 0));
}

// Global streaming stores at system scope (sc0 sc1 nt: written through to memory), for
// kernels that write each byte once and whose output the next launch reads back. No
// builtin sets these bits on a global store, hence the inline assembly; the compiler
// does not track these stores, which is safe as nothing in the kernel reads them back.
__device__ __forceinline__ void store_nt_sys(u32x4 v, void* p) {
  asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1 nt" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_nt_sys(u32x2 v, void* p) {
  asm volatile("global_store_dwordx2 %0, %1, off sc0 sc1 nt" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_nt_sys(uint32_t v, void* p) {
  asm volatile("global_store_dword %0, %1, off sc0 sc1 nt" ::"v"(p), "v"(v) : "memory");
}

// POL: the cache policy of an NT access (kBufNT or kBufNTSystem).
template <bool NT, int POL = kBufNT>
__device__ __forceinline__ void buf_st16(__amdgpu_buffer_rsrc_t r, u32x4 v, uint32_t off) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), r, off, 0, NT ? POL : 0);
}

// Store one output element at byte offset `off` of a row buffer (range-checked).
template <typename TO, bool NT, int POL = kBufNT>
__device__ __forceinline__ void buf_store1(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  if constexpr (TO::kBytes == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, NT ? POL : 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(pack2<TO>(v, 0.f) & 0xffffu), r, off, 0,
                                          NT ? POL : 0);
  }
}

// Pack N floats into N output elements (N * kBytes = 16 or 32 bytes) and store them
// through a row buffer at byte offset `off` (range-checked).
template <typename TO, int N, bool NT, int POL = kBufNT>
__device__ __forceinline__ void buf_store_vals(__amdgpu_buffer_rsrc_t r, uint32_t off, const float (&v)[N]) {
  if constexpr (TO::kBytes == 4) {
    static_assert(N % 4 == 0, "f32 output stores whole 16-byte vectors");
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
      u32x4 w = {__float_as_uint(v[4 * q]), __float_as_uint(v[4 * q + 1]), __float_as_uint(v[4 * q + 2]),
                 __float_as_uint(v[4 * q + 3])};
      buf_st16<NT, POL>(r, w, off + 16 * q);
    }
  } else {
    static_assert(N % 8 == 0, "16-bit output stores whole 16-byte vectors");
#pragma unroll
    for (int q = 0; q < N / 8; ++q) {
      u32x4 w = {pack2<TO>(v[8 * q], v[8 * q + 1]), pack2<TO>(v[8 * q + 2], v[8 * q + 3]),
                 pack2<TO>(v[8 * q + 4], v[8 * q + 5]), pack2<TO>(v[8 * q + 6], v[8 * q + 7])};
      buf_st16<NT, POL>(r, w, off + 16 * q);
    }
  }
}

// Store N floats as N output elements at element offset `elem` of `base`.
// N * kBytes is 8, 16 or 32 bytes; `base + elem` is aligned to that size.
template <typename TO, int N, bool NT>
__device__ __forceinline__ void store_vals(void* base, int64_t elem, const float (&v)[N]) {
  if constexpr (TO::kBytes == 4) {
    static_assert(N % 4 == 0, "f32 output stores whole 16-byte vectors");
    u32x4* p = reinterpret_cast<u32x4*>(static_cast<float*>(base) + elem);
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
      u32x4 w = {__float_as_uint(v[4 * q]), __float_as_uint(v[4 * q + 1]),
                 __float_as_uint(v[4 * q + 2]), __float_as_uint(v[4 * q + 3])};
      if constexpr (NT) __builtin_nontemporal_store(w, p + q);
      else p[q] = w;
    }
  } else {
    static_assert(N == 4 || N % 8 == 0, "16-bit output stores 8 or 16n bytes");
    if constexpr (N == 4) {
      u32x2* p = reinterpret_cast<u32x2*>(static_cast<uint16_t*>(base) + elem);
      u32x2 w = {pack2<TO>(v[0], v[1]), pack2<TO>(v[2], v[3])};
      if constexpr (NT) __builtin_nontemporal_store(w, p);
      else *p = w;
    } else {
      u32x4* p = reinterpret_cast<u32x4*>(static_cast<uint16_t*>(base) + elem);
#pragma unroll
      for (int q = 0; q < N / 8; ++q) {
        u32x4 w = {pack2<TO>(v[8 * q], v[8 * q + 1]), pack2<TO>(v[8 * q + 2], v[8 * q + 3]),
                   pack2<TO>(v[8 * q + 4], v[8 * q + 5]), pack2<TO>(v[8 * q + 6], v[8 * q + 7])};
        if constexpr (NT) __builtin_nontemporal_store(w, p + q);
        else p[q] = w;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Online log-sum-exp state in base-2 units: m = max(x) * log2(e),
// s = sum 2^(x*log2(e) - m). s == 0 means "no element yet" (m is then -inf).
// fmaxf ignores NaN, so NaN inputs never reach m; they reach s (2^NaN = NaN),
// and every step below keeps a NaN s as NaN (NaN * 0 = NaN), so a NaN logit
// always ends in a non-finite log-sum-exp. merge() is commutative bit-for-bit,
// so an xor-butterfly leaves every lane of a wave with the same value, and a
// fixed cross-wave order makes the result identical on every thread and run.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void ms_merge(float& m, float& s, float m2, float s2) {
  const float M = fmaxf(m, m2);
  const float a = (s == 0.f) ? 0.f : s * hw_exp2(m - M);
  const float b = (s2 == 0.f) ? 0.f : s2 * hw_exp2(m2 - M);
  m = M;
  s = a + b;
}

// Reference point for 2^(x*log2e - ref): the running max, or 0 while it is -inf
// (all elements so far -inf or NaN), so -inf terms give 0 and NaN terms NaN.
__device__ __forceinline__ float ms_ref(float m) { return (m == kNegInf) ? 0.f : m; }

// Rescale a running sum from reference m to reference nm (nm >= m).
__device__ __forceinline__ float ms_rescale(float s, float m, float nm) {
  return (s == 0.f) ? 0.f : s * hw_exp2(m - ms_ref(nm));
}

// log-sum-exp (natural units) of a merged state.
__device__ __forceinline__ float ms_lse(float m, float s) { return (m + log2f(s)) * kLn2; }

// Reduce two (m, s) pairs over the workgroup. `lds` holds 4 floats per wave.
// Returns the same values on every thread.
template <int BLOCK>
__device__ __forceinline__ void block_merge2(float& m1, float& s1, float& m2, float& s2,
                                             float* lds) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float om1 = __shfl_xor(m1, off), os1 = __shfl_xor(s1, off);
    const float om2 = __shfl_xor(m2, off), os2 = __shfl_xor(s2, off);
    ms_merge(m1, s1, om1, os1);
    ms_merge(m2, s2, om2, os2);
  }
  constexpr int NW = BLOCK / 64;
  if constexpr (NW > 1) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (lane == 0) {
      lds[4 * wid + 0] = m1;
      lds[4 * wid + 1] = s1;
      lds[4 * wid + 2] = m2;
      lds[4 * wid + 3] = s2;
    }
    __syncthreads();
    m1 = lds[0];
    s1 = lds[1];
    m2 = lds[2];
    s2 = lds[3];
#pragma unroll
    for (int w = 1; w < NW; ++w) {
      ms_merge(m1, s1, lds[4 * w + 0], lds[4 * w + 1]);
      ms_merge(m2, s2, lds[4 * w + 2], lds[4 * w + 3]);
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel argument block (passed by value) and per-row metadata.
// ---------------------------------------------------------------------------
// Handing values from one workgroup to another in the same launch (the last of a
// group of workgroups, chosen by an atomic ticket, reads what the others wrote). A
// device-scope release fence writes back the whole L2 of the XCD (buffer_wbl2), which
// cost microseconds per workgroup here. Instead each value is stored through to the
// device-coherent level (an agent-scope atomic store), the storing wave waits for its
// stores to complete before the ticket, and the reader, after the ticket, invalidates
// its caches' copies once (an agent-scope acquire fence: buffer_inv, no write-back) and
// loads as usual, so its loads go out together. (Agent-scope atomic loads would each
// wait for the one before.)
template <typename T>
__device__ __forceinline__ void store_coherent(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// This wave's stores complete (at the level they were issued to) before what follows.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Before reading what other workgroups stored with store_coherent (after the ticket).
__device__ __forceinline__ void acquire_coherent() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }

struct RowArgs {
  const void* logits;
  const void* ref_logits;  // nullptr => no reference pass
  const void* ids;
  const void* mask;        // nullptr => all ones
  const float* old_logp;   // nullptr => on-policy
  const float* adv;        // [n_seq]
  const float* seq_scale;  // [n_seq]: 1 / (loss_norm * max(sum mask, 1))
  void* dlogits;           // nullptr => forward only
  float* logp;
  float* ref_logp;
  float* token_loss;
  int* err;
  int* next_row;           // persistent row kernel: rows handed out past the first grid
  // Without zero-fill: the live rows' indices and their count, filled by
  // live_rows_kernel before the persistent row kernel, which then visits only those
  // rows. nullptr: every row in order.
  int* row_list;
  int* row_count;
  int64_t nrows;           // logits rows of the launch
  int64_t vocab;
  int64_t rows;
  int64_t logit_stride;
  int64_t tok_stride;
  int64_t tok_offset;
  int32_t ids_i64;
  int32_t mask_u8;
  int32_t loss_mode;
  int32_t zero_fill;
  int32_t counters_zeroed;  // next_row / row_count were zeroed earlier on the stream (step_prep_kernel)
  float clip_eps;
  float kl_beta;
};

struct RowMeta {
  int64_t row;   // logits row index
  int64_t tix;   // token index into ids/mask/per-token outputs (valid when tok)
  int64_t id;    // target token
  float w;       // mask weight
  int32_t seq;
  bool tok;      // row carries a token (t < rows)
  bool live;     // tok && w != 0 && id != ignore && id in range
};

__device__ __forceinline__ RowMeta row_meta(const RowArgs& a, int64_t row) {
  RowMeta r;
  r.row = row;
  const int64_t s = row / a.logit_stride;
  const int64_t t = row - s * a.logit_stride;
  r.seq = static_cast<int32_t>(s);
  r.tok = t < a.rows;
  r.tix = s * a.tok_stride + a.tok_offset + t;
  r.id = 0;
  r.w = 0.f;
  r.live = false;
  if (r.tok) {
    r.id = a.ids_i64 ? static_cast<const int64_t*>(a.ids)[r.tix]
                     : static_cast<int64_t>(static_cast<const int32_t*>(a.ids)[r.tix]);
    if (a.mask == nullptr) r.w = 1.f;
    else if (a.mask_u8) r.w = static_cast<const uint8_t*>(a.mask)[r.tix] ? 1.f : 0.f;
    else r.w = static_cast<const float*>(a.mask)[r.tix];
    const bool ignored = (r.id == PCP_IGNORE_INDEX);
    const bool in_range = (r.id >= 0) && (r.id < a.vocab);
    if (r.w != 0.f && !ignored && !in_range) {
      if (threadIdx.x == 0) atomicOr(a.err, kErrTokenRange);
    }
    r.live = (r.w != 0.f) && in_range;
  }
  return r;
}

// k3 KL estimator exp(d) - d - 1 without cancellation: for |d| < 0.5 the series
// d^2 * sum_k d^k / (k+2)! (truncated after d^7: relative error < 1e-9), else
// expm1(d) - d (cancellation below a factor of 4 there).
__device__ __forceinline__ float kl_k3(float d) {
  if (fabsf(d) < 0.5f) {
    float p = 1.f / 362880.f;
    p = fmaf(p, d, 1.f / 40320.f);
    p = fmaf(p, d, 1.f / 5040.f);
    p = fmaf(p, d, 1.f / 720.f);
    p = fmaf(p, d, 1.f / 120.f);
    p = fmaf(p, d, 1.f / 24.f);
    p = fmaf(p, d, 1.f / 6.f);
    p = fmaf(p, d, 0.5f);
    return d * d * p;
  }
  return expm1f(d) - d;
}

// Per-token loss term and d loss / d logp.
struct TokenTerms {
  float loss;  // m * l'
  float coef;  // c = d loss / d logp (already includes m / (loss_norm * L_s))
};

__device__ __forceinline__ TokenTerms token_terms(const RowArgs& a, const RowMeta& r, float lp,
                                                  float lr) {
  TokenTerms o;
  if (a.adv == nullptr) {  // forward-only request: no loss terms
    o.loss = 0.f;
    o.coef = 0.f;
    return o;
  }
  const float A = a.adv[r.seq];
  const float scale = a.seq_scale[r.seq] * r.w;
  if (a.loss_mode == PCP_LOSS_REINFORCE) {
    // token_losses = -logp * mask; seq_nll * adv; mean  (export_qwen_forward.py:156-163)
    o.loss = r.w * (-lp);
    o.coef = -A * scale;
  } else {
    const float old = a.old_logp ? a.old_logp[r.tix] : lp;
    const float rho = expf(lp - old);
    const float lo = 1.f - a.clip_eps, hi = 1.f + a.clip_eps;
    const float rc = fminf(fmaxf(rho, lo), hi);
    const float surr = fminf(rho * A, rc * A);
    const float dlr = lr - lp;
    o.loss = r.w * (-surr + a.kl_beta * kl_k3(dlr));
    // The min picks the unclipped branch (gradient -A*rho) unless the ratio left the
    // trust region on the side the advantage's sign rewards.
    const bool unclipped = (A >= 0.f) ? (rho <= hi) : (rho >= lo);
    const float dsurr = unclipped ? -A * rho : 0.f;
    // d k3 / d logp = 1 - exp(ref - logp) = -expm1(ref - logp)
    o.coef = scale * (dsurr - a.kl_beta * expm1f(dlr));
  }
  return o;
}

// Write per-token outputs of a token row (thread 0 only).
__device__ __forceinline__ void write_token_outputs(const RowArgs& a, const RowMeta& r, float lp,
                                                    float lr, float tl) {
  if (threadIdx.x != 0 || !r.tok) return;
  if (a.logp) a.logp[r.tix] = lp;
  if (a.ref_logp) a.ref_logp[r.tix] = lr;
  if (a.token_loss) a.token_loss[r.tix] = tl;
}

}  // namespace pcp
