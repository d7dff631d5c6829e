// Library context and status helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>

#include "pcp_grpo.h"

namespace pcp {
struct HostStager;
}

struct pcp_ctx {
  int device = 0;
  int backend = PCP_BACKEND_ROCM;
  char last_error[512] = {};      // fixed buffer: reporting an error allocates nothing
  int* d_err = nullptr;          // device error word (kErr* bits)
  int* d_next_row = nullptr;     // row counter of the persistent row kernel (same allocation)
  void* scratch = nullptr;       // per-call work buffers, grown on demand
  size_t scratch_bytes = 0;
  // Streams holding PCP_FLAG_ASYNC work (a fixed set, so recording one allocates nothing).
  static constexpr int kMaxPending = 32;
  hipStream_t pending[kMaxPending] = {};
  int n_pending = 0;
  void* noalloc_scratch = nullptr;  // this device's static work array (pcp_grpo_loss_fwd_bwd_noalloc)
  // Row-kernel timing (pcp_profile_start/stop): event pairs, next free pair.
  std::vector<hipEvent_t> prof_start, prof_stop;
  int prof_used = 0;
  bool prof_on = false;
  void* lm_dbuf = nullptr;        // LM-head backward operand (softmax cache / dlogits chunk), grown on demand
  size_t lm_dbuf_bytes = 0;
  int* sample_ticket = nullptr;   // the sampler's per-row tickets (zero between launches)
  pcp::HostStager* stager = nullptr;  // pinned staging ring of the host-bytes path
  hipStream_t xs[3] = {};         // host-bytes path: upload, compute and download streams
};

namespace pcp {

// Last failure message of the calling thread (a thread-local 512-byte buffer);
// pcp_last_error(NULL) returns it, so argument errors are reported even when no
// context exists.
char* thread_error();
constexpr size_t kErrLen = 512;

// Copy the calling thread's last message into ctx (argument errors found before the
// context was known).
inline void copy_thread_error(pcp_ctx* ctx) {
  if (!ctx) return;
  std::strncpy(ctx->last_error, thread_error(), kErrLen - 1);
  ctx->last_error[kErrLen - 1] = 0;
}

inline int fail(pcp_ctx* ctx, int code, const char* fmt, ...) {
  char* buf = thread_error();
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, kErrLen, fmt, ap);
  va_end(ap);
  copy_thread_error(ctx);
  return code;
}

inline int hip_fail(pcp_ctx* ctx, hipError_t e, const char* what) {
  return fail(ctx, PCP_ERR_DEVICE, "%s: %s (%d)", what, hipGetErrorString(e), static_cast<int>(e));
}

inline bool mul_overflows(int64_t a, int64_t b, int64_t* out) {
  return __builtin_mul_overflow(a, b, out);
}

inline int dtype_bytes(int dt) {
  switch (dt) {
    case PCP_F16: return 2;
    case PCP_BF16: return 2;
    case PCP_F32: return 4;
    case PCP_F64: return 8;
    case PCP_I32: return 4;
    case PCP_I64: return 8;
    case PCP_BOOL: return 1;
  }
  return 0;
}

// Make `bytes` of scratch available on ctx (grow-only; synchronises before a free).
int ensure_scratch(pcp_ctx* ctx, size_t bytes);

// After synchronising: read and clear the device error word, map it to a status.
int collect_device_errors(pcp_ctx* ctx);

// Record a stream that holds PCP_FLAG_ASYNC work for pcp_sync. When the fixed set is
// full the stream is synchronised at once instead (its errors still reach pcp_sync
// through the error word).
int add_pending(pcp_ctx* ctx, hipStream_t st);

// pcp_profile_start/stop: HIP events around a timed launch on its stream. prof_begin
// returns whether this launch is timed (profiling on and an event pair left).
inline bool prof_begin(pcp_ctx* ctx, hipStream_t st) {
  const bool timed = ctx->prof_on && ctx->prof_used < static_cast<int>(ctx->prof_start.size());
  if (timed && hipEventRecord(ctx->prof_start[ctx->prof_used], st) != hipSuccess) return false;
  return timed;
}
inline void prof_end(pcp_ctx* ctx, hipStream_t st, bool timed) {
  if (timed && hipEventRecord(ctx->prof_stop[ctx->prof_used], st) == hipSuccess) ++ctx->prof_used;
}

}  // namespace pcp
