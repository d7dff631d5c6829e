// On-disk and wire formats around the GRPO step (pcp_formats.h), read and written
// straight from and to HBM: the prompt dataset, the flat f32 master weights and the
// base64 UPDATE_WEIGHTS payload.
//
// References: tools/prepare_rl_dataset.py:28-40 and GRPO.loadPrompts
// (src/algorithms/grpo.zig:63-91); tools/convert_weights.py:39-44 and
// RLShepherd.loadWeightsFromFile (src/nodes/controllers/rl_shepherd.zig:141-229);
// broadcastNewWeights (rl_shepherd.zig:691-711) and Worker.handleUpdateWeights
// (src/nodes/workers/worker.zig:2631-2667), std.base64.standard.

#include <hip/hip_runtime.h>

#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "context.hpp"
#include "grpo_device.hpp"
#include "pcp_formats.h"

namespace pcp {
namespace {

constexpr size_t kStage = size_t(64) << 20;   // pinned staging chunk for weight files

struct File {
  FILE* f = nullptr;
  ~File() {
    if (f) std::fclose(f);
  }
};

// ---- base64 ----------------------------------------------------------------------------------

constexpr int kUnits = 4;   // 12-byte / 16-character units per thread in the fast kernels

// Bytewise x >= k for four bytes at once (every byte of x <= 127, k in [1, 128]): bit 7
// of each byte. The addend keeps every byte below 256, so no carry crosses a byte.
__device__ __forceinline__ uint32_t bytes_ge(uint32_t x, uint32_t k) {
  return (x + 0x01010101u * (128u - k)) & 0x80808080u;
}

// A 24-bit group -> its four characters, the first in the low byte, without branches:
// 'A' + x, then +6 from x = 26 ('a'), -75 from 52 ('0'), -15 at 62 ('+'), +3 at 63 ('/').
// Added terms stay <= 137 per byte and each byte's subtrahend is below its minuend, so
// no carry or borrow crosses a byte.
__device__ __forceinline__ uint32_t b64_quad(uint32_t b0, uint32_t b1, uint32_t b2) {
  const uint32_t v = (b0 << 16) | (b1 << 8) | b2;
  const uint32_t x = (v >> 18) | (((v >> 12) & 63) << 8) | (((v >> 6) & 63) << 16) | ((v & 63) << 24);
  const uint32_t m26 = bytes_ge(x, 26) >> 7, m52 = bytes_ge(x, 52) >> 7, m62 = bytes_ge(x, 62) >> 7,
                 m63 = bytes_ge(x, 63) >> 7;
  return x + 0x41414141u + m26 * 6 + m63 * 3 - (m52 * 75 + m62 * 15);
}

// Four characters (first in the low byte) -> their 6-bit values, packed the same way,
// without branches; bit 7 of a byte of `bad` is set where the character is outside the
// alphabet ('=' included). Classes are disjoint ranges and a valid byte's subtrahend
// is at most its minuend, so no borrow crosses a byte.
__device__ __forceinline__ uint32_t b64_values4(uint32_t w, uint32_t& bad) {
  const uint32_t x = w & 0x7f7f7f7fu;
  const uint32_t up = bytes_ge(x, 'A') & ~bytes_ge(x, 'Z' + 1), lo = bytes_ge(x, 'a') & ~bytes_ge(x, 'z' + 1),
                 dg = bytes_ge(x, '0') & ~bytes_ge(x, '9' + 1), pl = bytes_ge(x, '+') & ~bytes_ge(x, '+' + 1),
                 sl = bytes_ge(x, '/') & ~bytes_ge(x, '/' + 1);
  bad |= ~(up | lo | dg | pl | sl) | (w & 0x80808080u);
  const uint32_t add = (dg >> 7) * 4 + (pl >> 7) * 19 + (sl >> 7) * 16;
  const uint32_t sub = (up >> 7) * 65 + (lo >> 7) * 71;
  return x + add - sub;
}

// Four packed 6-bit values -> the 24-bit group they spell.
__device__ __forceinline__ uint32_t b64_group(uint32_t val) {
  return ((val & 63) << 18) | (((val >> 8) & 63) << 12) | (((val >> 16) & 63) << 6) | ((val >> 24) & 63);
}

// Fast encode over whole 12-byte units (src 4-byte aligned, dst 16-byte aligned): a lane
// loads one unit as three dwords and stores its 16 characters as one quad, so each wave
// instruction covers a contiguous 768-byte read or 1024-byte write. kUnits units per
// lane, 256 units apart, keep several loads in flight.
__global__ void __launch_bounds__(256) b64_encode_kernel(const uint32_t* __restrict__ src, int64_t nunits,
                                                         u32x4* __restrict__ dst) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * 256 * kUnits + threadIdx.x;
  uint32_t w[kUnits][3];
#pragma unroll
  for (int u = 0; u < kUnits; ++u) {
    const int64_t i = base + u * 256;
    if (i < nunits) {
      w[u][0] = __builtin_nontemporal_load(src + 3 * i);
      w[u][1] = __builtin_nontemporal_load(src + 3 * i + 1);
      w[u][2] = __builtin_nontemporal_load(src + 3 * i + 2);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnits; ++u) {
    const int64_t i = base + u * 256;
    if (i < nunits) {
      const uint32_t a = w[u][0], b = w[u][1], c = w[u][2];
      u32x4 o;
      o.x = b64_quad(a & 255, (a >> 8) & 255, (a >> 16) & 255);
      o.y = b64_quad(a >> 24, b & 255, (b >> 8) & 255);
      o.z = b64_quad((b >> 16) & 255, b >> 24, c & 255);
      o.w = b64_quad((c >> 8) & 255, (c >> 16) & 255, c >> 24);
      __builtin_nontemporal_store(o, dst + i);
    }
  }
}

// Groups [g0, ngroups) one per thread, byte by byte: the tail after the fast kernel, the
// final 1- or 2-byte group with '=' padding, and buffers the fast kernel's alignment
// excludes.
__global__ void __launch_bounds__(256) b64_encode_groups_kernel(const uint8_t* src, int64_t nbytes, int64_t g0,
                                                                uint8_t* dst) {
  const int64_t ngroups = (nbytes + 2) / 3;
  for (int64_t g = g0 + static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; g < ngroups;
       g += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t k = nbytes - 3 * g;   // bytes left from this group on: 1, 2 or >= 3
    const uint32_t b0 = src[3 * g], b1 = k > 1 ? src[3 * g + 1] : 0, b2 = k > 2 ? src[3 * g + 2] : 0;
    const uint32_t q = b64_quad(b0, b1, b2);
    dst[4 * g] = static_cast<uint8_t>(q);
    dst[4 * g + 1] = static_cast<uint8_t>(q >> 8);
    dst[4 * g + 2] = k > 1 ? static_cast<uint8_t>(q >> 16) : '=';
    dst[4 * g + 3] = k > 2 ? static_cast<uint8_t>(q >> 24) : '=';
  }
}

// Fast decode over whole 16-character units before the final quad (src 16-byte aligned,
// dst 4-byte aligned): one quad load and three dword stores per lane, contiguous across
// the wave. A character outside the alphabet sets kErrBadBase64.
__global__ void __launch_bounds__(256) b64_decode_kernel(const u32x4* __restrict__ src, int64_t nunits,
                                                         uint32_t* __restrict__ dst, int* err) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * 256 * kUnits + threadIdx.x;
  u32x4 w[kUnits];
#pragma unroll
  for (int u = 0; u < kUnits; ++u) {
    const int64_t i = base + u * 256;
    if (i < nunits) w[u] = __builtin_nontemporal_load(src + i);
  }
  uint32_t bad = 0;
#pragma unroll
  for (int u = 0; u < kUnits; ++u) {
    const int64_t i = base + u * 256;
    if (i < nunits) {
      const uint32_t v0 = b64_group(b64_values4(w[u].x, bad)), v1 = b64_group(b64_values4(w[u].y, bad)),
                     v2 = b64_group(b64_values4(w[u].z, bad)), v3 = b64_group(b64_values4(w[u].w, bad));
      // bytes of v0 (big-endian 24-bit), then v1, v2, v3, packed little-endian
      const uint32_t a = ((v0 >> 16) & 255) | (((v0 >> 8) & 255) << 8) | ((v0 & 255) << 16) | (((v1 >> 16) & 255) << 24);
      const uint32_t b = ((v1 >> 8) & 255) | ((v1 & 255) << 8) | (((v2 >> 16) & 255) << 16) | (((v2 >> 8) & 255) << 24);
      const uint32_t c = (v2 & 255) | (((v3 >> 16) & 255) << 8) | (((v3 >> 8) & 255) << 16) | ((v3 & 255) << 24);
      // Three dword stores 12 bytes apart per lane, nontemporal at device scope: at system
      // scope (store_nt_sys, written through in pieces of lines) the decode ran 3.5x slower.
      __builtin_nontemporal_store(a, dst + 3 * i);
      __builtin_nontemporal_store(b, dst + 3 * i + 1);
      __builtin_nontemporal_store(c, dst + 3 * i + 2);
    }
  }
  if (bad & 0x80808080u) atomicOr(err, kErrBadBase64);
}

// Quads [q0, nq) one per thread: the tail after the fast kernel and unaligned buffers.
// The final quad may carry padding, "xx==" (1 byte) or "xxx=" (2 bytes), and the bits
// below its last character must be zero (std.base64: InvalidPadding otherwise).
__global__ void __launch_bounds__(256) b64_decode_quads_kernel(const uint8_t* src, int64_t nq, int64_t q0,
                                                               uint8_t* dst, int* err) {
  uint32_t bad = 0;
  for (int64_t q = q0 + static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; q < nq;
       q += static_cast<int64_t>(gridDim.x) * 256) {
    const uint32_t c0 = src[4 * q], c1 = src[4 * q + 1];
    uint32_t c2 = src[4 * q + 2], c3 = src[4 * q + 3];
    int p = 0;
    if (q == nq - 1 && c3 == '=') p = c2 == '=' ? 2 : 1;
    if (p == 2) c2 = 'A';                // 'A' stands for the zero value of a padding position
    if (p >= 1) c3 = 'A';
    const uint32_t v = b64_group(b64_values4(c0 | (c1 << 8) | (c2 << 16) | (c3 << 24), bad));
    if (p == 2) bad |= (v & 0xFFFFu) ? 0x80u : 0u;   // leftover bits of "xx=="
    if (p == 1) bad |= (v & 0xFFu) ? 0x80u : 0u;     // leftover bits of "xxx="
    dst[3 * q] = static_cast<uint8_t>(v >> 16);
    if (p < 2) dst[3 * q + 1] = static_cast<uint8_t>(v >> 8);
    if (p < 1) dst[3 * q + 2] = static_cast<uint8_t>(v);
  }
  if (bad & 0x80808080u) atomicOr(err, kErrBadBase64);
}

// ---- weights ------------------------------------------------------------------------------------

__global__ void __launch_bounds__(256) to_bf16_kernel(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    y[i] = static_cast<uint16_t>(pack2<BF16T>(x[i], 0.f) & 0xFFFFu);
}

unsigned grid_for(int64_t n, int64_t per_block) {
  int64_t b = (n + per_block - 1) / per_block;
  if (b < 1) b = 1;
  if (b > 65536) b = 65536;
  return static_cast<unsigned>(b);
}

int io_fail(pcp_ctx* ctx, const char* what, const char* path) {
  return fail(ctx, PCP_ERR_IO, "%s %s: %s", what, path, std::strerror(errno));
}

}  // namespace
}  // namespace pcp

using namespace pcp;

extern "C" {

int pcp_prompts_load(pcp_ctx* ctx, const char* path, int64_t* tokens, int64_t tokens_cap, int64_t* offsets,
                     int64_t offsets_cap, int64_t* n_prompts, int64_t* n_tokens) {
  if (!path || !n_prompts || !n_tokens) return fail(ctx, PCP_ERR_INVALID_ARG, "path / n_prompts / n_tokens is NULL");
  File f;
  f.f = std::fopen(path, "rb");
  if (!f.f) return io_fail(ctx, "opening", path);
  std::vector<uint8_t> buf;
  uint8_t chunk[1 << 16];
  size_t got;
  while ((got = std::fread(chunk, 1, sizeof(chunk), f.f)) > 0) buf.insert(buf.end(), chunk, chunk + got);
  if (std::ferror(f.f)) return io_fail(ctx, "reading", path);
  size_t pos = 0;
  auto u32 = [&](uint32_t* v) {
    if (pos + 4 > buf.size()) return false;
    *v = uint32_t(buf[pos]) | uint32_t(buf[pos + 1]) << 8 | uint32_t(buf[pos + 2]) << 16 | uint32_t(buf[pos + 3]) << 24;
    pos += 4;
    return true;
  };
  uint32_t count;
  if (!u32(&count)) return fail(ctx, PCP_ERR_CORRUPT_STATE, "%s ends before its prompt count", path);
  std::vector<int64_t> off(1, 0), tok;
  for (uint32_t i = 0; i < count; ++i) {
    uint32_t n;
    if (!u32(&n)) return fail(ctx, PCP_ERR_CORRUPT_STATE, "%s ends inside prompt %u", path, i);
    if (pos + uint64_t(n) * 8 > buf.size()) return fail(ctx, PCP_ERR_CORRUPT_STATE, "%s ends inside prompt %u", path, i);
    for (uint32_t j = 0; j < n; ++j) {
      uint64_t v = 0;
      for (int b = 7; b >= 0; --b) v = (v << 8) | buf[pos + b];
      pos += 8;
      if (v > uint64_t(INT64_MAX)) return fail(ctx, PCP_ERR_OVERFLOW, "token %llu of prompt %u exceeds 2^63 - 1",
                                              (unsigned long long)v, i);
      tok.push_back(static_cast<int64_t>(v));
    }
    off.push_back(static_cast<int64_t>(tok.size()));
  }
  *n_prompts = count;
  *n_tokens = static_cast<int64_t>(tok.size());
  if (!tokens || !offsets) return PCP_OK;
  if (tokens_cap < *n_tokens || offsets_cap < *n_prompts + 1)
    return fail(ctx, PCP_ERR_OVERFLOW, "buffers hold %lld tokens / %lld offsets, the file needs %lld / %lld",
                (long long)tokens_cap, (long long)offsets_cap, (long long)*n_tokens, (long long)*n_prompts + 1);
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess && !tok.empty()) e = hipMemcpy(tokens, tok.data(), 8 * tok.size(), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(offsets, off.data(), 8 * off.size(), hipMemcpyHostToDevice);
  return e == hipSuccess ? PCP_OK : hip_fail(ctx, e, "uploading prompts");
}

int pcp_weights_load(pcp_ctx* ctx, const char* path, int n_tensors, const int64_t* counts, float* dev, void* bf16) {
  if (!path || n_tensors < 0 || (n_tensors > 0 && !counts)) return fail(ctx, PCP_ERR_INVALID_ARG, "path / counts is NULL");
  int64_t total = 0;
  for (int i = 0; i < n_tensors; ++i) {
    if (counts[i] < 0) return fail(ctx, PCP_ERR_INVALID_ARG, "counts[%d] < 0", i);
    if (total > (int64_t(1) << 40) - counts[i]) return fail(ctx, PCP_ERR_OVERFLOW, "more than 2^40 parameters");
    total += counts[i];
  }
  if (total > 0 && !dev) return fail(ctx, PCP_ERR_INVALID_ARG, "dev is NULL");
  File f;
  f.f = std::fopen(path, "rb");
  if (!f.f) return io_fail(ctx, "opening", path);
  if (std::fseek(f.f, 0, SEEK_END) != 0) return io_fail(ctx, "seeking", path);
  const long long size = std::ftell(f.f);
  if (size < 0 || std::fseek(f.f, 0, SEEK_SET) != 0) return io_fail(ctx, "seeking", path);
  if (static_cast<long long>(total) * 4 > size)
    return fail(ctx, PCP_ERR_CORRUPT_STATE, "%s holds %lld bytes, the tensors need %lld (WeightFileTooSmall)", path,
                size, (long long)total * 4);
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  // Two pinned chunks: the file read into one overlaps the copy out of the other.
  void* pin[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  hipStream_t st = nullptr;
  int rc = PCP_OK;
  const size_t bytes = static_cast<size_t>(total) * 4;
  for (int i = 0; i < 2 && rc == PCP_OK; ++i) {
    if ((e = hipHostMalloc(&pin[i], kStage)) != hipSuccess) rc = hip_fail(ctx, e, "hipHostMalloc");
    else if ((e = hipEventCreate(&done[i])) != hipSuccess) rc = hip_fail(ctx, e, "hipEventCreate");
  }
  if (rc == PCP_OK && (e = hipStreamCreate(&st)) != hipSuccess) rc = hip_fail(ctx, e, "hipStreamCreate");
  size_t off = 0;
  for (int k = 0; rc == PCP_OK && off < bytes; ++k) {
    const int b = k & 1;
    const size_t n = bytes - off < kStage ? bytes - off : kStage;
    if ((e = hipEventSynchronize(done[b])) != hipSuccess) {   // the copy out of this chunk has finished
      rc = hip_fail(ctx, e, "hipEventSynchronize");
      break;
    }
    if (std::fread(pin[b], 1, n, f.f) != n) {
      rc = io_fail(ctx, "reading", path);
      break;
    }
    char* d = reinterpret_cast<char*>(dev) + off;
    if ((e = hipMemcpyAsync(d, pin[b], n, hipMemcpyHostToDevice, st)) != hipSuccess ||
        (e = hipEventRecord(done[b], st)) != hipSuccess) {
      rc = hip_fail(ctx, e, "copying weights");
      break;
    }
    if (bf16) {
      const int64_t e0 = static_cast<int64_t>(off / 4), ne = static_cast<int64_t>(n / 4);
      to_bf16_kernel<<<grid_for(ne, 256 * 8), 256, 0, st>>>(dev + e0, static_cast<uint16_t*>(bf16) + e0, ne);
      if ((e = hipGetLastError()) != hipSuccess) {
        rc = hip_fail(ctx, e, "bf16 copy");
        break;
      }
    }
    off += n;
  }
  if (st && (e = hipStreamSynchronize(st)) != hipSuccess && rc == PCP_OK) rc = hip_fail(ctx, e, "hipStreamSynchronize");
  if (st) (void)hipStreamDestroy(st);
  for (int i = 0; i < 2; ++i) {
    if (done[i]) (void)hipEventDestroy(done[i]);
    if (pin[i]) (void)hipHostFree(pin[i]);
  }
  return rc;
}

int pcp_weights_save(pcp_ctx* ctx, const char* path, const float* dev, int64_t n) {
  if (!path || n < 0 || (n > 0 && !dev)) return fail(ctx, PCP_ERR_INVALID_ARG, "path / dev is NULL or n < 0");
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  File f;
  f.f = std::fopen(path, "wb");
  if (!f.f) return io_fail(ctx, "creating", path);
  void* pin = nullptr;
  if ((e = hipHostMalloc(&pin, kStage)) != hipSuccess) return hip_fail(ctx, e, "hipHostMalloc");
  int rc = PCP_OK;
  const size_t bytes = static_cast<size_t>(n) * 4;
  for (size_t off = 0; off < bytes;) {
    const size_t k = bytes - off < kStage ? bytes - off : kStage;
    if ((e = hipMemcpy(pin, reinterpret_cast<const char*>(dev) + off, k, hipMemcpyDeviceToHost)) != hipSuccess) {
      rc = hip_fail(ctx, e, "copying weights");
      break;
    }
    if (std::fwrite(pin, 1, k, f.f) != k) {
      rc = io_fail(ctx, "writing", path);
      break;
    }
    off += k;
  }
  (void)hipHostFree(pin);
  if (rc == PCP_OK && std::fflush(f.f) != 0) rc = io_fail(ctx, "writing", path);
  return rc;
}

int64_t pcp_base64_encoded_len(int64_t nbytes) { return nbytes < 0 ? PCP_ERR_INVALID_ARG : (nbytes + 2) / 3 * 4; }

int pcp_base64_encode(pcp_ctx* ctx, const void* src, int64_t nbytes, char* dst, void* stream) {
  if (nbytes < 0 || (nbytes > 0 && (!src || !dst))) return fail(ctx, PCP_ERR_INVALID_ARG, "src / dst is NULL or nbytes < 0");
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  if (nbytes == 0) return PCP_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool aligned = (reinterpret_cast<uintptr_t>(src) & 3u) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0;
  const int64_t nunits = aligned ? nbytes / 12 : 0;
  const bool timed = prof_begin(ctx, st);
  if (nunits > 0)
    b64_encode_kernel<<<static_cast<unsigned>((nunits + 256 * kUnits - 1) / (256 * kUnits)), 256, 0, st>>>(
        static_cast<const uint32_t*>(src), nunits, reinterpret_cast<u32x4*>(dst));
  const int64_t g0 = 4 * nunits, ngroups = (nbytes + 2) / 3;
  if (g0 < ngroups)
    b64_encode_groups_kernel<<<grid_for(ngroups - g0, 256), 256, 0, st>>>(static_cast<const uint8_t*>(src), nbytes, g0,
                                                                          reinterpret_cast<uint8_t*>(dst));
  prof_end(ctx, st, timed);
  if ((e = hipGetLastError()) != hipSuccess) return hip_fail(ctx, e, "base64 launch");
  if ((e = hipStreamSynchronize(st)) != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  return PCP_OK;
}

int pcp_base64_decode(pcp_ctx* ctx, const char* src, int64_t len, void* dst, int64_t* nbytes, void* stream) {
  if (!nbytes || len < 0 || (len > 0 && (!src || !dst))) return fail(ctx, PCP_ERR_INVALID_ARG, "src / dst / nbytes is NULL");
  *nbytes = 0;
  if (len % 4) return fail(ctx, PCP_ERR_INVALID_ARG, "base64 length %lld is not a multiple of 4 (InvalidPadding)",
                           (long long)len);
  if (!ctx) return fail(nullptr, PCP_ERR_INVALID_ARG, "context is NULL");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  if (len == 0) return PCP_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  char tail[2];
  if ((e = hipMemcpyAsync(tail, src + len - 2, 2, hipMemcpyDeviceToHost, st)) != hipSuccess ||
      (e = hipStreamSynchronize(st)) != hipSuccess)
    return hip_fail(ctx, e, "reading the padding");
  const int pad = tail[1] == '=' ? (tail[0] == '=' ? 2 : 1) : (tail[0] == '=' ? -1 : 0);
  if (pad < 0) return fail(ctx, PCP_ERR_INVALID_ARG, "'=' before a non-padding character (InvalidPadding)");
  const int64_t nq = len / 4;
  const bool aligned = (reinterpret_cast<uintptr_t>(src) & 15u) == 0 && (reinterpret_cast<uintptr_t>(dst) & 3u) == 0;
  const int64_t nunits = aligned ? (nq - 1) / 4 : 0;   // the final quad (padding) always takes the byte path
  const bool timed = prof_begin(ctx, st);
  if (nunits > 0)
    b64_decode_kernel<<<static_cast<unsigned>((nunits + 256 * kUnits - 1) / (256 * kUnits)), 256, 0, st>>>(
        reinterpret_cast<const u32x4*>(src), nunits, static_cast<uint32_t*>(dst), ctx->d_err);
  b64_decode_quads_kernel<<<grid_for(nq - 4 * nunits, 256), 256, 0, st>>>(
      reinterpret_cast<const uint8_t*>(src), nq, 4 * nunits, static_cast<uint8_t*>(dst), ctx->d_err);
  prof_end(ctx, st, timed);
  if ((e = hipGetLastError()) != hipSuccess) return hip_fail(ctx, e, "base64 launch");
  if ((e = hipStreamSynchronize(st)) != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  const int rc = collect_device_errors(ctx);
  if (rc != PCP_OK) return rc;
  *nbytes = nq * 3 - pad;
  return PCP_OK;
}

}  // extern "C"
