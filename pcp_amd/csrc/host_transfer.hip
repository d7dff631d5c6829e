// Host <-> device transfers of the host-bytes entry point: pinned staging ring for
// pageable inputs, pooled pinned buffers for large outputs, and a small pool of host
// threads for the staging copies.

#include "host_transfer.hpp"

#include <algorithm>
#include <condition_variable>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <thread>
#include <vector>

#include "context.hpp"

namespace pcp {

namespace {

constexpr size_t kChunk = size_t{64} << 20;          // bytes per staging slot
constexpr int kSlots = 3;                            // one filling, up to two in DMA flight
constexpr size_t kDirectMax = size_t{4} << 20;       // smaller inputs: one hipMemcpy
constexpr size_t kParallelMin = size_t{1} << 20;     // smaller host copies: one thread
constexpr size_t kPinnedOutMin = size_t{4} << 20;    // smaller outputs: malloc
constexpr size_t kPinnedRound = size_t{2} << 20;     // pinned capacities are multiples of this
constexpr size_t kPoolMaxBytes = size_t{64} << 30;   // idle pinned bytes kept for reuse

// A fixed set of host threads for large memcpy. copy() splits the range into one part
// per thread (the caller takes part 0) and returns when every part is done; calls
// from several threads take turns.
class CopyPool {
 public:
  static CopyPool& get() {
    static CopyPool* p = new CopyPool;   // never destroyed: workers may outlive static teardown
    return *p;
  }

  void copy(char* dst, const char* src, size_t n) {
    if (workers_.empty() || n < kParallelMin) {
      std::memcpy(dst, src, n);
      return;
    }
    std::lock_guard<std::mutex> turn(call_m_);
    const size_t parts = workers_.size() + 1;
    {
      std::lock_guard<std::mutex> lk(m_);
      dst_ = dst;
      src_ = src;
      n_ = n;
      per_ = ((n + parts - 1) / parts + 63) & ~size_t{63};
      left_ = workers_.size();
      ++gen_;
    }
    cv_.notify_all();
    part(0);
    std::unique_lock<std::mutex> lk(m_);
    done_cv_.wait(lk, [&] { return left_ == 0; });
  }

 private:
  CopyPool() {
    // At most 8 threads in all: the host share of one GPU, and enough to outrun one
    // DMA engine.
    const unsigned hw = std::thread::hardware_concurrency();
    const int n = hw >= 4 ? static_cast<int>(std::min(7u, hw / 2 - 1)) : 0;
    for (int i = 0; i < n; ++i) workers_.emplace_back([this, i] { run(static_cast<size_t>(i) + 1); });
    for (auto& t : workers_) t.detach();
  }

  void part(size_t k) const {
    const size_t b = std::min(n_, k * per_), e = std::min(n_, b + per_);
    if (e > b) std::memcpy(dst_ + b, src_ + b, e - b);
  }

  void run(size_t k) {
    uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> lk(m_);
        cv_.wait(lk, [&] { return gen_ != seen; });
        seen = gen_;
      }
      part(k);
      std::lock_guard<std::mutex> lk(m_);
      if (--left_ == 0) done_cv_.notify_one();
    }
  }

  std::mutex call_m_, m_;
  std::condition_variable cv_, done_cv_;
  std::vector<std::thread> workers_;
  char* dst_ = nullptr;
  const char* src_ = nullptr;
  size_t n_ = 0, per_ = 0, left_ = 0;
  uint64_t gen_ = 0;
};

// Pinned output buffers: handed out by host_out_alloc, recycled by host_out_free.
struct OutPool {
  std::mutex m;
  std::map<void*, size_t> live;          // handed out: buffer -> capacity
  std::multimap<size_t, void*> idle;     // capacity -> buffer
  size_t idle_bytes = 0;
};

OutPool& out_pool() {
  static OutPool* p = new OutPool;       // never destroyed: see CopyPool::get
  return *p;
}

}  // namespace

struct HostStager {
  char* slot[kSlots] = {};
  hipEvent_t done[kSlots] = {};
  bool busy[kSlots] = {};
  int next = 0;
};

namespace {

int make_stager(HostStager** out) {
  auto* s = new HostStager;
  for (int k = 0; k < kSlots; ++k) {
    void* p = nullptr;
    if (hipHostMalloc(&p, kChunk, hipHostMallocDefault) != hipSuccess ||
        hipEventCreateWithFlags(&s->done[k], hipEventDisableTiming) != hipSuccess) {
      if (p) (void)hipHostFree(p);
      for (int j = 0; j < k; ++j) {
        (void)hipHostFree(s->slot[j]);
        (void)hipEventDestroy(s->done[j]);
      }
      delete s;
      (void)hipGetLastError();
      return -1;
    }
    s->slot[k] = static_cast<char*>(p);
  }
  *out = s;
  return 0;
}

}  // namespace

hipError_t upload_pageable(pcp_ctx* ctx, void* dev_dst, const void* src, size_t n, hipStream_t st) {
  if (n <= kDirectMax) return hipMemcpy(dev_dst, src, n, hipMemcpyHostToDevice);
  if (!ctx->stager && make_stager(&ctx->stager) != 0) return hipMemcpy(dev_dst, src, n, hipMemcpyHostToDevice);
  HostStager* s = ctx->stager;
  const char* in = static_cast<const char*>(src);
  char* out = static_cast<char*>(dev_dst);
  for (size_t off = 0; off < n; off += kChunk) {
    const int k = s->next;
    s->next = (k + 1) % kSlots;
    if (s->busy[k]) {
      const hipError_t e = hipEventSynchronize(s->done[k]);   // the slot's previous DMA
      if (e != hipSuccess) return e;
    }
    const size_t len = std::min(kChunk, n - off);
    CopyPool::get().copy(s->slot[k], in + off, len);
    hipError_t e = hipMemcpyAsync(out + off, s->slot[k], len, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipEventRecord(s->done[k], st);
    if (e != hipSuccess) return e;
    s->busy[k] = true;
  }
  return hipSuccess;
}

void destroy_stager(pcp_ctx* ctx) {
  HostStager* s = ctx->stager;
  if (!s) return;
  for (int k = 0; k < kSlots; ++k) {
    if (s->busy[k]) (void)hipEventSynchronize(s->done[k]);
    (void)hipEventDestroy(s->done[k]);
    (void)hipHostFree(s->slot[k]);
  }
  delete s;
  ctx->stager = nullptr;
}

void* host_out_alloc(size_t n) {
  if (n < kPinnedOutMin) return std::malloc(n ? n : 1);
  OutPool& pool = out_pool();
  {
    std::lock_guard<std::mutex> lk(pool.m);
    auto it = pool.idle.lower_bound(n);
    if (it != pool.idle.end() && it->first <= 2 * n) {   // reuse a buffer at most twice the size
      void* p = it->second;
      pool.live[p] = it->first;
      pool.idle_bytes -= it->first;
      pool.idle.erase(it);
      return p;
    }
  }
  const size_t cap = (n + kPinnedRound - 1) / kPinnedRound * kPinnedRound;
  void* p = nullptr;
  if (hipHostMalloc(&p, cap, hipHostMallocDefault) != hipSuccess) {
    (void)hipGetLastError();
    return std::malloc(n);                                // pageable: slower to fill, same contract
  }
  std::lock_guard<std::mutex> lk(pool.m);
  pool.live[p] = cap;
  return p;
}

void host_out_free(void* p) {
  if (!p) return;
  OutPool& pool = out_pool();
  size_t cap = 0;
  {
    std::lock_guard<std::mutex> lk(pool.m);
    auto it = pool.live.find(p);
    if (it == pool.live.end()) {
      std::free(p);
      return;
    }
    cap = it->second;
    pool.live.erase(it);
    if (pool.idle_bytes + cap <= kPoolMaxBytes) {
      pool.idle.emplace(cap, p);
      pool.idle_bytes += cap;
      return;
    }
  }
  (void)hipHostFree(p);
}

}  // namespace pcp
