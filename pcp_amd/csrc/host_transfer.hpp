// Host <-> device transfers of the host-bytes entry point (pcp_execute).
//
// The caller's inputs are ordinary (pageable) host memory, which the DMA engines cannot
// read directly: a plain hipMemcpy stages them through the runtime's buffers with one
// host thread (~10 GB/s). Here they are staged through a per-context ring of pinned
// buffers that several host threads fill while the DMA engine moves the previous chunk.
// Large outputs are written by DMA straight into pinned host buffers, which pcp_free
// recycles into a process-wide pool instead of freeing.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

struct pcp_ctx;

namespace pcp {

struct HostStager;

// Copy n bytes of pageable host memory at src to dev_dst, ordered on stream st. On
// return src may be reused; the device copy completes in stream order.
hipError_t upload_pageable(pcp_ctx* ctx, void* dev_dst, const void* src, size_t n, hipStream_t st);

// Release a context's staging ring (pcp_destroy).
void destroy_stager(pcp_ctx* ctx);

// Host buffer for an output of n bytes: pinned (pooled) above kPinnedOutMin bytes, else
// malloc. Returns nullptr when no memory is available.
void* host_out_alloc(size_t n);
// Return a buffer from host_out_alloc (pinned buffers go back to the pool).
void host_out_free(void* p);

}  // namespace pcp
