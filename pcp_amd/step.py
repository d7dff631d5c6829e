"""Device-resident work around the loss head in one training step (include/pcp_step.h):
rollout packing, gradient statistics and the Nesterov update, over torch tensors in HBM.

Mirrors RLShepherd.trainStep (src/nodes/controllers/rl_shepherd.zig:487-515 packing,
:600-641 statistics, :643-682 update loop) and the host optimizer
(src/optimizers/nesterov.zig); the arithmetic runs in libpcp_grpo.so.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from ._lib import GradStats, NesterovMode, PcpError, check, lib
from .grpo import Context, _ptr, _stream_handle, default_context


def pack_rollouts(prompt_tokens: torch.Tensor, prompt_offsets: torch.Tensor, completion_tokens: torch.Tensor,
                  completion_offsets: torch.Tensor, n_rows: int, seq_len: int, *, stream=None,
                  ctx: Context | None = None):
    """Pack ragged rollouts (prompt then completion, truncated at seq_len) into
    ids int64 [n_rows, seq_len] and mask f32 [n_rows, seq_len] on the device."""
    dev = prompt_offsets.device
    ctx = ctx or default_context(dev.index or 0)
    for t in (prompt_tokens, prompt_offsets, completion_tokens, completion_offsets):
        if t.dtype != torch.int64:
            raise PcpError(-2, "token arrays and offsets must be int64")
    R = prompt_offsets.numel() - 1
    if completion_offsets.numel() != R + 1:
        raise PcpError(-1, "prompt and completion offsets differ in length")
    ids = torch.empty((n_rows, seq_len), dtype=torch.int64, device=dev)
    mask = torch.empty((n_rows, seq_len), dtype=torch.float32, device=dev)
    pt = _ptr(prompt_tokens) if prompt_tokens.numel() else None
    ct = _ptr(completion_tokens) if completion_tokens.numel() else None
    check(lib().pcp_pack_rollouts(ctx.handle, pt, prompt_tokens.numel(), _ptr(prompt_offsets), ct,
                                  completion_tokens.numel(), _ptr(completion_offsets), R, n_rows, seq_len,
                                  _ptr(ids), _ptr(mask), _stream_handle(stream)), ctx.handle)
    return ids, mask


def grad_stats(grads, *, stream=None, ctx: Context | None = None) -> dict:
    """rl_shepherd.zig:600-641 over one f32 tensor or a list of them."""
    grads = [grads] if isinstance(grads, torch.Tensor) else list(grads)
    ctx = ctx or default_context(grads[0].device.index or 0)
    st = GradStats()
    for i, g in enumerate(grads):
        if g.dtype != torch.float32:
            raise PcpError(-2, "gradients must be f32")
        check(lib().pcp_grad_stats_compute(ctx.handle, _ptr(g) if g.numel() else None, g.numel(), int(i > 0),
                                           ctypes.byref(st), _stream_handle(stream)), ctx.handle)
    return {"sumsq": st.sumsq, "l2_norm": st.l2_norm, "max_abs": st.max_abs, "nan_count": st.nan_count,
            "inf_count": st.inf_count, "elements": st.elements}


class Nesterov:
    """The reference's Nesterov optimizer (src/optimizers/nesterov.zig) with its
    velocities in HBM: init + initParameters -> __init__, update(index, param, grad),
    resetVelocity -> reset, serialize / deserialize; update_flat runs every tensor of a
    flat parameter buffer in one launch."""

    def __init__(self, counts, learning_rate: float = 0.01, momentum: float = 0.9,
                 mode: int = NesterovMode.sutskever, ctx: Context | None = None, device: int = 0):
        self.ctx = ctx or default_context(device)
        self.counts = [int(c) for c in counts]
        arr = (ctypes.c_int64 * len(self.counts))(*self.counts)
        h = ctypes.c_void_p()
        check(lib().pcp_nesterov_create(self.ctx.handle, float(learning_rate), float(momentum), int(mode),
                                        len(self.counts), arr, ctypes.byref(h)), self.ctx.handle)
        self.handle = h

    @property
    def total(self) -> int:
        return int(lib().pcp_nesterov_total(self.handle))

    def update(self, index: int, param: torch.Tensor, grad: torch.Tensor, stream=None) -> None:
        _f32(param, grad)
        check(lib().pcp_nesterov_update(self.handle, int(index), _ptr(param), _ptr(grad), param.numel(),
                                        _stream_handle(stream)), self.ctx.handle)

    def update_flat(self, params: torch.Tensor, grads: torch.Tensor, param_bf16: torch.Tensor | None = None,
                    stream=None) -> None:
        _f32(params, grads)
        if params.numel() != self.total or grads.numel() != self.total:
            raise PcpError(-12, f"flat buffers must hold {self.total} elements")
        if param_bf16 is not None and (param_bf16.dtype != torch.bfloat16 or param_bf16.numel() != self.total):
            raise PcpError(-2, "param_bf16 must be bf16 with one element per parameter")
        check(lib().pcp_nesterov_update_flat(self.handle, _ptr(params), _ptr(grads), _ptr(param_bf16),
                                             _stream_handle(stream)), self.ctx.handle)

    def reset(self) -> None:
        check(lib().pcp_nesterov_reset(self.handle, None), self.ctx.handle)

    def serialize(self) -> bytes:
        buf = np.empty(self.total, np.float32)
        check(lib().pcp_nesterov_serialize(self.handle, buf.ctypes.data if buf.size else None, buf.nbytes),
              self.ctx.handle)
        return buf.tobytes()

    def deserialize(self, data: bytes) -> None:
        raw = np.frombuffer(data, np.uint8) if len(data) else np.zeros(1, np.uint8)
        check(lib().pcp_nesterov_deserialize(self.handle, raw.ctypes.data, len(data)), self.ctx.handle)

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().pcp_nesterov_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _f32(*ts):
    for t in ts:
        if t.dtype != torch.float32:
            raise PcpError(-2, "parameters and gradients must be f32")


def sample_tokens(logits: torch.Tensor, temperature: float, uniforms: torch.Tensor | None = None, *,
                  ids: torch.Tensor | None = None, stream=None, ctx: Context | None = None,
                  sync: bool = True) -> torch.Tensor:
    """Sampler.sample (src/core/math.zig:21-58) on every row of logits [R, V] (f32 or
    bf16, HBM): greedy when temperature < 1e-6, else inverse-transform sampling with
    the caller's uniform draws (f32 [R] in [0, 1)). Returns int64 [R] token ids.
    sync=False only enqueues the launch on the stream (pcp_sample_tokens_async): the ids
    are ready in stream order, and ctx.sync() waits for them."""
    from ._lib import DType
    if logits.dim() != 2:
        raise PcpError(-1, "logits must be [rows, vocab]")
    code = {torch.float32: DType.f32, torch.bfloat16: DType.bf16}.get(logits.dtype)
    if code is None:
        raise PcpError(-2, "logits must be f32 or bf16")
    if logits.stride(1) != 1:
        raise PcpError(-1, "logits rows must be contiguous")
    R, V = logits.shape
    ctx = ctx or default_context(logits.device.index or 0)
    if ids is None:
        ids = torch.empty(R, dtype=torch.int64, device=logits.device)
    if uniforms is not None and (uniforms.dtype != torch.float32 or uniforms.numel() != R):
        raise PcpError(-1, "uniforms must be f32 with one value per row")
    fn = lib().pcp_sample_tokens if sync else lib().pcp_sample_tokens_async
    check(fn(ctx.handle, logits.data_ptr(), int(code), R, V, logits.stride(0), float(temperature), _ptr(uniforms),
             _ptr(ids), _stream_handle(stream)), ctx.handle)
    return ids
