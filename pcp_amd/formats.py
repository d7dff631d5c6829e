"""On-disk and wire formats around the GRPO step (include/pcp_formats.h), read and
written straight from and to HBM: the prompt dataset (.bin of
tools/prepare_rl_dataset.py:28-40 / grpo.zig:63-91), the flat f32 master weights
(tools/convert_weights.py:39-44 / rl_shepherd.zig:141-229) and the base64
UPDATE_WEIGHTS payload (rl_shepherd.zig:691-711 / worker.zig:2631-2667)."""
from __future__ import annotations

import ctypes

import torch

from ._lib import PcpError, check, lib
from .grpo import Context, _ptr, _stream_handle, default_context


def prompt_counts(path: str) -> tuple[int, int]:
    """(number of prompts, total tokens) of a prompt dataset file (host only)."""
    n_p, n_t = ctypes.c_int64(), ctypes.c_int64()
    check(lib().pcp_prompts_load(None, path.encode(), None, 0, None, 0, ctypes.byref(n_p), ctypes.byref(n_t)))
    return n_p.value, n_t.value


def load_prompts(path: str, *, device: int = 0, ctx: Context | None = None):
    """Prompts as device tensors in the layout of pack_rollouts: tokens int64 [n_tokens]
    (concatenated) and offsets int64 [n_prompts + 1]."""
    ctx = ctx or default_context(device)
    n_p, n_t = prompt_counts(path)
    dev = torch.device("cuda", device)
    tokens = torch.empty(max(n_t, 1), dtype=torch.int64, device=dev)
    offsets = torch.empty(n_p + 1, dtype=torch.int64, device=dev)
    a, b = ctypes.c_int64(), ctypes.c_int64()
    check(lib().pcp_prompts_load(ctx.handle, path.encode(), tokens.data_ptr(), tokens.numel(), offsets.data_ptr(),
                                 offsets.numel(), ctypes.byref(a), ctypes.byref(b)), ctx.handle)
    return tokens[:n_t], offsets


def load_weights(path: str, counts, *, bf16: bool = False, device: int = 0, ctx: Context | None = None):
    """The flat f32 weight file into one device buffer (tensor i at the sum of the
    previous counts); with bf16=True also its bf16 copy. Returns (f32, bf16 or None)."""
    ctx = ctx or default_context(device)
    counts = [int(c) for c in counts]
    total = sum(counts)
    dev = torch.device("cuda", device)
    w = torch.empty(max(total, 1), dtype=torch.float32, device=dev)
    wb = torch.empty(max(total, 1), dtype=torch.bfloat16, device=dev) if bf16 else None
    arr = (ctypes.c_int64 * max(len(counts), 1))(*counts)
    check(lib().pcp_weights_load(ctx.handle, path.encode(), len(counts), arr, w.data_ptr(),
                                 wb.data_ptr() if wb is not None else None), ctx.handle)
    return w[:total], (wb[:total] if wb is not None else None)


def save_weights(path: str, weights: torch.Tensor, *, ctx: Context | None = None) -> None:
    if weights.dtype != torch.float32 or not weights.is_contiguous():
        raise PcpError(-2, "weights must be a contiguous f32 tensor")
    ctx = ctx or default_context(weights.device.index or 0)
    check(lib().pcp_weights_save(ctx.handle, path.encode(), _ptr(weights), weights.numel()), ctx.handle)


def b64encode(data: torch.Tensor, *, out: torch.Tensor | None = None, stream=None,
              ctx: Context | None = None) -> torch.Tensor:
    """Base64 (standard alphabet, '=' padding) of a device tensor's bytes, as a device
    uint8 tensor of characters (written into `out` when given: uint8, at least
    pcp_base64_encoded_len(nbytes) elements)."""
    if not data.is_contiguous():
        raise PcpError(-1, "data must be contiguous")
    ctx = ctx or default_context(data.device.index or 0)
    nbytes = data.numel() * data.element_size()
    n_out = int(lib().pcp_base64_encoded_len(nbytes))
    out = _out_bytes(out, n_out, data.device)
    check(lib().pcp_base64_encode(ctx.handle, data.data_ptr() if nbytes else None, nbytes, out.data_ptr(),
                                  _stream_handle(stream)), ctx.handle)
    return out[:n_out]


def b64decode(text: torch.Tensor, *, out: torch.Tensor | None = None, stream=None,
              ctx: Context | None = None) -> torch.Tensor:
    """Decode device base64 characters (uint8) into a device uint8 tensor (into `out`
    when given: uint8, at least len // 4 * 3 elements)."""
    if text.dtype != torch.uint8 or not text.is_contiguous():
        raise PcpError(-2, "text must be a contiguous uint8 tensor")
    ctx = ctx or default_context(text.device.index or 0)
    n = text.numel()
    out = _out_bytes(out, n // 4 * 3, text.device)
    got = ctypes.c_int64()
    check(lib().pcp_base64_decode(ctx.handle, text.data_ptr() if n else None, n, out.data_ptr(), ctypes.byref(got),
                                  _stream_handle(stream)), ctx.handle)
    return out[:got.value]


def _out_bytes(out: torch.Tensor | None, n: int, device) -> torch.Tensor:
    if out is None:
        return torch.empty(max(n, 1), dtype=torch.uint8, device=device)
    if out.dtype != torch.uint8 or not out.is_contiguous() or out.numel() < n or out.device != device:
        raise PcpError(-1, f"out must be a contiguous uint8 tensor of at least {n} elements on {device}")
    return out
