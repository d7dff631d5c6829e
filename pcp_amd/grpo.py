"""Device-pointer API of the GRPO loss head over torch tensors resident in HBM.

torch provides device memory and the stream; all arithmetic runs in the HIP
kernels of libpcp_grpo.so. Layout (see include/pcp_grpo.h): logits [S, LS, V];
token arrays [S, TS]; row (s, t), t < rows, scores ids[s, tok_offset + t].
The aligned layout is rows = LS = TS, tok_offset = 0; the reference's shifted
layout (tools/export_qwen_forward.py:150-152) is rows = T-1, LS = TS = T,
tok_offset = 1.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import DType, LossMode, PcpError, check, lib

_TORCH_DTYPE = {
    torch.bfloat16: DType.bf16,
    torch.float16: DType.f16,
    torch.float32: DType.f32,
    torch.int64: DType.i64,
    torch.int32: DType.i32,
    torch.bool: DType.bool,
    torch.uint8: DType.bool,
}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return int(_TORCH_DTYPE[t.dtype])
    except KeyError:
        raise PcpError(-2, f"unsupported tensor dtype {t.dtype}") from None


class Context:
    """An initialised device context (~ IreeBackend.init(.rocm, device_id), iree.zig:84)."""

    def __init__(self, device_ordinal: int = 0):
        h = ctypes.c_void_p()
        check(lib().pcp_init(int(_lib.Backend.rocm), device_ordinal, ctypes.byref(h)))
        self.handle = h
        self.device = device_ordinal

    def close(self) -> None:
        if self.handle:
            lib().pcp_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sync(self) -> None:
        check(lib().pcp_sync(self.handle), self.handle)

    def release_workspace(self) -> None:
        """Free the context's device work buffers (the LM-head softmax cache among them);
        synchronises the device first. The next call allocates again."""
        check(lib().pcp_release_workspace(self.handle), self.handle)

    def workspace_bytes(self) -> int:
        """Bytes of device work buffers the context holds now."""
        return int(lib().pcp_workspace_bytes(self.handle))


_default_ctx: dict[int, Context] = {}


def default_context(device: int = 0) -> Context:
    if device not in _default_ctx:
        _default_ctx[device] = Context(device)
    return _default_ctx[device]


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise PcpError(-1, "tensor is not on the GPU")
    if not t.is_contiguous():
        raise PcpError(-1, "tensor is not contiguous")
    return t.data_ptr()


def _stream_handle(stream) -> int | None:
    """A torch stream, a raw hipStream_t handle (int) or None (torch's current stream)."""
    if isinstance(stream, int):
        return stream or None
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream or None


@dataclass
class GrpoOutputs:
    loss: torch.Tensor          # f32 scalar
    dlogits: torch.Tensor | None
    logp: torch.Tensor          # [S, TS] f32
    ref_logp: torch.Tensor | None
    token_loss: torch.Tensor    # [S, TS] f32
    advantages: torch.Tensor    # [S] f32


def _layout(logits, ids, rows, tok_offset):
    if logits.dim() != 3:
        raise PcpError(-1, "logits must be [S, LS, V]")
    if ids.dim() != 2 or ids.shape[0] != logits.shape[0]:
        raise PcpError(-1, "ids must be [S, TS] with the same S as logits")
    S, LS, V = logits.shape
    TS = ids.shape[1]
    rows = LS if rows is None else int(rows)
    return S, LS, V, TS, rows, int(tok_offset)


def fill_args(a: _lib.GrpoArgs, logits, ids, mask, rows, tok_offset, S, LS, V, TS) -> None:
    a.n_seq, a.rows, a.vocab = S, rows, V
    a.logit_seq_stride, a.tok_seq_stride, a.tok_offset = LS, TS, tok_offset
    a.logits_dtype = dtype_code(logits)
    a.ids_dtype = dtype_code(ids)
    a.logits = _ptr(logits)
    a.ids = _ptr(ids)
    if mask is not None:
        a.mask = _ptr(mask)
        a.mask_dtype = dtype_code(mask)


def grpo_loss_fwd_bwd(logits: torch.Tensor, ids: torch.Tensor, mask: torch.Tensor | None = None, *,
                      advantages: torch.Tensor | None = None, rewards: torch.Tensor | None = None,
                      group_size: int = 1, ref_logits: torch.Tensor | None = None,
                      old_logp: torch.Tensor | None = None, loss_mode: int = LossMode.REINFORCE,
                      clip_eps: float = 0.2, kl_beta: float = 0.04, loss_norm: float = 0.0,
                      std_eps: float = 1e-8, rows: int | None = None, tok_offset: int = 0,
                      want_dlogits: bool = True, dlogits: torch.Tensor | None = None,
                      dlogits_dtype: torch.dtype | None = None, zero_fill: bool = True,
                      force_streaming: bool = False, exact_bf16: bool = False,
                      outputs: GrpoOutputs | None = None, sync: bool = True, stream=None,
                      ctx: Context | None = None, noalloc: bool = False) -> GrpoOutputs:
    """Fused loss forward + dlogits backward (pcp_grpo_loss_fwd_bwd).

    Pass ``outputs`` (from a previous call of the same shape) to reuse its buffers
    instead of allocating: the benchmark does this so the timed region only runs
    the kernels. ``noalloc`` calls pcp_grpo_loss_fwd_bwd_noalloc, whose work buffers
    are the GPU's static array instead of the context's.
    """
    ctx = ctx or default_context(logits.device.index or 0)
    S, LS, V, TS, rows, tok_offset = _layout(logits, ids, rows, tok_offset)
    dev = logits.device
    if outputs is None:
        if want_dlogits and dlogits is None:
            dlogits = torch.empty((S, LS, V), dtype=dlogits_dtype or logits.dtype, device=dev)
        outputs = GrpoOutputs(
            loss=torch.zeros((), dtype=torch.float32, device=dev),
            dlogits=dlogits if want_dlogits else None,
            logp=torch.zeros((S, TS), dtype=torch.float32, device=dev),
            ref_logp=torch.zeros((S, TS), dtype=torch.float32, device=dev) if ref_logits is not None else None,
            token_loss=torch.zeros((S, TS), dtype=torch.float32, device=dev),
            advantages=torch.zeros((S,), dtype=torch.float32, device=dev))
    a = _lib.default_args()
    fill_args(a, logits, ids, mask, rows, tok_offset, S, LS, V, TS)
    a.group_size = int(group_size)
    a.ref_logits = _ptr(ref_logits)
    a.old_logp = _ptr(old_logp)
    a.advantages = _ptr(advantages)
    a.rewards = _ptr(rewards)
    a.dlogits = _ptr(outputs.dlogits)
    a.dlogits_dtype = dtype_code(outputs.dlogits) if outputs.dlogits is not None else a.logits_dtype
    a.logp = _ptr(outputs.logp)
    a.ref_logp = _ptr(outputs.ref_logp)
    a.token_loss = _ptr(outputs.token_loss)
    a.advantages_out = _ptr(outputs.advantages)
    a.loss = _ptr(outputs.loss)
    a.loss_mode = int(loss_mode)
    a.clip_eps, a.kl_beta, a.std_eps, a.loss_norm = clip_eps, kl_beta, std_eps, loss_norm
    a.flags = ((0 if sync else _lib.FLAG_ASYNC) | (0 if zero_fill else _lib.FLAG_NO_ZERO_FILL)
               | (_lib.FLAG_FORCE_STREAMING if force_streaming else 0)
               | (_lib.FLAG_EXACT_BF16 if exact_bf16 else 0))
    a.stream = _stream_handle(stream)
    fn = lib().pcp_grpo_loss_fwd_bwd_noalloc if noalloc else lib().pcp_grpo_loss_fwd_bwd
    check(fn(ctx.handle, ctypes.byref(a)), ctx.handle)
    return outputs


def logprob_fwd(logits: torch.Tensor, ids: torch.Tensor, ref_logits: torch.Tensor | None = None, *,
                rows: int | None = None, tok_offset: int = 0, mask: torch.Tensor | None = None,
                force_streaming: bool = False, sync: bool = True, stream=None, ctx: Context | None = None):
    """Per-token log-probs of ids under logits (and ref_logits): pcp_grpo_logprob_fwd.
    Returns (logp, ref_logp or None), each [S, TS] f32."""
    ctx = ctx or default_context(logits.device.index or 0)
    S, LS, V, TS, rows, tok_offset = _layout(logits, ids, rows, tok_offset)
    logp = torch.zeros((S, TS), dtype=torch.float32, device=logits.device)
    ref_logp = torch.zeros_like(logp) if ref_logits is not None else None
    a = _lib.default_args()
    fill_args(a, logits, ids, mask, rows, tok_offset, S, LS, V, TS)
    a.ref_logits = _ptr(ref_logits)
    a.logp = _ptr(logp)
    a.ref_logp = _ptr(ref_logp)
    a.flags = (0 if sync else _lib.FLAG_ASYNC) | (_lib.FLAG_FORCE_STREAMING if force_streaming else 0)
    a.stream = _stream_handle(stream)
    check(lib().pcp_grpo_logprob_fwd(ctx.handle, ctypes.byref(a)), ctx.handle)
    return logp, ref_logp


def advantages(rewards: torch.Tensor, group_size: int, std_eps: float = 1e-8, *, stream=None,
               ctx: Context | None = None) -> torch.Tensor:
    """Group-relative advantages on the device (bit-exact with rl_shepherd.zig:462-479)."""
    ctx = ctx or default_context(rewards.device.index or 0)
    if rewards.dtype != torch.float32 or rewards.dim() != 1:
        raise PcpError(-2, "rewards must be a 1-D float32 tensor")
    out = torch.empty_like(rewards)
    check(lib().pcp_grpo_advantages(ctx.handle, _ptr(rewards), rewards.numel(), int(group_size),
                                    ctypes.c_float(std_eps), _ptr(out), _stream_handle(stream)), ctx.handle)
    return out


@dataclass
class LmheadOutputs:
    loss: torch.Tensor          # f32 scalar
    logp: torch.Tensor          # [S, T] f32
    ref_logp: torch.Tensor | None
    token_loss: torch.Tensor    # [S, T] f32
    advantages: torch.Tensor    # [S] f32
    dhidden: torch.Tensor | None  # [S*T, H] f32 (dL/dh before the final norm when it is fused)
    dweight: torch.Tensor | None  # [V, H] f32
    dnorm_weight: torch.Tensor | None = None  # [H] f32, with the fused final norm


def lmhead_fwd_bwd(hidden: torch.Tensor, weight: torch.Tensor, ids: torch.Tensor, mask: torch.Tensor | None = None,
                   *, ref_weight: torch.Tensor | None = None, advantages: torch.Tensor | None = None,
                   rewards: torch.Tensor | None = None, group_size: int = 1, old_logp: torch.Tensor | None = None,
                   loss_mode: int = LossMode.REINFORCE, clip_eps: float = 0.2, kl_beta: float = 0.04,
                   loss_norm: float = 0.0, std_eps: float = 1e-8, want_grads: bool = True, vocab_chunk: int = 0,
                   norm_weight: torch.Tensor | None = None, norm_eps: float = 1e-6, exact_bf16: bool = False,
                   low_memory_chunks: bool = False,
                   outputs: LmheadOutputs | None = None, sync: bool = True, stream=None,
                   ctx: Context | None = None) -> LmheadOutputs:
    """Fused LM-head + GRPO loss (pcp_grpo_lmhead_fwd_bwd). hidden [S*T, H] bf16,
    weight / ref_weight [V, H] bf16, ids / mask / old_logp [S, T]. With norm_weight
    (f32 [H]) the decoder's final RMSNorm is fused in: hidden is the last layer's
    output before the norm, and dhidden / dnorm_weight are the gradients there.
    vocab_chunk 0 lets the library keep the forward's softmax terms for the backward:
    f16 by default, f32 with exact_bf16 (PCP_FLAG_EXACT_BF16; the bf16 dlogits are then
    the f32 value rounded once); a chunk width recomputes the logits per chunk
    instead, and low_memory_chunks (PCP_FLAG_FORCE_STREAMING) selects that backward's
    form without transposed copies (which it takes by itself when they do not fit)."""
    ctx = ctx or default_context(hidden.device.index or 0)
    if ids.dim() != 2:
        raise PcpError(-1, "ids must be [S, T]")
    S, T = ids.shape
    N, H = hidden.shape
    V = weight.shape[0]
    if N != S * T or weight.shape[1] != H:
        raise PcpError(-1, "hidden must be [S*T, H] and weight [V, H]")
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise PcpError(-2, "hidden and weight must be bf16")
    dev = hidden.device
    if outputs is None:
        outputs = LmheadOutputs(
            loss=torch.zeros((), dtype=torch.float32, device=dev),
            logp=torch.zeros((S, T), dtype=torch.float32, device=dev),
            ref_logp=torch.zeros((S, T), dtype=torch.float32, device=dev) if ref_weight is not None else None,
            token_loss=torch.zeros((S, T), dtype=torch.float32, device=dev),
            advantages=torch.zeros((S,), dtype=torch.float32, device=dev),
            dhidden=torch.empty((N, H), dtype=torch.float32, device=dev) if want_grads else None,
            dweight=torch.empty((V, H), dtype=torch.float32, device=dev) if want_grads else None,
            dnorm_weight=torch.empty(H, dtype=torch.float32, device=dev)
            if want_grads and norm_weight is not None else None)
    if norm_weight is not None and (norm_weight.dtype != torch.float32 or norm_weight.numel() != H
                                    or not norm_weight.is_contiguous()):
        raise PcpError(-2, "norm_weight must be a contiguous f32 tensor of H elements")
    a = _lib.LmheadArgs()
    lib().pcp_lmhead_args_init(ctypes.byref(a))
    a.n_seq, a.rows, a.hidden, a.vocab, a.group_size, a.vocab_chunk = S, T, H, V, int(group_size), int(vocab_chunk)
    a.ids_dtype = dtype_code(ids)
    a.hidden_states, a.weight, a.ref_weight = _ptr(hidden), _ptr(weight), _ptr(ref_weight)
    a.ids = _ptr(ids)
    if mask is not None:
        a.mask = _ptr(mask)
        a.mask_dtype = dtype_code(mask)
    a.old_logp, a.advantages, a.rewards = _ptr(old_logp), _ptr(advantages), _ptr(rewards)
    a.logp, a.ref_logp, a.token_loss = _ptr(outputs.logp), _ptr(outputs.ref_logp), _ptr(outputs.token_loss)
    a.advantages_out, a.loss = _ptr(outputs.advantages), _ptr(outputs.loss)
    a.dhidden, a.dweight = _ptr(outputs.dhidden), _ptr(outputs.dweight)
    a.norm_weight, a.dnorm_weight, a.norm_eps = _ptr(norm_weight), _ptr(outputs.dnorm_weight), norm_eps
    a.loss_mode = int(loss_mode)
    a.clip_eps, a.kl_beta, a.std_eps, a.loss_norm = clip_eps, kl_beta, std_eps, loss_norm
    a.flags = ((0 if sync else _lib.FLAG_ASYNC) | (_lib.FLAG_EXACT_BF16 if exact_bf16 else 0)
               | (_lib.FLAG_FORCE_STREAMING if low_memory_chunks else 0))
    a.stream = _stream_handle(stream)
    check(lib().pcp_grpo_lmhead_fwd_bwd(ctx.handle, ctypes.byref(a)), ctx.handle)
    return outputs
