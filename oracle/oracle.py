"""TEST INFRASTRUCTURE — Python face of the CPU oracle (oracle/libpcp_oracle.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker (or the timed CPU baseline); the product
path (pcp_amd) never does.

What each function restates (reference file:line):
  advantages   src/nodes/controllers/rl_shepherd.zig:462-479 (bit-exact f32)
  logprob      tools/export_qwen_forward.py:154-156, models/tests/qwen_test.mlir:257-277
  grpo_rows    export_qwen_forward.py:156-163 (REINFORCE), its autodiff backward
               (src/compiler/graph_builder.zig:302-426, src/autodiff/vjp_rules.zig rules
               cited in grpo_oracle.cpp) and the clipped-ratio + k3-KL loss
  grpo_full    the whole loss head over [S, T, V] with the kernels' row layout
               (seq lengths = clamp(mask.sum(1), min=1), export_qwen_forward.py:160)
  check_dlogits  grpo_rows' exact dlogits compared in place with a device's rows
  lmhead_*     export_qwen_forward.py:147 (lm_head) and matmulVJP, vjp_rules.zig:426-497
  rmsnorm_*    the final norm before lm_head (export_qwen_forward.py:112, model.norm =
               Qwen2RMSNorm of transformers' modeling_qwen2) and its VJP
  nesterov     src/optimizers/nesterov.zig:86-97 and nesterov_mlir.zig:93-99
  grad_stats   src/nodes/controllers/rl_shepherd.zig:607-641
  pack         src/nodes/controllers/rl_shepherd.zig:487-515
  sample       src/core/math.zig:21-73 (Sampler.sample with the uniform draw given)

Pinning: every function is checked in tests/test_oracle.py against the reference's
known-answer tests (src/examples/isolated_vjp_tests.zig), closed forms, brute force
in float64, finite differences and torch CPU autograd.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.environ.get("PCP_ORACLE_LIB") or os.path.join(_HERE, "libpcp_oracle.so")

F16, BF16, F32, F64 = 0, 1, 2, 3
EXACT, REF_F32, FAITHFUL = 0, 1, 2
REINFORCE, CLIP_KL = 0, 1
IGNORE_INDEX = -100


class _RowsArgs(ctypes.Structure):
    _fields_ = [
        ("nrows", ctypes.c_int64), ("vocab", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("logits", ctypes.c_void_p), ("ref_logits", ctypes.c_void_p),
        ("ids", ctypes.c_void_p), ("w", ctypes.c_void_p), ("adv", ctypes.c_void_p),
        ("seq_len", ctypes.c_void_p), ("old_logp", ctypes.c_void_p),
        ("loss_norm", ctypes.c_float), ("loss_mode", ctypes.c_int32),
        ("clip_eps", ctypes.c_float), ("kl_beta", ctypes.c_float),
        ("precision", ctypes.c_int32), ("nthreads", ctypes.c_int32),
        ("lp", ctypes.c_void_p), ("lr", ctypes.c_void_p), ("token_loss", ctypes.c_void_p),
        ("coef", ctypes.c_void_p), ("dlogits", ctypes.c_void_p),
    ]


class _CheckArgs(ctypes.Structure):
    _fields_ = [
        ("nrows", ctypes.c_int64), ("vocab", ctypes.c_int64), ("dtype", ctypes.c_int32),
        ("logits", ctypes.c_void_p), ("ids", ctypes.c_void_p), ("coef", ctypes.c_void_p),
        ("floor_row", ctypes.c_void_p), ("got_dtype", ctypes.c_int32), ("got", ctypes.c_void_p),
        ("rel", ctypes.c_double), ("kfloor", ctypes.c_double), ("sub", ctypes.c_double),
        ("rel_min", ctypes.c_double), ("nthreads", ctypes.c_int32),
        ("max_usage", ctypes.c_void_p), ("max_abs", ctypes.c_void_p), ("max_rel", ctypes.c_void_p),
        ("n_bad", ctypes.c_void_p),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_f32_to_bf16_array.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.oracle_advantages.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_float,
                                        ctypes.c_void_p]
        L.oracle_logprob.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64,
                                     ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                     ctypes.c_void_p]
        L.oracle_grpo_rows.argtypes = [ctypes.POINTER(_RowsArgs)]
        L.oracle_grpo_rows.restype = ctypes.c_int
        L.oracle_max_threads.restype = ctypes.c_int
        L.oracle_check_dlogits.argtypes = [ctypes.POINTER(_CheckArgs)]
        L.oracle_check_dlogits.restype = ctypes.c_int
        _VP, _I64 = ctypes.c_void_p, ctypes.c_int64
        L.oracle_nesterov.argtypes = [_VP, _VP, _VP, _I64, ctypes.c_float, ctypes.c_float, ctypes.c_int]
        L.oracle_nesterov.restype = None
        L.oracle_grad_stats.argtypes = [_VP, _I64, _VP, _VP, _VP, _VP]
        L.oracle_grad_stats.restype = None
        L.oracle_pack.argtypes = [_VP, _I64, _VP, _VP, _I64, _VP, _I64, _I64, _I64, _VP, _VP]
        L.oracle_pack.restype = ctypes.c_int
        L.oracle_sample.argtypes = [_VP, _I64, ctypes.c_float, ctypes.c_float]
        L.oracle_sample.restype = _I64
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---- element codecs --------------------------------------------------------

def bf16_from_f32(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16_array(_ptr(x), _ptr(out), x.size)
    return out


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns to f32."""
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def lmhead_logits(hidden_bits: np.ndarray, weight_bits: np.ndarray) -> np.ndarray:
    """Exact float64 logits hidden * W^T of bf16 operands (bit patterns, uint16): the
    LM head of tools/export_qwen_forward.py:147 evaluated without rounding."""
    return bf16_to_f32(hidden_bits).astype(np.float64) @ bf16_to_f32(weight_bits).astype(np.float64).T


def lmhead_grads(hidden_bits: np.ndarray, weight_bits: np.ndarray, logits: np.ndarray, lse: np.ndarray,
                 coef: np.ndarray, ids: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """float64 (dhidden, dW) of the LM head: D = c * (onehot - softmax), dhidden = D W,
    dW = D^T hidden (matmulVJP, src/autodiff/vjp_rules.zig:426-497)."""
    N, V = logits.shape
    D = -np.exp(logits - lse[:, None]) * coef[:, None]
    live = (coef != 0) & (ids >= 0) & (ids < V)
    D[np.nonzero(live)[0], ids[live]] += coef[live]
    h = bf16_to_f32(hidden_bits).astype(np.float64)
    W = bf16_to_f32(weight_bits).astype(np.float64)
    return D @ W, D.T @ h


def rmsnorm_operand(h_bits: np.ndarray, gamma: np.ndarray, eps: float) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Qwen2RMSNorm of bf16 rows h [N, H] as the LM head's bf16 operand, in f32 with a
    stated summation order, so the result is a function of the inputs alone:
      ss = sum_k h_k^2: each of 256 lanes adds columns lane, lane + 256, ... in turn;
           lanes 64w..64w+63 reduce by halving (a[i] + a[i + 32], then + 16, ..., + 1);
           the four wave sums add as ((w0 + w1) + w2) + w3
      r  = 1 / sqrt(ss / H + eps)           (correctly rounded f32)
      x  = bf16(h * r)                      (Qwen2RMSNorm's .to(input_dtype))
      y  = bf16(gamma * x)                  (the bf16 operand of lm_head)
    Returns (y bits uint16 [N, H], r f32 [N], x bits uint16 [N, H])."""
    h = bf16_to_f32(h_bits)
    N, H = h.shape
    per = -(-H // 256)
    hp = np.zeros((N, per * 256), np.float32)
    hp[:, :H] = h
    hp = hp.reshape(N, per, 256)
    acc = np.zeros((N, 256), np.float32)
    for i in range(per):
        acc = acc + hp[:, i, :] * hp[:, i, :]
    w = acc.reshape(N, 4, 64)
    half = 32
    while half >= 1:
        w = w[..., :half] + w[..., half:2 * half]
        half //= 2
    w = w[..., 0]
    ss = ((w[:, 0] + w[:, 1]) + w[:, 2]) + w[:, 3]
    r = np.float32(1) / np.sqrt(ss / np.float32(H) + np.float32(eps))
    x_bits = bf16_from_f32(h * r[:, None])
    y_bits = bf16_from_f32(np.asarray(gamma, np.float32)[None, :] * bf16_to_f32(x_bits))
    return y_bits, r.astype(np.float32), x_bits


def rmsnorm_vjp(h_bits: np.ndarray, gamma: np.ndarray, eps: float, x_bits: np.ndarray,
                dy: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """float64 (dh, dgamma) of y = gamma * x, x = h / sqrt(mean(h^2) + eps), given dL/dy;
    the bf16 roundings of x and y pass gradients through (a dtype cast under autograd),
    and dgamma multiplies dy by the rounded x that the forward used:
      g = dy * gamma,  dh = r g - h r^3 (sum_k g_k h_k) / H,  dgamma = sum_n dy_n * x_n."""
    h = bf16_to_f32(h_bits).astype(np.float64)
    H = h.shape[1]
    r = 1.0 / np.sqrt((h * h).mean(axis=1) + eps)
    g = dy * np.asarray(gamma, np.float64)[None, :]
    dot = (g * h).sum(axis=1)
    dh = r[:, None] * g - h * (r ** 3 * dot / H)[:, None]
    dgamma = (dy * bf16_to_f32(x_bits).astype(np.float64)).sum(axis=0)
    return dh, dgamma


def widen(x: np.ndarray, dtype: int) -> np.ndarray:
    """Logits array in its storage form (uint16 for bf16, float16, float32) -> float64."""
    if dtype == BF16:
        return bf16_to_f32(x).astype(np.float64)
    return np.asarray(x).astype(np.float64)


def storage_dtype_code(x: np.ndarray, bf16: bool = False) -> int:
    if bf16 or x.dtype == np.uint16:
        return BF16
    if x.dtype == np.float16:
        return F16
    if x.dtype == np.float32:
        return F32
    if x.dtype == np.float64:
        return F64
    raise TypeError(f"unsupported logits storage {x.dtype}")


# ---- a3: advantages ---------------------------------------------------------

def advantages(rewards: np.ndarray, group_size: int, eps: float = 1e-8) -> np.ndarray:
    r = np.ascontiguousarray(rewards, dtype=np.float32)
    out = np.empty_like(r)
    lib().oracle_advantages(_ptr(r), r.size, int(group_size), ctypes.c_float(eps), _ptr(out))
    return out


# ---- a1: log-prob gather ------------------------------------------------------

def logprob(logits: np.ndarray, ids: np.ndarray, dtype: int | None = None, precision: int = EXACT,
            nthreads: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """logits [N, V] in storage form; ids [N]. Returns (lp, lse) in float64."""
    x = np.ascontiguousarray(logits)
    dt = storage_dtype_code(x) if dtype is None else dtype
    N, V = x.shape
    ids64 = np.ascontiguousarray(ids, dtype=np.int64)
    lp = np.empty(N, np.float64)
    lse = np.empty(N, np.float64)
    lib().oracle_logprob(_ptr(x), dt, N, V, _ptr(ids64), precision, nthreads, _ptr(lp), _ptr(lse))
    return lp, lse


# ---- a2+a4+a5: rows ---------------------------------------------------------------

@dataclass
class RowsResult:
    lp: np.ndarray
    lr: np.ndarray
    token_loss: np.ndarray
    coef: np.ndarray
    dlogits: np.ndarray | None


def grpo_rows(logits: np.ndarray, ids: np.ndarray, w: np.ndarray, adv: np.ndarray, seq_len: np.ndarray,
              loss_norm: float, *, ref_logits: np.ndarray | None = None, old_logp: np.ndarray | None = None,
              loss_mode: int = REINFORCE, clip_eps: float = 0.2, kl_beta: float = 0.04,
              precision: int = EXACT, want_dlogits: bool = True, dtype: int | None = None,
              nthreads: int = 0) -> RowsResult:
    """Loss terms of independent rows. Per-row metadata: ids, mask weight w, the
    advantage and clamped length of the row's sequence, old log-prob."""
    x = np.ascontiguousarray(logits)
    dt = storage_dtype_code(x) if dtype is None else dtype
    N, V = x.shape
    ref = None if ref_logits is None else np.ascontiguousarray(ref_logits)
    ids64 = np.ascontiguousarray(ids, dtype=np.int64).reshape(N)
    wf = np.ascontiguousarray(w, dtype=np.float32).reshape(N)
    af = np.ascontiguousarray(adv, dtype=np.float32).reshape(N)
    lf = np.ascontiguousarray(seq_len, dtype=np.float32).reshape(N)
    of = None if old_logp is None else np.ascontiguousarray(old_logp, dtype=np.float32).reshape(N)
    res = RowsResult(np.empty(N), np.empty(N), np.empty(N), np.empty(N),
                     np.empty((N, V), np.float32) if want_dlogits else None)
    a = _RowsArgs(N, V, dt, _ptr(x), _ptr(ref), _ptr(ids64), _ptr(wf), _ptr(af), _ptr(lf), _ptr(of),
                  float(loss_norm), loss_mode, clip_eps, kl_beta, precision, nthreads,
                  _ptr(res.lp), _ptr(res.lr), _ptr(res.token_loss), _ptr(res.coef), _ptr(res.dlogits))
    rc = lib().oracle_grpo_rows(ctypes.byref(a))
    if rc != 0:
        raise ValueError("oracle_grpo_rows rejected its arguments")
    return res


@dataclass
class CheckResult:
    max_usage: np.ndarray   # per row: max err / tol
    max_abs: np.ndarray     # per row: max |got - exact|
    max_rel: np.ndarray     # per row: max err / |exact| over |exact| >= rel_min * |coef|
    n_bad: np.ndarray       # per row: elements with err > tol


def check_dlogits(logits: np.ndarray, ids: np.ndarray, coef: np.ndarray, floor_row: np.ndarray, got: np.ndarray,
                  got_dtype: int, rel: float, kfloor: float, sub: float = 0.0, rel_min: float = 2.0 ** -14,
                  dtype: int | None = None, nthreads: int = 0) -> CheckResult:
    """Compare a device's dlogits rows (storage form: uint16 bf16 / float16 / float32)
    with the exact float64 rows coef * (onehot(ids) - softmax(logits)), element by
    element against tol = rel * |exact| + kfloor * floor_row + sub, without holding the
    exact rows in memory. coef: the oracle's exact coefficients (grpo_rows). Rows must be
    live (0 <= id < V)."""
    x = np.ascontiguousarray(logits)
    dt = storage_dtype_code(x) if dtype is None else dtype
    N, V = x.shape
    g = np.ascontiguousarray(got)
    assert g.shape == (N, V)
    ids64 = np.ascontiguousarray(ids, dtype=np.int64).reshape(N)
    assert ((ids64 >= 0) & (ids64 < V)).all()
    cf = np.ascontiguousarray(coef, dtype=np.float64).reshape(N)
    fl = np.ascontiguousarray(floor_row, dtype=np.float64).reshape(N)
    res = CheckResult(np.empty(N), np.empty(N), np.empty(N), np.empty(N, np.int64))
    a = _CheckArgs(N, V, dt, _ptr(x), _ptr(ids64), _ptr(cf), _ptr(fl), int(got_dtype), _ptr(g), float(rel),
                   float(kfloor), float(sub), float(rel_min), nthreads, _ptr(res.max_usage), _ptr(res.max_abs),
                   _ptr(res.max_rel), _ptr(res.n_bad))
    if lib().oracle_check_dlogits(ctypes.byref(a)) != 0:
        raise ValueError("oracle_check_dlogits rejected its arguments")
    return res


# ---- full problem -------------------------------------------------------------------

@dataclass
class FullResult:
    loss: float
    lp: np.ndarray          # [S, TS] indexed like ids (unaddressed entries 0)
    lr: np.ndarray
    token_loss: np.ndarray
    coef: np.ndarray
    adv: np.ndarray         # [S] f32
    seq_len: np.ndarray     # [S] f32
    dlogits: np.ndarray | None  # [S, LS, V] f32


def seq_lengths(mask: np.ndarray, rows: int, tok_offset: int) -> np.ndarray:
    """max(sum_t mask[s, tok_offset + t], 1) over the rows that carry tokens (f32)."""
    m = np.asarray(mask, dtype=np.float32)[:, tok_offset:tok_offset + rows]
    return np.maximum(m.astype(np.float64).sum(axis=1), 1.0).astype(np.float32)


def grpo_full(logits: np.ndarray, ids: np.ndarray, mask: np.ndarray | None, *, rows: int, tok_offset: int = 0,
              advantages_in: np.ndarray | None = None, rewards: np.ndarray | None = None, group_size: int = 1,
              ref_logits: np.ndarray | None = None, old_logp: np.ndarray | None = None,
              loss_mode: int = REINFORCE, clip_eps: float = 0.2, kl_beta: float = 0.04,
              loss_norm: float = 0.0, std_eps: float = 1e-8, precision: int = EXACT,
              want_dlogits: bool = True, dtype: int | None = None, nthreads: int = 0) -> FullResult:
    """The loss head over logits [S, LS, V] (storage form) and token arrays [S, TS]:
    row (s, t < rows) scores ids[s, tok_offset + t]; rows >= rows are pad rows."""
    x = np.asarray(logits)
    S, LS, V = x.shape
    ids = np.asarray(ids)
    TS = ids.shape[1]
    m = np.ones(ids.shape, np.float32) if mask is None else np.asarray(mask, dtype=np.float32)
    if advantages_in is not None:
        adv = np.ascontiguousarray(advantages_in, dtype=np.float32)
    else:
        adv = advantages(rewards, group_size, std_eps)
    L = seq_lengths(m, rows, tok_offset)
    G = float(loss_norm) if loss_norm > 0 else float(S)
    sel_rows = x[:, :rows, :].reshape(S * rows, V)
    sel_ref = None if ref_logits is None else np.asarray(ref_logits)[:, :rows, :].reshape(S * rows, V)
    tix = slice(tok_offset, tok_offset + rows)
    r = grpo_rows(sel_rows, ids[:, tix].reshape(-1), m[:, tix].reshape(-1),
                  np.repeat(adv, rows), np.repeat(L, rows), G, ref_logits=sel_ref,
                  old_logp=None if old_logp is None else np.asarray(old_logp)[:, tix].reshape(-1),
                  loss_mode=loss_mode, clip_eps=clip_eps, kl_beta=kl_beta, precision=precision,
                  want_dlogits=want_dlogits, dtype=dtype, nthreads=nthreads)

    def place(v):
        out = np.zeros((S, TS), np.float64)
        out[:, tix] = v.reshape(S, rows)
        return out

    tl = r.token_loss.reshape(S, rows)
    seq = tl.sum(axis=1) / L.astype(np.float64)
    if loss_mode == REINFORCE:
        seq = seq * adv.astype(np.float64)
    loss = float(seq.sum() / G)
    dl = None
    if want_dlogits:
        dl = np.zeros((S, LS, V), np.float32)
        dl[:, :rows, :] = r.dlogits.reshape(S, rows, V)
    return FullResult(loss, place(r.lp), place(r.lr), place(r.token_loss), place(r.coef), adv, L, dl)


# ---- the work around the loss head in one step (step_oracle.cpp) ---------------------

def nesterov(p: np.ndarray, v: np.ndarray, g: np.ndarray, lr: float, mu: float, mode: int = 0):
    """One update, f32 op by op: mode 0 = nesterov.zig:86-97 (v = mu*v + g;
    p = p - lr*(g + mu*v)), mode 1 = nesterov_mlir.zig:93-99 (v = mu*v + lr*g; p = p - v).
    Returns new (p, v) arrays."""
    p = np.array(p, dtype=np.float32, copy=True)
    v = np.array(v, dtype=np.float32, copy=True)
    g = np.ascontiguousarray(g, dtype=np.float32)
    lib().oracle_nesterov(_ptr(p), _ptr(v), _ptr(g), p.size, ctypes.c_float(lr), ctypes.c_float(mu), int(mode))
    return p, v


def grad_stats(g: np.ndarray) -> dict:
    """rl_shepherd.zig:607-641: f64 sum of squares and max |g| over the finite values,
    NaN and Inf counts (sequential, as the reference)."""
    g = np.ascontiguousarray(g, dtype=np.float32).reshape(-1)
    s, m = ctypes.c_double(), ctypes.c_float()
    nn, ni = ctypes.c_int64(), ctypes.c_int64()
    lib().oracle_grad_stats(_ptr(g), g.size, ctypes.byref(s), ctypes.byref(m), ctypes.byref(nn), ctypes.byref(ni))
    return {"sumsq": s.value, "l2_norm": float(np.sqrt(s.value)), "max_abs": m.value, "nan_count": nn.value,
            "inf_count": ni.value, "elements": g.size}


def pack(prompt_tokens, prompt_offsets, completion_tokens, completion_offsets, n_rows: int, seq_len: int):
    """rl_shepherd.zig:487-515 packing. Returns (ids int64 [n_rows, T], mask f32, ok)."""
    pt = np.ascontiguousarray(prompt_tokens, dtype=np.int64)
    po = np.ascontiguousarray(prompt_offsets, dtype=np.int64)
    ct = np.ascontiguousarray(completion_tokens, dtype=np.int64)
    co = np.ascontiguousarray(completion_offsets, dtype=np.int64)
    R = po.size - 1
    ids = np.empty((n_rows, seq_len), np.int64)
    mask = np.empty((n_rows, seq_len), np.float32)
    rc = lib().oracle_pack(_ptr(pt), pt.size, _ptr(po), _ptr(ct), ct.size, _ptr(co), R, n_rows, seq_len,
                           _ptr(ids), _ptr(mask))
    return ids, mask, rc == 0


def sample(logits: np.ndarray, temperature: float, u: float = 0.0) -> int:
    """math.zig:21-73 Sampler.sample on one f32 row with the uniform draw u given
    (the reference draws it with prng.random().float(f32))."""
    x = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1)
    return int(lib().oracle_sample(_ptr(x), x.size, ctypes.c_float(temperature), ctypes.c_float(u)))
