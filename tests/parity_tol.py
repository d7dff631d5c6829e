"""Tolerances of the parity tests, derived by forward error analysis, and host/device
array helpers (shared by the logits-input and the fused LM-head tests).

  log-probs, token losses (f32 math):  |d| <= 1e-5 * max(1, |lse|)      (rel 1e-5 of the row scale)
  loss:                                the log-prob bar propagated through dloss/dlogp and
                                       dloss/dref, plus 1e-5 of the sum of |contributions|
  dlogits, f32 output:                 |d| <= 1e-4 (north star) and <= 1e-5*|exact| + floor_row
  dlogits, bf16 output:                |d| <= (2^-8 + 2^-11 + 1.3e-5)*|exact| + (1 + 2^-6)*floor_row
  dlogits, bf16 output, exact mode:    |d| <= (2^-8 + 1.1e-5)*|exact| + (1 + 2^-7)*floor_row
floor_row (coef_floor) is what the f32 log-prob error allows in the row's
coefficient c: c is built from exp(logp - old) and expm1(ref - logp), whose terms
can cancel.

The 16-bit bars follow from the f32 bar. Let o' be the f32 result, with
|o' - d| <= 1e-5*|d| + floor_row (the f32 bar). A 16-bit output rounded to nearest
even is off by at most its unit roundoff times the value: 2^-8 for bf16 (8 significant
bits), 2^-11 for f16.
  Exact mode (PCP_FLAG_EXACT_BF16, and every path other than bf16 -> bf16 resident
  rows): out = round(o'), so |out - d| <= 2^-8*|o'| + |o' - d|
  <= (2^-8 + 1.1e-5)*|d| + (1 + 2^-7)*floor_row.
  Default bf16 -> bf16 resident rows scale the sum pass's softmax terms, kept as f16,
  into dlogits: o = f * f16(e) with f = -c * 2^(m - lse) and e <= 1. The f16 rounding
  adds at most 2^-11 of the term (2^-25 absolute below f16's normal range, which is
  |c| * 2^-25 in o, since 2^(m - lse) <= 1), so |o - o'| <= 2^-11*|o'| + |c|*2^-25 and
    |out - d| <= 2^-8*|o| + |o - o'| + |o' - d|
              <= (2^-8 + 2^-11 + 2^-19)*|o'| + |o' - d| + (1 + 2^-8)*|c|*2^-25
              <= (2^-8 + 2^-11 + 1.3e-5)*|d| + (1 + 2^-6)*floor_row,
  using |o'| <= |d| + |o' - d| and floor_row >= 1e-5*|c| (so |c|*2^-24 < 2^-7*floor_row).
"""
import numpy as np
import torch

from oracle import oracle as orc

DEV = torch.device("cuda:0")


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(DEV).view(torch.bfloat16)
    return torch.from_numpy(a).to(DEV)


def host_bits(t):
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def token_scale(logits, ids, rows, off, dtype):
    """max(1, |lse|) of every token-carrying row, placed at its token index: the
    scale of the per-token log-prob tolerance (1e-5 * this)."""
    S, LS, V = logits.shape
    sel = np.ascontiguousarray(logits[:, :rows]).reshape(S * rows, V)
    _, lse = orc.logprob(sel, np.clip(ids[:, off:off + rows].reshape(-1), 0, None), dtype=dtype)
    out = np.zeros(ids.shape, np.float64)
    out[:, off:off + rows] = np.maximum(1.0, np.abs(lse)).reshape(S, rows)
    return out


def loss_tolerance(token_loss, coef, lp, lr, mask, adv, seq_len, G, reinforce, beta, tscale):
    """Forward-error bound of the loss given the per-token log-prob bar: each token's
    logp / ref logp may be off by 1e-5*max(1,|lse|), which moves the loss by
    |dloss/dlogp| + |dloss/dref| times that; the reduction adds 1e-5 of the sum of
    |contributions| (the loss can be a near-cancellation of those terms)."""
    L = np.asarray(seq_len, np.float64)[:, None]
    per = np.abs(token_loss) / L
    if reinforce:
        per = per * np.abs(np.asarray(adv, np.float64))[:, None]
        dref = 0.0
    else:
        dref = np.abs(beta * np.expm1(lr - lp)) * np.abs(mask) / (G * L)
    delta = 1e-5 * tscale
    return 1e-5 * per.sum() / G + ((np.abs(coef) + dref) * delta).sum() + 1e-12


def full_loss_tol(r, logits, ids, mask, rows, off, dtype, reinforce, beta, G):
    return loss_tolerance(r.token_loss, r.coef, r.lp, r.lr, mask, r.adv, r.seq_len, G, reinforce, beta,
                          token_scale(logits, ids, rows, off, dtype))


def lse_scale(logits_rows, ids_rows, dtype):
    _, lse = orc.logprob(logits_rows, np.clip(ids_rows, 0, None), dtype=dtype)
    return np.maximum(1.0, np.abs(lse))


def coef_floor(coef, lp, lr, w, adv, seq_len, G, old, reinforce, beta, eps, tscale):
    """Per-row absolute error allowed in dlogits = c*(onehot - softmax), from the f32
    log-prob error delta = 1e-5*max(1,|lse|): c = scale*(-A*rho*[unclipped] - beta*expm1(d))
    with rho = exp(logp - old), d = ref - logp moves by scale*(|A|*rho + 2*beta*e^d)*delta
    (its terms can cancel, so this is not relative to c), and the softmax by |c|*delta."""
    delta = 1e-5 * tscale
    if reinforce:
        return np.abs(coef) * (delta + 1e-5)
    scale = np.abs(w) / (G * np.asarray(seq_len, np.float64))
    rho = np.exp(lp - old)
    unclipped = np.where(adv >= 0, rho <= 1 + eps, rho >= 1 - eps)
    dc = scale * (np.abs(adv) * rho * unclipped + 2 * beta * np.exp(lr - lp)) * delta
    return dc + np.abs(coef) * delta + 1e-5 * np.abs(coef)


def full_floor(r, mask, old, G, reinforce, beta, eps, tscale):
    """coef_floor over a FullResult ([S, TS] token arrays)."""
    L = np.asarray(r.seq_len, np.float64)[:, None]
    A = np.asarray(r.adv, np.float64)[:, None]
    old = r.lp if old is None else np.asarray(old, np.float64)
    return coef_floor(r.coef, r.lp, r.lr, np.asarray(mask, np.float64), A, L, G, old, reinforce, beta, eps, tscale)


def tok_to_rows(a, rows, off, LS):
    """[S, TS] token-indexed array -> [S, LS] logits-row-indexed (pad rows 0)."""
    out = np.zeros((a.shape[0], LS), np.float64)
    out[:, :rows] = a[:, off:off + rows]
    return out


BF16_CACHED_REL = 2.0 ** -8 + 2.0 ** -11 + 1.3e-5
BF16_EXACT_REL = 2.0 ** -8 + 1.1e-5


def assert_dlogits(got, want, floor_rows, bf16_out, exact=False, f16_out=False):
    """floor_rows: per-row absolute floor (coef_floor), broadcast over the vocabulary.
    bf16_out: a 16-bit output (bf16 or f16). exact: the output is the f32 result rounded
    once (PCP_FLAG_EXACT_BF16, or a path without the f16 softmax cache). f16_out: the
    output is f16, whose values below 2^-14 are subnormal with a fixed spacing of 2^-24,
    so a correctly rounded one is off by up to 2^-25 absolutely, whatever its size (rows
    whose coefficient nearly cancels reach that range)."""
    got = got.astype(np.float64)
    want = want.astype(np.float64)
    fl = np.asarray(floor_rows, np.float64)[..., None]
    err = np.abs(got - want)
    sub = 2.0 ** -25 if f16_out else 0.0
    if bf16_out and exact:
        tol = BF16_EXACT_REL * np.abs(want) + (1 + 2.0 ** -7) * fl + sub
    elif bf16_out:
        tol = BF16_CACHED_REL * np.abs(want) + (1 + 2.0 ** -6) * fl + sub
    else:
        tol = 1e-5 * np.abs(want) + fl
        assert err.max() <= 1e-4
    bad = err > tol
    assert not bad.any(), f"{bad.sum()} dlogits out of tolerance; worst {err.max():.3e}"


def emulate_block_sum(x, block):
    """float32 value of the device's fixed-order workgroup sum of x over `block` lanes:
    lane j adds x[j], x[j + block], ... in order; each 64-lane wave then reduces by the
    xor butterfly (every lane adds the value of lane ^ off, off = 32, 16, ..., 1); the
    wave sums add in wave order."""
    x = np.asarray(x, np.float32).reshape(-1)
    acc = np.zeros(block, np.float32)
    for k in range(0, len(x), block):
        c = x[k:k + block]
        acc[:len(c)] = acc[:len(c)] + c
    w = acc.reshape(block // 64, 64)
    lanes = np.arange(64)
    for off in (32, 16, 8, 4, 2, 1):
        w = w + w[:, lanes ^ off]
    v = w[0, 0]
    for i in range(1, block // 64):
        v = np.float32(v + w[i, 0])
    return np.float32(v)


def emulate_loss(token_loss, mask, adv, reinforce, loss_norm):
    """The loss the device's reduction forms from its own f32 token losses [S, T] (the
    token-carrying columns) and 0/1 mask: per sequence the 256-lane sum over its tokens
    divided by max(sum mask, 1) (times the advantage in REINFORCE), then the 1024-lane
    sum of those over the sequences divided by loss_norm, every step in float32."""
    tl = np.asarray(token_loss, np.float32)
    S = tl.shape[0]
    seq_len = np.maximum(np.asarray(mask, np.float32).sum(1, dtype=np.float32), np.float32(1))
    vals = np.empty(S, np.float32)
    for s in range(S):
        v = np.float32(emulate_block_sum(tl[s], 256) / seq_len[s])
        vals[s] = np.float32(v * np.float32(adv[s])) if reinforce else v
    return np.float32(emulate_block_sum(vals, 1024) / np.float32(loss_norm))
