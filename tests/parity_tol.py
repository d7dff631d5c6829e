"""Tolerances of the parity tests, derived by forward error analysis, and host/device
array helpers (shared by the logits-input and the fused LM-head tests).

  log-probs, token losses (f32 math):  |d| <= 1e-5 * max(1, |lse|)      (rel 1e-5 of the row scale)
  loss:                                the log-prob bar propagated through dloss/dlogp and
                                       dloss/dref, plus 1e-5 of the sum of |contributions|
  dlogits, f32 output:                 |d| <= 1e-4 (north star) and <= 1e-5*|exact| + floor_row
  dlogits, bf16 output:                |d| <= (2^-8 + 4e-6)*|exact| + floor_row
floor_row (coef_floor) is what the f32 log-prob error allows in the row's
coefficient c: c is built from exp(logp - old) and expm1(ref - logp), whose terms
can cancel.
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


def assert_dlogits(got, want, floor_rows, bf16_out):
    """floor_rows: per-row absolute floor (coef_floor), broadcast over the vocabulary."""
    got = got.astype(np.float64)
    want = want.astype(np.float64)
    fl = np.asarray(floor_rows, np.float64)[..., None]
    err = np.abs(got - want)
    if bf16_out:
        tol = (2.0 ** -8 + 4e-6) * np.abs(want) + fl
    else:
        tol = 1e-5 * np.abs(want) + fl
        assert err.max() <= 1e-4
    bad = err > tol
    assert not bad.any(), f"{bad.sum()} dlogits out of tolerance; worst {err.max():.3e}"
