"""Parity of the fused LM-head + GRPO loss (pcp_grpo_lmhead_fwd_bwd) with the oracle.

The oracle evaluates the logits hidden . W^T of the same bf16 operands exactly in
float64 (oracle.lmhead_logits), runs the loss head on them (grpo_full on F64
logits), and forms the float64 gradients D.W and D^T.hidden with
D = c (onehot - softmax) (oracle.lmhead_grads). At the full configuration-5 size,
where a float64 CPU evaluation would take minutes, the reference is torch fp32 on
the GPU (token chunks of the same products), and the loss is checked against the
reduction of the device's own token losses.

Tolerances:
  log-probs, token losses, loss: as the logits-input path (parity_tol). The tile
    kernel sums products of bf16 values, each exact in f32, so its f32 accumulation
    error is far below the 1e-5 * max(1, |lse|) bar.
  dhidden, dW: the device rounds D to bf16 (2^-8 relative at most) before the two
    GEMMs and c carries the coef_floor error, so elementwise
    |dh - dh*| <= E . |W| and |dW - dW*| <= E^T . |hidden| with
    E = (2^-8 + 1e-4) |D| + 2 floor_n (onehot + p).
    By default (vocab_chunk 0) the backward takes the softmax terms from the forward:
    e = 2^(x log2e - m_b), with m_b the largest logit of the 128-entry block b holding
    v, stored as f16 (2^-11 relative, or 2^-25 absolute below f16's normal range) and
    scaled by 2^(m_b - lse). Off the target that adds
    (1 + 2^-7) |c| (2^-11 p + 2^-25 exp(m_b - lse)) to E (the 2^-7 covers the bf16
    rounding of the larger value); the target's D comes from the f32 target logit as
    without the cache.
"""
import time

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from pcp_amd import grpo, synth
from pcp_amd._lib import LossMode, PcpError
from parity_tol import coef_floor, dev, loss_tolerance

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
ORC_MODE = {LossMode.REINFORCE: orc.REINFORCE, LossMode.GRPO_CLIP_KL: orc.CLIP_KL}


def bf16_bits(rng, shape, std):
    return orc.bf16_from_f32((rng.standard_normal(shape) * std).astype(np.float32))


def make_case(S, T, H, V, G, seed, lengths=None, logit_std=2.0):
    """hidden ~ N(0, 1), W ~ N(0, logit_std^2 / H) (logits ~ N(0, logit_std^2)),
    W_ref = W + 5% noise, all rounded to bf16."""
    rng = np.random.default_rng(seed)
    N = S * T
    w_std = logit_std / np.sqrt(H)
    hb = bf16_bits(rng, (N, H), 1.0)
    wb = bf16_bits(rng, (V, H), w_std)
    rb = orc.bf16_from_f32(orc.bf16_to_f32(wb) + (rng.standard_normal((V, H)) * w_std * 0.05).astype(np.float32))
    ids = rng.integers(0, V, size=(S, T)).astype(np.int64)
    lengths = np.asarray(lengths if lengths is not None else rng.integers(1, T + 1, size=S))
    mask = synth.mask_from_lengths(lengths, T)
    rewards = rng.integers(0, 2, size=S).astype(np.float32)
    noise = (rng.standard_normal((S, T)) * 0.01).astype(np.float32)
    return dict(S=S, T=T, H=H, V=V, G=G, hb=hb, wb=wb, rb=rb, ids=ids, mask=mask, rewards=rewards, noise=noise)


def oracle_case(c, mode, clip_eps=0.2, kl_beta=0.04):
    S, T, V = c["S"], c["T"], c["V"]
    L = orc.lmhead_logits(c["hb"], c["wb"])
    R = orc.lmhead_logits(c["hb"], c["rb"])
    idsf = c["ids"].reshape(-1)
    lp0, lse = orc.logprob(L, np.clip(idsf, 0, V - 1), dtype=orc.F64)
    _, rlse = orc.logprob(R, np.clip(idsf, 0, V - 1), dtype=orc.F64)
    old = (lp0.reshape(S, T) + c["noise"]).astype(np.float32)
    r = orc.grpo_full(L.reshape(S, T, V), c["ids"], c["mask"], rows=T, rewards=c["rewards"], group_size=c["G"],
                      ref_logits=R.reshape(S, T, V), old_logp=old, loss_mode=ORC_MODE[mode], clip_eps=clip_eps,
                      kl_beta=kl_beta, want_dlogits=False, dtype=orc.F64)
    return L, lse, rlse, old, r


def run_device(c, mode, old, *, vocab_chunk=0, want_grads=True, ids=None, mask=None, clip_eps=0.2, kl_beta=0.04,
               exact_bf16=False, low_memory=False):
    return grpo.lmhead_fwd_bwd(dev(c["hb"]), dev(c["wb"]), dev(c["ids"]) if ids is None else ids,
                               dev(c["mask"]) if mask is None else mask, ref_weight=dev(c["rb"]),
                               rewards=dev(c["rewards"]), group_size=c["G"], old_logp=dev(old), loss_mode=mode,
                               clip_eps=clip_eps, kl_beta=kl_beta, vocab_chunk=vocab_chunk, want_grads=want_grads,
                               exact_bf16=exact_bf16, low_memory_chunks=low_memory)


def cache_error(L, lse, coef, ids):
    """Per-element bound on what the f16 softmax cache adds to D (module docstring)."""
    N, V = L.shape
    nb = (V + 127) // 128
    Lp = np.full((N, nb * 128), -np.inf)
    Lp[:, :V] = L
    blk = np.repeat(Lp.reshape(N, nb, 128).max(2), 128, axis=1)[:, :V]
    X = (1 + 2.0 ** -7) * np.abs(coef)[:, None] * (2.0 ** -11 * np.exp(L - lse[:, None])
                                                   + 2.0 ** -25 * np.exp(blk - lse[:, None]))
    live = (coef != 0) & (ids >= 0) & (ids < V)
    X[np.nonzero(live)[0], ids[live]] = 0.0
    return X


def grad_bounds(c, L, lse, r, mode, old, kl_beta=0.04, clip_eps=0.2, cached=True):
    """(want_dh, tol_dh, want_dw, tol_dw) in float64. cached: the backward used the
    forward's softmax cache (vocab_chunk 0 without PCP_FLAG_EXACT_BF16)."""
    S, T, V = c["S"], c["T"], c["V"]
    ids = c["ids"].reshape(-1)
    coef = r.coef.reshape(-1)
    tscale = np.maximum(1.0, np.abs(lse)).reshape(S, T)
    fl = coef_floor(r.coef, r.lp, r.lr, c["mask"].astype(np.float64), r.adv.astype(np.float64)[:, None],
                    r.seq_len.astype(np.float64)[:, None], float(S), old.astype(np.float64),
                    mode == LossMode.REINFORCE, kl_beta, clip_eps, tscale).reshape(-1)
    dh, dw = orc.lmhead_grads(c["hb"], c["wb"], L, lse, coef, ids)
    P = np.exp(L - lse[:, None])
    D = -P * coef[:, None]
    live = (coef != 0) & (ids >= 0) & (ids < V)
    D[np.nonzero(live)[0], ids[live]] += coef[live]
    onehot = np.zeros_like(P)
    onehot[np.arange(len(ids)), np.clip(ids, 0, V - 1)] = 1.0
    E = (2.0 ** -8 + 1e-4) * np.abs(D) + 2.0 * fl[:, None] * (onehot + P)
    E[fl == 0] = (2.0 ** -8 + 1e-4) * np.abs(D[fl == 0])
    if cached:
        E += cache_error(L, lse, coef, ids)
    W = np.abs(orc.bf16_to_f32(c["wb"]).astype(np.float64))
    h = np.abs(orc.bf16_to_f32(c["hb"]).astype(np.float64))
    return dh, E @ W + 1e-30, dw, E.T @ h + 1e-30


def check_forward(c, out, L, lse, rlse, r, mode):
    S, T = c["S"], c["T"]
    sc = np.maximum(1.0, np.abs(lse)).reshape(S, T)
    rsc = np.maximum(1.0, np.abs(rlse)).reshape(S, T)
    lp = out.logp.cpu().numpy()
    assert np.all(np.abs(lp - r.lp) <= 1e-5 * sc), np.abs(lp - r.lp).max()
    assert np.all(lp[c["mask"] == 0] == 0)
    if mode == LossMode.GRPO_CLIP_KL:
        lr = out.ref_logp.cpu().numpy()
        assert np.all(np.abs(lr - r.lr) <= 1e-5 * rsc), np.abs(lr - r.lr).max()
    tl = out.token_loss.cpu().numpy()
    assert np.all(np.abs(tl - r.token_loss) <= 1e-5 * sc), np.abs(tl - r.token_loss).max()
    assert np.array_equal(out.advantages.cpu().numpy(), r.adv)
    tol = loss_tolerance(r.token_loss, r.coef, r.lp, r.lr, c["mask"], r.adv, r.seq_len, float(S),
                         mode == LossMode.REINFORCE, 0.04, np.maximum(sc, rsc))
    assert abs(float(out.loss.cpu()) - r.loss) <= tol, (float(out.loss.cpu()), r.loss, tol)


def check_grads(out, want_dh, tol_dh, want_dw, tol_dw):
    dh = out.dhidden.cpu().numpy().astype(np.float64)
    dw = out.dweight.cpu().numpy().astype(np.float64)
    edh, edw = np.abs(dh - want_dh), np.abs(dw - want_dw)
    assert not np.any(edh > tol_dh), f"dhidden: {(edh > tol_dh).sum()} out of tolerance, worst {edh.max():.3e}"
    assert not np.any(edw > tol_dw), f"dW: {(edw > tol_dw).sum()} out of tolerance, worst {edw.max():.3e}"


# ---- ragged small shapes against the float64 oracle -----------------------------------------

SMALL = [
    # S, T, H, V, G, chunk, lengths: 150 tokens (two token tiles, the second ragged),
    # an odd number of K stages, a ragged last vocab tile and several vocab chunks.
    (3, 50, 192, 1000, 3, 256, [50, 31, 7]),
    (2, 64, 64, 129, 2, 0, [64, 1]),
    (1, 7, 128, 4096, 1, 1024, [5]),
    # 6,000 live tokens = 24 token tiles: forward tile groups of 9, 9 and 6;
    # 10,900 = 43 token tiles: one forward group, backward groups of 4 and a last of 3.
    (2, 3000, 64, 300, 2, 256, [3000, 3000]),
    (4, 3000, 64, 300, 2, 256, [3000, 3000, 3000, 1900]),
    # 3,100 live of 6,000 tokens: grids sized for 24 token tiles run 13, and dhidden
    # accumulates over two chunks, so a tile computed twice would show.
    (2, 3000, 64, 300, 2, 256, [3000, 100]),
    (2, 3000, 64, 300, 2, 0, [3000, 100]),
]


def _random_shapes(n, seed=77):
    # Seeded shapes for the same check: hidden sizes of 2, 6 and 10 K stages,
    # vocabularies off the 128 / 256 tile widths, token counts off the 32-column
    # MFMA blocks, empty sequences, chunk widths including ones past V.
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        S = int(rng.integers(1, 4))
        T = int(rng.integers(5, 160))
        H = int(rng.choice([64, 192, 320]))
        V = int(rng.integers(1, 2500))
        chunk = int(rng.choice([0, 256, 768, 4096]))
        lengths = [int(x) for x in rng.integers(0, T + 1, size=S)]
        out.append((S, T, H, V, S, chunk, lengths))
    return out


SMALL += _random_shapes(6)


@pytest.mark.parametrize("mode", [LossMode.REINFORCE, LossMode.GRPO_CLIP_KL])
@pytest.mark.parametrize("shape", SMALL, ids=lambda s: f"S{s[0]}T{s[1]}H{s[2]}V{s[3]}c{s[5]}")
def test_lmhead_small_vs_oracle(shape, mode):
    S, T, H, V, G, chunk, lengths = shape
    c = make_case(S, T, H, V, G, seed=S * 1000 + V, lengths=lengths)
    L, lse, rlse, old, r = oracle_case(c, mode)
    print(f"lmhead small S={S} T={T} H={H} V={V} chunk={chunk} mode={int(mode)}", flush=True)
    out = run_device(c, mode, old, vocab_chunk=chunk)
    torch.cuda.synchronize()
    check_forward(c, out, L, lse, rlse, r, mode)
    check_grads(out, *grad_bounds(c, L, lse, r, mode, old, cached=chunk == 0))


@pytest.mark.parametrize("shape", [s for s in SMALL if s[5] > 0], ids=lambda s: f"S{s[0]}T{s[1]}H{s[2]}V{s[3]}c{s[5]}")
def test_lmhead_small_low_memory_chunks_vs_oracle(shape):
    """The chunked backward's low-memory form (K-major operands read with LDS transpose
    loads, no transposed copies), which it takes when the copies do not fit: the same
    shapes against the oracle, and the same forward as the default chunked form."""
    S, T, H, V, G, chunk, lengths = shape
    c = make_case(S, T, H, V, G, seed=S * 1000 + V, lengths=lengths)
    mode = LossMode.GRPO_CLIP_KL
    L, lse, rlse, old, r = oracle_case(c, mode)
    print(f"lmhead small low-memory chunks S={S} T={T} H={H} V={V} chunk={chunk}", flush=True)
    lo = run_device(c, mode, old, vocab_chunk=chunk, low_memory=True)
    hi = run_device(c, mode, old, vocab_chunk=chunk)
    torch.cuda.synchronize()
    check_forward(c, lo, L, lse, rlse, r, mode)
    check_grads(lo, *grad_bounds(c, L, lse, r, mode, old, cached=False))
    for f in ("loss", "logp", "ref_logp", "token_loss"):
        assert torch.equal(getattr(lo, f), getattr(hi, f)), f


@pytest.mark.parametrize("shape", SMALL, ids=lambda s: f"S{s[0]}T{s[1]}H{s[2]}V{s[3]}")
def test_lmhead_small_exact_vs_oracle(shape):
    """PCP_FLAG_EXACT_BF16 (f32 softmax terms) at the same ragged shapes, the shape's
    chunk ignored: under the bound without the cache term."""
    S, T, H, V, G, _, lengths = shape
    c = make_case(S, T, H, V, G, seed=S * 1000 + V + 7, lengths=lengths)
    mode = LossMode.GRPO_CLIP_KL
    L, lse, rlse, old, r = oracle_case(c, mode)
    print(f"lmhead small exact S={S} T={T} H={H} V={V}", flush=True)
    out = run_device(c, mode, old, exact_bf16=True)
    torch.cuda.synchronize()
    check_forward(c, out, L, lse, rlse, r, mode)
    check_grads(out, *grad_bounds(c, L, lse, r, mode, old, cached=False))


def _variant_shapes(n, seed=2024):
    # Seeded shapes for all four backward forms: up to 8 sequences of up to 700 tokens
    # (empty ones included), hidden sizes of 1 to 16 stages, vocabularies up to 40,000
    # and chunk widths below and past them, capped so the float64 oracle stays quick.
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        S = int(rng.integers(1, 9))
        T = int(rng.integers(3, 700))
        H = int(rng.choice([64, 128, 192, 256, 448, 640, 1024]))
        V = int(rng.integers(1, 40000))
        G = int(rng.choice([d for d in range(1, S + 1) if S % d == 0]))
        lengths = [int(x) for x in rng.integers(0, T + 1, size=S)]
        chunk = int(rng.choice([256, 512, 1024, 4096, 16384]))
        std = float(rng.choice([1.0, 2.0, 4.0]))
        mode = LossMode.GRPO_CLIP_KL if rng.random() < 0.7 else LossMode.REINFORCE
        if S * T * V * H <= 3e9:
            out.append((S, T, H, V, G, chunk, lengths, std, mode))
    return out


@pytest.mark.parametrize("case", _variant_shapes(12), ids=lambda s: f"S{s[0]}T{s[1]}H{s[2]}V{s[3]}c{s[5]}")
def test_lmhead_random_variants_vs_oracle(case):
    """Each backward form on the same seeded random inputs: the default (f16 softmax
    terms), PCP_FLAG_EXACT_BF16 (f32 terms), the chunked recompute with transposed
    copies and in its low-memory form, each under its bound; the forward outputs of
    all four are identical."""
    S, T, H, V, G, chunk, lengths, std, mode = case
    c = make_case(S, T, H, V, G, seed=S * 7919 + V, lengths=lengths, logit_std=std)
    L, lse, rlse, old, r = oracle_case(c, mode)
    first = None
    for name, kw in (("cached", {}), ("exact", dict(exact_bf16=True)), ("chunked", dict(vocab_chunk=chunk)),
                     ("low-memory", dict(vocab_chunk=chunk, low_memory=True))):
        print(f"lmhead random S={S} T={T} H={H} V={V} chunk={chunk} mode={int(mode)} {name}", flush=True)
        out = run_device(c, mode, old, **kw)
        torch.cuda.synchronize()
        check_forward(c, out, L, lse, rlse, r, mode)
        check_grads(out, *grad_bounds(c, L, lse, r, mode, old, cached=name == "cached"))
        if first is None:
            first = out
        for f in ("loss", "logp", "token_loss"):
            assert torch.equal(getattr(out, f), getattr(first, f)), (name, f)


def test_lmhead_ignore_index_int32_bool_mask_and_no_grads():
    c = make_case(2, 40, 128, 700, 2, seed=11, lengths=[40, 25])
    c["ids"][0, 3] = -100          # live by mask, ignored by id: no loss, no gradient, no error
    L, lse, rlse, old, r = oracle_case(c, LossMode.GRPO_CLIP_KL)
    ids32 = dev(c["ids"].astype(np.int32))
    maskb = dev(c["mask"].astype(bool))
    out = run_device(c, LossMode.GRPO_CLIP_KL, old, ids=ids32, mask=maskb)
    torch.cuda.synchronize()
    check_forward(c, out, L, lse, rlse, r, LossMode.GRPO_CLIP_KL)
    check_grads(out, *grad_bounds(c, L, lse, r, LossMode.GRPO_CLIP_KL, old))
    fwd = run_device(c, LossMode.GRPO_CLIP_KL, old, want_grads=False)
    torch.cuda.synchronize()
    assert fwd.dhidden is None and fwd.dweight is None
    assert torch.equal(fwd.logp, out.logp) and torch.equal(fwd.loss, out.loss)


def test_lmhead_all_masked_and_no_mask():
    """No live token: the loss, log-probs and every gradient are 0 on the cached (f16 and
    f32 terms) and the chunked backward (the live count stays on the device; the products run with no
    token tiles / an empty K), with and without the fused final norm; outputs are
    pre-filled with NaN so that a skipped write shows. Then mask = NULL."""
    c = make_case(2, 20, 64, 500, 2, seed=9, lengths=[20, 20])
    old = np.full((2, 20), -6.0, np.float32)
    zero = torch.zeros((2, 20), dtype=torch.float32, device=DEV)
    nan = float("nan")
    for chunk, exact in ((0, False), (256, False), (0, True)):
        outs = grpo.LmheadOutputs(loss=torch.full((), nan, device=DEV), logp=torch.full((2, 20), nan, device=DEV),
                                  ref_logp=torch.full((2, 20), nan, device=DEV),
                                  token_loss=torch.full((2, 20), nan, device=DEV),
                                  advantages=torch.full((2,), nan, device=DEV),
                                  dhidden=torch.full((40, 64), nan, device=DEV), dweight=torch.full((500, 64), nan, device=DEV))
        out = grpo.lmhead_fwd_bwd(dev(c["hb"]), dev(c["wb"]), dev(c["ids"]), zero, ref_weight=dev(c["rb"]),
                                  rewards=dev(c["rewards"]), group_size=2, old_logp=dev(old),
                                  loss_mode=LossMode.GRPO_CLIP_KL, vocab_chunk=chunk, exact_bf16=exact, outputs=outs)
        torch.cuda.synchronize()
        assert float(out.loss) == 0.0 and not out.logp.any() and not out.token_loss.any()
        assert not out.dhidden.any() and not out.dweight.any()
        cn = make_norm_case(2, 20, 64, 500, 2, seed=10, lengths=[20, 20])
        outs = grpo.LmheadOutputs(loss=torch.full((), nan, device=DEV), logp=torch.full((2, 20), nan, device=DEV),
                                  ref_logp=None, token_loss=torch.full((2, 20), nan, device=DEV),
                                  advantages=torch.full((2,), nan, device=DEV),
                                  dhidden=torch.full((40, 64), nan, device=DEV), dweight=torch.full((500, 64), nan, device=DEV),
                                  dnorm_weight=torch.full((64,), nan, device=DEV))
        out = grpo.lmhead_fwd_bwd(dev(cn["h"]), dev(cn["wb"]), dev(cn["ids"]), zero, rewards=dev(cn["rewards"]),
                                  group_size=2, vocab_chunk=chunk, exact_bf16=exact, norm_weight=dev(cn["gamma"]),
                                  outputs=outs)
        torch.cuda.synchronize()
        assert float(out.loss) == 0.0 and not out.logp.any()
        assert not out.dhidden.any() and not out.dweight.any() and not out.dnorm_weight.any()
    # mask = NULL: every token with an in-range id is live (same result as an all-ones mask).
    L, lse, rlse, old, r = oracle_case(c, LossMode.GRPO_CLIP_KL)
    out = grpo.lmhead_fwd_bwd(dev(c["hb"]), dev(c["wb"]), dev(c["ids"]), None, ref_weight=dev(c["rb"]),
                              rewards=dev(c["rewards"]), group_size=2, old_logp=dev(old),
                              loss_mode=LossMode.GRPO_CLIP_KL)
    torch.cuda.synchronize()
    check_forward(c, out, L, lse, rlse, r, LossMode.GRPO_CLIP_KL)
    check_grads(out, *grad_bounds(c, L, lse, r, LossMode.GRPO_CLIP_KL, old))


def test_execute_lmhead_shifted_vs_oracle():
    """The host-bytes function: hidden row t scores token t+1 (the reference's shift)."""
    from pcp_amd._lib import DType
    from pcp_amd.backend import HipGrpoBackend

    S, T, H, V, G = 2, 33, 128, 600, 2
    c = make_case(S, T, H, V, G, seed=21, lengths=[33, 20])
    L = orc.lmhead_logits(c["hb"], c["wb"]).reshape(S, T, V)
    R = orc.lmhead_logits(c["hb"], c["rb"]).reshape(S, T, V)
    old = np.full((S, T), -6.0, np.float32)
    r = orc.grpo_full(L, c["ids"], c["mask"], rows=T - 1, tok_offset=1, rewards=c["rewards"], group_size=G,
                      ref_logits=R, old_logp=old, loss_mode=orc.CLIP_KL, want_dlogits=False, dtype=orc.F64)
    hyper = np.array([G, 0.2, 0.04, 0, 1], np.float32)
    ins = [c["hb"].reshape(S, T, H), c["wb"], c["rb"], c["ids"], c["mask"], old, c["rewards"], hyper]
    be = HipGrpoBackend.init()
    outs = be.executeFunction(None, "grpo_lmhead_fwd_bwd", ins, [x.shape for x in ins],
                              [DType.bf16, DType.bf16, DType.bf16, DType.i64, DType.f32, DType.f32, DType.f32,
                               DType.f32])
    be.deinit()
    loss = np.frombuffer(outs[0], np.float32)[0]
    dh = np.frombuffer(outs[1], np.float32).reshape(S, T, H)
    dw = np.frombuffer(outs[2], np.float32).reshape(V, H)
    lp = np.frombuffer(outs[3], np.float32).reshape(S, T)
    lr = np.frombuffer(outs[4], np.float32).reshape(S, T)
    _, lse = orc.logprob(L.reshape(-1, V), np.zeros(S * T, np.int64), dtype=orc.F64)
    sc = np.maximum(1.0, np.abs(lse)).reshape(S, T)
    sc_tok = np.ones((S, T))
    sc_tok[:, 1:] = sc[:, :-1]
    assert np.all(np.abs(lp - r.lp) <= 1e-5 * sc_tok) and np.all(lp[:, 0] == 0)
    assert np.all(np.abs(lr - r.lr) <= 1e-5 * sc_tok + 1e-5)
    tol = loss_tolerance(r.token_loss, r.coef, r.lp, r.lr, c["mask"], r.adv, r.seq_len, float(S), False, 0.04,
                         sc_tok)
    assert abs(loss - r.loss) <= tol
    assert np.array_equal(np.frombuffer(outs[5], np.float32), r.adv)
    # Gradients: rows t < T-1 carry token t+1's coefficient; the last row is 0.
    crow = np.zeros((S, T))
    crow[:, :-1] = r.coef[:, 1:]
    irow = np.zeros((S, T), np.int64)
    irow[:, :-1] = c["ids"][:, 1:]
    want_dh, want_dw = orc.lmhead_grads(c["hb"], c["wb"], L.reshape(-1, V), lse, crow.reshape(-1), irow.reshape(-1))
    assert not dh[:, -1].any()
    scale_h = np.abs(want_dh).max()
    scale_w = np.abs(want_dw).max()
    assert np.abs(dh.reshape(-1, H) - want_dh).max() <= 2.0 ** -7 * scale_h
    assert np.abs(dw - want_dw).max() <= 2.0 ** -7 * scale_w


def test_execute_lmhead_final_norm_shifted():
    """The host-bytes function with the ninth input (final norm weight, eps in hyper[5]):
    the same outputs as the device-pointer call on the shifted token arrays, plus
    dnorm_weight as the seventh output."""
    from pcp_amd._lib import DType
    from pcp_amd.backend import HipGrpoBackend

    S, T, H, V, G = 2, 33, 192, 500, 2
    c = make_norm_case(S, T, H, V, G, seed=23, lengths=[33, 21])
    c["eps"] = 1e-5
    old = np.full((S, T), -6.0, np.float32)
    hyper = np.array([G, 0.2, 0.04, 0, 1, c["eps"]], np.float32)
    ins = [c["h"].reshape(S, T, H), c["wb"], c["rb"], c["ids"], c["mask"], old, c["rewards"], hyper, c["gamma"]]
    be = HipGrpoBackend.init()
    outs = be.executeFunction(None, "grpo_lmhead_fwd_bwd", ins, [x.shape for x in ins],
                              [DType.bf16, DType.bf16, DType.bf16, DType.i64, DType.f32, DType.f32, DType.f32,
                               DType.f32, DType.f32])
    be.deinit()
    assert len(outs) == 7
    # The device-pointer call on the shifted arrays (row t scores token t + 1).
    sid = np.zeros_like(c["ids"])
    sid[:, :-1] = c["ids"][:, 1:]
    smask = np.zeros_like(c["mask"])
    smask[:, :-1] = c["mask"][:, 1:]
    sold = np.zeros_like(old)
    sold[:, :-1] = old[:, 1:]
    ref = grpo.lmhead_fwd_bwd(dev(c["h"]), dev(c["wb"]), dev(sid), dev(smask), ref_weight=dev(c["rb"]),
                              rewards=dev(c["rewards"]), group_size=G, old_logp=dev(sold),
                              loss_mode=LossMode.GRPO_CLIP_KL, norm_weight=dev(c["gamma"]), norm_eps=c["eps"])
    torch.cuda.synchronize()
    assert np.frombuffer(outs[0], np.float32)[0] == float(ref.loss.cpu())
    assert np.array_equal(np.frombuffer(outs[1], np.float32), ref.dhidden.cpu().numpy().reshape(-1))
    assert np.array_equal(np.frombuffer(outs[2], np.float32), ref.dweight.cpu().numpy().reshape(-1))
    lp = np.frombuffer(outs[3], np.float32).reshape(S, T)
    assert np.array_equal(lp[:, 1:], ref.logp.cpu().numpy()[:, :-1]) and not lp[:, 0].any()
    assert np.array_equal(np.frombuffer(outs[6], np.float32), ref.dnorm_weight.cpu().numpy())


@pytest.mark.parametrize("chunk, exact, low", [(512, False, False), (512, False, True), (0, False, False),
                                              (0, True, False)], ids=["chunked", "chunked-low-memory", "cached", "exact"])
def test_lmhead_deterministic(chunk, exact, low):
    c = make_case(2, 70, 128, 900, 2, seed=5, lengths=[70, 33])
    old = np.full((2, 70), -7.0, np.float32)
    a = run_device(c, LossMode.GRPO_CLIP_KL, old, vocab_chunk=chunk, exact_bf16=exact, low_memory=low)
    b = run_device(c, LossMode.GRPO_CLIP_KL, old, vocab_chunk=chunk, exact_bf16=exact, low_memory=low)
    torch.cuda.synchronize()
    for f in ("loss", "logp", "ref_logp", "token_loss", "dhidden", "dweight"):
        assert torch.equal(getattr(a, f), getattr(b, f)), f


def test_lmhead_exact_flag():
    """PCP_FLAG_EXACT_BF16 keeps the forward's softmax terms as f32, so the backward's
    bf16 dlogits are the f32 value rounded once: inside the bound without the cache
    term, as the recomputing backward (an explicit chunk) is. With an explicit chunk the
    flag changes nothing, bit for bit. The forward outputs of the default, exact and
    chunked calls are identical; the default backward meets its own bound."""
    c = make_case(3, 90, 192, 2500, 3, seed=31, lengths=[90, 61, 12])
    mode = LossMode.GRPO_CLIP_KL
    L, lse, rlse, old, r = oracle_case(c, mode)
    ex = run_device(c, mode, old, exact_bf16=True)
    ch = run_device(c, mode, old, vocab_chunk=16384)
    chx = run_device(c, mode, old, vocab_chunk=16384, exact_bf16=True)
    ca = run_device(c, mode, old)
    torch.cuda.synchronize()
    for f in ("loss", "logp", "ref_logp", "token_loss", "dhidden", "dweight"):
        assert torch.equal(getattr(chx, f), getattr(ch, f)), f
    for f in ("loss", "logp", "ref_logp", "token_loss"):
        assert torch.equal(getattr(ca, f), getattr(ex, f)), f
        assert torch.equal(getattr(ch, f), getattr(ex, f)), f
    check_forward(c, ex, L, lse, rlse, r, mode)
    exact_bounds = grad_bounds(c, L, lse, r, mode, old, cached=False)
    check_grads(ex, *exact_bounds)
    check_grads(ch, *exact_bounds)
    check_grads(ca, *grad_bounds(c, L, lse, r, mode, old, cached=True))


@pytest.mark.parametrize("variant", ["exact", "chunked", "cached"])
def test_lmhead_dlogits_rounded_once(variant):
    """The bf16 dlogits operand itself. With one live token the dW product has K = 1, so
    dW[v, k] = D_v * h_k exactly (a product of two bf16 values is exact in f32) and
    D_v = dW[v, k0] / h_k0 exactly in float64. With PCP_FLAG_EXACT_BF16 (f32 softmax
    terms) and with the recomputing backward (an explicit chunk), every D_v is the
    float64 D = c (onehot - softmax) rounded to nearest even, except where D lies within
    1e-4 of a rounding midpoint relative to |D| (the f32 logits, exponentials and c stay
    far inside that). The default f16 terms (2^-11 relative) fail the same check on a
    share of the elements, which shows that the check tells the two apart."""
    T, H, V = 16, 256, 5000
    c = make_case(1, T, H, V, 1, seed=61, lengths=[T], logit_std=3.0)
    L = orc.lmhead_logits(c["hb"], c["wb"])
    h = orc.bf16_to_f32(c["hb"]).astype(np.float64)
    adv = 0.75
    kw = {"exact": dict(exact_bf16=True), "chunked": dict(vocab_chunk=1024), "cached": {}}[variant]
    bf16 = lambda x: orc.bf16_from_f32(np.asarray(x, np.float64).astype(np.float32))
    checked = wrong = 0
    for t in np.random.default_rng(62).choice(T, 4, replace=False):
        mask = np.zeros((1, T), np.float32)
        mask[0, t] = 1.0
        print(f"dlogits rounded once: {variant}, live token {t}", flush=True)
        out = grpo.lmhead_fwd_bwd(dev(c["hb"]), dev(c["wb"]), dev(c["ids"]), dev(mask),
                                  rewards=dev(np.ones(1, np.float32)), advantages=dev(np.full(1, adv, np.float32)), **kw)
        torch.cuda.synchronize()
        dw = out.dweight.cpu().numpy().astype(np.float64)
        k0 = int(np.argmax(np.abs(h[t])))
        d_dev = dw[:, k0] / h[t, k0]
        assert np.array_equal(orc.bf16_to_f32(bf16(d_dev)).astype(np.float64), d_dev), "D is not a bf16 value"
        # REINFORCE, one sequence of one live token: d loss / d logp = -adv.
        coef = -adv
        x = L[t]
        p = np.exp(x - (x.max() + np.log(np.exp(x - x.max()).sum())))
        d = -coef * p
        d[c["ids"][0, t]] += coef
        clear = bf16(d * (1 + 1e-4)) == bf16(d * (1 - 1e-4))
        checked += int(clear.sum())
        wrong += int((bf16(d_dev) != bf16(d))[clear].sum())
    assert checked > 0.9 * 4 * V, checked
    if variant == "cached":
        assert wrong > 0, "the check does not tell f16 terms from exact rounding"
    else:
        assert wrong == 0, f"{wrong} of {checked} dlogits are not the exact value rounded once"


def test_lmhead_async_does_not_wait():
    """PCP_FLAG_ASYNC: the call only enqueues (the live-token count is never read back).
    Queued behind a bounded spin kernel of ~0.2 s, the call returns long before the spin
    ends, and the results equal a synchronous call's."""
    c = make_case(2, 70, 128, 900, 2, seed=5, lengths=[70, 33])
    old = np.full((2, 70), -7.0, np.float32)
    want = run_device(c, LossMode.GRPO_CLIP_KL, old)
    args = (dev(c["hb"]), dev(c["wb"]), dev(c["ids"]), dev(c["mask"]))
    kw = dict(ref_weight=dev(c["rb"]), rewards=dev(c["rewards"]), group_size=2, old_logp=dev(old),
              loss_mode=LossMode.GRPO_CLIP_KL)
    ctx = grpo.default_context(0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    torch.cuda._sleep(400_000_000)             # a bounded spin: ~0.2 s at 2 GHz
    t1 = time.perf_counter()
    got = grpo.lmhead_fwd_bwd(*args, sync=False, ctx=ctx, **kw)
    t2 = time.perf_counter()
    busy = not torch.cuda.current_stream().query()
    ctx.sync()
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    print(f"async LM head: enqueue {1e3 * (t2 - t1):.2f} ms, spin + call {1e3 * (t3 - t0):.1f} ms", flush=True)
    assert busy and t3 - t0 > 0.05, "the spin kernel did not hold the stream"
    assert t2 - t1 < 0.5 * (t3 - t0), "the async call waited for the device"
    for f in ("loss", "logp", "ref_logp", "token_loss", "dhidden", "dweight"):
        assert torch.equal(getattr(got, f), getattr(want, f)), f


@pytest.mark.parametrize("chunk, exact", [(0, False), (512, False), (0, True)], ids=["cached", "chunked", "exact"])
def test_lmhead_graph_capture_replays(chunk, exact):
    """The call captured in a HIP graph (asynchronous, no host read): three replays with
    eager work between them (outputs overwritten with NaN) each equal an eager call bit
    for bit."""
    c = make_case(2, 70, 128, 900, 2, seed=43, lengths=[70, 41])
    old = np.full((2, 70), -7.0, np.float32)
    args = (dev(c["hb"]), dev(c["wb"]), dev(c["ids"]), dev(c["mask"]))
    kw = dict(ref_weight=dev(c["rb"]), rewards=dev(c["rewards"]), group_size=2, old_logp=dev(old),
              loss_mode=LossMode.GRPO_CLIP_KL, vocab_chunk=chunk, exact_bf16=exact)
    want = grpo.lmhead_fwd_bwd(*args, **kw)
    out = grpo.lmhead_fwd_bwd(*args, **kw)     # the graph's outputs; buffers already grown
    ctx = grpo.default_context(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        grpo.lmhead_fwd_bwd(*args, outputs=out, sync=False, ctx=ctx, **kw)
    ctx.sync()
    fields = ("loss", "logp", "ref_logp", "token_loss", "advantages", "dhidden", "dweight")
    for rep in range(3):
        for f in fields:
            getattr(out, f).fill_(float("nan"))
        torch.cuda.synchronize()
        print(f"graph replay {rep} ({'chunked' if chunk else 'exact' if exact else 'cached'})", flush=True)
        g.replay()
        torch.cuda.synchronize()
        for f in fields:
            assert torch.equal(getattr(out, f), getattr(want, f)), (rep, f)
    ctx.sync()


def test_release_workspace_then_call_again():
    """pcp_release_workspace frees the context's work buffers (the loss path's scratch and
    the LM head's softmax cache); calls after it allocate again and give the same bits as
    before (no state lives only in a freed buffer), and pcp_workspace_bytes reads 0 in
    between. A private context, so the other tests' default context keeps its buffers."""
    c = make_case(2, 70, 128, 900, 2, seed=47, lengths=[70, 33])
    old = np.full((2, 70), -7.0, np.float32)
    args = (dev(c["hb"]), dev(c["wb"]), dev(c["ids"]), dev(c["mask"]))
    kw = dict(ref_weight=dev(c["rb"]), rewards=dev(c["rewards"]), group_size=2, old_logp=dev(old),
              loss_mode=LossMode.GRPO_CLIP_KL)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(5)
    logits = (torch.randn((4, 64, 1000), generator=gen, device="cuda:0") * 3).to(torch.bfloat16)
    ids = torch.randint(0, 1000, (4, 64), generator=gen, device="cuda:0")
    mask = (torch.arange(64, device="cuda:0")[None] < torch.tensor([[64], [10], [40], [1]], device="cuda:0")).float()
    rewards = torch.rand((4,), generator=gen, device="cuda:0")
    ctx = grpo.Context(0)
    try:
        def run():
            lm = grpo.lmhead_fwd_bwd(*args, ctx=ctx, **kw)
            loss = grpo.grpo_loss_fwd_bwd(logits, ids, mask, rewards=rewards, group_size=2, ctx=ctx)
            return lm, loss
        want_lm, want_loss = run()
        assert ctx.workspace_bytes() > 0
        ctx.release_workspace()
        assert ctx.workspace_bytes() == 0
        ctx.release_workspace()   # nothing held: returns at once
        got_lm, got_loss = run()
        assert ctx.workspace_bytes() > 0
        for f in ("loss", "logp", "ref_logp", "token_loss", "advantages", "dhidden", "dweight"):
            assert torch.equal(getattr(got_lm, f), getattr(want_lm, f)), f
        for f in ("loss", "dlogits", "logp", "token_loss", "advantages"):
            assert torch.equal(getattr(got_loss, f), getattr(want_loss, f)), f
    finally:
        ctx.close()


def test_synth_lmhead_tokens_gumbel_argmax():
    """pcp_synth_lmhead_tokens (config 5's target ids) draws argmax_v(logit + g) per row
    with g = -log(-log u), u from Philox(seed + chunk index, tag 3, row-in-chunk * V + v)
    as pcp_synth_sample_tokens draws. With the noise recomputed on the host (the Philox
    is pinned by known answers in test_abi.py) and the logits exact in float64, every
    drawn id scores within 1e-4 of its row's best (the device forms f32 logits and f32
    logarithms); chunks of 16 over 40 rows cover the per-chunk seeds."""
    rng = np.random.default_rng(91)
    N, H, V, seed, chunk = 40, 128, 700, 1234, 16
    hb = bf16_bits(rng, (N, H), 1.0)
    wb = bf16_bits(rng, (V, H), 0.25)
    ids = synth.sample_lmhead_ids(dev(hb), dev(wb), seed, chunk=chunk).cpu().numpy()
    assert ids.shape == (N,) and ids.min() >= 0 and ids.max() < V
    L = orc.lmhead_logits(hb, wb)
    scale = np.float32(2.3283064365386963e-10)
    for r in range(N):
        k, rl = divmod(r, chunk)
        sk = seed + k
        flat = rl * V + np.arange(V)
        u = np.empty(V, np.uint32)
        for q in range(flat[0] // 4, flat[-1] // 4 + 1):
            words = synth.philox([q & 0xFFFFFFFF, q >> 32, 3, 0], [sk & 0xFFFFFFFF, sk >> 32])
            for j in range(4):
                v = 4 * q + j - rl * V
                if 0 <= v < V:
                    u[v] = words[j]
        uf = (u.astype(np.float32) + np.float32(0.5)) * scale
        score = L[r] - np.log(-np.log(uf.astype(np.float64)))
        assert score[ids[r]] >= score.max() - 1e-4 * max(1.0, abs(score.max())), (r, ids[r], int(score.argmax()))
    assert len(set(ids.tolist())) > N // 2


def test_lmhead_errors():
    c = make_case(1, 16, 64, 300, 1, seed=3, lengths=[16])
    old = np.zeros((1, 16), np.float32)
    bad = c["ids"].copy()
    bad[0, 2] = 300
    with pytest.raises(PcpError) as ei:
        run_device(c, LossMode.REINFORCE, old, ids=dev(bad))
    assert ei.value.code == -3
    hb = c["hb"].copy()
    hb[5] = orc.bf16_from_f32(np.full(64, np.nan, np.float32))
    with pytest.raises(PcpError) as ei:
        grpo.lmhead_fwd_bwd(dev(hb), dev(c["wb"]), dev(c["ids"]), dev(c["mask"]), rewards=dev(c["rewards"]))
    assert ei.value.code == -4
    # A NaN hidden row of a masked token is not an error (its loss weight is 0).
    mask = c["mask"].copy()
    mask[0, 5] = 0
    out = grpo.lmhead_fwd_bwd(dev(hb), dev(c["wb"]), dev(c["ids"]), dev(mask), rewards=dev(c["rewards"]))
    torch.cuda.synchronize()
    assert np.isfinite(float(out.loss.cpu()))
    with pytest.raises(PcpError) as ei:
        grpo.lmhead_fwd_bwd(dev(c["hb"][:, :32].copy()), dev(c["wb"][:, :32].copy()), dev(c["ids"]),
                            rewards=dev(c["rewards"]))
    assert ei.value.code == -1   # hidden must be a multiple of 64


# ---- the decoder's final RMSNorm fused at both ends ------------------------------------------

def make_norm_case(S, T, H, V, G, seed, lengths, logit_std=2.0):
    """make_case plus the pre-norm hidden states h (rows of scales e^-2 .. e^3), a norm
    weight near 1 (bf16 values) and eps 1e-6. The oracle's LM-head operand hb is the
    norm's bf16 output, reproduced bit for bit by oracle.rmsnorm_operand."""
    c = make_case(S, T, H, V, G, seed, lengths, logit_std)
    rng = np.random.default_rng(seed + 7)
    scale = np.exp(rng.uniform(-2, 3, size=(S * T, 1)))
    c["h"] = orc.bf16_from_f32((rng.standard_normal((S * T, H)) * scale).astype(np.float32))
    c["gamma"] = orc.bf16_to_f32(orc.bf16_from_f32((1 + 0.2 * rng.standard_normal(H)).astype(np.float32)))
    c["eps"] = 1e-6
    c["hb"], c["rstd"], c["xb"] = orc.rmsnorm_operand(c["h"], c["gamma"], c["eps"])
    return c


def run_device_norm(c, mode, old, *, vocab_chunk=0, outputs=None):
    return grpo.lmhead_fwd_bwd(dev(c["h"]), dev(c["wb"]), dev(c["ids"]), dev(c["mask"]), ref_weight=dev(c["rb"]),
                               rewards=dev(c["rewards"]), group_size=c["G"], old_logp=dev(old), loss_mode=mode,
                               vocab_chunk=vocab_chunk, norm_weight=dev(c["gamma"]), norm_eps=c["eps"],
                               outputs=outputs)


def norm_grad_bounds(c, want_dy, tol_dy, n_live):
    """float64 (dh, tol_dh, dgamma, tol_dgamma) through the norm's VJP. The bound on the
    LM head's dy propagates as |d(dh)| <= r (tg + |x| sum_k tg_k |x_k| / H) with
    tg = tol_dy |gamma| and x = h r; f32 slack covers the device's dot products and its
    f32 r; dgamma adds its f32 sum over live rows (block partials, then blocks)."""
    h = orc.bf16_to_f32(c["h"]).astype(np.float64)
    H = h.shape[1]
    r = 1.0 / np.sqrt((h * h).mean(1) + c["eps"])
    x = h * r[:, None]
    gam = np.abs(c["gamma"].astype(np.float64))
    dh, dg = orc.rmsnorm_vjp(c["h"], c["gamma"], c["eps"], c["xb"], want_dy)
    tg = tol_dy * gam[None, :]
    g = np.abs(want_dy) * gam[None, :]
    tol_dh = r[:, None] * (tg + np.abs(x) * ((tg * np.abs(x)).sum(1) / H)[:, None])
    tol_dh += 8e-6 * r[:, None] * (g + np.abs(x) * ((g * np.abs(x)).sum(1) / H)[:, None])
    xr = np.abs(orc.bf16_to_f32(c["xb"]).astype(np.float64))
    tol_dg = (tol_dy * xr).sum(0) + (n_live + 600) * 2.0 ** -24 * (np.abs(want_dy) * xr).sum(0)
    return dh, tol_dh + 1e-30, dg, tol_dg + 1e-30


NORM_SHAPES = [
    # S, T, H, V, G, chunk, lengths: H = 192 (one column per thread, ragged), Qwen2.5-0.5B's
    # H = 896 (four columns per thread, the last ragged), H = 4096 (sixteen).
    (3, 50, 192, 1000, 3, 256, [50, 31, 7]),
    (2, 64, 896, 2048, 2, 0, [64, 20]),
    (1, 40, 4096, 1024, 1, 512, [33]),
]


@pytest.mark.parametrize("mode", [LossMode.REINFORCE, LossMode.GRPO_CLIP_KL])
@pytest.mark.parametrize("shape", NORM_SHAPES, ids=lambda s: f"S{s[0]}T{s[1]}H{s[2]}V{s[3]}")
def test_lmhead_final_norm_vs_oracle(shape, mode):
    S, T, H, V, G, chunk, lengths = shape
    c = make_norm_case(S, T, H, V, G, seed=S * 100 + H, lengths=lengths)
    L, lse, rlse, old, r = oracle_case(c, mode)
    print(f"lmhead final norm S={S} T={T} H={H} V={V} mode={int(mode)}", flush=True)
    out = run_device_norm(c, mode, old, vocab_chunk=chunk)
    torch.cuda.synchronize()
    check_forward(c, out, L, lse, rlse, r, mode)
    want_dy, tol_dy, want_dw, tol_dw = grad_bounds(c, L, lse, r, mode, old, cached=chunk == 0)
    dw = out.dweight.cpu().numpy().astype(np.float64)
    assert not np.any(np.abs(dw - want_dw) > tol_dw), np.abs(dw - want_dw).max()
    n_live = int((c["mask"] != 0).sum())
    want_dh, tol_dh, want_dg, tol_dg = norm_grad_bounds(c, want_dy, tol_dy, n_live)
    dh = out.dhidden.cpu().numpy().astype(np.float64)
    edh = np.abs(dh - want_dh)
    assert not np.any(edh > tol_dh), f"dh: {(edh > tol_dh).sum()} out of tolerance, worst {edh.max():.3e}"
    assert np.all(dh[c["mask"].reshape(-1) == 0] == 0)
    dg = out.dnorm_weight.cpu().numpy().astype(np.float64)
    edg = np.abs(dg - want_dg)
    assert not np.any(edg > tol_dg), f"dgamma: {(edg > tol_dg).sum()} out of tolerance, worst {edg.max():.3e}"


def test_lmhead_final_norm_operand_bit_exact():
    """The norm's bf16 output, the LM head's operand, equals oracle.rmsnorm_operand bit
    for bit. With one live token the dW GEMM has K = 1, so dW[v, k] = D_v * y_k exactly
    (a product of two bf16 values is exact in f32), and y = y* holds iff
    dW[v, k] * y*_k0 == dW[v, k0] * y*_k for every k, exactly in float64."""
    T, H, V = 64, 896, 300
    c = make_norm_case(1, T, H, V, 1, seed=21, lengths=[T])
    ypos = orc.bf16_to_f32(c["hb"]).astype(np.float64)
    rng = np.random.default_rng(22)
    for t in rng.choice(T, 8, replace=False):
        mask = np.zeros((1, T), np.float32)
        mask[0, t] = 1.0
        print(f"final norm operand: live token {t}", flush=True)
        out = grpo.lmhead_fwd_bwd(dev(c["h"]), dev(c["wb"]), dev(c["ids"]), dev(mask), rewards=dev(np.ones(1, np.float32)),
                                  advantages=dev(np.full(1, 0.75, np.float32)), norm_weight=dev(c["gamma"]),
                                  norm_eps=c["eps"])
        torch.cuda.synchronize()
        dw = out.dweight.cpu().numpy().astype(np.float64)
        y = ypos[t]
        v = int(np.argmax(np.abs(dw).sum(1)))
        k0 = int(np.argmax(np.abs(y)))
        assert dw[v, k0] != 0 and y[k0] != 0
        assert np.array_equal(dw[v] * y[k0], dw[v, k0] * y), np.nonzero(dw[v] * y[k0] != dw[v, k0] * y)[0][:8]
        assert np.all(np.isfinite(dw))


def test_lmhead_final_norm_partial_gradients_and_errors():
    """dW alone (no gradient through the norm is formed), dgamma alone, the same values as
    with every gradient; dnorm_weight without norm_weight and hidden > 8192 are rejected."""
    c = make_norm_case(2, 32, 256, 700, 2, seed=9, lengths=[32, 9])
    mode = LossMode.REINFORCE
    old = np.zeros((2, 32), np.float32)
    full = run_device_norm(c, mode, old)
    mk = lambda **kw: grpo.LmheadOutputs(
        loss=torch.zeros((), device=DEV), logp=torch.zeros((2, 32), device=DEV), ref_logp=None,
        token_loss=torch.zeros((2, 32), device=DEV), advantages=torch.zeros(2, device=DEV), **kw)
    only_w = run_device_norm(c, mode, old, outputs=mk(dhidden=None, dweight=torch.empty((700, 256), device=DEV)))
    only_g = run_device_norm(c, mode, old, outputs=mk(dhidden=None, dweight=None,
                                                      dnorm_weight=torch.empty(256, device=DEV)))
    torch.cuda.synchronize()
    assert torch.equal(only_w.dweight, full.dweight)
    assert torch.equal(only_g.dnorm_weight, full.dnorm_weight)
    assert torch.equal(only_w.loss, full.loss)
    with pytest.raises(PcpError) as ei:
        grpo.lmhead_fwd_bwd(dev(c["h"]), dev(c["wb"]), dev(c["ids"]), dev(c["mask"]), rewards=dev(c["rewards"]),
                            outputs=mk(dhidden=None, dweight=None, dnorm_weight=torch.empty(256, device=DEV)))
    assert ei.value.code == -1
    hb = torch.zeros((64, 8256), dtype=torch.bfloat16, device=DEV)
    wb = torch.zeros((8, 8256), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(PcpError) as ei:
        grpo.lmhead_fwd_bwd(hb, wb, torch.zeros((1, 64), dtype=torch.int64, device=DEV),
                            rewards=torch.zeros(1, device=DEV), norm_weight=torch.ones(8256, device=DEV))
    assert ei.value.code == -1


# ---- real hidden and vocabulary sizes, few tokens, against the float64 oracle ---------------

@pytest.mark.parametrize("H", [4096, 896], ids=["H4096", "H896"])
def test_lmhead_qwen_vocab_vs_oracle(H):
    """The Qwen vocabulary with config 5's hidden size (4096) and Qwen2.5-0.5B's (896: 14
    stages, a half-filled last tile of the products' H side), 205 live tokens: the default
    (f16 softmax terms) backward, the exact one (PCP_FLAG_EXACT_BF16, f32 terms) and the
    recomputing one (16384-wide chunks) against the float64 oracle, each under its own
    bound."""
    cfg = synth.LMHEAD
    c = make_case(2, 128, H, cfg.V, 2, seed=17 + H, lengths=[128, 77], logit_std=cfg.std_w * np.sqrt(H))
    L, lse, rlse, old, r = oracle_case(c, LossMode.GRPO_CLIP_KL)
    bounds = {cached: grad_bounds(c, L, lse, r, LossMode.GRPO_CLIP_KL, old, cached=cached) for cached in (True, False)}
    for name, kw in (("cached", {}), ("exact", dict(exact_bf16=True)), ("chunked", dict(vocab_chunk=16384))):
        print(f"lmhead qwen-vocab N=256 H={H} V=151936 {name}", flush=True)
        out = run_device(c, LossMode.GRPO_CLIP_KL, old, **kw)
        torch.cuda.synchronize()
        check_forward(c, out, L, lse, rlse, r, LossMode.GRPO_CLIP_KL)
        check_grads(out, *bounds[name == "cached"])


# ---- configuration 5 at full size against torch fp32 ------------------------------------------

def _clip_kl_coef(lp, lr, old, adv, mask, cfg, lse):
    """Per-token clip + KL coefficients c from reference log-probs lp / lr (float64 [N]),
    formed by the oracle: the two-entry row [x, 0] with x = -log(expm1(-lp)) has
    log-softmax lp at its first entry, so oracle_grpo_rows on such rows (float64
    storage) computes c exactly as on the full rows. Also each token's coef_floor, what
    the 1e-5 * max(1, |lse|) log-prob bar allows in c."""
    S, T = mask.shape
    w = mask.reshape(-1).astype(np.float32)
    live = w != 0
    lpd = np.minimum(np.where(live, lp, -1.0), -1e-30)
    lrd = np.minimum(np.where(live, lr, -1.0), -1e-30)
    rows = lambda v: np.ascontiguousarray(np.stack([-np.log(np.expm1(-v)), np.zeros_like(v)], 1))
    L = np.maximum(mask.astype(np.float64).sum(1), 1.0).astype(np.float32)
    Ltok, Atok = np.repeat(L, T), np.repeat(adv, T)
    old = old.reshape(-1).astype(np.float32)
    r = orc.grpo_rows(rows(lpd), np.zeros(S * T, np.int64), w, Atok, Ltok, float(S), ref_logits=rows(lrd),
                      old_logp=old, loss_mode=orc.CLIP_KL, clip_eps=cfg.clip_eps, kl_beta=cfg.kl_beta,
                      dtype=orc.F64, want_dlogits=False)
    assert np.abs(r.lp[live] - lpd[live]).max() <= 1e-12 * np.abs(lpd[live]).max()
    tscale = np.maximum(1.0, np.abs(lse))
    fl = coef_floor(r.coef, r.lp, r.lr, w.astype(np.float64), Atok.astype(np.float64), Ltok.astype(np.float64),
                    float(S), old.astype(np.float64), False, cfg.kl_beta, cfg.clip_eps, tscale)
    return r.coef, fl, r.token_loss


def _torch_reference(inp, coef=None, chunk=2048, floor=None, cache_terms=None):
    """fp32 logp / lse per token, and with coef the gradients and their bounds; floor
    (per token) is the error c itself may carry (clip + KL: coef_floor), else c is
    exact up to f32 rounding (REINFORCE). The bounds include the f16 softmax terms'
    error, unless cache_terms (a dict) is given: that part of the bounds then goes to
    cache_terms["dh"] and cache_terms["dw"] (the bounds returned are those of dlogits
    rounded once, PCP_FLAG_EXACT_BF16)."""
    h, W, ids = inp["hidden"], inp["weight"], inp["ids"].reshape(-1)
    Wf = W.float()
    N = h.shape[0]
    lp = torch.empty(N, dtype=torch.float32, device=DEV)
    lse = torch.empty_like(lp)
    dh = tol_dh = dw = tol_dw = None
    if coef is not None:
        dh = torch.empty((N, Wf.shape[1]), dtype=torch.float32, device=DEV)
        tol_dh = torch.empty_like(dh)
        dw = torch.zeros_like(Wf)
        tol_dw = torch.zeros_like(Wf)
        Wa = Wf.abs()
        if cache_terms is not None:
            cache_terms["dh"] = torch.empty_like(dh)
            cache_terms["dw"] = torch.zeros_like(Wf)
    for n0 in range(0, N, chunk):
        hc = h[n0:n0 + chunk].float()
        Lc = hc @ Wf.T
        l = torch.logsumexp(Lc, dim=1)
        lse[n0:n0 + chunk] = l
        idc = ids[n0:n0 + chunk]
        lp[n0:n0 + chunk] = Lc.gather(1, idc[:, None])[:, 0] - l
        if coef is not None:
            cc = coef[n0:n0 + chunk]
            P = torch.exp(Lc - l[:, None])
            D = -P * cc[:, None]
            D.scatter_add_(1, idc[:, None], cc[:, None])
            E = (2.0 ** -8 + 1e-4) * D.abs()
            if floor is None:
                # c is exact up to f32 rounding (REINFORCE), so the softmax term carries
                # only the log-prob error: |c| * 1e-5 * max(1, |lse|) * p.
                E += (cc.abs() * 1e-5 * l.abs().clamp(min=1.0))[:, None] * P
            else:
                # The device's c and this one each lie within floor of the exact c:
                # 2 floor (onehot + p), as in grad_bounds.
                fc = 2.0 * floor[n0:n0 + chunk]
                E += fc[:, None] * P
                E.scatter_add_(1, idc[:, None], fc[:, None])
            # The default backward's f16 softmax cache (cache_error, in torch).
            V = Lc.shape[1]
            nb = (V + 127) // 128
            blk = torch.nn.functional.pad(Lc, (0, nb * 128 - V), value=-float("inf")).view(-1, nb, 128).amax(2)
            X = torch.exp(blk - l[:, None]).repeat_interleave(128, dim=1)[:, :V]
            X = (1 + 2.0 ** -7) * cc.abs()[:, None] * (2.0 ** -11 * P + 2.0 ** -25 * X)
            X.scatter_(1, idc[:, None], 0.0)
            if cache_terms is None:
                E += X
            else:
                cache_terms["dh"][n0:n0 + chunk] = X @ Wa
                cache_terms["dw"] += X.T @ hc.abs()
            del P, X, blk, Lc
            dh[n0:n0 + chunk] = D @ Wf
            tol_dh[n0:n0 + chunk] = E @ Wa
            dw += D.T @ hc
            tol_dw += E.T @ hc.abs()
            del D, E
    return lp, lse, dh, tol_dh, dw, tol_dw


def test_config5_full_size():
    cfg = synth.LMHEAD
    inp = synth.make_lmhead_inputs(cfg, DEV)
    S, T = cfg.S, cfg.T
    print("config 5 full size: reference log-probs", flush=True)
    lp_ref, lse_ref, *_ = _torch_reference(inp)
    old = (lp_ref.reshape(S, T) + inp["old_shift"]).contiguous()
    for mode in (LossMode.REINFORCE, LossMode.GRPO_CLIP_KL):
        print(f"config 5 full size: device mode={int(mode)}", flush=True)
        out = grpo.lmhead_fwd_bwd(inp["hidden"], inp["weight"], inp["ids"], inp["mask"],
                                  ref_weight=inp["ref_weight"], rewards=inp["rewards"], group_size=cfg.group,
                                  old_logp=old, loss_mode=mode, clip_eps=cfg.clip_eps, kl_beta=cfg.kl_beta)
        torch.cuda.synchronize()
        m = inp["mask"].reshape(-1) != 0
        sc = lse_ref.abs().clamp(min=1.0)
        err = (out.logp.reshape(-1) - lp_ref).abs()
        assert bool((err[m] <= 1e-5 * sc[m]).all()), float(err[m].max())
        e_lp = float((err / sc)[m].max())
        assert bool((out.logp.reshape(-1)[~m] == 0).all())
        # The loss is the masked sequence mean of the device's own token losses.
        L = inp["mask"].double().sum(1).clamp(min=1.0)
        tl = out.token_loss.double()
        seq = tl.sum(1) / L
        if mode == LossMode.REINFORCE:
            seq = seq * out.advantages.double()
        want = float(seq.sum() / S)
        assert abs(float(out.loss) - want) <= 1e-5 * float((tl.abs().sum(1) / L).sum() / S) + 1e-12
        adv = orc.advantages(inp["rewards"].cpu().numpy(), cfg.group)
        assert np.array_equal(out.advantages.cpu().numpy(), adv)
        if mode == LossMode.REINFORCE:
            # REINFORCE: c = -A * w / (L * G) needs no log-prob, so the gradients have
            # a reference independent of the device's forward.
            coef = (-torch.from_numpy(adv).to(DEV).double()[:, None] * inp["mask"].double() / (L[:, None] * S))
            print("config 5 full size: reference gradients", flush=True)
            cache = {}
            _, _, dh, tol_dh, dw, tol_dw = _torch_reference(inp, coef.float().reshape(-1), cache_terms=cache)
            # The default backward (f16 softmax terms) under the bound with their term, and
            # PCP_FLAG_EXACT_BF16 (f32 terms) under the bound of dlogits rounded once.
            exact = grpo.lmhead_fwd_bwd(inp["hidden"], inp["weight"], inp["ids"], inp["mask"],
                                        ref_weight=inp["ref_weight"], rewards=inp["rewards"], group_size=cfg.group,
                                        old_logp=old, loss_mode=mode, exact_bf16=True)
            torch.cuda.synchronize()
            assert torch.equal(exact.logp, out.logp) and torch.equal(exact.loss, out.loss)
            # The loss from the fp32 reference log-probs: -A * sum_t m lp / L, averaged.
            seq_ref = -(inp["mask"].double() * lp_ref.double().reshape(S, T)).sum(1) / L
            loss_ref = float((seq_ref * torch.from_numpy(adv).to(DEV).double()).sum() / S)
            e_loss = abs(float(out.loss) - loss_ref) / max(abs(loss_ref), 1e-30)
            terms = float(((inp["mask"].double() * lp_ref.double().reshape(S, T)).abs().sum(1) / L
                           * torch.from_numpy(np.abs(adv)).to(DEV).double()).sum() / S)
            e_terms = abs(float(out.loss) - loss_ref) / terms
            for name, res, th, tw in (("default", out, tol_dh + cache["dh"], tol_dw + cache["dw"]),
                                      ("exact", exact, tol_dh, tol_dw)):
                bad_h = ((res.dhidden - dh).abs() > th + 1e-6 * th.max()).sum().item()
                bad_w = ((res.dweight - dw).abs() > tw + 1e-6 * tw.max()).sum().item()
                used_h = float(((res.dhidden - dh).abs() / (th + 1e-30)).max())
                used_w = float(((res.dweight - dw).abs() / (tw + 1e-30)).max())
                print(f"  REINFORCE gradients, {name}: largest error / bound: dhidden {used_h:.3f}, dW {used_w:.3f}",
                      flush=True)
                print(f"PARITY-TABLE config5 reinforce {name}: |dlogp|/max(1,|lse|) {e_lp:.2e} (bar 1e-5); loss rel "
                      f"{e_loss:.2e}, per sum of |terms| {e_terms:.2e} (vs fp32 torch); dhidden max abs "
                      f"{float((res.dhidden - dh).abs().max()):.2e} "
                      f"({used_h:.3f} of its bound); dW max abs {float((res.dweight - dw).abs().max()):.2e} "
                      f"({used_w:.3f} of its bound)", flush=True)
                assert bad_h == 0 and bad_w == 0, (name, bad_h, bad_w)
            del dh, tol_dh, dw, tol_dw, cache, exact
        else:
            lr_ref, rlse_ref = _torch_reference({**inp, "weight": inp["ref_weight"]})[:2]
            err = (out.ref_logp.reshape(-1) - lr_ref).abs()
            assert bool((err[m] <= 1e-5 * sc[m] + 1e-5).all()), float(err[m].max())
            # clip + KL (the benchmark's mode): c from the fp32 reference log-probs through
            # the oracle, each token's coef_floor in the bound.
            print("config 5 full size: clip-KL reference gradients", flush=True)
            scale = torch.maximum(lse_ref.abs(), rlse_ref.abs()).double().cpu().numpy()
            coef, fl, tl_ref = _clip_kl_coef(lp_ref.double().cpu().numpy(), lr_ref.double().cpu().numpy(),
                                             old.cpu().numpy(), adv, inp["mask"].cpu().numpy(), cfg, scale)
            Lh = L.cpu().numpy()
            loss_ref = float((tl_ref.reshape(S, T).sum(1) / Lh).sum() / S)
            e_loss = abs(float(out.loss) - loss_ref) / max(abs(loss_ref), 1e-30)
            e_terms = abs(float(out.loss) - loss_ref) / float((np.abs(tl_ref).reshape(S, T).sum(1) / Lh).sum() / S)
            e_lr = float(((out.ref_logp.reshape(-1) - lr_ref).abs() / rlse_ref.abs().clamp(min=1.0))[m].max())
            _, _, dh, tol_dh, dw, tol_dw = _torch_reference(inp, torch.from_numpy(coef).float().to(DEV),
                                                            floor=torch.from_numpy(fl).float().to(DEV))
            bad_h = ((out.dhidden - dh).abs() > tol_dh + 1e-6 * tol_dh.max()).sum().item()
            bad_w = ((out.dweight - dw).abs() > tol_dw + 1e-6 * tol_dw.max()).sum().item()
            used_h = float(((out.dhidden - dh).abs() / (tol_dh + 1e-30)).max())
            used_w = float(((out.dweight - dw).abs() / (tol_dw + 1e-30)).max())
            print(f"  clip-KL gradients: largest error / bound: dhidden {used_h:.3f}, dW {used_w:.3f}", flush=True)
            print(f"PARITY-TABLE config5 clip_kl default: |dlogp|/max(1,|lse|) {e_lp:.2e} (bar 1e-5); ref {e_lr:.2e}; "
                  f"loss rel {e_loss:.2e}, per sum of |terms| {e_terms:.2e} (vs fp32 torch); dhidden max abs "
                  f"{float((out.dhidden - dh).abs().max()):.2e} "
                  f"({used_h:.3f} of its bound); dW max abs {float((out.dweight - dw).abs().max()):.2e} "
                  f"({used_w:.3f} of its bound)", flush=True)
            assert bad_h == 0 and bad_w == 0, (bad_h, bad_w)
            del dh, tol_dh, dw, tol_dw
        del out
        torch.cuda.empty_cache()


def test_lmhead_large_batch_cached_matches_chunked():
    """A batch whose backward workspace (about 26 GB at 40,960 tokens, V = 151,936,
    H = 4,096) is past the old 16 GiB cap takes the cached path and agrees with the
    chunked path on the same inputs: identical log-probs and loss terms (the same
    forward tiles), gradients within the f16 term's rounding (a misplaced tile or row
    would be off by O(1)), and not bit-identical (so the cache path did run)."""
    from dataclasses import replace
    cfg = replace(synth.LMHEAD, prompts=10)
    inp = synth.make_lmhead_inputs(cfg, DEV)
    print(f"lmhead large batch: {cfg.S * cfg.T} tokens", flush=True)
    kw = dict(ref_weight=inp["ref_weight"], rewards=inp["rewards"], group_size=cfg.group,
              loss_mode=LossMode.GRPO_CLIP_KL, clip_eps=cfg.clip_eps, kl_beta=cfg.kl_beta)
    first = grpo.lmhead_fwd_bwd(inp["hidden"], inp["weight"], inp["ids"], inp["mask"], want_grads=False, **kw)
    old = (first.logp + inp["old_shift"]).contiguous()
    del first
    cached = grpo.lmhead_fwd_bwd(inp["hidden"], inp["weight"], inp["ids"], inp["mask"], old_logp=old, **kw)
    torch.cuda.synchronize()
    chunked = grpo.lmhead_fwd_bwd(inp["hidden"], inp["weight"], inp["ids"], inp["mask"], old_logp=old,
                                  vocab_chunk=16384, **kw)
    torch.cuda.synchronize()
    assert torch.equal(cached.logp, chunked.logp) and torch.equal(cached.ref_logp, chunked.ref_logp)
    assert torch.equal(cached.token_loss, chunked.token_loss) and float(cached.loss) == float(chunked.loss)
    for name in ("dhidden", "dweight"):
        a, b = getattr(cached, name), getattr(chunked, name)
        rel = float((a - b).norm() / b.norm())
        worst = float((a - b).abs().max() / b.abs().max())
        print(f"  {name}: relative Frobenius difference {rel:.2e}, largest {worst:.2e}", flush=True)
        assert bool(torch.isfinite(a).all()) and rel < 2 ** -8 and worst < 2 ** -6, (name, rel, worst)
    assert not torch.equal(cached.dweight, chunked.dweight)
    # The chunked backward's low-memory form (K-major operands on the 32x32x16 tile, 32-bit
    # offsets within each 40,960 x 16,384 chunk): the same D as the chunked form. (Measured
    # bit-identical, both MFMA shapes adding the k products in the same order; the bar
    # leaves room for a different one.)
    del cached
    low = grpo.lmhead_fwd_bwd(inp["hidden"], inp["weight"], inp["ids"], inp["mask"], old_logp=old,
                              vocab_chunk=16384, low_memory_chunks=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(low.logp, chunked.logp) and float(low.loss) == float(chunked.loss)
    for name in ("dhidden", "dweight"):
        a, b = getattr(low, name), getattr(chunked, name)
        rel = float((a - b).norm() / b.norm())
        worst = float((a - b).abs().max() / b.abs().max())
        print(f"  low-memory {name}: relative Frobenius difference {rel:.2e}, largest {worst:.2e}", flush=True)
        assert bool(torch.isfinite(a).all()) and rel < 2 ** -16 and worst < 2 ** -12, (name, rel, worst)
