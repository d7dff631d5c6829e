"""Seeded random sweep of the loss head (pcp_grpo_loss_fwd_bwd) against the CPU oracle:
vocabulary sizes from 1 to 151,936, f32 / bf16 / f16 logits, the aligned and the
reference's shifted layout, ignored (-100) ids, empty sequences, both loss modes, and
the resident and streaming kernels. The bars are those of tests/parity_tol.py.
A one-off run of the same generator over seeds 16-175 (both kernels, all passing with
the f16 subnormal term of assert_dlogits) found the cases that term covers."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from pcp_amd import grpo
from pcp_amd._lib import LossMode
from parity_tol import assert_dlogits, dev, full_floor, full_loss_tol, host_bits, lse_scale, tok_to_rows

pytestmark = pytest.mark.gpu

VOCABS = [1, 2, 7, 64, 129, 1000, 4095, 8192, 8193, 20000, 151936, 300, 5000, 16, 3000, 12345]
DTYPES = ["f32", "bf16", "f16"]


def make_case(k):
    rng = np.random.default_rng(1000 + k)
    V = VOCABS[k % len(VOCABS)]
    dt = DTYPES[k % 3]
    G = 1 if k % 8 == 0 else int(rng.choice([2, 3]))           # G = 1: zero advantages
    S = G * int(rng.integers(1, 3))
    T = 3 if V > 100000 else int(rng.integers(2, 40))
    shifted = bool(k % 2)
    rows, off = (T - 1, 1) if shifted else (T, 0)
    mode = LossMode.GRPO_CLIP_KL if k % 4 < 2 else LossMode.REINFORCE
    x = rng.standard_normal((S, T, V)).astype(np.float32) * float(rng.choice([1.0, 3.0]))
    if V > 1 and k % 5 == 0:
        x[0, 0, rng.integers(0, V)] = 60.0                       # one dominant logit
    ref = x + rng.standard_normal((S, T, V)).astype(np.float32) * 0.1
    lengths = rng.integers(0, T + 1, size=S)                     # empty sequences allowed
    mask = (np.arange(T)[None] < lengths[:, None]).astype(np.float32)
    ids = rng.integers(0, V, size=(S, T)).astype(np.int64)
    ids[rng.random((S, T)) < 0.1] = -100                         # ignored tokens, masked or not
    rewards = rng.random(S).astype(np.float32) if k % 3 else rng.integers(0, 2, size=S).astype(np.float32)
    if dt == "bf16":
        store, ref_store, odt = orc.bf16_from_f32(x), orc.bf16_from_f32(ref), orc.BF16
    elif dt == "f16":
        store, ref_store, odt = x.astype(np.float16), ref.astype(np.float16), orc.F16
    else:
        store, ref_store, odt = x, ref, orc.F32
    old = None
    if mode == LossMode.GRPO_CLIP_KL:
        sel = np.ascontiguousarray(store[:, :rows]).reshape(S * rows, V)
        lp, _ = orc.logprob(sel, np.clip(ids[:, off:off + rows].reshape(-1), 0, None), dtype=odt)
        old = np.zeros((S, T), np.float32)
        old[:, off:off + rows] = (lp.reshape(S, rows) + rng.standard_normal((S, rows)) * 0.1).astype(np.float32)
    return dict(S=S, T=T, V=V, G=G, rows=rows, off=off, mode=mode, dt=dt, odt=odt, store=store,
                ref=ref_store if mode == LossMode.GRPO_CLIP_KL else None, ids=ids, mask=mask, rewards=rewards, old=old)


@pytest.mark.parametrize("streaming", [False, True])
# Three passes over the vocabularies with other seeds, and two seeds whose clip-KL rows
# have coefficients near 1e-5, which puts their f16 dlogits among f16's subnormals.
@pytest.mark.parametrize("k", list(range(3 * len(VOCABS))) + [77, 125])
def test_random_case_vs_oracle(k, streaming):
    c = make_case(k)
    S, T, V, rows, off = c["S"], c["T"], c["V"], c["rows"], c["off"]
    reinforce = c["mode"] == LossMode.REINFORCE
    print(f"random case {k}: S={S} T={T} V={V} {c['dt']} rows={rows} off={off} mode={int(c['mode'])} "
          f"streaming={streaming}", flush=True)
    kw = dict(rewards=dev(c["rewards"]), group_size=c["G"], loss_mode=c["mode"], rows=rows, tok_offset=off,
              force_streaming=streaming)
    if c["ref"] is not None:
        kw["ref_logits"] = dev(c["ref"])
        kw["old_logp"] = dev(c["old"])
    out = grpo.grpo_loss_fwd_bwd(dev(c["store"]), dev(c["ids"]), dev(c["mask"]), **kw)
    torch.cuda.synchronize()
    want = orc.grpo_full(c["store"], c["ids"], c["mask"], rows=rows, tok_offset=off, rewards=c["rewards"],
                         group_size=c["G"], ref_logits=c["ref"], old_logp=c["old"],
                         loss_mode=orc.REINFORCE if reinforce else orc.CLIP_KL, dtype=c["odt"])
    sel = np.ascontiguousarray(c["store"][:, :rows]).reshape(S * rows, V)
    scale = np.ones((S, T))
    scale[:, off:off + rows] = lse_scale(sel, c["ids"][:, off:off + rows].reshape(-1), c["odt"]).reshape(S, rows)
    assert np.all(np.abs(out.logp.cpu().numpy() - want.lp) <= 1e-5 * scale)
    if not reinforce:
        rsel = np.ascontiguousarray(c["ref"][:, :rows]).reshape(S * rows, V)
        rscale = np.ones((S, T))
        rscale[:, off:off + rows] = lse_scale(rsel, c["ids"][:, off:off + rows].reshape(-1), c["odt"]).reshape(S, rows)
        assert np.all(np.abs(out.ref_logp.cpu().numpy() - want.lr) <= 1e-5 * rscale)
    assert np.all(np.abs(out.token_loss.cpu().numpy() - want.token_loss) <= 1e-5 * scale)
    assert np.array_equal(out.advantages.cpu().numpy(), want.adv)
    assert abs(float(out.loss.cpu()) - want.loss) <= full_loss_tol(
        want, c["store"], c["ids"], c["mask"], rows, off, c["odt"], reinforce, 0.04, S)
    floor = tok_to_rows(full_floor(want, c["mask"], c["old"], S, reinforce, 0.04, 0.2, scale), rows, off, T)
    got = host_bits(out.dlogits)
    got = orc.bf16_to_f32(got) if c["dt"] == "bf16" else got.astype(np.float32)
    assert_dlogits(got, want.dlogits, floor, c["dt"] != "f32", f16_out=c["dt"] == "f16")
    # rows without a live token (masked, ignored, pad) are exactly zero
    d = host_bits(out.dlogits)
    for s in range(S):
        for t in range(T):
            dead = t >= rows or c["mask"][s, off + t] == 0 or c["ids"][s, off + t] == -100
            if dead:
                assert not np.any(d[s, t]), (s, t)
