"""Row-kernel cases the sweep does not reach: peaked bf16 rows, where the resident
kernel's f16 softmax terms matter, and calls that leave dead rows unwritten
(PCP_FLAG_NO_ZERO_FILL) on every row kernel. Bars: tests/parity_tol.py."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from pcp_amd import grpo
from pcp_amd._lib import LossMode
from parity_tol import (assert_dlogits, dev, full_floor, full_loss_tol, host_bits, token_scale,
                        tok_to_rows)

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def peaked_case(V, S, T, seed):
    """bf16 rows whose two largest logits sit in one 16-byte vector (so one lane holds
    both, and the lane's largest term is 1), near-tied, with softmax mass 0.3-0.5 each."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((S, T, V)).astype(np.float32)
    ids = rng.integers(0, V, size=(S, T)).astype(np.int64)
    level = np.log(2.0 * V * np.exp(0.5))            # e^level = 2 * sum of the other terms
    for s in range(S):
        for t in range(T):
            q = int(rng.integers(0, V // 8))
            a, b = rng.choice(8, size=2, replace=False)
            i, j = 8 * q + a, 8 * q + b
            x[s, t, i] = level + rng.uniform(0.0, 0.3)
            x[s, t, j] = level + rng.uniform(0.0, 0.3)
            r = rng.random()
            ids[s, t] = i if r < 0.3 else (j if r < 0.5 else ids[s, t])
    ref = x + rng.standard_normal(x.shape).astype(np.float32) * 0.1
    lengths = rng.integers(T // 2, T + 1, size=S)
    mask = (np.arange(T)[None] < lengths[:, None]).astype(np.float32)
    rewards = rng.random(S).astype(np.float32)
    return orc.bf16_from_f32(x), orc.bf16_from_f32(ref), ids, mask, rewards


@pytest.mark.parametrize("V,S,T", [(1000, 8, 16), (151936, 4, 8)])
def test_peaked_bf16_rows(V, S, T):
    """Two near-tied dominant logits per row (p ~ 0.3-0.5 each) in one lane. By default
    the kernel's f16 softmax terms carry up to 2^-11 of these large dlogits, inside the
    cached bar; with PCP_FLAG_EXACT_BF16 every output is the f32 result rounded once,
    inside the exact bar. Where the term is in f16's normal range (|d| >= 2^-14 |c|) the
    two differ by at most one bf16 ulp, since 2^-11 of a value is under half its ulp."""
    x, ref, ids, mask, rewards = peaked_case(V, S, T, seed=V + S)
    G = 2
    sel = np.ascontiguousarray(x).reshape(S * T, V)
    lp, _ = orc.logprob(sel, ids.reshape(-1), dtype=orc.BF16)
    old = (lp.reshape(S, T) + np.random.default_rng(1).standard_normal((S, T)) * 0.05).astype(np.float32)
    want = orc.grpo_full(x, ids, mask, rows=T, rewards=rewards, group_size=G, ref_logits=ref, old_logp=old,
                         loss_mode=orc.CLIP_KL, dtype=orc.BF16)
    # The rows are peaked as intended: the largest softmax term of every row is 0.25 or more.
    xs = orc.bf16_to_f32(sel).astype(np.float64)
    p = np.exp(xs - xs.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert p.max(1).min() >= 0.25
    ts = token_scale(x, ids, T, 0, orc.BF16)
    fl = tok_to_rows(full_floor(want, mask, old, S, False, 0.04, 0.2, ts), T, 0, T)
    bits = {}
    for exact in (False, True):
        print(f"peaked bf16 rows: V={V} S={S} T={T} exact={exact}", flush=True)
        out = grpo.grpo_loss_fwd_bwd(dev(x), dev(ids), dev(mask), rewards=dev(rewards), group_size=G,
                                     ref_logits=dev(ref), old_logp=dev(old), loss_mode=LossMode.GRPO_CLIP_KL,
                                     exact_bf16=exact)
        torch.cuda.synchronize()
        assert np.all(np.abs(out.logp.cpu().numpy() - want.lp) <= 1e-5 * ts)
        bits[exact] = host_bits(out.dlogits)
        got = orc.bf16_to_f32(bits[exact])
        assert_dlogits(got, want.dlogits, fl, True, exact=exact)
        err = np.abs(got.astype(np.float64) - want.dlogits)
        cabs = np.abs(want.coef)[..., None]
        big = (np.abs(want.dlogits) >= 0.05 * cabs) & (cabs > 0)
        rel = (err[big] / np.abs(want.dlogits[big])).max()
        print(f"  worst relative error where |d| >= 0.05|c|: {rel:.3e} (bf16 unit roundoff {2.0 ** -8:.3e})",
              flush=True)
        assert abs(float(out.loss.cpu()) - want.loss) <= full_loss_tol(want, x, ids, mask, T, 0, orc.BF16, False,
                                                                       0.04, S)
    c = np.abs(want.coef)[..., None] * np.ones((1, 1, V))
    normal = np.abs(want.dlogits) >= 2.0 ** -14 * c
    a = bits[False].astype(np.int32)
    b = bits[True].astype(np.int32)
    same_sign = (a >> 15) == (b >> 15)
    ulps = np.abs((a & 0x7FFF) - (b & 0x7FFF))
    assert np.all(same_sign[normal] | (ulps[normal] == 0)) and ulps[normal].max() <= 1
    print(f"  cached vs exact: {np.mean(ulps[normal] != 0):.2%} of normal-range elements one ulp apart", flush=True)


# (kind, logits dtype, V, dlogits dtype, force_streaming, shifted layout, live fraction of the mask)
ZF_CASES = [
    ("resident", "bf16", 4096, "bf16", False, False, 0.7),
    ("resident-sparse", "bf16", 4096, "bf16", False, False, 0.25),
    ("resident-shifted", "bf16", 151936, "bf16", False, True, 0.7),
    ("resident-shifted-sparse", "bf16", 151936, "bf16", False, True, 0.2),
    ("resident-edge", "bf16", 5003, "bf16", False, True, 0.7),
    ("resident-edge-sparse", "bf16", 5003, "bf16", False, False, 0.3),
    ("resident-f32", "f32", 3000, "f32", False, False, 0.7),
    ("resident-f32-sparse", "f32", 3000, "f32", False, True, 0.25),
    ("resident-bf16-to-f32", "bf16", 4096, "f32", False, True, 0.7),
    ("resident-bf16-to-f32-qwen", "bf16", 151936, "f32", False, False, 0.7),
    ("resident-bf16-to-f32-qwen-sparse", "bf16", 151936, "f32", False, True, 0.25),
    ("stream-vec", "bf16", 4096, "bf16", True, True, 0.7),
    ("stream-scalar", "bf16", 5003, "f32", False, False, 0.7),
]


@pytest.mark.parametrize("kind,dt,V,odt,stream,shifted,live", ZF_CASES, ids=[c[0] for c in ZF_CASES])
def test_no_zero_fill_leaves_dead_rows(kind, dt, V, odt, stream, shifted, live):
    """PCP_FLAG_NO_ZERO_FILL: dlogits rows of masked, ignored (-100) and pad tokens keep
    what the caller put there, bit for bit; live rows match the oracle. Resident
    (aligned and off-16-byte rows), f32 and mixed-precision, and both streaming kernels.
    The persistent kernels visit only the listed live rows when fewer than half the rows
    are live (the sparse cases) and every row otherwise."""
    rng = np.random.default_rng(V + 7 * len(kind))
    S, T, G = 4, 9, 2
    rows, off = (T - 1, 1) if shifted else (T, 0)
    x32 = rng.standard_normal((S, T, V)).astype(np.float32) * 3
    r32 = x32 + rng.standard_normal((S, T, V)).astype(np.float32) * 0.1
    if dt == "bf16":
        x, ref, odt_orc = orc.bf16_from_f32(x32), orc.bf16_from_f32(r32), orc.BF16
    else:
        x, ref, odt_orc = x32, r32, orc.F32
    ids = rng.integers(0, V, size=(S, T)).astype(np.int64)
    ids[rng.random((S, T)) < 0.15] = -100
    mask = (rng.random((S, T)) < live).astype(np.float32)
    mask[1] = 0.0                                        # one empty sequence
    rewards = np.array([1.0, 0.0, 0.25, 0.75], np.float32)
    sel = np.ascontiguousarray(x[:, :rows]).reshape(S * rows, V)
    lp, _ = orc.logprob(sel, np.clip(ids[:, off:off + rows].reshape(-1), 0, None), dtype=odt_orc)
    old = np.zeros((S, T), np.float32)
    old[:, off:off + rows] = (lp.reshape(S, rows) + rng.standard_normal((S, rows)) * 0.05).astype(np.float32)
    tdt = {"bf16": torch.bfloat16, "f32": torch.float32}[odt]
    sentinel = -3.5
    dl = torch.full((S, T, V), sentinel, dtype=tdt, device=DEV)
    print(f"no zero-fill: {kind} {dt}->{odt} V={V} streaming={stream} shifted={shifted}", flush=True)
    out = grpo.grpo_loss_fwd_bwd(dev(x), dev(ids), dev(mask), rewards=dev(rewards), group_size=G,
                                 ref_logits=dev(ref), old_logp=dev(old), loss_mode=LossMode.GRPO_CLIP_KL,
                                 rows=rows, tok_offset=off, dlogits=dl, zero_fill=False, force_streaming=stream)
    torch.cuda.synchronize()
    want = orc.grpo_full(x, ids, mask, rows=rows, tok_offset=off, rewards=rewards, group_size=G, ref_logits=ref,
                         old_logp=old, loss_mode=orc.CLIP_KL, dtype=odt_orc)
    got_bits = host_bits(out.dlogits)
    sent_bits = host_bits(torch.full((1,), sentinel, dtype=tdt))[0]
    dead = np.zeros((S, T), bool)
    for s in range(S):
        for t in range(T):
            dead[s, t] = t >= rows or mask[s, off + t] == 0 or ids[s, off + t] == -100
    assert dead.any() and (~dead).any()
    assert np.all(got_bits[dead] == sent_bits), "a dead row was written"
    ts = token_scale(x, ids, rows, off, odt_orc)
    fl = tok_to_rows(full_floor(want, mask, old, S, False, 0.04, 0.2, ts), rows, off, T)
    got = orc.bf16_to_f32(got_bits) if odt == "bf16" else got_bits.astype(np.float32)
    assert_dlogits(got[~dead], want.dlogits[~dead], fl[~dead], odt == "bf16")
    assert abs(float(out.loss.cpu()) - want.loss) <= full_loss_tol(want, x, ids, mask, rows, off, odt_orc, False,
                                                                   0.04, S)


# (logits dtype, V, dlogits dtype): aligned rows, several listed rows per workgroup
LISTED_CASES = [("bf16", 32768, "bf16"), ("bf16", 32768, "f32"), ("f32", 8192, "f32")]


@pytest.mark.parametrize("dt,V,odt", LISTED_CASES, ids=[f"{c[0]}-{c[1]}-{c[2]}" for c in LISTED_CASES])
def test_no_zero_fill_listed_rows_prefetch(dt, V, odt):
    """Without zero-fill and a quarter of the rows live, the resident kernel walks the
    listed live rows, several per workgroup here, loading each next row's policy chunks
    during the current row's dlogits pass (on 1024-lane instances of 2 and 4 chunks and
    the split-half bf16 -> f32 instance). Every live row against the oracle, dead rows
    untouched bit for bit."""
    rng = np.random.default_rng(V + len(dt) + len(odt))
    S, T, G = 16, 512, 4
    x32 = rng.standard_normal((S, T, V)).astype(np.float32) * 3
    r32 = x32 + rng.standard_normal((S, T, V)).astype(np.float32) * 0.1
    if dt == "bf16":
        x, ref, odt_orc = orc.bf16_from_f32(x32), orc.bf16_from_f32(r32), orc.BF16
    else:
        x, ref, odt_orc = x32, r32, orc.F32
    del x32, r32
    ids = rng.integers(0, V, size=(S, T)).astype(np.int64)
    ids[rng.random((S, T)) < 0.05] = -100
    mask = (rng.random((S, T)) < 0.27).astype(np.float32)
    rewards = rng.random(S).astype(np.float32)
    lp, _ = orc.logprob(np.ascontiguousarray(x).reshape(S * T, V), np.clip(ids.reshape(-1), 0, None), dtype=odt_orc)
    old = (lp.reshape(S, T) + rng.standard_normal((S, T)) * 0.05).astype(np.float32)
    tdt = {"bf16": torch.bfloat16, "f32": torch.float32}[odt]
    sentinel = -3.5
    dl = torch.full((S, T, V), sentinel, dtype=tdt, device=DEV)
    dead = (mask == 0) | (ids == -100)
    assert 2 * int((~dead).sum()) < S * T          # the listed path
    print(f"listed rows: {dt}->{odt} V={V}, {int((~dead).sum())} live of {S * T}", flush=True)
    out = grpo.grpo_loss_fwd_bwd(dev(x), dev(ids), dev(mask), rewards=dev(rewards), group_size=G,
                                 ref_logits=dev(ref), old_logp=dev(old), loss_mode=LossMode.GRPO_CLIP_KL,
                                 dlogits=dl, zero_fill=False)
    torch.cuda.synchronize()
    want = orc.grpo_full(x, ids, mask, rows=T, rewards=rewards, group_size=G, ref_logits=ref, old_logp=old,
                         loss_mode=orc.CLIP_KL, dtype=odt_orc)
    got_bits = host_bits(out.dlogits)
    sent_bits = host_bits(torch.full((1,), sentinel, dtype=tdt))[0]
    assert np.all(got_bits[dead] == sent_bits), "a dead row was written"
    ts = token_scale(x, ids, T, 0, odt_orc)
    fl = tok_to_rows(full_floor(want, mask, old, S, False, 0.04, 0.2, ts), T, 0, T)
    got = orc.bf16_to_f32(got_bits) if odt == "bf16" else got_bits.astype(np.float32)
    assert_dlogits(got[~dead], want.dlogits[~dead], fl[~dead], odt == "bf16")
    assert abs(float(out.loss.cpu()) - want.loss) <= full_loss_tol(want, x, ids, mask, T, 0, odt_orc, False, 0.04, S)


# Live-row counts around the persistent grid's size (one workgroup per resident slot,
# a few hundred to about a thousand here): none, one, fewer than the grid, between one
# and two grids (the second rows come from the first claim, not the counter), more,
# and either side of the switch to visiting every row (half of 8192 rows).
LIVE_COUNTS = [0, 1, 37, 255, 256, 257, 511, 512, 513, 767, 1023, 1024, 1025, 1537, 2049, 4095, 4096]


@pytest.fixture(scope="module")
def count_inputs():
    S, T, V = 16, 512, 4096
    gen = torch.Generator(device=DEV)
    gen.manual_seed(77)
    x = torch.randn((S, T, V), generator=gen, device=DEV) * 3
    r = x + torch.randn((S, T, V), generator=gen, device=DEV) * 0.1
    ids = torch.randint(0, V, (S, T), generator=gen, device=DEV)
    old = torch.randn((S, T), generator=gen, device=DEV) * 0.05 - float(np.log(V))
    rewards = torch.rand((S,), generator=gen, device=DEV)
    return dict(S=S, T=T, V=V, x={"bf16": x.to(torch.bfloat16), "f32": x}, r={"bf16": r.to(torch.bfloat16), "f32": r},
                ids=ids, old=old, rewards=rewards)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("n_live", LIVE_COUNTS)
def test_no_zero_fill_live_counts(count_inputs, n_live, dt):
    """Exactly n_live live rows at random places: the call without zero-fill (listed rows
    with the next-row prefetch below half live, every row in order from half on) gives
    the zero-fill call's outputs bit for bit on live rows and leaves every dead row's
    dlogits as they were."""
    c = count_inputs
    S, T, V = c["S"], c["T"], c["V"]
    rng = np.random.default_rng(1000 + n_live)
    flat = np.zeros(S * T, np.float32)
    flat[rng.choice(S * T, size=n_live, replace=False)] = 1.0
    mask = torch.from_numpy(flat.reshape(S, T)).to(DEV)
    kw = dict(rewards=c["rewards"], group_size=4, ref_logits=c["r"][dt], old_logp=c["old"],
              loss_mode=LossMode.GRPO_CLIP_KL)
    x = c["x"][dt]
    sentinel = -3.5
    dl = torch.full((S, T, V), sentinel, dtype=x.dtype, device=DEV)
    print(f"live rows {n_live} of {S * T} ({dt})", flush=True)
    got = grpo.grpo_loss_fwd_bwd(x, c["ids"], mask, dlogits=dl, zero_fill=False, **kw)
    want = grpo.grpo_loss_fwd_bwd(x, c["ids"], mask, **kw)
    torch.cuda.synchronize()
    live = mask != 0
    assert torch.equal(got.dlogits[live], want.dlogits[live])
    assert bool((got.dlogits[~live] == sentinel).all()), "a dead row was written"
    assert bool((want.dlogits[~live] == 0).all())
    for f in ("loss", "logp", "ref_logp", "token_loss", "advantages"):
        assert torch.equal(getattr(got, f), getattr(want, f)), f
