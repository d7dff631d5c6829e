"""pcp_grpo_loss_fwd_bwd_noalloc against pcp_grpo_loss_fwd_bwd, through the C ABI.

The allocation-free entry point runs the same kernels on work buffers taken from the
GPU's static array, so its results must equal the allocating entry point's bit for bit.
Two calls in a row, the second on a smaller input, check that contents the first call
left in the shared array do not leak into the second. Both the per-token losses in the
array (token_loss NULL) and caller-supplied ones are covered, and the loss is checked
against the CPU oracle as well.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from pcp_amd import _lib, grpo
from pcp_amd._lib import LossMode, check, lib

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def make_case(seed, S, T, V, G, mode, max_len=None):
    rng = np.random.default_rng(seed)
    pol = (rng.standard_normal((S, T, V), dtype=np.float32) * 3).astype(np.float32)
    ref = pol + rng.standard_normal((S, T, V), dtype=np.float32) * 0.1
    ids = rng.integers(0, V, size=(S, T)).astype(np.int64)
    lengths = rng.integers(1, (max_len or T) + 1, size=S)
    mask = (np.arange(T)[None] < lengths[:, None]).astype(np.float32)
    rewards = rng.random(S).astype(np.float32)
    old = (rng.standard_normal((S, T)) * 0.01 - np.log(V)).astype(np.float32)
    return dict(pol=orc.bf16_from_f32(pol), ref=orc.bf16_from_f32(ref), ids=ids, mask=mask, rewards=rewards,
                old=old, S=S, T=T, V=V, G=G, mode=mode)


def bf16_dev(h):
    return torch.from_numpy(h.view(np.int16)).to(DEV).view(torch.bfloat16)


def run(c, noalloc, token_loss_out, flags=0):
    """One call through the C ABI; token_loss_out False leaves token_loss NULL so the
    library keeps the per-token losses in its work buffers. dlogits start as 7.0, so
    rows a PCP_FLAG_NO_ZERO_FILL call leaves untouched keep that value."""
    S, T, V = c["S"], c["T"], c["V"]
    pol, ref = bf16_dev(c["pol"]), bf16_dev(c["ref"])
    ids = torch.from_numpy(c["ids"]).to(DEV)
    mask = torch.from_numpy(c["mask"]).to(DEV)
    rewards = torch.from_numpy(c["rewards"]).to(DEV)
    old = torch.from_numpy(c["old"]).to(DEV)
    dl = torch.full((S, T, V), 7.0, dtype=torch.bfloat16, device=DEV)
    logp = torch.zeros((S, T), dtype=torch.float32, device=DEV)
    ref_logp = torch.zeros_like(logp)
    tl = torch.zeros_like(logp) if token_loss_out else None
    adv = torch.zeros(S, dtype=torch.float32, device=DEV)
    loss = torch.zeros((), dtype=torch.float32, device=DEV)
    a = _lib.default_args()
    grpo.fill_args(a, pol, ids, mask, T, 0, S, T, V, T)
    a.group_size = c["G"]
    a.ref_logits = ref.data_ptr() if c["mode"] == LossMode.GRPO_CLIP_KL else None
    a.old_logp = old.data_ptr()
    a.rewards = rewards.data_ptr()
    a.dlogits = dl.data_ptr()
    a.dlogits_dtype = int(_lib.DType.bf16)
    a.logp, a.ref_logp = logp.data_ptr(), ref_logp.data_ptr()
    a.token_loss = tl.data_ptr() if tl is not None else None
    a.advantages_out, a.loss = adv.data_ptr(), loss.data_ptr()
    a.loss_mode = int(c["mode"])
    a.flags = flags
    a.stream = torch.cuda.current_stream().cuda_stream or None
    ctx = grpo.default_context(0)
    fn = lib().pcp_grpo_loss_fwd_bwd_noalloc if noalloc else lib().pcp_grpo_loss_fwd_bwd
    check(fn(ctx.handle, ctypes.byref(a)), ctx.handle)
    torch.cuda.synchronize()
    out = dict(loss=loss.cpu().numpy(), dl=dl.view(torch.int16).cpu().numpy(), logp=logp.cpu().numpy(),
               ref_logp=ref_logp.cpu().numpy(), adv=adv.cpu().numpy())
    if tl is not None:
        out["tl"] = tl.cpu().numpy()
    return out


def assert_same(got, want):
    for k in want:
        g, w = np.atleast_1d(got[k]), np.atleast_1d(want[k])
        assert g.shape == w.shape and np.array_equal(g.view(np.uint8), w.view(np.uint8)), f"{k} differs"


@pytest.mark.parametrize("token_loss_out", [False, True])
def test_noalloc_matches_allocating_entry_point_two_calls(token_loss_out):
    big = make_case(1, S=8, T=96, V=5003, G=4, mode=LossMode.GRPO_CLIP_KL)
    small = make_case(2, S=4, T=40, V=3000, G=2, mode=LossMode.REINFORCE)
    print(f"noalloc: token_loss_out={token_loss_out} big S=8 T=96 V=5003 then small S=4 T=40 V=3000", flush=True)
    for c in (big, small):
        got = run(c, True, token_loss_out)
        want = run(c, False, token_loss_out)
        assert_same(got, want)
        exp = orc.grpo_full(c["pol"], c["ids"], c["mask"], rows=c["T"], rewards=c["rewards"], group_size=c["G"],
                            ref_logits=c["ref"] if c["mode"] == LossMode.GRPO_CLIP_KL else None,
                            old_logp=c["old"], loss_mode=int(c["mode"]), dtype=orc.BF16)
        # The f32 log-prob bar (1e-5 of the row scale, here |lse| < 20) through the loss's
        # linear aggregation: at most 1e-5 * 20 * mean_s |A_s| * (|rho| + beta) per sequence.
        scale = 20.0 * float(np.abs(exp.adv).mean() * 1.5 + 0.04) + abs(exp.loss)
        assert abs(float(got["loss"]) - exp.loss) <= 1e-5 * scale, (got["loss"], exp.loss)


def test_noalloc_without_zero_fill_walks_the_listed_rows():
    """PCP_FLAG_NO_ZERO_FILL keeps the live-row list and its count in the static array.
    With under half the rows live the row kernel visits the listed rows only; the
    results equal the allocating call's bit for bit, dead rows keep their 7.0 fill, and
    a second, smaller call on the shared array does the same."""
    big = make_case(3, S=8, T=96, V=5003, G=4, mode=LossMode.GRPO_CLIP_KL, max_len=30)
    small = make_case(4, S=4, T=40, V=3000, G=2, mode=LossMode.REINFORCE, max_len=12)
    print("noalloc no-zero-fill: big S=8 T=96 V=5003 then small S=4 T=40 V=3000", flush=True)
    seven = np.array([7.0], np.float32).view(np.uint32)[0] >> 16
    for c in (big, small):
        assert 2 * int(c["mask"].sum()) < c["mask"].size, "the case must leave under half the rows live"
        got = run(c, True, False, _lib.FLAG_NO_ZERO_FILL)
        want = run(c, False, False, _lib.FLAG_NO_ZERO_FILL)
        assert_same(got, want)
        dead = c["mask"] == 0
        assert (got["dl"][dead].view(np.uint16) == seven).all(), "a dead row was written"
        assert not (got["dl"][~dead].view(np.uint16) == seven).all(axis=-1).any(), "a live row was not written"
        exp = orc.grpo_full(c["pol"], c["ids"], c["mask"], rows=c["T"], rewards=c["rewards"], group_size=c["G"],
                            ref_logits=c["ref"] if c["mode"] == LossMode.GRPO_CLIP_KL else None,
                            old_logp=c["old"], loss_mode=int(c["mode"]), dtype=orc.BF16)
        scale = 20.0 * float(np.abs(exp.adv).mean() * 1.5 + 0.04) + abs(exp.loss)
        assert abs(float(got["loss"]) - exp.loss) <= 1e-5 * scale, (got["loss"], exp.loss)


@pytest.mark.parametrize("overflow", ["token_loss", "row_list"])
def test_noalloc_rejects_requests_beyond_its_array(overflow):
    # 2^20 + 1 rows do not fit next to the other buffers in 4 MiB: as per-token losses
    # (token_loss NULL), or as the live-row list alone (token_loss given, dlogits without
    # zero-fill: one 4-byte entry per row).
    a = _lib.default_args()
    a.n_seq, a.rows, a.vocab, a.group_size = 1, (1 << 20) + 1, 16, 1
    a.logits, a.ids, a.advantages = 0x1000, 0x2000, 0x3000
    if overflow == "row_list":
        a.token_loss, a.dlogits, a.flags = 0x4000, 0x5000, _lib.FLAG_NO_ZERO_FILL
    ctx = grpo.default_context(0)
    rc = lib().pcp_grpo_loss_fwd_bwd_noalloc(ctx.handle, ctypes.byref(a))
    assert rc == -9
    assert b"allocation-free" in lib().pcp_last_error(ctx.handle)
