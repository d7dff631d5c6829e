"""Token-array dtypes through the C ABI: ids as i64 or i32, masks as f32 or bool (u8).

The kernels read either id width and either mask type through the same index
arithmetic, so a 0/1 mask and its bool (or 0/1 uint8) form, and an id array and its i32
copy, must give the same outputs bit for bit on every path: the resident row kernel
(bf16 and f32 logits), the streaming fallback, the listed rows without zero-fill, the
shifted reference layout, forward-only log-probs and the fused LM head. The i64 / f32
forms are the ones every other GPU test checks against the oracle.
"""
import numpy as np
import pytest
import torch

from pcp_amd import grpo
from pcp_amd._lib import LossMode

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
S, T, V, G = 8, 64, 4096, 4

# (ids dtype, mask dtype); the first is the reference form.
FORMS = [(torch.int64, torch.float32), (torch.int32, torch.float32), (torch.int64, torch.bool),
         (torch.int32, torch.bool), (torch.int32, torch.uint8)]
FORM_IDS = ["i64-f32", "i32-f32", "i64-bool", "i32-bool", "i32-u8"]


def token_arrays(seed, max_len):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, V, size=(S, T)).astype(np.int64)
    ids[rng.random((S, T)) < 0.1] = -100
    lengths = rng.integers(1, max_len + 1, size=S)
    mask = (np.arange(T)[None] < lengths[:, None]).astype(np.float32)
    mask[rng.random((S, T)) < 0.05] = 0.0      # holes inside the live spans
    return torch.from_numpy(ids).to(DEV), torch.from_numpy(mask).to(DEV)


def as_form(ids, mask, form):
    idt, mdt = form
    return ids.to(idt), (mask != 0).to(mdt) if mdt != torch.float32 else mask


@pytest.fixture(scope="module")
def logits():
    gen = torch.Generator(device=DEV)
    gen.manual_seed(11)
    x = torch.randn((S, T, V), generator=gen, device=DEV) * 3
    r = x + torch.randn((S, T, V), generator=gen, device=DEV) * 0.1
    old = torch.randn((S, T), generator=gen, device=DEV) * 0.05 - float(np.log(V))
    rewards = torch.rand((S,), generator=gen, device=DEV)
    return dict(x=x, r=r, old=old, rewards=rewards)


LOSS_PATHS = {
    # name: (logits dtype, max sequence length, keyword arguments)
    "resident-bf16": (torch.bfloat16, T, {}),
    "resident-f32": (torch.float32, T, {}),
    "streaming-bf16": (torch.bfloat16, T, dict(force_streaming=True)),
    "listed-no-zero-fill": (torch.bfloat16, 20, dict(zero_fill=False)),
    "shifted-bf16": (torch.bfloat16, T, dict(rows=T - 1, tok_offset=1)),
}


@pytest.mark.parametrize("path", list(LOSS_PATHS))
def test_loss_token_dtypes_bit_identical(logits, path):
    dt, max_len, kw = LOSS_PATHS[path]
    ids, mask = token_arrays(len(path), max_len)
    x, r = logits["x"].to(dt), logits["r"].to(dt)
    outs = []
    for form, name in zip(FORMS, FORM_IDS):
        i, m = as_form(ids, mask, form)
        dl = torch.full((S, T, V), -2.0, dtype=dt, device=DEV)   # rows left unwritten keep this
        print(f"loss path {path}, ids / mask {name}", flush=True)
        outs.append(grpo.grpo_loss_fwd_bwd(x, i, m, rewards=logits["rewards"], group_size=G, ref_logits=r,
                                           old_logp=logits["old"], loss_mode=LossMode.GRPO_CLIP_KL,
                                           dlogits=dl, **kw))
    live = int((mask != 0).sum())
    assert 0 < live < S * T
    for o, name in zip(outs[1:], FORM_IDS[1:]):
        for f in ("loss", "dlogits", "logp", "ref_logp", "token_loss", "advantages"):
            assert torch.equal(getattr(o, f), getattr(outs[0], f)), (path, name, f)


@pytest.mark.parametrize("force_streaming", [False, True], ids=["forward-kernel", "streaming"])
def test_logprob_token_dtypes_bit_identical(logits, force_streaming):
    ids, mask = token_arrays(5, T)
    x, r = logits["x"].to(torch.bfloat16), logits["r"].to(torch.bfloat16)
    outs = []
    for form in FORMS:
        i, m = as_form(ids, mask, form)
        outs.append(grpo.logprob_fwd(x, i, r, mask=m, force_streaming=force_streaming))
    for (lp, rlp), name in zip(outs[1:], FORM_IDS[1:]):
        assert torch.equal(lp, outs[0][0]), name
        assert torch.equal(rlp, outs[0][1]), name


@pytest.mark.parametrize("exact", [False, True], ids=["cached", "exact"])
def test_lmhead_token_dtypes_bit_identical(exact):
    St, Tt, H, Vl = 2, 70, 128, 900
    gen = torch.Generator(device=DEV)
    gen.manual_seed(21)
    hidden = torch.randn((St * Tt, H), generator=gen, device=DEV).to(torch.bfloat16)
    w = (torch.randn((Vl, H), generator=gen, device=DEV) * 0.25).to(torch.bfloat16)
    wr = (w.float() + torch.randn((Vl, H), generator=gen, device=DEV) * 0.01).to(torch.bfloat16)
    rng = np.random.default_rng(23)
    ids = rng.integers(0, Vl, size=(St, Tt)).astype(np.int64)
    ids[rng.random((St, Tt)) < 0.1] = -100
    mask = (np.arange(Tt)[None] < np.array([[70], [41]])).astype(np.float32)
    ids, mask = torch.from_numpy(ids).to(DEV), torch.from_numpy(mask).to(DEV)
    old = torch.full((St, Tt), -7.0, device=DEV)
    rewards = torch.rand((St,), generator=gen, device=DEV)
    outs = []
    for form, name in zip(FORMS, FORM_IDS):
        i, m = as_form(ids, mask, form)
        print(f"LM head, ids / mask {name}", flush=True)
        outs.append(grpo.lmhead_fwd_bwd(hidden, w, i, m, ref_weight=wr, rewards=rewards, group_size=2, old_logp=old,
                                        loss_mode=LossMode.GRPO_CLIP_KL, exact_bf16=exact))
    for o, name in zip(outs[1:], FORM_IDS[1:]):
        for f in ("loss", "logp", "ref_logp", "token_loss", "advantages", "dhidden", "dweight"):
            assert torch.equal(getattr(o, f), getattr(outs[0], f)), (name, f)
