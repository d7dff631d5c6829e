"""Device-side error reporting on every row-kernel form.

A live token id outside [0, V) (and not -100) is PCP_ERR_TOKEN_RANGE (-3); a NaN or +Inf
in a live row of the policy or reference logits is PCP_ERR_NONFINITE (-4). Dead rows
(mask 0) are not read for the loss, so a NaN there is not an error. After a failing call
the error word is cleared: the next clean call succeeds and gives the clean outputs bit
for bit. Paths: the resident kernel (bf16 and f32 logits), the streaming fallback, the
calls without zero-fill (listed rows below half live, every row above), and the
forward-only log-prob kernels.
"""
import numpy as np
import pytest
import torch

from pcp_amd import grpo
from pcp_amd._lib import LossMode, PcpError

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
S, T, V = 4, 32, 4096

PATHS = {
    # name: (logits dtype, sequence lengths, loss keyword arguments or None for forward-only)
    "resident-bf16": (torch.bfloat16, [32, 20, 9, 30], {}),
    "resident-f32": (torch.float32, [32, 20, 9, 30], {}),
    "streaming": (torch.bfloat16, [32, 20, 9, 30], dict(force_streaming=True)),
    "listed-no-zero-fill": (torch.bfloat16, [12, 3, 9, 7], dict(zero_fill=False)),
    "every-row-no-zero-fill": (torch.bfloat16, [32, 20, 29, 30], dict(zero_fill=False)),
    "logprob": (torch.bfloat16, [32, 20, 9, 30], None),
    "logprob-streaming": (torch.bfloat16, [32, 20, 9, 30], dict(force_streaming=True, logprob=True)),
}


def inputs(dt, lengths):
    gen = torch.Generator(device=DEV)
    gen.manual_seed(3)
    x = (torch.randn((S, T, V), generator=gen, device=DEV) * 3).to(dt)
    r = (x.float() + torch.randn((S, T, V), generator=gen, device=DEV) * 0.1).to(dt)
    ids = torch.randint(0, V, (S, T), generator=gen, device=DEV)
    mask = (torch.arange(T, device=DEV)[None] < torch.tensor(lengths, device=DEV)[:, None]).float()
    rewards = torch.rand((S,), generator=gen, device=DEV)
    old = torch.randn((S, T), generator=gen, device=DEV) * 0.05 - float(np.log(V))
    return dict(x=x, r=r, ids=ids, mask=mask, rewards=rewards, old=old)


def call(path, d):
    _, _, kw = PATHS[path]
    if kw is None or kw.get("logprob"):
        lp, rlp = grpo.logprob_fwd(d["x"], d["ids"], d["r"], mask=d["mask"],
                                   force_streaming=bool(kw and kw.get("force_streaming")))
        return dict(logp=lp, ref_logp=rlp)
    out = grpo.grpo_loss_fwd_bwd(d["x"], d["ids"], d["mask"], rewards=d["rewards"], group_size=2, ref_logits=d["r"],
                                 old_logp=d["old"], loss_mode=LossMode.GRPO_CLIP_KL,
                                 dlogits=torch.zeros_like(d["x"]), **kw)
    return {f: getattr(out, f) for f in ("loss", "dlogits", "logp", "ref_logp", "token_loss")}


def same(a, b):
    return all(torch.equal(a[k], b[k]) for k in a)


@pytest.mark.parametrize("path", list(PATHS))
def test_device_errors_on_every_row_path(path):
    dt, lengths, _ = PATHS[path]
    d = inputs(dt, lengths)
    clean = call(path, d)
    torch.cuda.synchronize()

    def expect(code, what, **override):
        print(f"{path}: {what}", flush=True)
        with pytest.raises(PcpError) as e:
            call(path, {**d, **override})
        assert e.value.code == code, (path, what, e.value.code)
        assert same(call(path, d), clean), (path, what, "clean call after the error")

    bad_ids = d["ids"].clone()
    bad_ids[1, 2] = V                       # live (lengths[1] > 2)
    expect(-3, "live id == V", ids=bad_ids)
    bad_ids = d["ids"].clone()
    bad_ids[2, 0] = -5                      # negative, not the ignore index
    expect(-3, "live id -5", ids=bad_ids)
    x = d["x"].clone()
    x[0, 4, 1000] = float("nan")
    expect(-4, "NaN in a live policy row", x=x)
    r = d["r"].clone()
    r[3, 1, 7] = float("inf")
    expect(-4, "+Inf in a live reference row", r=r)
    # A NaN in a dead row (mask 0) is not read for the loss: no error, same outputs on
    # every live row (the dead row's own outputs are its fill).
    x = d["x"].clone()
    x[2, T - 1, 11] = float("nan")          # lengths[2] < T: a dead row
    print(f"{path}: NaN in a dead row", flush=True)
    got = call(path, {**d, "x": x})
    torch.cuda.synchronize()
    assert same(got, clean), path
