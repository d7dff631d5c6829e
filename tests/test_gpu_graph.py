"""The loss path (pcp_grpo_loss_fwd_bwd and its allocation-free form) captured in a HIP graph.

With PCP_FLAG_ASYNC the call only enqueues kernels once its work buffer has grown: no
allocation, no memset, no host read. The per-call counters (the row kernel's row counter,
the live-row count without zero-fill) are zeroed by step_prep_kernel's stores, and
loss_reduce_kernel leaves its ticket at 0, so a captured call can be replayed. Each
replay here runs on new inputs written into the captured tensors, with eager calls of the
same entry point (and synchronisations) between the replays, and must equal an eager
call on those inputs bit for bit: every kernel of the path is deterministic (fixed
summation orders; without zero-fill the live-row list order varies, but each row's
outputs depend on its own data only). Without zero-fill the dead dlogits rows keep the
sentinel both buffers were filled with.
"""
import numpy as np
import pytest
import torch

from pcp_amd import grpo
from pcp_amd._lib import LossMode

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
S, T, V, G = 16, 96, 8192, 4
SENTINEL = 7.0


def fresh_inputs(seed, dtype, lens):
    """Seeded inputs of one shape (written into the captured tensors before a replay);
    sequence lengths uniform in lens = (lo, hi)."""
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    pol = torch.randn((S, T, V), generator=gen, device=DEV) * 3
    ref = pol + torch.randn((S, T, V), generator=gen, device=DEV) * 0.1
    ids = torch.randint(0, V, (S, T), generator=gen, device=DEV, dtype=torch.int64)
    rng = np.random.default_rng(seed)
    lengths = rng.integers(lens[0], lens[1] + 1, size=S)
    mask = torch.from_numpy((np.arange(T)[None] < lengths[:, None]).astype(np.float32)).to(DEV)
    rewards = torch.rand((S,), generator=gen, device=DEV)
    old = torch.randn((S, T), generator=gen, device=DEV) * 0.01 - float(np.log(V))
    return dict(pol=pol.to(dtype), ref=ref.to(dtype), ids=ids, mask=mask, rewards=rewards, old=old)


def call(x, out, **kw):
    return grpo.grpo_loss_fwd_bwd(x["pol"], x["ids"], x["mask"], rewards=x["rewards"], group_size=G,
                                  ref_logits=x["ref"], old_logp=x["old"], loss_mode=LossMode.GRPO_CLIP_KL,
                                  outputs=out, **kw)


def new_outputs(x, f32_out):
    dt = torch.float32 if f32_out else x["pol"].dtype
    return grpo.GrpoOutputs(
        loss=torch.zeros((), dtype=torch.float32, device=DEV),
        dlogits=torch.full((S, T, V), SENTINEL, dtype=dt, device=DEV),
        logp=torch.zeros((S, T), dtype=torch.float32, device=DEV),
        ref_logp=torch.zeros((S, T), dtype=torch.float32, device=DEV),
        token_loss=torch.zeros((S, T), dtype=torch.float32, device=DEV),
        advantages=torch.zeros((S,), dtype=torch.float32, device=DEV))


FIELDS = ("loss", "dlogits", "logp", "ref_logp", "token_loss", "advantages")

CASES = {
    # name: (logits dtype, f32 dlogits, zero_fill, length range, extra keyword arguments).
    # Without zero-fill the row kernel walks the live-row list below half live rows
    # (lengths 1..40 of 96: at most 42% live) and every row otherwise (60..96: over 62%).
    "bf16": (torch.bfloat16, False, True, (1, T), {}),
    "bf16-exact": (torch.bfloat16, False, True, (1, T), dict(exact_bf16=True)),
    "bf16-f32-out": (torch.bfloat16, True, True, (1, T), {}),
    "f32": (torch.float32, False, True, (1, T), {}),
    "bf16-streaming": (torch.bfloat16, False, True, (1, T), dict(force_streaming=True)),
    "bf16-nzf-listed": (torch.bfloat16, False, False, (1, 40), {}),
    "bf16-nzf-every-row": (torch.bfloat16, False, False, (60, T), {}),
    "bf16-noalloc-nzf-listed": (torch.bfloat16, False, False, (1, 40), dict(noalloc=True)),
    "bf16-noalloc": (torch.bfloat16, False, True, (1, T), dict(noalloc=True)),
}


@pytest.mark.parametrize("case", list(CASES))
def test_loss_graph_capture_replays(case):
    dtype, f32_out, zero_fill, lens, kw = CASES[case]
    kw = dict(kw, zero_fill=zero_fill)
    ctx = grpo.default_context(0)
    x = fresh_inputs(100, dtype, lens)
    out = new_outputs(x, f32_out)
    call(x, out, **kw)                        # grows the work buffer; warms the launch caches
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(x, out, sync=False, ctx=ctx, **kw)
    ctx.sync()
    for rep in range(3):
        y = fresh_inputs(200 + rep, dtype, lens)
        for k in x:
            x[k].copy_(y[k])
        want = new_outputs(x, f32_out)
        call(x, want, **kw)                   # eager, synchronous, on the replay's inputs
        for f in FIELDS:
            t = getattr(out, f)
            t.fill_(SENTINEL if f == "dlogits" else float("nan"))
        torch.cuda.synchronize()
        print(f"loss graph replay {rep} ({case})", flush=True)
        g.replay()
        torch.cuda.synchronize()
        ctx.sync()                            # device-side error word
        for f in FIELDS:
            assert torch.equal(getattr(out, f), getattr(want, f)), (case, rep, f)
        if not zero_fill:
            dead = x["mask"] == 0
            assert bool((out.dlogits[dead] == SENTINEL).all()), (case, rep)
    del g
    torch.cuda.synchronize()
