"""The HBM stream probes (pcp_hbm_stream) compute what they claim: copy, the 2-read :
1-write mix (XOR), the write pattern, and a read that leaves its output alone, for
every shape and both load / store kinds, on sizes off the workgroup's span."""
import ctypes

import pytest
import torch

from pcp_amd._lib import PcpError, check, lib
from pcp_amd.grpo import default_context

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("vpt", [1, 2, 4, 8])
@pytest.mark.parametrize("nt", [0, 1])
def test_hbm_stream_kinds(vpt, nt):
    ctx = default_context(0)
    n = 256 * 1024 + 12                   # int32 words: 16-byte multiple, not a multiple of any span
    g = torch.Generator(device=DEV).manual_seed(vpt * 2 + nt)
    a = torch.randint(-2 ** 31, 2 ** 31 - 1, (n,), dtype=torch.int32, device=DEV, generator=g)
    b = torch.randint(-2 ** 31, 2 ** 31 - 1, (n,), dtype=torch.int32, device=DEV, generator=g)
    c = torch.zeros_like(a)
    st = torch.cuda.current_stream().cuda_stream or None
    run = lambda kind: check(lib().pcp_hbm_stream(ctx.handle, kind, nt, vpt, a.data_ptr(), b.data_ptr(), c.data_ptr(),
                                                  4 * n, st), ctx.handle)
    print(f"hbm stream probes: vpt={vpt} nt={nt}", flush=True)
    run(2)
    torch.cuda.synchronize()
    assert torch.equal(c, a)
    run(3)
    torch.cuda.synchronize()
    assert torch.equal(c, a ^ b)
    c.zero_()
    run(0)                                # read only: c stays zero (the sink is written for an all-ones XOR only)
    torch.cuda.synchronize()
    assert not c.any()
    run(1)
    torch.cuda.synchronize()
    w = c.view(-1, 4).cpu()
    idx = torch.arange(n // 4, dtype=torch.int64)
    assert torch.equal(w[:, 0].to(torch.int64) & 0xFFFFFFFF, idx & 0xFFFFFFFF)
    assert torch.equal(w[:, 1:], torch.tensor([1, 2, 3], dtype=torch.int32).expand(n // 4, 3))


def test_hbm_stream_rejects_bad_shape_on_device():
    ctx = default_context(0)
    a = torch.zeros(1024, dtype=torch.int32, device=DEV)
    with pytest.raises(PcpError) as e:
        check(lib().pcp_hbm_stream(ctx.handle, 2, 0, 3, a.data_ptr(), None, a.data_ptr(), 4096, None), ctx.handle)
    assert e.value.code == -1 and "vectors_per_lane" in str(e.value)
