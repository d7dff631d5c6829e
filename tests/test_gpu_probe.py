"""The HBM stream probes (pcp_hbm_stream) compute what they claim: copy, the 2-read :
1-write mix (XOR), the write pattern, and a read that leaves its output alone, for
every shape and both load / store kinds, on sizes off the workgroup's span. The MFMA
probe (pcp_mfma_peak) computes the products it counts: its accumulators against a
float64 product of the same operands in the documented fragment layout."""
import ctypes

import numpy as np
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


def _probe_bf16(seed: int, idx: np.ndarray) -> np.ndarray:
    """The probe's operand values: a murmur3-style mix of (seed, idx), mapped to
    [-1, 1) and truncated to bf16 (as float64)."""
    m = np.uint64(0xFFFFFFFF)
    x = (np.uint64(seed) ^ ((idx.astype(np.uint64) * np.uint64(0x9E3779B9)) & m)) & m
    x ^= x >> np.uint64(16)
    x = (x * np.uint64(0x85EBCA6B)) & m
    x ^= x >> np.uint64(13)
    x = (x * np.uint64(0xC2B2AE35)) & m
    x ^= x >> np.uint64(16)
    f = ((x >> np.uint64(8)).astype(np.int64) - (1 << 23)).astype(np.float32) * np.float32(2.0 ** -23)
    return ((f.view(np.uint32) >> np.uint32(16)) << np.uint32(16)).view(np.float32).astype(np.float64)


def test_mfma_peak_products_and_clocks():
    """Workgroup 0's wave 0 accumulators equal iters/2 x (A_0 B_0^T + A_1 B_1^T) per 32 x 32
    block, with A fragment lane l holding row l % 32 at k = 8 (l / 32) + e and the result
    lane l column l % 32 at rows 8 (r / 4) + 4 (l / 32) + r % 4; the clocks advance."""
    ctx = default_context(0)
    wg, iters, seed = 3, 64, 12345
    out = torch.full((8192,), float("nan"), dtype=torch.float32, device=DEV)
    clocks = torch.zeros((wg, 4), dtype=torch.int64, device=DEV)
    print(f"mfma probe: workgroups={wg} iters={iters}", flush=True)
    check(lib().pcp_mfma_peak(ctx.handle, wg, iters, seed, out.data_ptr(), clocks.data_ptr(), None), ctx.handle)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64).reshape(4, 2, 16, 64)
    lane, e = np.arange(64)[:, None], np.arange(8)[None, :]
    k = 8 * (lane // 32) + e                                     # [64, 8]
    exp = np.zeros((4, 2, 32, 32))
    for s in range(2):
        for i in range(4):
            A = np.zeros((32, 16))
            A[np.broadcast_to(lane % 32, k.shape), k] = _probe_bf16(seed, ((s * 4 + i) * 64 + lane) * 8 + e)
            for j in range(2):
                B = np.zeros((32, 16))
                B[np.broadcast_to(lane % 32, k.shape), k] = _probe_bf16(seed, 4096 + ((s * 2 + j) * 64 + lane) * 8 + e)
                exp[i, j] += (iters // 2) * (A @ B.T)
    r, ln = np.arange(16)[:, None], np.arange(64)[None, :]
    want = exp[:, :, 8 * (r // 4) + 4 * (ln // 32) + r % 4, ln % 32]   # [4, 2, 16, 64]
    err = np.abs(got - want).max()
    assert err <= 1e-4 * np.abs(want).max(), err
    c = clocks.cpu().numpy()
    assert (c[:, 1] > c[:, 0]).all() and (c[:, 3] > c[:, 2]).all()


def test_mfma_peak_rejects_odd_iters_on_device():
    ctx = default_context(0)
    out = torch.zeros(8192, dtype=torch.float32, device=DEV)
    with pytest.raises(PcpError) as e:
        check(lib().pcp_mfma_peak(ctx.handle, 1, 3, 0, out.data_ptr(), None, None), ctx.handle)
    assert e.value.code == -1 and "iters" in str(e.value)
