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


@pytest.mark.parametrize("shape", [0, 1], ids=["32x32x16", "16x16x32"])
def test_mfma_peak_products_and_clocks(shape):
    """Workgroup 0's wave 0 accumulators equal iters/2 x (A_0 B_0^T + A_1 B_1^T) per block,
    with the documented fragment layouts: an A (B) fragment lane holds row (column)
    lane % M at k = 8 (lane / M) + e, and the result lane column lane % M at rows
    8 (r / 4) + 4 (lane / 32) + r % 4 (M = 32) or 4 (lane / 16) + r (M = 16). The
    LM-head tile kernel relies on the same layouts. The clocks advance."""
    ctx = default_context(0)
    wg, iters, seed = 3, 64, 12345
    M, K = (32, 16) if shape == 0 else (16, 32)
    NI, NJ, NR = (4, 2, 16) if shape == 0 else (8, 4, 4)
    out = torch.full((8192,), float("nan"), dtype=torch.float32, device=DEV)
    clocks = torch.zeros((wg, 4), dtype=torch.int64, device=DEV)
    print(f"mfma probe: shape={shape} workgroups={wg} iters={iters}", flush=True)
    check(lib().pcp_mfma_peak(ctx.handle, shape, wg, iters, seed, out.data_ptr(), clocks.data_ptr(), None),
          ctx.handle)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64).reshape(NI, NJ, NR, 64)
    lane, e = np.arange(64)[:, None], np.arange(8)[None, :]
    k = 8 * (lane // M) + e                                      # [64, 8]
    rows = np.broadcast_to(lane % M, k.shape)
    boff = 4096 if shape == 0 else 8192
    exp = np.zeros((NI, NJ, M, M))
    for s in range(2):
        for i in range(NI):
            A = np.zeros((M, K))
            A[rows, k] = _probe_bf16(seed, ((s * NI + i) * 64 + lane) * 8 + e)
            for j in range(NJ):
                B = np.zeros((M, K))
                B[rows, k] = _probe_bf16(seed, boff + ((s * NJ + j) * 64 + lane) * 8 + e)
                exp[i, j] += (iters // 2) * (A @ B.T)
    r, ln = np.arange(NR)[:, None], np.arange(64)[None, :]
    rrow = 8 * (r // 4) + 4 * (ln // 32) + r % 4 if shape == 0 else 4 * (ln // 16) + r
    want = exp[:, :, rrow, ln % M]                               # [NI, NJ, NR, 64]
    err = np.abs(got - want).max()
    assert err <= 1e-4 * np.abs(want).max(), err
    c = clocks.cpu().numpy()
    assert (c[:, 1] > c[:, 0]).all() and (c[:, 3] > c[:, 2]).all()


def test_mfma_peak_rejects_odd_iters_on_device():
    ctx = default_context(0)
    out = torch.zeros(8192, dtype=torch.float32, device=DEV)
    with pytest.raises(PcpError) as e:
        check(lib().pcp_mfma_peak(ctx.handle, 1, 1, 3, 0, out.data_ptr(), None, None), ctx.handle)
    assert e.value.code == -1 and "iters" in str(e.value)
