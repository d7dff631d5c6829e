"""Parity of the step around the loss head (include/pcp_step.h) with the CPU oracle:
Nesterov update (both formulations), gradient statistics and rollout packing.

Bars: the update, the bf16 shadow copy, packing and the statistics' counts and max are
bit-exact; the f64 sum of squares runs in a different (fixed) order than the
reference's sequential loop, so it is checked to 1e-12 relative.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from pcp_amd import grpo, step
from pcp_amd._lib import NesterovMode, PcpError

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


@pytest.mark.parametrize("mode", [NesterovMode.sutskever, NesterovMode.mlir])
def test_nesterov_flat_bit_exact(mode):
    rng = np.random.default_rng(11)
    counts = [3, 1000, 5, 65537, 7, 4096]           # ragged: tensor offsets are not 16-byte aligned
    n = sum(counts)
    p = rng.standard_normal(n).astype(np.float32)
    lr, mu = 0.01, 0.9
    opt = step.Nesterov(counts, lr, mu, mode)
    pd = t(p)
    shadow = torch.empty(n, dtype=torch.bfloat16, device=DEV)
    v = np.zeros(n, np.float32)
    for k in range(3):
        g = rng.standard_normal(n).astype(np.float32)
        opt.update_flat(pd, t(g), shadow)
        p, v = orc.nesterov(p, v, g, lr, mu, int(mode))
        assert np.array_equal(bits(pd.cpu().numpy()), bits(p)), f"step {k}"
        assert np.array_equal(shadow.view(torch.int16).cpu().numpy().view(np.uint16), orc.bf16_from_f32(p))
    assert np.array_equal(bits(np.frombuffer(opt.serialize(), np.float32)), bits(v))
    opt.close()


def test_nesterov_per_tensor_matches_flat_and_errors():
    rng = np.random.default_rng(12)
    counts = [5, 17, 1024, 3, 333]
    n = sum(counts)
    offs = np.concatenate([[0], np.cumsum(counts)])
    p0 = rng.standard_normal(n).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    opt = step.Nesterov(counts, 0.05, 0.8)
    flat = t(p0)                                     # per-tensor views of one flat buffer
    gd = t(g)
    for i in range(len(counts)):
        opt.update(i, flat[offs[i]:offs[i + 1]], gd[offs[i]:offs[i + 1]])
    want, v = orc.nesterov(p0, np.zeros(n, np.float32), g, 0.05, 0.8)
    assert np.array_equal(bits(flat.cpu().numpy()), bits(want))
    assert np.array_equal(bits(np.frombuffer(opt.serialize(), np.float32)), bits(v))
    # standalone (separately allocated, aligned) tensors give the same values
    opt2 = step.Nesterov(counts, 0.05, 0.8)
    parts = [t(p0[offs[i]:offs[i + 1]]) for i in range(len(counts))]
    for i, pt in enumerate(parts):
        opt2.update(i, pt, gd[offs[i]:offs[i + 1]].clone())
    assert np.array_equal(bits(torch.cat(parts).cpu().numpy()), bits(want))
    with pytest.raises(PcpError) as e:
        opt.update(len(counts), parts[0], parts[0])
    assert e.value.code == -11
    with pytest.raises(PcpError) as e:
        opt.update(1, parts[0], parts[0])
    assert e.value.code == -12
    opt.close()
    opt2.close()


def test_nesterov_state_round_trip_and_reset():
    rng = np.random.default_rng(13)
    counts = [100, 28]
    n = sum(counts)
    opt = step.Nesterov(counts, 0.1, 0.9)
    pd = t(rng.standard_normal(n).astype(np.float32))
    opt.update_flat(pd, t(rng.standard_normal(n).astype(np.float32)))
    state = opt.serialize()
    assert len(state) == 4 * n and np.any(np.frombuffer(state, np.float32))
    opt.reset()
    assert not np.any(np.frombuffer(opt.serialize(), np.float32))
    opt.deserialize(state + b"extra bytes are ignored")
    assert opt.serialize() == state
    with pytest.raises(PcpError) as e:
        opt.deserialize(state[:-4])
    assert e.value.code == -13
    assert opt.serialize() == state                 # a rejected state changes nothing
    opt.close()


@pytest.mark.parametrize("offset", [0, 1])
def test_grad_stats_match_oracle(offset):
    rng = np.random.default_rng(14)
    g = (rng.standard_normal(1 << 20) * 2).astype(np.float32)
    g[[3, 77777]] = np.nan
    g[[10, 500000]] = np.inf
    g[99] = -np.inf
    gd = t(g)[offset:]                              # offset 1: a pointer that is not 16-byte aligned
    got = step.grad_stats(gd)
    want = orc.grad_stats(g[offset:])
    for k in ("nan_count", "inf_count", "elements"):
        assert got[k] == want[k], k
    assert got["max_abs"] == want["max_abs"]
    assert abs(got["sumsq"] - want["sumsq"]) <= 1e-12 * want["sumsq"]
    # two tensors accumulate like the reference's loop over gradients
    both = step.grad_stats([gd[:1000], gd[1000:]])
    assert both["nan_count"] == want["nan_count"] and both["max_abs"] == want["max_abs"]
    assert abs(both["sumsq"] - want["sumsq"]) <= 1e-12 * want["sumsq"]
    assert both["elements"] == want["elements"]


def test_grad_stats_sum_of_squares_in_f64():
    x = np.array([1e20, 3.0, -1e20], np.float32)                         # squares overflow f32
    got = step.grad_stats(t(x))
    big = float(x[0]) ** 2
    assert got["sumsq"] == (big + 9.0) + big and np.isfinite(got["l2_norm"]) and got["max_abs"] == x[0]


def test_grad_stats_deterministic():
    g = t(np.random.default_rng(15).standard_normal(3_000_001).astype(np.float32))
    a, b = step.grad_stats(g), step.grad_stats(g)
    assert a == b


def test_pack_rollouts_match_oracle():
    rng = np.random.default_rng(16)
    R, n_rows, T = 13, 16, 512
    lp = rng.integers(0, 300, R)
    lc = rng.integers(0, 400, R)
    lp[0], lc[1] = 0, 0
    lp[4], lc[4] = 500, 100                         # truncated at T
    pt = rng.integers(0, 151936, lp.sum())
    ct = rng.integers(0, 151936, lc.sum())
    po = np.concatenate([[0], np.cumsum(lp)])
    co = np.concatenate([[0], np.cumsum(lc)])
    ids, mask = step.pack_rollouts(t(pt), t(po), t(ct), t(co), n_rows, T)
    want_ids, want_mask, ok = orc.pack(pt, po, ct, co, n_rows, T)
    assert ok
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    assert np.array_equal(mask.cpu().numpy(), want_mask)


def test_pack_rollouts_bad_offsets_are_reported():
    po = np.array([0, 5, 3, 6], np.int64)            # rollout 1 ends before it starts
    co = np.array([0, 2, 4, 100], np.int64)          # rollout 2 runs past the completion tokens
    pt = np.arange(1, 7, dtype=np.int64)
    ct = np.arange(11, 17, dtype=np.int64)
    with pytest.raises(PcpError) as e:
        step.pack_rollouts(t(pt), t(po), t(ct), t(co), 3, 8)
    assert e.value.code == -1
    ids, mask = step.pack_rollouts(t(pt), t(np.array([0, 5, 6, 6])), t(ct), t(np.array([0, 2, 4, 6])), 3, 8)
    want_ids, want_mask, ok = orc.pack(pt, [0, 5, 6, 6], ct, [0, 2, 4, 6], 3, 8)
    assert ok and np.array_equal(ids.cpu().numpy(), want_ids) and np.array_equal(mask.cpu().numpy(), want_mask)


def test_nesterov_full_model_size_sampled():
    """494,032,768 parameters (Qwen2.5-0.5B): the update is elementwise, so the oracle
    checks a random sample of 2^20 elements bit for bit."""
    P = 494_032_768
    gen = torch.Generator(device=DEV).manual_seed(0)
    p = torch.randn(P, device=DEV, generator=gen)
    g = torch.randn(P, device=DEV, generator=gen)
    idx = torch.from_numpy(np.random.default_rng(17).integers(0, P, 1 << 20)).to(DEV)
    p_s, g_s = p[idx].cpu().numpy(), g[idx].cpu().numpy()
    opt = step.Nesterov([P], 1e-5, 0.9)
    shadow = torch.empty(P, dtype=torch.bfloat16, device=DEV)
    opt.update_flat(p, g, shadow)
    opt.update_flat(p, g, shadow)
    torch.cuda.synchronize()
    want, _ = orc.nesterov(p_s, np.zeros_like(p_s), g_s, 1e-5, 0.9)
    want, _ = orc.nesterov(want, orc.nesterov(p_s, np.zeros_like(p_s), g_s, 1e-5, 0.9)[1], g_s, 1e-5, 0.9)
    assert np.array_equal(bits(p[idx].cpu().numpy()), bits(want))
    assert np.array_equal(shadow[idx].view(torch.int16).cpu().numpy().view(np.uint16), orc.bf16_from_f32(want))
    opt.close()


# ---- the rollout sampler (math.zig:21-58) -------------------------------------------------

def _exact_cdf(x, T):
    x64 = x.astype(np.float64)
    m = x64.max()
    return np.cumsum(np.exp((x64 - m) / T))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sampler_greedy_bit_exact(dtype):
    rng = np.random.default_rng(21)
    R, V = 40, 151936
    x = (rng.standard_normal((R, V)) * 3).astype(np.float32)
    x[1, [5, 90000, 151935]] = 50.0                   # ties: the first maximum wins
    x[2, :] = -np.inf                                 # nothing above -inf: index 0
    x[3, [0, 7]] = np.nan
    x[3, 100] = 40.0                                  # NaN never wins
    x[4, 151935] = 60.0                               # maximum in the ragged last block
    xd = torch.from_numpy(x).to(DEV).to(dtype)
    got = step.sample_tokens(xd, 0.0).cpu().numpy()
    xh = xd.float().cpu().numpy()
    want = np.array([orc.sample(xh[r], 0.0) for r in range(R)])
    assert np.array_equal(got, want)


@pytest.mark.parametrize("T", [0.7, 1.0, 1.6])
def test_sampler_exact_cdf_and_reference_drift(T):
    """The GPU sums f32 terms in float64, so its index is the exact inverse CDF to 1e-6
    of the sum. The reference adds 151936 f32 terms one by one, which absorbs small
    terms: its cumulative drifts from the exact one (by ~2e-4 of the sum here), and a
    draw whose threshold falls in that gap picks another token. Every disagreement with
    the reference restatement must lie inside the reference's own drift, measured per
    row with numpy's sequential float32 cumsum."""
    rng = np.random.default_rng(22)
    R, V = 256, 151936
    x = (rng.standard_normal((R, V)) * 2.5).astype(np.float32)
    u = rng.random(R).astype(np.float32)
    got = step.sample_tokens(t(x), T, t(u)).cpu().numpy()
    for r in range(R):
        c = _exact_cdf(x[r], T)
        thr = float(u[r]) * c[-1]
        g = got[r]
        assert c[g] >= thr - 1e-6 * c[-1] and (g == 0 or c[g - 1] <= thr + 1e-6 * c[-1]), (r, g)
        if r % 4 == 0:                                # the sequential oracle is slow: every 4th row
            want = orc.sample(x[r], T, float(u[r]))
            if g != want:
                e32 = np.exp(((x[r] - x[r].max()) / np.float32(T)).astype(np.float32))
                drift = np.abs(np.cumsum(e32, dtype=np.float32).astype(np.float64) - c).max()
                lo, hi = min(g, want), max(g, want)
                assert c[hi - 1] - drift <= thr <= c[lo] + drift + 1e-6 * c[-1], (r, g, want)


def test_sampler_closed_forms_and_specials():
    V = 151936
    x = np.zeros((6, V), np.float32)                  # uniform rows: index = ceil(u V) - 1
    u = np.array([0.25, 0.5, 0.999, 1e-7, 0.0, 0.33333334], np.float32)
    got = step.sample_tokens(t(x), 1.0, t(u)).cpu().numpy()
    want = np.maximum(np.ceil(u.astype(np.float64) * V) - 1, 0).astype(np.int64)
    assert np.array_equal(got, want), (got, want)
    y = np.full((4, 1000), -30.0, np.float32)
    y[0, 417] = 30.0                                  # one dominant logit
    y[1, 3] = np.nan                                  # NaN: the reference's sum is NaN -> n - 1
    y[2, :] = -np.inf                                 # -inf row: NaN sum -> n - 1
    y[3, 9] = np.inf                                  # +inf: inf - inf -> n - 1
    got = step.sample_tokens(t(y), 1.0, t(np.full(4, 0.5, np.float32))).cpu().numpy()
    assert list(got) == [417, 999, 999, 999]
    assert [orc.sample(y[r], 1.0, 0.5) for r in range(4)] == [417, 999, 999, 999]


@pytest.mark.parametrize("V", [1001, 5003, 151937])
def test_sampler_odd_bf16_rows_last_element(V):
    """bf16 rows of odd length: the last element shares its dword with the bytes after
    the row, so it is read on its own. The maximum (greedy) or all the mass (sampling)
    at index V - 1, in a wider buffer whose bytes after the row hold a larger value."""
    rng = np.random.default_rng(V)
    R, LD = 8, V + 7
    full = (rng.standard_normal((R, LD)) * 2).astype(np.float32)
    full[:, V - 1] = 40.0
    full[:, V:] = 90.0                                # outside the rows: never read
    xd = torch.from_numpy(full).to(DEV).to(torch.bfloat16)
    rows = torch.empty((R, (LD + 7) // 8 * 8), dtype=torch.bfloat16, device=DEV)
    rows[:, :LD] = xd
    view = rows[:, :V]
    assert int(step.sample_tokens(view, 0.0)[0]) == V - 1
    assert np.all(step.sample_tokens(view, 0.0).cpu().numpy() == V - 1)
    u = rng.random(R).astype(np.float32)
    got = step.sample_tokens(view, 1.0, t(u)).cpu().numpy()
    assert np.all(got == V - 1), got
    full[:, V - 1] = -40.0                            # and when the last element carries nothing
    rows[:, :LD] = torch.from_numpy(full).to(DEV).to(torch.bfloat16)
    got = step.sample_tokens(view, 0.0).cpu().numpy()
    want = np.array([orc.sample(rows[r, :V].float().cpu().numpy(), 0.0) for r in range(R)])
    assert np.array_equal(got, want) and not np.any(got == V - 1)


def test_sampler_nan_and_inf_temperature():
    """math.zig:23 takes the greedy branch only for temperature < 1e-6. NaN samples and
    every term is NaN, so the row gives len - 1; +Inf makes every finite term 1 (a
    uniform draw); -Inf is greedy."""
    rng = np.random.default_rng(25)
    R, V = 6, 4096
    x = (rng.standard_normal((R, V)) * 2).astype(np.float32)
    u = np.array([0.1, 0.5, 0.9, 0.0, 0.33, 0.75], np.float32)
    got = step.sample_tokens(t(x), float("nan"), t(u)).cpu().numpy()
    assert np.all(got == V - 1)
    assert [orc.sample(x[r], float("nan"), float(u[r])) for r in range(R)] == [V - 1] * R
    got = step.sample_tokens(t(x), float("inf"), t(u)).cpu().numpy()
    want = np.maximum(np.ceil(u.astype(np.float64) * V) - 1, 0).astype(np.int64)
    assert np.array_equal(got, want), (got, want)
    got = step.sample_tokens(t(x), float("-inf")).cpu().numpy()
    assert np.array_equal(got, x.argmax(1))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T", [0.0, 0.7])
def test_sampler_few_rows_match_batch(dtype, T):
    """Small batches (the reference samples one row per generated token): the first rows
    of a 5-row call and the same rows alone give the same tokens, and each is the exact
    inverse CDF (greedy: the first maximum)."""
    rng = np.random.default_rng(26)
    V = 151936
    x = (rng.standard_normal((5, V)) * 2.5).astype(np.float32)
    x[2, [7, 90001]] = 40.0                           # a tie: the first maximum wins
    xd = torch.from_numpy(x).to(DEV).to(dtype)
    u = rng.random(5).astype(np.float32)
    five = step.sample_tokens(xd, T, t(u) if T > 0 else None).cpu().numpy()
    xh = xd.float().cpu().numpy()
    for R in (1, 3, 4):
        few = step.sample_tokens(xd[:R], T, t(u[:R]) if T > 0 else None).cpu().numpy()
        assert np.array_equal(few, five[:R]), (R, few, five[:R])
    for r in range(5):
        if T == 0.0:
            assert five[r] == int(np.argmax(xh[r]))
            continue
        c = _exact_cdf(xh[r], T)
        thr = float(u[r]) * c[-1]
        g = five[r]
        assert c[g] >= thr - 1e-6 * c[-1] and (g == 0 or c[g - 1] <= thr + 1e-6 * c[-1]), (r, g)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T", [0.0, 0.7])
def test_sampler_async_enqueues_behind_the_producer(dtype, T):
    """pcp_sample_tokens_async: a decode loop's pattern. On one stream, each step writes
    a row of logits (a torch kernel standing for the forward), then the sampler is only
    enqueued behind it; no host wait until the end. The tokens equal the synchronous
    entry point's on the same rows, one row per call (the reference's pattern) and 64
    rows per call, over consecutive calls (each launch leaves its row tickets at zero)."""
    rng = np.random.default_rng(27)
    V, steps = 151936, 12
    base = torch.from_numpy((rng.standard_normal((steps, V)) * 2.5).astype(np.float32)).to(DEV).to(dtype)
    u = torch.from_numpy(rng.random(steps).astype(np.float32)).to(DEV)
    ctx = grpo.Context(0)
    st = torch.cuda.Stream()
    row = torch.empty((1, V), dtype=dtype, device=DEV)
    out = torch.empty((steps, 1), dtype=torch.int64, device=DEV)
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        for i in range(steps):
            row.copy_(base[i:i + 1])              # the producer, on the same stream
            step.sample_tokens(row, T, u[i:i + 1] if T > 0 else None, ids=out[i], stream=st.cuda_stream, ctx=ctx,
                               sync=False)
    ctx.sync()
    torch.cuda.synchronize()
    want = torch.stack([step.sample_tokens(base[i:i + 1], T, u[i:i + 1] if T > 0 else None, ctx=ctx)
                        for i in range(steps)])
    assert torch.equal(out, want)
    many = step.sample_tokens(base, T, u if T > 0 else None, ctx=ctx, sync=False)
    ctx.sync()
    assert torch.equal(many.view(-1, 1), want)
    ctx.close()


def test_sampler_bf16_and_strided_rows():
    rng = np.random.default_rng(23)
    R, V, LD = 16, 5000, 5120                         # rows inside a wider buffer
    full = (rng.standard_normal((R, LD)) * 2).astype(np.float32)
    xd = torch.from_numpy(full).to(DEV).to(torch.bfloat16)[:, :V]
    u = rng.random(R).astype(np.float32)
    got = step.sample_tokens(xd, 0.8, t(u)).cpu().numpy()
    xh = xd.float().cpu().numpy()
    for r in range(R):
        c = _exact_cdf(xh[r], 0.8)
        thr = float(u[r]) * c[-1]
        g = got[r]
        assert c[g] >= thr - 1e-6 * c[-1] and (g == 0 or c[g - 1] <= thr + 1e-6 * c[-1])


def test_sampler_successive_calls_reuse_counters_and_partials():
    """Successive calls on the same logits buffer and the context's scratch partials,
    alternating greedy and sampled rows, changing row counts and single-workgroup rows:
    each call selects from its own data."""
    rng = np.random.default_rng(24)
    V = 151936
    buf = torch.empty((64, V), dtype=torch.float32, device=DEV)
    for call, (R, T) in enumerate([(64, 0.9), (64, 0.0), (17, 1.3), (64, 0.9), (1, 0.0), (33, 0.7)]):
        x = (rng.standard_normal((R, V)) * 2.0).astype(np.float32)
        x[:, rng.integers(0, V, R)] += 8.0 * (call + 1)   # the mass moves between calls
        buf[:R].copy_(t(x))
        u = rng.random(R).astype(np.float32)
        got = step.sample_tokens(buf[:R], T, t(u) if T > 0 else None).cpu().numpy()
        for r in range(R):
            if T == 0.0:
                assert got[r] == int(np.argmax(x[r])), (call, r)
                continue
            c = _exact_cdf(x[r], T)
            thr = float(u[r]) * c[-1]
            g = got[r]
            assert c[g] >= thr - 1e-6 * c[-1] and (g == 0 or c[g - 1] <= thr + 1e-6 * c[-1]), (call, r, g)
    small = torch.tensor([[0.5, 2.0, -1.0, -3.0]], device=DEV)   # one block, one workgroup
    assert int(step.sample_tokens(small, 0.0)[0]) == 1
    assert int(step.sample_tokens(small, 1.0, t(np.array([0.0], np.float32)))[0]) == 0
