"""Parity of the HIP path (libpcp_grpo.so through its C ABI) with the CPU oracle.

Tolerances (plus tighter engineering bars where the math allows):
  log-probs, token losses (f32 math):  |d| <= 1e-5 * max(1, |lse|)      (rel 1e-5 of the row scale)
  loss:                                the log-prob bar propagated through dloss/dlogp and
                                       dloss/dref, plus 1e-5 of the sum of |contributions|
  dlogits, f32 output:                 |d| <= 1e-4 (north star) and <= 1e-5*|exact| + floor_row
  dlogits, bf16 output:                |d| <= (2^-8 + 2^-11 + 1.3e-5)*|exact| + (1 + 2^-6)*floor_row
  dlogits, bf16 output, exact mode:    |d| <= (2^-8 + 1.1e-5)*|exact| + (1 + 2^-7)*floor_row
  advantages, ids, masks, zero rows:   bit-exact
(the bars and their derivation are in parity_tol.py). floor_row (coef_floor) is what
the f32 log-prob error allows in the row's coefficient c: c is built from
exp(logp - old) and expm1(ref - logp), whose terms can cancel. A bf16 output rounded to
nearest even is off by up to 2^-8 of the value (8 significant bits); the default
bf16 -> bf16 rows also scale f16 softmax terms (2^-11 of the term, 2^-25 absolute below
f16's normal range). The north star's "bf16 paths rel 2e-3" is met by the log-probs and
loss computed from bf16 logits.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from pcp_amd import grpo, synth
from pcp_amd._lib import DType, LossMode, PcpError
from pcp_amd.backend import HipGrpoBackend
from parity_tol import (BF16_CACHED_REL, BF16_EXACT_REL, assert_dlogits, coef_floor, dev, emulate_loss, full_floor,
                        full_loss_tol, host_bits, loss_tolerance, lse_scale, tok_to_rows, token_scale)

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden")
DEV = torch.device("cuda:0")


def load_cases():
    z = np.load(os.path.join(GOLD, "cases.npz"))
    cases = {}
    for k in z.files:
        name, field = k.split("/", 1)
        cases.setdefault(name, {})[field] = z[k]
    return cases


CASES = load_cases()


def run_case(c, **kw):
    args = dict(rows=int(c["rows"]), tok_offset=int(c["tok_offset"]), group_size=int(c["group_size"]),
                loss_mode=int(c["loss_mode"]), clip_eps=float(c["clip_eps"]), kl_beta=float(c["kl_beta"]),
                loss_norm=float(c["loss_norm"]))
    if "advantages" in c:
        args["advantages"] = dev(c["advantages"])
    else:
        args["rewards"] = dev(c["rewards"])
    if "ref_logits" in c:
        args["ref_logits"] = dev(c["ref_logits"])
    if "old_logp" in c:
        args["old_logp"] = dev(c["old_logp"])
    args.update(kw)
    out = grpo.grpo_loss_fwd_bwd(dev(c["logits"]), dev(c["ids"]), dev(c["mask"]), **args)
    torch.cuda.synchronize()
    return out


def golden_loss_tol(c):
    off, rows = int(c["tok_offset"]), int(c["rows"])
    dt = orc.BF16 if c["logits"].dtype == np.uint16 else orc.F32
    L = np.maximum(c["mask"][:, off:off + rows].astype(np.float64).sum(1), 1.0)
    G = float(c["loss_norm"]) if float(c["loss_norm"]) > 0 else float(c["ids"].shape[0])
    return loss_tolerance(c["exp_token_loss"], c["exp_coef"], c["exp_lp"], c["exp_lr"], c["mask"], c["exp_adv"],
                          L, G, int(c["loss_mode"]) == 0, float(c["kl_beta"]),
                          token_scale(c["logits"], c["ids"], rows, off, dt))


def golden_floor_rows(c):
    S, LS, V = c["logits"].shape
    off, rows = int(c["tok_offset"]), int(c["rows"])
    dt = orc.BF16 if c["logits"].dtype == np.uint16 else orc.F32
    L = np.maximum(c["mask"][:, off:off + rows].astype(np.float64).sum(1), 1.0)[:, None]
    G = float(c["loss_norm"]) if float(c["loss_norm"]) > 0 else float(S)
    old = c["old_logp"].astype(np.float64) if "old_logp" in c else c["exp_lp"]
    fl = coef_floor(c["exp_coef"], c["exp_lp"], c["exp_lr"], c["mask"].astype(np.float64),
                    c["exp_adv"].astype(np.float64)[:, None], L, G, old, int(c["loss_mode"]) == 0,
                    float(c["kl_beta"]), float(c["clip_eps"]), token_scale(c["logits"], c["ids"], rows, off, dt))
    return tok_to_rows(fl, rows, off, LS)


# ---- golden fixtures through the device path ----------------------------------------

@pytest.mark.parametrize("streaming", [False, True])
@pytest.mark.parametrize("name", sorted(CASES))
def test_golden_cases(name, streaming):
    c = CASES[name]
    out = run_case(c, force_streaming=streaming)
    S, LS, V = c["logits"].shape
    rows, off = int(c["rows"]), int(c["tok_offset"])
    bf16 = c["logits"].dtype == np.uint16
    dt = orc.BF16 if bf16 else orc.F32
    sel = c["logits"][:, :rows].reshape(S * rows, V)
    ids = c["ids"][:, off:off + rows].reshape(-1)
    scale = lse_scale(sel, ids, dt).reshape(S, rows)
    lp = out.logp.cpu().numpy()[:, off:off + rows]
    assert np.all(np.abs(lp - c["exp_lp"][:, off:off + rows]) <= 1e-5 * scale)
    tl = out.token_loss.cpu().numpy()[:, off:off + rows]
    assert np.all(np.abs(tl - c["exp_token_loss"][:, off:off + rows]) <= 1e-5 * scale)
    assert abs(float(out.loss.cpu()) - c["exp_loss"]) <= golden_loss_tol(c)
    assert np.array_equal(out.advantages.cpu().numpy(), c["exp_adv"])
    assert_dlogits(host_bits(out.dlogits).astype(np.float32) if not bf16 else orc.bf16_to_f32(host_bits(out.dlogits)),
                   c["exp_dlogits"], golden_floor_rows(c), bf16)
    # masked / ignored / pad rows are exactly zero
    d = host_bits(out.dlogits)
    for s in range(S):
        for t in range(LS):
            dead = t >= rows or c["mask"][s, off + t] == 0 or c["ids"][s, off + t] == -100
            if dead:
                assert not np.any(d[s, t]), (s, t)


def test_golden_bf16_in_f32_out():
    c = CASES["v130_bf16_clip_kl"]
    out = run_case(c, dlogits_dtype=torch.float32)
    assert out.dlogits.dtype == torch.float32
    S, LS, V = c["logits"].shape
    assert_dlogits(out.dlogits.cpu().numpy(), c["exp_dlogits"], golden_floor_rows(c), False)


# ---- advantages -----------------------------------------------------------------------

def test_advantages_bit_exact():
    with open(os.path.join(GOLD, "advantages.json")) as f:
        d = json.load(f)
    for c in d["cases"]:
        r = np.array(c["rewards_bits"], np.uint32).view(np.float32)
        got = grpo.advantages(dev(r), c["group"], d["eps"]).cpu().numpy().view(np.uint32)
        assert np.array_equal(got, np.array(c["adv_bits"], np.uint32)), c["name"]


# ---- config 1 (toy-qwen), full problem ----------------------------------------------------

@pytest.mark.parametrize("mode", [LossMode.REINFORCE, LossMode.GRPO_CLIP_KL])
def test_config1_full(mode):
    cfg = synth.CONFIGS[1]
    inp = synth.make_device_inputs(cfg, DEV)
    out = grpo.grpo_loss_fwd_bwd(inp["logits"], inp["ids"], inp["mask"], rewards=inp["rewards"],
                                 group_size=cfg.group, ref_logits=inp["ref_logits"], old_logp=inp["old_logp"],
                                 loss_mode=mode, clip_eps=cfg.clip_eps, kl_beta=cfg.kl_beta)
    torch.cuda.synchronize()
    h = {k: (v.cpu().numpy() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    want = orc.grpo_full(h["logits"], h["ids"], h["mask"], rows=cfg.T, rewards=h["rewards"], group_size=cfg.group,
                         ref_logits=h["ref_logits"], old_logp=h["old_logp"],
                         loss_mode=orc.CLIP_KL if mode == LossMode.GRPO_CLIP_KL else orc.REINFORCE,
                         clip_eps=cfg.clip_eps, kl_beta=cfg.kl_beta, dtype=orc.F32)
    scale = lse_scale(h["logits"].reshape(-1, cfg.V), h["ids"].reshape(-1), orc.F32).reshape(cfg.S, cfg.T)
    assert np.all(np.abs(out.logp.cpu().numpy() - want.lp) <= 1e-5 * scale)
    if mode == LossMode.GRPO_CLIP_KL:
        assert np.all(np.abs(out.ref_logp.cpu().numpy() - want.lr) <= 1e-5 * scale)
    assert np.all(np.abs(out.token_loss.cpu().numpy() - want.token_loss) <= 1e-5 * scale)
    assert abs(float(out.loss.cpu()) - want.loss) <= full_loss_tol(
        want, h["logits"], h["ids"], h["mask"], cfg.T, 0, orc.F32, mode == LossMode.REINFORCE, cfg.kl_beta, cfg.S)
    tsc = token_scale(h["logits"], h["ids"], cfg.T, 0, orc.F32)
    fl = full_floor(want, h["mask"], h["old_logp"], cfg.S, mode == LossMode.REINFORCE, cfg.kl_beta, cfg.clip_eps, tsc)
    got_d = out.dlogits.cpu().numpy()
    assert_dlogits(got_d, want.dlogits, fl, False)
    live = h["mask"] != 0
    e_lp = (np.abs(out.logp.cpu().numpy() - want.lp) / scale)[live].max()
    e_lr = (np.abs(out.ref_logp.cpu().numpy() - want.lr) / scale)[live].max() if mode == LossMode.GRPO_CLIP_KL else 0.0
    e_tl = (np.abs(out.token_loss.cpu().numpy() - want.token_loss) / scale)[live].max()
    ltol = full_loss_tol(want, h["logits"], h["ids"], h["mask"], cfg.T, 0, orc.F32, mode == LossMode.REINFORCE,
                         cfg.kl_beta, cfg.S)
    e_loss = abs(float(out.loss.cpu()) - want.loss)
    terms = np.abs(want.token_loss).sum(1) / want.seq_len.astype(np.float64)
    if mode == LossMode.REINFORCE:
        terms = terms * np.abs(want.adv.astype(np.float64))
    d_abs = np.abs(got_d.astype(np.float64) - want.dlogits.astype(np.float64))
    print(f"PARITY-TABLE config1 {'clip_kl' if mode == LossMode.GRPO_CLIP_KL else 'reinforce'}: live rows "
          f"{int(live.sum())} of {live.size}; |dlogp|/max(1,|lse|) {e_lp:.2e} (bar 1e-5); ref {e_lr:.2e}; token loss "
          f"{e_tl:.2e}; loss rel {e_loss / max(abs(want.loss), 1e-30):.2e}, per sum of |terms| "
          f"{e_loss / (terms.sum() / cfg.S):.2e} ({e_loss / ltol:.3f} of its bar); f32 "
          f"dlogits max abs {d_abs.max():.2e} (bar 1e-4)", flush=True)


def test_config1_reference_faithful_gap():
    # The reference backward's 1e-4 guards stay inside the dlogits budget.
    cfg = synth.CONFIGS[1]
    inp = synth.make_device_inputs(cfg, DEV)
    adv = torch.from_numpy(orc.advantages(inp["rewards"].cpu().numpy(), cfg.group)).to(DEV)
    out = grpo.grpo_loss_fwd_bwd(inp["logits"], inp["ids"], inp["mask"], advantages=adv)
    torch.cuda.synchronize()
    h = {k: (v.cpu().numpy() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    fa = orc.grpo_full(h["logits"], h["ids"], h["mask"], rows=cfg.T, advantages_in=adv.cpu().numpy(),
                       precision=orc.FAITHFUL, dtype=orc.F32)
    assert np.abs(out.dlogits.cpu().numpy() - fa.dlogits).max() <= 1e-4
    assert abs(float(out.loss.cpu()) - fa.loss) <= full_loss_tol(fa, h["logits"], h["ids"], h["mask"], cfg.T, 0,
                                                                  orc.F32, True, 0.0, cfg.S)


def test_logprob_fwd_matches_oracle():
    cfg = synth.CONFIGS[1]
    inp = synth.make_device_inputs(cfg, DEV)
    lp, lr = grpo.logprob_fwd(inp["logits"], inp["ids"], inp["ref_logits"])
    torch.cuda.synchronize()
    L = inp["logits"].cpu().numpy().reshape(-1, cfg.V)
    R = inp["ref_logits"].cpu().numpy().reshape(-1, cfg.V)
    ids = inp["ids"].cpu().numpy().reshape(-1)
    want, lse = orc.logprob(L, ids)
    want_r, lse_r = orc.logprob(R, ids)
    assert np.all(np.abs(lp.cpu().numpy().reshape(-1) - want) <= 1e-5 * np.maximum(1, np.abs(lse)))
    assert np.all(np.abs(lr.cpu().numpy().reshape(-1) - want_r) <= 1e-5 * np.maximum(1, np.abs(lse_r)))


def test_logprob_fwd_config2_forward_streaming_and_loss_path():
    """Forward-only log-probs at config 2 (bf16, V = 151936): the forward kernel, the
    streaming kernel and the loss path (resident kernel) agree within
    2e-5 * max(1, |lse|) on live tokens, masked tokens read exactly 0, and sampled rows
    match the float64 oracle within 1e-5 * max(1, |lse|)."""
    cfg = synth.CONFIGS[2]
    inp = synth.make_device_inputs(cfg, DEV)
    print("config 2 forward-only log-probs: forward kernel, streaming, loss path", flush=True)
    lp, lr = grpo.logprob_fwd(inp["logits"], inp["ids"], inp["ref_logits"], mask=inp["mask"])
    lps, lrs = grpo.logprob_fwd(inp["logits"], inp["ids"], inp["ref_logits"], mask=inp["mask"], force_streaming=True)
    out = grpo.grpo_loss_fwd_bwd(inp["logits"], inp["ids"], inp["mask"], rewards=inp["rewards"], group_size=cfg.group,
                                 ref_logits=inp["ref_logits"], old_logp=inp["old_logp"],
                                 loss_mode=LossMode.GRPO_CLIP_KL)
    torch.cuda.synchronize()
    m = inp["mask"] != 0
    for t in (lp, lr, lps, lrs):
        assert not bool(t[~m].any())
    rng = np.random.default_rng(7)
    rows = rng.choice(np.nonzero(m.cpu().numpy().reshape(-1))[0], 24, replace=False)
    L = inp["logits"].reshape(-1, cfg.V)[torch.from_numpy(rows).to(DEV)].float().cpu().numpy()
    R = inp["ref_logits"].reshape(-1, cfg.V)[torch.from_numpy(rows).to(DEV)].float().cpu().numpy()
    ids = inp["ids"].reshape(-1).cpu().numpy()[rows]
    want, lse = orc.logprob(L.astype(np.float64), ids, dtype=orc.F64)
    want_r, lse_r = orc.logprob(R.astype(np.float64), ids, dtype=orc.F64)
    idt = inp["ids"].reshape(-1, 1)
    for got, got_s, got_l, logits, w, l in ((lp, lps, out.logp, inp["logits"], want, lse),
                                            (lr, lrs, out.ref_logp, inp["ref_logits"], want_r, lse_r)):
        for g in (got, got_s, got_l):
            g = g.reshape(-1).cpu().numpy()[rows]
            assert np.all(np.abs(g - w) <= 1e-5 * np.maximum(1, np.abs(l))), np.abs(g - w).max()
        # All three are within 1e-5 * max(1, |lse|) of the truth, lse = x_y - logp per token.
        xy = logits.reshape(-1, cfg.V).gather(1, idt).float().reshape(got.shape)
        tol = 2e-5 * torch.clamp((xy - got).abs(), min=1.0)
        for other in (got_s, got_l):
            assert bool(((got - other).abs()[m] <= tol[m]).all()), float((got - other).abs()[m].max())


def _fwd_logits(rng, n, V, dtype, neg_inf):
    x = (rng.standard_normal((n, V)) * 3.0).astype(np.float32)
    x[:, rng.integers(0, V, 3)] += 12.0                   # a few dominant columns
    if neg_inf:
        x[::2, rng.integers(0, V, max(1, V // 5))] = -np.inf  # masked-out vocabulary entries
    if dtype == "bf16":
        bits = orc.bf16_from_f32(x)
        return bits, orc.bf16_to_f32(bits).astype(np.float64)
    if dtype == "f16":
        h = x.astype(np.float16)
        return h, h.astype(np.float64)
    return x, x.astype(np.float64)


@pytest.mark.parametrize("dtype,V,lead", [("bf16", 8, 0), ("bf16", 136, 0), ("bf16", 16408, 0), ("bf16", 151936, 0),
                                          ("f16", 24, 0), ("f16", 32776, 0), ("f32", 4, 0), ("f32", 8196, 0),
                                          ("f32", 50000, 0), ("bf16", 3, 0), ("bf16", 50257, 0), ("bf16", 151936, 5),
                                          ("f16", 130, 3), ("f32", 1027, 1), ("f32", 7, 3)])
@pytest.mark.parametrize("with_ref", [False, True])
def test_logprob_fwd_kernel_shapes(dtype, V, lead, with_ref):
    """The forward-only kernel over one-vector rows, a ragged last batch, multi-batch
    rows and the config-2 width, and rows off 16 bytes: V not a multiple of the 16-byte
    vector (every row starts at a different offset) and logits viewed `lead` elements
    into their allocation (so even row 0 has a head). -inf vocabulary entries included.
    Log-probs within 1e-5 * max(1, |lse|) of the float64 oracle, the streaming kernel
    within 2e-5 * max(1, |lse|), masked and ignored tokens 0."""
    rng = np.random.default_rng(V * 3 + with_ref + 7 * lead)
    S, T = 3, 5
    n = S * T
    x, x64 = _fwd_logits(rng, n, V, dtype, neg_inf=True)
    r, r64 = _fwd_logits(rng, n, V, dtype, neg_inf=False)
    ids = rng.integers(0, V, n).astype(np.int64)
    ids[x64[np.arange(n), ids] == -np.inf] = int(np.argmax(x64[0]))   # keep targets finite
    ids = ids.reshape(S, T)
    ids[1, 2] = -100
    mask = np.ones((S, T), np.float32)
    mask[0, 4] = 0.0
    print(f"forward kernel {dtype} V={V} lead={lead} ref={with_ref}", flush=True)
    sh = (S, T, V)

    def placed(a):
        flat = dev(np.concatenate([a.reshape(-1)[:lead] if lead else a.reshape(-1)[:0], a.reshape(-1)]))
        return flat[lead:].view(sh)

    lt, rt = placed(x), placed(r)
    args = dict(mask=dev(mask))
    lp, lr = grpo.logprob_fwd(lt, dev(ids), rt if with_ref else None, **args)
    lps, lrs = grpo.logprob_fwd(lt, dev(ids), rt if with_ref else None, force_streaming=True, **args)
    torch.cuda.synchronize()
    live = (mask != 0) & (ids != -100)
    fid = np.where(ids.reshape(-1) < 0, 0, ids.reshape(-1))
    pairs = [(lp, lps, x64)] + ([(lr, lrs, r64)] if with_ref else [])
    for got, got_s, ref64 in pairs:
        want, lse = orc.logprob(ref64, fid, dtype=orc.F64)
        g = got.cpu().numpy().reshape(-1)
        gs = got_s.cpu().numpy().reshape(-1)
        lv = live.reshape(-1)
        tol = 1e-5 * np.maximum(1, np.abs(lse))
        assert np.all(np.abs(g - want)[lv] <= tol[lv]), np.abs(g - want)[lv].max()
        assert np.all(np.abs(g - gs)[lv] <= 2 * tol[lv])
        assert np.all(g[~lv] == 0) and np.all(gs[~lv] == 0)
    if not with_ref:
        assert lr is None


@pytest.mark.parametrize("dtype,V,lead,dlead", [("bf16", 50257, 0, 0), ("bf16", 130, 3, 3), ("bf16", 130, 3, 4),
                                               ("f16", 24, 5, 5), ("f32", 1027, 1, 1), ("f32", 7, 3, 0),
                                               ("bf16", 151937, 0, 0)])
def test_loss_rows_off_16_bytes(dtype, V, lead, dlead):
    """The loss path (fwd + bwd) on rows that start off 16 bytes: V not a multiple of the
    16-byte vector, and logits / dlogits viewed lead / dlead elements into their
    allocations. When dlogits share the logits' offset mod 16 the rows stay resident
    (aligned interior as vectors, head and tail element-wise); otherwise they stream.
    Log-probs, dlogits and the loss against the float64 oracle at the golden bars; the
    dlogits before and after the viewed rows are untouched."""
    rng = np.random.default_rng(V + 13 * lead + dlead)
    S, T, G = 4, 5, 2
    x, x64 = _fwd_logits(rng, S * T, V, dtype, neg_inf=False)
    noisy = (x64 + rng.standard_normal(x64.shape) * 0.1).astype(np.float32)   # ref = policy + N(0, 0.1^2)
    rr = {"bf16": orc.bf16_from_f32, "f16": lambda v: v.astype(np.float16), "f32": lambda v: v}[dtype](noisy)
    ids = rng.integers(0, V, (S, T)).astype(np.int64)
    mask = (rng.random((S, T)) < 0.8).astype(np.float32)
    old = (rng.standard_normal((S, T)) * 0.05 - np.log(V)).astype(np.float32)
    rewards = np.array([1, 0, 0.5, 0.25], np.float32)
    sh = (S, T, V)
    print(f"loss rows off 16 bytes: {dtype} V={V} lead={lead} dlead={dlead}", flush=True)

    def placed(a, k):
        flat = dev(np.concatenate([a.reshape(-1)[:k], a.reshape(-1)]))
        return flat[k:].view(sh)

    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    guard = 11
    dl_alloc = torch.full((dlead + S * T * V + guard,), 7.0, dtype=tdt, device=DEV)
    dl = dl_alloc[dlead:dlead + S * T * V].view(sh)
    out = grpo.grpo_loss_fwd_bwd(placed(x, lead), dev(ids), dev(mask), rewards=dev(rewards), group_size=G,
                                 ref_logits=placed(rr, 2 * lead), old_logp=dev(old),
                                 loss_mode=LossMode.GRPO_CLIP_KL, dlogits=dl)
    torch.cuda.synchronize()
    assert bool((dl_alloc[:dlead] == 7.0).all()) and bool((dl_alloc[dlead + S * T * V:] == 7.0).all())
    odt = {"bf16": orc.BF16, "f16": orc.F16, "f32": orc.F32}[dtype]
    want = orc.grpo_full(x.reshape(sh), ids, mask, rows=T, tok_offset=0, rewards=rewards, group_size=G,
                         ref_logits=rr.reshape(sh), old_logp=old, loss_mode=orc.CLIP_KL, dtype=odt)
    xs = x.reshape(sh)
    ts = token_scale(xs, ids, T, 0, odt)
    assert np.all(np.abs(out.logp.cpu().numpy() - want.lp) <= 1e-5 * ts)
    fl = full_floor(want, mask, old, S, False, 0.04, 0.2, ts)
    got = out.dlogits.float().cpu().numpy()
    assert_dlogits(got, want.dlogits, tok_to_rows(fl, T, 0, T), dtype != "f32", f16_out=dtype == "f16")
    assert abs(float(out.loss.cpu()) - want.loss) <= full_loss_tol(want, xs, ids, mask, T, 0, odt, False, 0.04, S)


# ---- host-bytes path (the WorkerBackend face) ------------------------------------------------

def test_execute_reference_signature():
    c = CASES["v64_shifted"]
    be = HipGrpoBackend.init()
    wb = be.asWorkerBackend()
    S, T, V = c["logits"].shape
    args = ([c["logits"], c["ids"], c["mask"], c["advantages"]],
            [c["logits"].shape, c["ids"].shape, c["mask"].shape, c["advantages"].shape],
            [DType.f32, DType.i64, DType.f32, DType.f32])
    outs = wb.executeFunction(None, "grpo_loss_fwd_bwd", *args)
    with pytest.raises(PcpError) as e:   # the whole step ("main") is not this library's
        wb.executeTrainingStep(None, *args)
    assert e.value.code == -10
    loss = np.frombuffer(outs[0], np.float32)[0]
    dl = np.frombuffer(outs[1], np.float32).reshape(S, T, V)
    assert abs(loss - c["exp_loss"]) <= golden_loss_tol(c)
    assert_dlogits(dl, c["exp_dlogits"], golden_floor_rows(c), False)
    assert not np.any(dl[:, T - 1])  # the sliced-off last position gets a zero gradient
    be.deinit()


C_HOST = r"""
/* A C caller of the host-bytes boundary, making the calls a Zig binding of the
 * reference's WorkerBackend would: pcp_init -> pcp_execute("grpo_loss_fwd_bwd") ->
 * pcp_free -> pcp_destroy.
 * argv: S T V dir; reads dir/{logits,ids,mask,adv}.bin, writes dir/{loss,dlogits}.bin. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "pcp_grpo.h"
static void* slurp(const char* dir, const char* name, size_t n) {
  char path[1024]; snprintf(path, sizeof path, "%s/%s", dir, name);
  FILE* f = fopen(path, "rb"); void* p = malloc(n);
  if (!f || !p || fread(p, 1, n, f) != n) { fprintf(stderr, "read %s\n", path); exit(3); }
  fclose(f); return p;
}
static void spill(const char* dir, const char* name, const void* p, size_t n) {
  char path[1024]; snprintf(path, sizeof path, "%s/%s", dir, name);
  FILE* f = fopen(path, "wb");
  if (!f || fwrite(p, 1, n, f) != n) { fprintf(stderr, "write %s\n", path); exit(3); }
  fclose(f);
}
int main(int argc, char** argv) {
  if (argc != 5) return 2;
  const int64_t S = atoll(argv[1]), T = atoll(argv[2]), V = atoll(argv[3]);
  const char* dir = argv[4];
  const size_t nb[4] = {(size_t)(S * T * V) * 4, (size_t)(S * T) * 8, (size_t)(S * T) * 4, (size_t)S * 4};
  const void* data[4] = {slurp(dir, "logits.bin", nb[0]), slurp(dir, "ids.bin", nb[1]),
                         slurp(dir, "mask.bin", nb[2]), slurp(dir, "adv.bin", nb[3])};
  const int64_t s0[3] = {S, T, V}, s1[2] = {S, T}, s3[1] = {S};
  const int64_t* shapes[4] = {s0, s1, s1, s3};
  const int ranks[4] = {3, 2, 2, 1};
  const int dtypes[4] = {PCP_F32, PCP_I64, PCP_F32, PCP_F32};
  pcp_ctx* ctx = NULL;
  int rc = pcp_init(PCP_BACKEND_ROCM, 0, &ctx);
  if (rc != PCP_OK) { fprintf(stderr, "pcp_init %d: %s\n", rc, pcp_last_error(NULL)); return 4; }
  int n_out = 0; void** outs = NULL; size_t* sizes = NULL;
  rc = pcp_execute(ctx, "grpo_loss_fwd_bwd", 4, data, nb, shapes, ranks, dtypes, &n_out, &outs, &sizes);
  if (rc != PCP_OK) { fprintf(stderr, "pcp_execute %d: %s\n", rc, pcp_last_error(ctx)); return 5; }
  if (n_out != 2 || sizes[0] != 4 || sizes[1] != nb[0]) { fprintf(stderr, "outputs %d\n", n_out); return 6; }
  spill(dir, "loss.bin", outs[0], sizes[0]);
  spill(dir, "dlogits.bin", outs[1], sizes[1]);
  pcp_free(ctx, n_out, outs, sizes);
  pcp_destroy(ctx);
  for (int i = 0; i < 4; ++i) free((void*)data[i]);
  printf("ok %d outputs\n", n_out);
  return 0;
}
"""


def test_c_host_execute_end_to_end(tmp_path):
    """The binding's call sequence (init, execute, free, destroy) from a compiled C host on the golden case
    v64_shifted (the reference's shifted layout): the loss and dlogits it writes match the
    torch float64 fixture at the golden bars."""
    import subprocess
    from pcp_amd import _lib

    c = CASES["v64_shifted"]
    S, T, V = c["logits"].shape
    for name, key, dt in [("logits.bin", "logits", np.float32), ("ids.bin", "ids", np.int64),
                          ("mask.bin", "mask", np.float32), ("adv.bin", "advantages", np.float32)]:
        np.ascontiguousarray(c[key], dtype=dt).tofile(tmp_path / name)
    src = tmp_path / "host.c"
    src.write_text(C_HOST)
    exe = tmp_path / "host"
    inc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
    libdir = os.path.dirname(_lib.LIB_PATH)
    subprocess.run(["gcc", "-std=c99", "-O1", "-I", inc, str(src), "-L", libdir, "-lpcp_grpo",
                    f"-Wl,-rpath,{libdir}", "-o", str(exe)], check=True)
    print(f"C host: pcp_execute(grpo_loss_fwd_bwd) on v64_shifted S={S} T={T} V={V}", flush=True)
    r = subprocess.run([str(exe), str(S), str(T), str(V), str(tmp_path)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    loss = np.fromfile(tmp_path / "loss.bin", np.float32)[0]
    dl = np.fromfile(tmp_path / "dlogits.bin", np.float32).reshape(S, T, V)
    assert abs(loss - c["exp_loss"]) <= golden_loss_tol(c)
    assert_dlogits(dl, c["exp_dlogits"], golden_floor_rows(c), False)
    assert not np.any(dl[:, T - 1])


def test_execute_clip_kl_and_logprob():
    rng = np.random.default_rng(7)
    S, T, V, G = 4, 9, 300, 2
    logits = (rng.standard_normal((S, T, V)) * 2).astype(np.float32)
    ref = (logits + rng.standard_normal((S, T, V)) * 0.1).astype(np.float32)
    ids = rng.integers(0, V, (S, T)).astype(np.int64)
    mask = (rng.random((S, T)) < 0.8).astype(np.float32)
    old = (rng.standard_normal((S, T)) * 0.05 - 6).astype(np.float32)
    rewards = np.array([1, 0, 0.5, 0.5], np.float32)
    hyper = np.array([G, 0.2, 0.04, 0], np.float32)
    be = HipGrpoBackend.init()
    ins = [logits, ref, ids, mask, old, rewards, hyper]
    outs = be.executeFunction(None, "grpo_clip_kl_fwd_bwd", ins, [x.shape for x in ins],
                              [DType.f32, DType.f32, DType.i64, DType.f32, DType.f32, DType.f32, DType.f32])
    want = orc.grpo_full(logits, ids, mask, rows=T - 1, tok_offset=1, rewards=rewards, group_size=G,
                         ref_logits=ref, old_logp=old, loss_mode=orc.CLIP_KL, dtype=orc.F32)
    loss = np.frombuffer(outs[0], np.float32)[0]
    assert abs(loss - want.loss) <= full_loss_tol(want, logits, ids, mask, T - 1, 1, orc.F32, False, 0.04, S)
    dl = np.frombuffer(outs[1], np.float32).reshape(S, T, V)
    fl = full_floor(want, mask, old, S, False, 0.04, 0.2, token_scale(logits, ids, T - 1, 1, orc.F32))
    assert_dlogits(dl, want.dlogits, tok_to_rows(fl, T - 1, 1, T), False)
    lp = np.frombuffer(outs[2], np.float32).reshape(S, T)
    assert np.allclose(lp, want.lp, rtol=1e-5, atol=2e-5)
    assert np.array_equal(np.frombuffer(outs[4], np.float32), want.adv)
    outs2 = be.executeFunction(None, "grpo_logprob_fwd", [logits, ids], [logits.shape, ids.shape],
                               [DType.f32, DType.i64])
    lp2 = np.frombuffer(outs2[0], np.float32).reshape(S, T)
    want_lp, _ = orc.logprob(logits[:, :-1].reshape(-1, V), ids[:, 1:].reshape(-1))
    assert np.allclose(lp2[:, 1:].reshape(-1), want_lp, rtol=1e-5, atol=2e-5)
    assert np.all(lp2[:, 0] == 0)
    adv = be.executeFunction(None, "grpo_advantages", [rewards, np.array(G, np.int64)], [(S,), ()],
                             [DType.f32, DType.i64])
    assert np.array_equal(np.frombuffer(adv[0], np.float32), orc.advantages(rewards, G))
    be.deinit()


@pytest.mark.parametrize("group_mib", [None, 48])
def test_execute_large_inputs_staged_and_pinned_outputs(group_mib, monkeypatch):
    """Inputs of 4 MiB and more go to the device through the context's pinned staging
    ring (three 64 MiB slots: a 158 MB logits tensor spans it and the reference tensor
    wraps it), outputs of 4 MiB and more come back in pooled pinned buffers. With
    PCP_EXECUTE_GROUP_MIB=48 the loss runs over groups of one sequence (40 MB of
    logits), uploads, kernels and downloads overlapping on three streams. Two successive
    host-bytes calls on fresh data each equal the device-pointer call on the same data
    bit for bit (loss, dlogits, log-probs, advantages)."""
    if group_mib:
        monkeypatch.setenv("PCP_EXECUTE_GROUP_MIB", str(group_mib))
    rng = np.random.default_rng(31)
    S, T, V, G = 4, 130, 151936, 2
    be = HipGrpoBackend.init()
    for call in range(2):
        print(f"host-bytes call {call}: [{S}, {T}, {V}] bf16, group MiB {group_mib}", flush=True)
        x = (rng.standard_normal((S, T, V)) * 3).astype(np.float32)
        logits = orc.bf16_from_f32(x)
        ref = orc.bf16_from_f32(x + (rng.standard_normal((S, T, V)) * 0.1).astype(np.float32))
        del x
        ids = rng.integers(0, V, (S, T)).astype(np.int64)
        mask = (rng.random((S, T)) < 0.8).astype(np.float32)
        old = (rng.standard_normal((S, T)) * 0.05 - 12).astype(np.float32)
        rewards = rng.random(S).astype(np.float32)
        hyper = np.array([G, 0.2, 0.04, 0], np.float32)
        ins = [logits, ref, ids, mask, old, rewards, hyper]
        outs = be.executeFunction(None, "grpo_clip_kl_fwd_bwd", ins, [a.shape for a in ins],
                                  [DType.bf16, DType.bf16, DType.i64, DType.f32, DType.f32, DType.f32, DType.f32])
        out = grpo.grpo_loss_fwd_bwd(dev(logits), dev(ids), dev(mask), rows=T - 1, tok_offset=1,
                                     rewards=dev(rewards), group_size=G, ref_logits=dev(ref), old_logp=dev(old),
                                     loss_mode=LossMode.GRPO_CLIP_KL, clip_eps=0.2, kl_beta=0.04)
        torch.cuda.synchronize()
        assert np.frombuffer(outs[0], np.float32)[0] == float(out.loss.cpu())
        assert np.array_equal(np.frombuffer(outs[1], np.uint16).reshape(S, T, V), host_bits(out.dlogits))
        assert np.array_equal(np.frombuffer(outs[2], np.float32).reshape(S, T)[:, 1:],
                              out.logp.cpu().numpy()[:, 1:])
        assert np.array_equal(np.frombuffer(outs[4], np.float32), out.advantages.cpu().numpy())
        del outs, out
    be.deinit()


# ---- device error reporting ---------------------------------------------------------------

def test_device_errors_are_reported_and_cleared():
    c = CASES["v7_ignore_empty"]
    ids = c["ids"].copy()
    ids[0, 0] = 7           # == V, on a live token
    with pytest.raises(PcpError) as e:
        run_case({**c, "ids": ids})
    assert e.value.code == -3
    out = run_case(c)       # the error word was cleared
    assert abs(float(out.loss.cpu()) - c["exp_loss"]) <= golden_loss_tol(c)
    # A NaN or +inf logit in a live row must surface, also when it is the only
    # element a lane holds (V=7: one element per lane) and on the resident path (V=1024).
    for name, bad in (("v7_ignore_empty", np.nan), ("v1024_clip_kl", np.nan), ("v1024_clip_kl", np.inf)):
        cc = CASES[name]
        lg = cc["logits"].copy()
        lg[0, 0, 3] = bad
        with pytest.raises(PcpError) as e:
            run_case({**cc, "logits": lg})
        assert e.value.code == -4, (name, bad)
    out = run_case(c)
    assert abs(float(out.loss.cpu()) - c["exp_loss"]) <= golden_loss_tol(c)


@pytest.mark.parametrize("S,T", [(1, 5), (3, 300), (64, 512), (1500, 7), (2100, 3)])
@pytest.mark.parametrize("mode", [LossMode.REINFORCE, LossMode.GRPO_CLIP_KL])
def test_loss_reduction_order_bit_exact(S, T, mode):
    """The one-launch loss reduction (per-sequence sums, then the last workgroup's sum
    over the sequences) equals, bit for bit, a float32 emulation of its fixed summation
    order applied to the device's own token losses: 256 lanes per sequence, 1024 lanes
    over the sequences (S = 1500 and 2100 take the second and third pass of that sum).
    The advantages it computes in the same launch as the lengths are the oracle's bits."""
    print(f"loss reduction order S={S} T={T} mode={int(mode)}", flush=True)
    rng = np.random.default_rng(S * 7 + T)
    V, G = 8, (3 if S % 3 == 0 else (2 if S % 2 == 0 else 1))
    x = torch.from_numpy(rng.standard_normal((S, T, V)).astype(np.float32) * 2).to(DEV)
    ids = torch.from_numpy(rng.integers(0, V, (S, T))).to(DEV)
    lengths = rng.integers(0, T + 1, S)
    mask = torch.from_numpy((np.arange(T)[None] < lengths[:, None]).astype(np.float32)).to(DEV)
    rewards = torch.from_numpy(rng.random(S).astype(np.float32)).to(DEV)
    old = torch.from_numpy((rng.standard_normal((S, T)) * 0.1 - 2).astype(np.float32)).to(DEV)
    ref = (x + 0.1 * torch.from_numpy(rng.standard_normal((S, T, V)).astype(np.float32)).to(DEV)).contiguous()
    out = grpo.grpo_loss_fwd_bwd(x, ids, mask, rewards=rewards, group_size=G, ref_logits=ref, old_logp=old,
                                 loss_mode=mode, want_dlogits=False)
    torch.cuda.synchronize()
    adv = orc.advantages(rewards.cpu().numpy(), G)
    assert np.array_equal(out.advantages.cpu().numpy().view(np.uint32), adv.view(np.uint32))
    want = emulate_loss(out.token_loss.cpu().numpy(), mask.cpu().numpy(), adv, mode == LossMode.REINFORCE, S)
    got = out.loss.cpu().numpy().astype(np.float32)
    assert got.view(np.uint32) == want.view(np.uint32), (float(got), float(want))
    # and again on the same context: the reduction's ticket was left at zero
    out2 = grpo.grpo_loss_fwd_bwd(x, ids, mask, rewards=rewards, group_size=G, ref_logits=ref, old_logp=old,
                                  loss_mode=mode, want_dlogits=False)
    torch.cuda.synchronize()
    assert torch.equal(out2.loss, out.loss)


def test_deterministic_repeat():
    c = CASES["v1024_clip_kl"]
    a = run_case(c)
    b = run_case(c)
    assert torch.equal(a.dlogits, b.dlogits) and torch.equal(a.loss, b.loss) and torch.equal(a.logp, b.logp)


# ---- full-size configurations: every live row against the oracle + global properties ---------

BF16_CACHED_BAR = (BF16_CACHED_REL, 1 + 2.0 ** -6)
BF16_EXACT_BAR = (BF16_EXACT_REL, 1 + 2.0 ** -7)


def _all_live_rows_check(cfg, inp, out, mode, exact, label, chunk=4096, f32_out=False):
    """Every live row of a full-size configuration against the oracle, in chunks of
    `chunk` rows: log-prob, reference log-prob and token loss of each against the f32
    bar, every dlogits element against the bf16 bar (oracle.check_dlogits compares the
    exact float64 rows in place), and the loss against the oracle's loss over all rows.
    Prints the largest error of each quantity and the largest share of its bar used."""
    S, T, V = inp["logits"].shape
    flat = inp["logits"].view(-1, V)
    rflat = inp["ref_logits"].view(-1, V)
    dflat = out.dlogits.view(-1, V)
    ids_all = inp["ids"].view(-1).cpu().numpy()
    mask = inp["mask"].cpu().numpy()
    w_all = mask.reshape(-1)
    rewards = inp["rewards"].cpu().numpy()
    adv = orc.advantages(rewards, cfg.group)
    assert np.array_equal(out.advantages.cpu().numpy().view(np.uint32), adv.view(np.uint32))
    Ls = orc.seq_lengths(mask, T, 0)
    old_all = inp["old_logp"].view(-1).cpu().numpy()
    lp_all = out.logp.view(-1).cpu().numpy()
    lr_all = out.ref_logp.view(-1).cpu().numpy() if out.ref_logp is not None else None
    tl_all = out.token_loss.view(-1).cpu().numpy()
    m = orc.CLIP_KL if mode == LossMode.GRPO_CLIP_KL else orc.REINFORCE
    rel, kf = (1e-5, 1.0) if f32_out else (BF16_EXACT_BAR if exact else BF16_CACHED_BAR)
    live = np.nonzero((w_all != 0) & (ids_all >= 0) & (ids_all < V))[0]
    st = dict(lp=0.0, lr=0.0, tl=0.0, usage=0.0, abs=0.0, rel=0.0)
    tl_exact = np.zeros(S * T)
    coef_exact = np.zeros(S * T)
    lse_exact = np.zeros(S * T)
    lp_exact = np.zeros(S * T)
    lr_exact = np.zeros(S * T)
    for i0 in range(0, len(live), chunk):
        rows = live[i0:i0 + chunk]
        n = len(rows)
        idx = torch.as_tensor(rows, device=DEV)
        L = host_bits(flat.index_select(0, idx))
        R = host_bits(rflat.index_select(0, idx)) if m == orc.CLIP_KL else None
        D = host_bits(dflat.index_select(0, idx))
        ids = ids_all[rows]
        seq = rows // T
        w = w_all[rows]
        want = orc.grpo_rows(L, ids, w, adv[seq], Ls[seq], float(S), ref_logits=R, old_logp=old_all[rows],
                             loss_mode=m, clip_eps=cfg.clip_eps, kl_beta=cfg.kl_beta, dtype=orc.BF16,
                             want_dlogits=False)
        lse = orc.bf16_to_f32(L[np.arange(n), ids]).astype(np.float64) - want.lp
        sc = np.maximum(1.0, np.abs(lse))
        e_lp = np.abs(lp_all[rows] - want.lp) / sc
        e_tl = np.abs(tl_all[rows] - want.token_loss) / sc
        assert e_lp.max() <= 1e-5 and e_tl.max() <= 1e-5, (label, e_lp.max(), e_tl.max())
        if m == orc.CLIP_KL:
            rlse = orc.bf16_to_f32(R[np.arange(n), ids]).astype(np.float64) - want.lr
            e_lr = np.abs(lr_all[rows] - want.lr) / np.maximum(1.0, np.abs(rlse))
            assert e_lr.max() <= 1e-5, (label, e_lr.max())
            st["lr"] = max(st["lr"], float(e_lr.max()))
        fl = coef_floor(want.coef, want.lp, want.lr, w, adv[seq].astype(np.float64), Ls[seq].astype(np.float64),
                        float(S), old_all[rows].astype(np.float64), m == orc.REINFORCE, cfg.kl_beta, cfg.clip_eps,
                        sc)
        res = orc.check_dlogits(L, ids, want.coef, fl, D, orc.F32 if f32_out else orc.BF16, rel, kf, dtype=orc.BF16)
        assert int(res.n_bad.sum()) == 0, (label, int(res.n_bad.sum()), float(res.max_usage.max()))
        if f32_out:
            assert float(res.max_abs.max()) <= 1e-4, (label, float(res.max_abs.max()))
        st["lp"] = max(st["lp"], float(e_lp.max()))
        st["tl"] = max(st["tl"], float(e_tl.max()))
        st["usage"] = max(st["usage"], float(res.max_usage.max()))
        st["abs"] = max(st["abs"], float(res.max_abs.max()))
        st["rel"] = max(st["rel"], float(res.max_rel.max()))
        tl_exact[rows] = want.token_loss
        coef_exact[rows] = want.coef
        lse_exact[rows] = lse
        lp_exact[rows] = want.lp
        lr_exact[rows] = want.lr
    # The loss from the oracle's token losses of every live row.
    tl2 = tl_exact.reshape(S, T)
    seqv = tl2.sum(1) / Ls.astype(np.float64)
    if m == orc.REINFORCE:
        seqv = seqv * adv.astype(np.float64)
    loss_exact = float(seqv.sum() / S)
    tol = loss_tolerance(tl2, coef_exact.reshape(S, T), lp_exact.reshape(S, T), lr_exact.reshape(S, T), mask,
                         adv, Ls, float(S), m == orc.REINFORCE, cfg.kl_beta,
                         np.maximum(1.0, np.abs(lse_exact)).reshape(S, T))
    got_loss = float(out.loss.cpu())
    assert abs(got_loss - loss_exact) <= tol, (label, got_loss, loss_exact, tol)
    st["loss_rel"] = abs(got_loss - loss_exact) / max(abs(loss_exact), 1e-30)
    st["loss_use"] = abs(got_loss - loss_exact) / tol
    terms = np.abs(tl2).sum(1) / Ls.astype(np.float64)
    if m == orc.REINFORCE:
        terms = terms * np.abs(adv.astype(np.float64))
    st["loss_rel_terms"] = abs(got_loss - loss_exact) / (terms.sum() / S)
    print(f"PARITY-TABLE {label}: live rows {len(live)} of {S * T}; |dlogp|/max(1,|lse|) {st['lp']:.2e}"
          f" (bar 1e-5); ref {st['lr']:.2e}; token loss {st['tl']:.2e}; loss rel {st['loss_rel']:.2e}, per sum of"
          f" |terms| {st['loss_rel_terms']:.2e} ({st['loss_use']:.3f} of its bar); {'f32' if f32_out else 'bf16'}"
          f" dlogits max abs {st['abs']:.2e}{' (bar 1e-4)' if f32_out else ''}, max rel (p >= 2^-14) {st['rel']:.3e}"
          f"{'' if f32_out else ' (2^-8 = 3.906e-03)'}, bar used {st['usage']:.3f}", flush=True)
    return st


def _full_config(key, mode, exact=False, n_seq=None, f32_out=False, zero_fill=True):
    cfg = synth.CONFIGS[key]
    inp = synth.make_device_inputs(cfg, DEV, n_seq=n_seq)
    S = inp["logits"].shape[0]
    label = (f"config{key} {'clip_kl' if mode == LossMode.GRPO_CLIP_KL else 'reinforce'}" + (" exact" if exact else "")
             + (f" f32 dlogits, {S} sequences" if f32_out else "") + ("" if zero_fill else " no zero-fill"))
    print(f"full-size {label}", flush=True)
    sentinel = -3.5
    dl = None if zero_fill else torch.full(inp["logits"].shape, sentinel,
                                           dtype=torch.float32 if f32_out else torch.bfloat16, device=DEV)
    out = grpo.grpo_loss_fwd_bwd(inp["logits"], inp["ids"], inp["mask"], rewards=inp["rewards"], group_size=cfg.group,
                                 ref_logits=inp["ref_logits"], old_logp=inp["old_logp"], loss_mode=mode,
                                 clip_eps=cfg.clip_eps, kl_beta=cfg.kl_beta, exact_bf16=exact,
                                 dlogits_dtype=torch.float32 if f32_out else None, dlogits=dl, zero_fill=zero_fill)
    torch.cuda.synchronize()
    T = cfg.T
    _all_live_rows_check(cfg, inp, out, mode, exact, label, f32_out=f32_out)
    # every masked row of dlogits is exactly zero, or without zero-fill untouched
    lengths = inp["lengths"]
    for s in range(S):
        ln = int(lengths[s])
        if ln < T:
            if zero_fill:
                assert float(out.dlogits[s, ln:].abs().amax()) == 0.0
            else:
                assert bool((out.dlogits[s, ln:] == sentinel).all())
    # loss == the f64 aggregation of the kernel's own token losses (reduce kernels)
    tl = out.token_loss.double().cpu().numpy()
    Ls = orc.seq_lengths(inp["mask"].cpu().numpy(), T, 0).astype(np.float64)
    seqv = tl.sum(1) / Ls
    if mode == LossMode.REINFORCE:
        seqv = seqv * out.advantages.double().cpu().numpy()
    scale = (np.abs(tl).sum(1) / Ls * (np.abs(out.advantages.double().cpu().numpy())
                                        if mode == LossMode.REINFORCE else 1.0)).sum() / S
    assert abs(float(out.loss.cpu()) - seqv.sum() / S) <= 1e-5 * scale
    # log-probs of every row agree with the forward-only kernel
    lp2, _ = grpo.logprob_fwd(inp["logits"], inp["ids"])
    m = inp["mask"] != 0
    assert float((out.logp - lp2).abs()[m].max()) <= 2e-5 * 20
    return inp, out


@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("mode", [LossMode.GRPO_CLIP_KL, LossMode.REINFORCE])
def test_config2_full_size(mode, exact):
    _full_config(2, mode, exact)


def test_config2_rows_f32_dlogits():
    """bf16 logits with f32 dlogits (the resident kernel's split-half instance) at
    configuration 2's row shape, 8 of its sequences, every live row against the oracle
    under the f32 bar (max-abs 1e-4)."""
    _full_config(2, LossMode.GRPO_CLIP_KL, n_seq=8, f32_out=True)


@pytest.mark.parametrize("exact", [False, True])
def test_config3_full_size(exact):
    _full_config(3, LossMode.GRPO_CLIP_KL, exact)


@pytest.mark.parametrize("exact", [False, True])
def test_config4_full_size(exact):
    _full_config(4, LossMode.GRPO_CLIP_KL, exact)


@pytest.mark.parametrize("key", [2, 4])
def test_full_size_no_zero_fill(key):
    """PCP_FLAG_NO_ZERO_FILL at full size. Config 4 (21% of rows live) takes the listed
    path, where each workgroup runs about 53 live rows in turn and loads each next row's
    policy chunks during the current row's dlogits pass; config 2 (57% live) visits
    every row. Every live row against the oracle, dead rows untouched."""
    _full_config(key, LossMode.GRPO_CLIP_KL, zero_fill=False)


def test_config4_rows_f32_dlogits_no_zero_fill():
    """bf16 logits, f32 dlogits, no zero-fill at configuration 4 (21% of rows live): the
    listed path with the next-row prefetch on the split-half instance, about 53 rows per
    workgroup. Every live row against the oracle under the f32 bar, dead rows untouched."""
    _full_config(4, LossMode.GRPO_CLIP_KL, f32_out=True, zero_fill=False)


@pytest.mark.parametrize("V", [(1 << 29) - 4, (1 << 29) + 4])
def test_logprob_fwd_two_gib_rows(V):
    """f32 rows just under 2 GiB (the forward kernel, 32-bit buffer offsets) and just
    over (the streaming kernel): log-probs within 1e-5 * max(1, |lse|) of a float64
    log-sum-exp on the host. The target, three elements before the row end where the
    offsets are largest, holds e^8 times the rest of the row's mass: a kernel that
    missed or misplaced it would be off by ~8. (With no dominant term, each lane's f32
    sum of ~2M small terms drops those below half an ulp, ~0.3% of the sum here.)"""
    print(f"forward-only f32 row of V={V}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(V & 0xFFFF)
    x = torch.randn((1, 1, V), device=DEV, generator=g) * 2.0
    ids = torch.tensor([[V - 3]], device=DEV)
    x[0, 0, V - 3] = 30.0
    lp, _ = grpo.logprob_fwd(x, ids)
    torch.cuda.synchronize()
    h = x.view(-1).cpu().numpy()
    del x
    m = float(h.max())
    s = 0.0
    for i in range(0, V, 1 << 26):
        s += float(np.exp(h[i:i + (1 << 26)].astype(np.float64) - m).sum())
    lse = m + np.log(s)
    want = 30.0 - lse
    assert abs(float(lp[0, 0]) - want) <= 1e-5 * max(1.0, abs(lse)), (float(lp[0, 0]), want)
