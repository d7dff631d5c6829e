"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the HIP path.

Each oracle function is checked against something it was not derived from:
the reference's known-answer tests (src/examples/isolated_vjp_tests.zig), the
committed golden fixtures (torch CPU float64 autograd, numpy float32 simulation),
closed forms, brute force and finite differences in float64. The mutation tests
at the end plant plausible mistakes in oracle outputs and show the checks catch
them.
"""
import json
import os

import numpy as np
import pytest
import torch

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def load_cases():
    z = np.load(os.path.join(GOLD, "cases.npz"))
    cases = {}
    for k in z.files:
        name, field = k.split("/", 1)
        cases.setdefault(name, {})[field] = z[k]
    return cases


CASES = load_cases()


def run_oracle_case(orc, c, precision=0):
    dt = orc.BF16 if c["logits"].dtype == np.uint16 else orc.F32
    kw = {}
    if "advantages" in c:
        kw["advantages_in"] = c["advantages"]
    else:
        kw["rewards"] = c["rewards"]
    return orc.grpo_full(c["logits"], c["ids"], c["mask"], rows=int(c["rows"]), tok_offset=int(c["tok_offset"]),
                         group_size=int(c["group_size"]), ref_logits=c.get("ref_logits"),
                         old_logp=c.get("old_logp"), loss_mode=int(c["loss_mode"]), clip_eps=float(c["clip_eps"]),
                         kl_beta=float(c["kl_beta"]), loss_norm=float(c["loss_norm"]), precision=precision,
                         dtype=dt, **kw)


# ---- codecs ------------------------------------------------------------------------

def test_bf16_rne_matches_torch(orc):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.005859375, 1.0078125, 3.0e38, -1e-40, np.inf, -np.inf],
                                 np.float32)])
    # exact ties: mantissa ...1 1000 0000 0000 0000 and ...0 1000 ...
    ties = (np.arange(1000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = orc.bf16_from_f32(x)
    assert np.array_equal(got, want)
    back = orc.bf16_to_f32(got)
    assert np.array_equal(back, torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy())


# ---- a3 advantages -----------------------------------------------------------------

def test_advantages_bit_exact_against_fixture(orc):
    with open(os.path.join(GOLD, "advantages.json")) as f:
        d = json.load(f)
    assert len(d["cases"]) >= 9
    for c in d["cases"]:
        r = np.array(c["rewards_bits"], np.uint32).view(np.float32)
        want = np.array(c["adv_bits"], np.uint32)
        got = orc.advantages(r, c["group"], d["eps"]).view(np.uint32)
        assert np.array_equal(got, want), c["name"]


def test_advantages_hand_values(orc):
    # G=4, r=[1,0,0,0]: mean 0.25, std sqrt(0.1875) + 1e-8.
    a = orc.advantages(np.array([1, 0, 0, 0], np.float32), 4)
    sd = np.float32(np.sqrt(np.float32(0.1875))) + np.float32(1e-8)
    assert a[0] == np.float32(np.float32(0.75) / sd)
    assert a[1] == np.float32(np.float32(-0.25) / sd)
    # binary all-equal groups give exactly 0; partial last group uses its own n
    a = orc.advantages(np.array([1, 1, 1, 0, 1], np.float32), 3)
    assert np.all(a[:3] == 0) and a[3] == -1 and a[4] == 1


def test_advantages_degenerate_groups_are_rounding_noise(orc):
    # The reference adds 1e-8 to the std *outside* the sqrt, so an all-equal group of
    # non-representable rewards gives (r - mean)/(tiny + 1e-8), not 0.
    a = orc.advantages(np.full(16, 0.7, np.float32), 16)
    assert np.all(a == a[0]) and a[0] != 0 and abs(a[0]) < 1.0


# ---- a1 log-prob ---------------------------------------------------------------------

def test_logprob_closed_forms(orc):
    V = 1000
    x = np.full((3, V), 0.37, np.float32)
    lp, lse = orc.logprob(x, np.array([0, 5, 999]))
    assert np.allclose(lp, -np.log(V), rtol=0, atol=1e-12)
    lp1, _ = orc.logprob(np.array([[3.5], [-7.0]], np.float32), np.array([0, 0]))
    assert np.all(lp1 == 0.0)
    rng = np.random.default_rng(1)
    y = rng.standard_normal((5, 77)).astype(np.float32)
    ids = rng.integers(0, 77, 5)
    a, _ = orc.logprob(y, ids)
    b, _ = orc.logprob((y + np.float32(40.0)).astype(np.float32), ids)  # shift invariance (exact shift in f32? not always)
    assert np.allclose(a, b, atol=2e-5)


def test_logprob_brute_force_and_torch(orc):
    rng = np.random.default_rng(2)
    y = (rng.standard_normal((64, 513)) * 3).astype(np.float32)
    ids = rng.integers(0, 513, 64)
    lp, lse = orc.logprob(y, ids)
    y64 = y.astype(np.float64)
    m = y64.max(1, keepdims=True)
    brute = y64[np.arange(64), ids] - (m[:, 0] + np.log(np.exp(y64 - m).sum(1)))
    assert np.allclose(lp, brute, rtol=0, atol=1e-12)
    ce = torch.nn.functional.cross_entropy(torch.from_numpy(y), torch.from_numpy(ids), reduction="none").numpy()
    lpf, _ = orc.logprob(y, ids, precision=orc.REF_F32)
    assert np.allclose(-lpf, ce, rtol=1e-5, atol=1e-5)
    assert np.allclose(lpf, lp, rtol=1e-5, atol=1e-5)


def test_reference_kat_cross_entropy_stability(orc):
    with open(os.path.join(GOLD, "reference_kats.json")) as f:
        kat = json.load(f)["cross_entropy_stability"]
    x = np.array([kat["logits"]], np.float32)
    ids = np.array([kat["target"]])
    for prec in (orc.EXACT, orc.REF_F32, orc.FAITHFUL):
        # loss = -lp with upstream 1: one sequence, A = 1, L = 1, G = 1.
        r = orc.grpo_rows(x, ids, [1.0], [1.0], [1.0], 1.0, precision=prec)
        assert abs(r.token_loss[0] - kat["expect_loss"]) <= kat["atol"]
        assert np.all(np.abs(r.dlogits[0] - np.array(kat["expect_grad"])) <= kat["atol"])


def test_reference_kat_reduce_max_routes_to_the_max(orc):
    # reduceMaxVJP sends the upstream gradient to the element equal to the max
    # ([1,5,3] -> [0,1,0]); in the faithful backward that is the only place the
    # 1e-4 leak of the log guard appears.
    with open(os.path.join(GOLD, "reference_kats.json")) as f:
        kat = json.load(f)["reduce_max_grad"]
    x = np.array([kat["x"]], np.float32)
    ex = orc.grpo_rows(x, np.array([2]), [1.0], [1.0], [1.0], 1.0, precision=orc.EXACT)
    fa = orc.grpo_rows(x, np.array([2]), [1.0], [1.0], [1.0], 1.0, precision=orc.FAITHFUL)
    diff = fa.dlogits[0] - ex.dlogits[0]
    route = np.array(kat["expect_grad"])
    leak = diff[np.argmax(route)]
    assert leak != 0
    others = diff - leak * route
    assert np.all(np.abs(others) < 1e-4 * 2 * abs(ex.coef[0]))


# ---- a2/a4/a5 against the torch-autograd fixtures ---------------------------------------

@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_golden(orc, name):
    c = CASES[name]
    r = run_oracle_case(orc, c)
    np.testing.assert_allclose(r.loss, c["exp_loss"], rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(r.lp, c["exp_lp"], rtol=1e-12, atol=1e-12)
    if "ref_logits" in c:
        np.testing.assert_allclose(r.lr, c["exp_lr"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(r.token_loss, c["exp_token_loss"], rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(r.coef, c["exp_coef"], rtol=1e-10, atol=1e-16)
    assert np.array_equal(r.adv, c["exp_adv"])
    scale = max(np.abs(c["exp_coef"]).max(), 1e-30)
    np.testing.assert_allclose(r.dlogits, c["exp_dlogits"], rtol=1e-6, atol=1e-7 * scale)


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_f32_order_within_north_star_tolerance(orc, name):
    c = CASES[name]
    ex = run_oracle_case(orc, c, orc.EXACT)
    f = run_oracle_case(orc, c, orc.REF_F32)
    lse_scale = np.maximum(1.0, np.abs(ex.lp))
    assert np.all(np.abs(f.lp - ex.lp) <= 1e-5 * lse_scale + 1e-5)
    assert abs(f.loss - ex.loss) <= 1e-5 * max(1.0, abs(ex.loss))
    assert np.abs(f.dlogits - ex.dlogits).max() <= 1e-4


def test_faithful_reference_ad_within_dlogits_budget(orc):
    for name in ("v7_ignore_empty", "v64_shifted", "v2_ties_large"):
        c = CASES[name]
        ex = run_oracle_case(orc, c, orc.EXACT)
        fa = run_oracle_case(orc, c, orc.FAITHFUL)
        gap = np.abs(fa.dlogits - ex.dlogits).max()
        assert gap <= 1e-4
        # the guards perturb each row by about 1e-4 relative to its coefficient
        assert gap <= 3e-4 * np.abs(ex.coef).max() + 1e-7


def test_dlogits_invariants(orc):
    c = CASES["v1024_clip_kl"]
    r = run_oracle_case(orc, c)
    S, LS, V = r.dlogits.shape
    row_sums = r.dlogits.astype(np.float64).sum(-1)
    assert np.abs(row_sums).max() <= 1e-6 * np.abs(r.coef).max()
    dead = c["mask"][:, :LS] == 0
    assert np.all(r.dlogits[dead] == 0)


def test_clip_kl_special_cases(orc):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((6, 50)) * 2).astype(np.float32)
    ids = rng.integers(0, 50, 6)
    w, A, L = np.ones(6), np.array([1, -1, 0.5, -2, 1, 1], np.float32), np.full(6, 3.0)
    base = orc.grpo_rows(x, ids, w, A, L, 2.0)  # REINFORCE
    # beta = 0 and old = lp (ratio 1): the clip-KL gradient reduces to the reference's.
    on = orc.grpo_rows(x, ids, w, A, L, 2.0, ref_logits=x, loss_mode=orc.CLIP_KL, kl_beta=0.0)
    np.testing.assert_allclose(on.coef, base.coef, rtol=1e-14)
    np.testing.assert_allclose(on.dlogits, base.dlogits, rtol=1e-6, atol=1e-12)
    # ref = policy: KL term and its gradient vanish for any beta.
    kl = orc.grpo_rows(x, ids, w, A, L, 2.0, ref_logits=x, loss_mode=orc.CLIP_KL, kl_beta=0.5)
    np.testing.assert_allclose(kl.coef, on.coef, rtol=1e-14)
    # ratio beyond the trust region on the side the advantage rewards: zero gradient.
    lp = base.lp
    old = lp - np.where(A > 0, 1.0, -1.0)   # rho = e (A>0) or 1/e (A<0)
    cl = orc.grpo_rows(x, ids, w, A, L, 2.0, ref_logits=x, old_logp=old, loss_mode=orc.CLIP_KL, kl_beta=0.0)
    assert np.all(cl.coef == 0)
    # ...and the unclipped side keeps -A*rho.
    old2 = (lp + np.where(A > 0, 1.0, -1.0)).astype(np.float32)   # the ABI carries old_logp as f32
    uc = orc.grpo_rows(x, ids, w, A, L, 2.0, ref_logits=x, old_logp=old2, loss_mode=orc.CLIP_KL, kl_beta=0.0)
    rho = np.exp(lp - old2.astype(np.float64))
    np.testing.assert_allclose(uc.coef, -A * rho / (2.0 * 3.0), rtol=1e-12)


def test_finite_differences_tiny(orc):
    rng = np.random.default_rng(4)
    V = 9
    x = (rng.standard_normal((1, V)) * 1.5).astype(np.float64)
    ref = (x + rng.standard_normal((1, V)) * 0.3)
    ids = np.array([4])
    args = dict(ref_logits=ref.astype(np.float32), old_logp=np.array([-2.0], np.float32), loss_mode=orc.CLIP_KL,
                kl_beta=0.3, clip_eps=0.2)

    def loss_at(xx):
        r = orc.grpo_rows(xx.astype(np.float32), ids, [1.0], [0.8], [1.0], 1.0, want_dlogits=False, **args)
        return r.token_loss[0]

    # f32 inputs: probe with steps large enough for f32 storage, central differences.
    g = orc.grpo_rows(x.astype(np.float32), ids, [1.0], [0.8], [1.0], 1.0, **args).dlogits[0]
    x32 = x.astype(np.float32).astype(np.float64)
    h = 1e-2
    fd = np.array([(loss_at(x32 + h * np.eye(V)[v]) - loss_at(x32 - h * np.eye(V)[v])) / (2 * h) for v in range(V)])
    np.testing.assert_allclose(g, fd, rtol=2e-3, atol=2e-4)


def test_check_dlogits_agrees_with_numpy_and_catches_planted_mistakes(orc):
    """check_dlogits (the in-place element-wise comparison the full-size GPU tests use)
    against the same statistics computed in numpy from grpo_rows' materialised exact
    rows, on bf16 and f32 device-like outputs; then planted mistakes in the compared
    rows (a sign, a shifted index, a dropped onehot term, one element off by two bf16
    ulps) are counted."""
    rng = np.random.default_rng(11)
    N, V = 12, 777
    x = orc.bf16_from_f32((rng.standard_normal((N, V)) * 3).astype(np.float32))
    ids = rng.integers(0, V, N)
    A = rng.standard_normal(N).astype(np.float32)
    r = orc.grpo_rows(x, ids, np.ones(N), A, np.full(N, 5.0), 2.0, dtype=orc.BF16)
    exact = orc.grpo_rows(x, ids, np.ones(N), A, np.full(N, 5.0), 2.0, dtype=orc.BF16).dlogits
    # grpo_rows stores f32; recompute the float64 rows for the numpy side.
    xd = orc.bf16_to_f32(x).astype(np.float64)
    lse = np.log(np.exp(xd - xd.max(1, keepdims=True)).sum(1)) + xd.max(1)
    d = -np.exp(xd - lse[:, None]) * r.coef[:, None]
    d[np.arange(N), ids] += r.coef
    np.testing.assert_allclose(exact, d.astype(np.float32), rtol=0, atol=0)
    fl = 1e-5 * np.abs(r.coef)
    rel, kf = 2.0 ** -8 + 1.1e-5, 1 + 2.0 ** -7
    for dt, got in ((orc.BF16, orc.bf16_from_f32(d.astype(np.float32))), (orc.F32, d.astype(np.float32))):
        res = orc.check_dlogits(x, ids, r.coef, fl, got, dt, rel, kf, dtype=orc.BF16)
        g = orc.bf16_to_f32(got).astype(np.float64) if dt == orc.BF16 else got.astype(np.float64)
        err = np.abs(g - d)
        tol = rel * np.abs(d) + kf * fl[:, None]
        # The two log-sum-exps differ in summation order (~1e-16 relative), which moves
        # the tiny f32 errors by ~1e-17 absolute.
        np.testing.assert_allclose(res.max_abs, err.max(1), rtol=1e-6, atol=1e-15)
        np.testing.assert_allclose(res.max_usage, (err / tol).max(1), rtol=1e-6, atol=1e-9)
        big = np.abs(d) >= 2.0 ** -14 * np.abs(r.coef)[:, None]
        np.testing.assert_allclose(res.max_rel, np.where(big, err / np.where(big, np.abs(d), 1), 0).max(1),
                                   rtol=1e-6, atol=1e-12)
        assert (res.n_bad == 0).all() and res.max_usage.max() <= 1.0
        if dt == orc.BF16:
            assert res.max_rel.max() <= 2.0 ** -8 and res.max_rel.max() > 2.0 ** -10   # RNE rounding is seen
    good = orc.bf16_from_f32(d.astype(np.float32))

    def bad_rows(g):
        return int((orc.check_dlogits(x, ids, r.coef, fl, g, orc.BF16, rel, kf, dtype=orc.BF16).n_bad > 0).sum())

    assert bad_rows(orc.bf16_from_f32(-d.astype(np.float32))) == N            # sign of the coefficient
    assert bad_rows(np.ascontiguousarray(np.roll(good, 1, axis=1))) == N      # off-by-one vocabulary index
    no_onehot = d.copy()
    no_onehot[np.arange(N), ids] -= r.coef
    assert bad_rows(orc.bf16_from_f32(no_onehot.astype(np.float32))) == N     # dropped onehot term
    one = good.copy()
    one[3, ids[3]] = one[3, ids[3]] + 2 if abs(d[3, ids[3]]) > 0 else one[3, ids[3]]   # two ulps at the target
    assert bad_rows(one) == 1


# ---- mutation tests: plausible mistakes in the oracle are caught -----------------

def test_checks_catch_planted_mistakes(orc):
    c = CASES["v1024_clip_kl"]
    r = run_oracle_case(orc, c)
    want = c["exp_dlogits"]
    scale = np.abs(c["exp_coef"]).max()

    def passes(d):
        return np.allclose(d, want, rtol=1e-6, atol=1e-7 * scale)

    assert passes(r.dlogits)
    assert not passes(-r.dlogits)                                   # sign of the coefficient
    shifted = np.roll(r.dlogits, 1, axis=-1)                        # off-by-one gather index
    assert not passes(shifted)
    no_onehot = r.dlogits.copy()                                    # dropped onehot term
    S, LS, V = no_onehot.shape
    for s in range(S):
        for t in range(int(c["rows"])):
            i = c["ids"][s, t]
            if c["mask"][s, t] != 0:
                no_onehot[s, t, i] -= r.coef[s, t]
    assert not passes(no_onehot)
    assert not np.allclose(r.loss * (1 + 1e-4), c["exp_loss"], rtol=1e-12)   # a dropped eps-level term
    transposed = np.transpose(r.dlogits, (1, 0, 2)).reshape(r.dlogits.shape) if S != LS else None
    if transposed is not None:
        assert not passes(transposed)


# ---- a6: LM-head oracle -------------------------------------------------------------

def test_lmhead_logits_brute_force_and_torch(orc):
    """logits = hidden . W^T of the exact bf16 values: brute-force dot products on a tiny
    case, torch float64 matmul on a larger one, and a transposed-operand mistake fails."""
    rng = np.random.default_rng(3)
    hb = orc.bf16_from_f32(rng.standard_normal((3, 5)).astype(np.float32))
    wb = orc.bf16_from_f32(rng.standard_normal((4, 5)).astype(np.float32))
    got = orc.lmhead_logits(hb, wb)
    h, w = orc.bf16_to_f32(hb).astype(np.float64), orc.bf16_to_f32(wb).astype(np.float64)
    brute = np.array([[sum(h[n, k] * w[v, k] for k in range(5)) for v in range(4)] for n in range(3)])
    np.testing.assert_allclose(got, brute, rtol=1e-14, atol=1e-14)
    hb = orc.bf16_from_f32(rng.standard_normal((17, 64)).astype(np.float32))
    wb = orc.bf16_from_f32(rng.standard_normal((33, 64)).astype(np.float32))
    ref = torch.from_numpy(orc.bf16_to_f32(hb).astype(np.float64)) @ torch.from_numpy(
        orc.bf16_to_f32(wb).astype(np.float64)).T
    np.testing.assert_allclose(orc.lmhead_logits(hb, wb), ref.numpy(), rtol=1e-13, atol=1e-13)
    assert not np.allclose(orc.lmhead_logits(hb, wb)[:, :17], ref.numpy()[:17, :17].T, rtol=1e-3)


def test_lmhead_grads_match_torch_autograd(orc):
    """dhidden = D.W and dW = D^T.hidden with D = c (onehot - softmax) against torch float64
    autograd of L = sum_n c_n * logp_n(hidden . W^T) (the LM head's VJP, matmulVJP,
    src/autodiff/vjp_rules.zig:426-497). Masked tokens (c = 0) and an ignored id carry no gradient."""
    rng = np.random.default_rng(4)
    N, H, V = 9, 16, 23
    hb = orc.bf16_from_f32(rng.standard_normal((N, H)).astype(np.float32))
    wb = orc.bf16_from_f32((rng.standard_normal((V, H)) * 0.5).astype(np.float32))
    ids = rng.integers(0, V, N)
    ids[4] = -100
    coef = rng.standard_normal(N)
    coef[2] = 0.0
    coef[4] = 0.0
    h = torch.tensor(orc.bf16_to_f32(hb).astype(np.float64), requires_grad=True)
    w = torch.tensor(orc.bf16_to_f32(wb).astype(np.float64), requires_grad=True)
    logits = h @ w.T
    lp = torch.log_softmax(logits, dim=1).gather(1, torch.from_numpy(np.clip(ids, 0, None))[:, None])[:, 0]
    (torch.from_numpy(coef) * lp).sum().backward()
    L = logits.detach().numpy()
    lse = torch.logsumexp(logits, dim=1).detach().numpy()
    dh, dw = orc.lmhead_grads(hb, wb, L, lse, coef, ids)
    np.testing.assert_allclose(dh, h.grad.numpy(), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(dw, w.grad.numpy(), rtol=1e-12, atol=1e-13)
    assert not np.any(dh[[2, 4]])
    # planted mistakes: a flipped sign, a dropped onehot term
    assert not np.allclose(-dh, h.grad.numpy(), rtol=1e-6)
    D = -np.exp(L - lse[:, None]) * coef[:, None]
    assert not np.allclose(D @ orc.bf16_to_f32(wb).astype(np.float64), h.grad.numpy(), rtol=1e-6)


# ---- the final RMSNorm before the LM head -------------------------------------------------

def test_rmsnorm_operand_closed_forms_order_and_torch(orc):
    """Qwen2RMSNorm as the LM head's bf16 operand (oracle.rmsnorm_operand):
    closed forms (constant rows, a one-hot row), the stated f32 summation order against
    a scalar loop over the same order, and the transformers formula in torch f32."""
    H = 320
    gamma = orc.bf16_to_f32(orc.bf16_from_f32(np.linspace(0.5, 1.5, H).astype(np.float32)))
    # constant 2.0 rows, eps = 0: r = 1/2 exactly, x = 1, y = gamma
    hb = orc.bf16_from_f32(np.full((2, H), 2.0, np.float32))
    y, r, x = orc.rmsnorm_operand(hb, gamma, 0.0)
    assert np.all(r == 0.5) and np.all(orc.bf16_to_f32(x) == 1.0)
    assert np.array_equal(y, np.broadcast_to(orc.bf16_from_f32(gamma), (2, H)))
    # one-hot row a = 3 at k = 7: r = sqrt(H) / 3 (eps = 0), x_k = sqrt(H)
    h = np.zeros((1, H), np.float32)
    h[0, 7] = 3.0
    y, r, x = orc.rmsnorm_operand(orc.bf16_from_f32(h), gamma, 0.0)
    assert abs(float(r[0]) - np.sqrt(H) / 3) <= 2e-7 * np.sqrt(H) / 3
    xv = orc.bf16_to_f32(x)[0]
    assert xv[7] == orc.bf16_to_f32(orc.bf16_from_f32(np.float32([np.sqrt(H)])))[0] and not np.any(np.delete(xv, 7))
    # the summation order, scalar by scalar
    rng = np.random.default_rng(5)
    hb = orc.bf16_from_f32((rng.standard_normal((3, H)) * 3).astype(np.float32))
    eps = np.float32(1e-6)
    y, r, x = orc.rmsnorm_operand(hb, gamma, eps)
    hf = orc.bf16_to_f32(hb)
    for n in range(3):
        lanes = []
        for t in range(256):
            a = np.float32(0)
            for k in range(t, H, 256):
                a = np.float32(a + np.float32(hf[n, k] * hf[n, k]))
            lanes.append(a)
        waves = []
        for w in range(4):
            v = lanes[64 * w:64 * w + 64]
            while len(v) > 1:
                v = [np.float32(v[i] + v[i + len(v) // 2]) for i in range(len(v) // 2)]
            waves.append(v[0])
        ss = np.float32(np.float32(np.float32(waves[0] + waves[1]) + waves[2]) + waves[3])
        want = np.float32(1) / np.sqrt(np.float32(ss / np.float32(H)) + eps)
        assert r[n] == want
    # transformers' Qwen2RMSNorm in torch f32 (another summation order): y equal but for
    # rare one-ulp flips at bf16 rounding boundaries
    N = 64
    hb = orc.bf16_from_f32((rng.standard_normal((N, 896)) * 2).astype(np.float32))
    g2 = orc.bf16_to_f32(orc.bf16_from_f32((1 + 0.1 * rng.standard_normal(896)).astype(np.float32)))
    y, r, x = orc.rmsnorm_operand(hb, g2, 1e-6)
    ht = torch.from_numpy(orc.bf16_to_f32(hb)).to(torch.bfloat16)
    hs = ht.float()
    var = hs.pow(2).mean(-1, keepdim=True)
    xt = (hs * torch.rsqrt(var + 1e-6)).to(torch.bfloat16)
    yt = (torch.from_numpy(g2).to(torch.bfloat16) * xt).view(torch.int16).numpy().view(np.uint16)
    d = np.abs(y.astype(np.int32) - yt.astype(np.int32))
    assert d.max() <= 1 and (d > 0).mean() < 1e-3
    r64 = 1 / np.sqrt((orc.bf16_to_f32(hb).astype(np.float64) ** 2).mean(1) + 1e-6)
    assert np.all(np.abs(r - r64) <= 1e-6 * r64)


def test_rmsnorm_vjp_matches_torch_autograd(orc):
    """dh and dgamma (oracle.rmsnorm_vjp) against torch float64 autograd of
    L = sum(dy * gamma * x) with the bf16 rounding of x passing gradients through;
    central differences; scale invariance (eps = 0: sum_k dh_k h_k = 0); and two planted
    mistakes (a flipped sign, a dropped r^3 term) fail."""
    rng = np.random.default_rng(6)
    N, H, eps = 5, 192, 1e-6
    hb = orc.bf16_from_f32((rng.standard_normal((N, H)) * 2).astype(np.float32))
    gamma = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    dy = rng.standard_normal((N, H))
    _, _, xb = orc.rmsnorm_operand(hb, gamma, eps)
    dh, dg = orc.rmsnorm_vjp(hb, gamma, eps, xb, dy)
    h = torch.tensor(orc.bf16_to_f32(hb).astype(np.float64), requires_grad=True)
    g = torch.tensor(gamma.astype(np.float64), requires_grad=True)
    x = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    xr = x + (torch.from_numpy(orc.bf16_to_f32(xb).astype(np.float64)) - x).detach()
    (torch.from_numpy(dy) * (g * xr)).sum().backward()
    np.testing.assert_allclose(dh, h.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dg, g.grad.numpy(), rtol=1e-12, atol=1e-12)

    def F(hh):
        return float((dy * gamma.astype(np.float64) * hh / np.sqrt((hh * hh).mean(1, keepdims=True) + eps)).sum())
    h0 = orc.bf16_to_f32(hb).astype(np.float64)
    for (n, k) in [(0, 0), (2, 17), (4, 191)]:
        e = np.zeros_like(h0)
        e[n, k] = 1e-6
        fd = (F(h0 + e) - F(h0 - e)) / 2e-6
        assert abs(fd - dh[n, k]) <= 1e-6 * max(1.0, abs(dh[n, k]))
    dh0, _ = orc.rmsnorm_vjp(hb, gamma, 0.0, xb, dy)
    assert np.all(np.abs((dh0 * h0).sum(1)) <= 1e-12 * (np.abs(dh0 * h0)).sum(1))
    # planted mistakes
    r = 1 / np.sqrt((h0 * h0).mean(1) + eps)
    gg = dy * gamma[None, :]
    dot = (gg * h0).sum(1)
    flipped = r[:, None] * gg + h0 * (r ** 3 * dot / H)[:, None]
    no_r3 = r[:, None] * gg - h0 * (r * dot / H)[:, None]
    for bad in (flipped, no_r3):
        assert not np.allclose(bad, h.grad.numpy(), rtol=1e-6)


# ---- the step around the loss head: Nesterov, gradient statistics, packing ----------------

def test_nesterov_mlir_reference_kat(orc):
    """The reference's known answer (src/examples/mlir_optimizer_test.zig:176-256):
    p=0.5, v=0, g=0.2, lr=0.1, mu=0.9 -> p=0.48, v=0.02 (within 1e-6)."""
    p, v = orc.nesterov([0.5], [0.0], [0.2], 0.1, 0.9, mode=1)
    assert abs(p[0] - 0.48) <= 1e-6 and abs(v[0] - 0.02) <= 1e-6
    p, v = orc.nesterov([0.5], [0.0], [0.2], 0.1, 0.9, mode=0)   # the other formulation differs
    assert abs(p[0] - 0.48) > 1e-3


def test_nesterov_matches_torch_sgd(orc):
    """nesterov.zig's update is torch.optim.SGD(momentum=mu, nesterov=True, dampening=0):
    buf = mu*buf + g; p -= lr*(g + mu*buf). torch may fuse into FMAs, so a few ulp."""
    rng = np.random.default_rng(5)
    n, lr, mu = 4099, 0.03, 0.9
    p0 = rng.standard_normal(n).astype(np.float32)
    pt = torch.tensor(p0.copy(), requires_grad=True)
    opt = torch.optim.SGD([pt], lr=lr, momentum=mu, nesterov=True, dampening=0.0)
    p, v = p0.copy(), np.zeros(n, np.float32)
    pb, vb = p0.copy(), np.zeros(n, np.float32)     # planted mistake: lookahead on the old velocity
    tol = dict(rtol=4e-7, atol=4e-7 * np.abs(p0).max())
    for step in range(5):
        g = rng.standard_normal(n).astype(np.float32)
        pt.grad = torch.from_numpy(g.copy())
        opt.step()
        p, v = orc.nesterov(p, v, g, lr, mu, mode=0)
        np.testing.assert_allclose(p, pt.detach().numpy(), **tol)
        np.testing.assert_allclose(v, opt.state[pt]["momentum_buffer"].numpy(), rtol=4e-7, atol=1e-6)
        pb = (pb - np.float32(lr) * (g + np.float32(mu) * vb)).astype(np.float32)
        vb = (np.float32(mu) * vb + g).astype(np.float32)
    assert not np.allclose(pb, pt.detach().numpy(), **tol)


def test_nesterov_closed_forms(orc):
    """Constant gradient from v0 = 0: v_k = g (1 - mu^k) / (1 - mu) and
    p_k = p0 - lr * sum_j (g + mu v_j) (float64); mu = 0 is plain SGD bit for bit."""
    g = np.array([0.25, -1.5, 3.0], np.float32)
    p0 = np.array([1.0, 2.0, -0.5], np.float32)
    lr, mu, k = 0.05, 0.8, 7
    p, v = p0.copy(), np.zeros(3, np.float32)
    for _ in range(k):
        p, v = orc.nesterov(p, v, g, lr, mu, mode=0)
    gd, vs = g.astype(np.float64), [g.astype(np.float64) * (1 - mu ** j) / (1 - mu) for j in range(1, k + 1)]
    want_p = p0 - lr * sum(gd + mu * vj for vj in vs)
    np.testing.assert_allclose(v, vs[-1], rtol=2e-6)
    np.testing.assert_allclose(p, want_p, rtol=2e-6)
    p1, v1 = orc.nesterov(p0, np.zeros(3, np.float32), g, lr, 0.0, mode=0)
    assert np.array_equal(p1, (p0 - np.float32(lr) * g).astype(np.float32)) and np.array_equal(v1, g)
    p2, _ = orc.nesterov(p0, np.ones(3, np.float32), g, 0.0, mu, mode=0)
    assert np.array_equal(p2, p0)


def test_grad_stats_against_numpy(orc):
    rng = np.random.default_rng(6)
    g = (rng.standard_normal(100003) * 3).astype(np.float32)
    g[[5, 77, 901]] = np.nan
    g[[13, 4000]] = np.inf
    g[20] = -np.inf
    s = orc.grad_stats(g)
    fin = g[np.isfinite(g)].astype(np.float64)
    assert s["nan_count"] == 3 and s["inf_count"] == 3 and s["elements"] == g.size
    assert s["max_abs"] == np.float32(np.abs(fin).max())
    assert abs(s["sumsq"] - float(np.sum(fin * fin))) <= 1e-12 * float(np.sum(fin * fin))
    assert abs(s["l2_norm"] - float(np.linalg.norm(fin))) <= 1e-12 * float(np.linalg.norm(fin))
    z = orc.grad_stats(np.zeros(0, np.float32))
    assert z["max_abs"] == 0 and z["sumsq"] == 0


def test_pack_against_numpy(orc):
    """Row k = concat(prompt_k, completion_k)[:T] with mask 1 there; missing rollouts
    give zero rows; bad offsets are reported and their rows stay zero."""
    rng = np.random.default_rng(7)
    R, n_rows, T = 5, 7, 12
    lp = rng.integers(0, 8, R)
    lc = rng.integers(0, 9, R)
    lp[2], lc[3] = 0, 0
    prompts = [rng.integers(1, 1000, n) for n in lp]
    comps = [rng.integers(1, 1000, n) for n in lc]
    po = np.concatenate([[0], np.cumsum(lp)])
    co = np.concatenate([[0], np.cumsum(lc)])
    ids, mask, ok = orc.pack(np.concatenate(prompts), po, np.concatenate(comps), co, n_rows, T)
    assert ok
    for k in range(n_rows):
        row = np.concatenate([prompts[k], comps[k]])[:T] if k < R else np.zeros(0, np.int64)
        assert np.array_equal(ids[k, :len(row)], row) and not ids[k, len(row):].any()
        assert mask[k].sum() == len(row) and np.all(mask[k, :len(row)] == 1)
    bad = po.copy()
    bad[2] = bad[3] + 1                           # decreasing pair for rollout 2
    ids2, mask2, ok2 = orc.pack(np.concatenate(prompts), bad, np.concatenate(comps), co, n_rows, T)
    assert not ok2 and not mask2[2].any()


# ---- the rollout sampler (math.zig:21-73) -------------------------------------------------

def test_sampler_reference_kat(orc):
    """math.zig:76-89: greedy [1, 5, 2] -> 1; [1, 10, 1] at T = 1 -> 1 for the draws in
    [p0, p0 + p1) = [1.2e-4, 0.99988) (p1 = 0.99975), 0 below, 2 above."""
    assert orc.sample([1.0, 5.0, 2.0], 0.0) == 1
    for u in (0.001, 0.3, 0.9998):
        assert orc.sample([1.0, 10.0, 1.0], 1.0, u) == 1
    assert orc.sample([1.0, 10.0, 1.0], 1.0, 0.0) == 0
    assert orc.sample([1.0, 10.0, 1.0], 1.0, 0.00005) == 0
    assert orc.sample([1.0, 10.0, 1.0], 1.0, 0.99999) == 2


def test_sampler_against_inverse_cdf(orc):
    """Inverse-transform sampling: index = first i with cumsum(p)_i >= u (numpy float64
    searchsorted on the exact CDF), up to the f32 sum's rounding near a boundary."""
    rng = np.random.default_rng(8)
    for T in (0.7, 1.0, 2.5):
        x = (rng.standard_normal(3000) * 2).astype(np.float32)
        p = np.exp((x.astype(np.float64) - x.max()) / T)
        c = np.cumsum(p)
        for u in rng.random(200).astype(np.float32):
            got = orc.sample(x, T, float(u))
            want = int(np.searchsorted(c, float(u) * c[-1], side="left"))
            if got != want:                              # only at a rounding boundary
                assert abs(c[min(got, want)] - float(u) * c[-1]) <= 1e-5 * c[-1]


def test_sampler_closed_forms(orc):
    V = 1000
    assert orc.sample(np.zeros(V, np.float32), 1.0, 0.25) == 249      # uniform: ceil(u V) - 1
    assert orc.sample(np.zeros(V, np.float32), 1.0, 0.0) == 0
    x = np.full(V, -30.0, np.float32)
    x[417] = 30.0
    assert orc.sample(x, 1.0, 0.5) == 417                              # one dominant logit
    ties = np.array([3.0, 7.0, 7.0, 1.0], np.float32)
    assert orc.sample(ties, 0.0) == 1                                  # first maximum
    assert orc.sample(np.array([np.nan, 2.0, np.nan, 5.0], np.float32), 0.0) == 3   # NaN never wins
    assert orc.sample(np.full(4, -np.inf, np.float32), 0.0) == 0
    assert orc.sample(np.array([1.0, np.nan, 2.0], np.float32), 1.0, 0.5) == 2       # NaN sum: n - 1


def test_sampler_is_the_sequential_f32_cumsum_rule(orc):
    """The restatement picks the first index where numpy's sequential float32 cumsum of
    the f32 terms reaches float32(u) * total (math.zig:35-53's loop)."""
    rng = np.random.default_rng(9)
    for T in (0.7, 1.3):
        for _ in range(12):
            x = (rng.standard_normal(20000) * 2.5).astype(np.float32)
            u = np.float32(rng.random())
            e32 = np.exp(((x - x.max()) / np.float32(T)).astype(np.float32))
            c32 = np.cumsum(e32, dtype=np.float32)
            want = int(np.argmax(c32 >= u * c32[-1])) if np.any(c32 >= u * c32[-1]) else x.size - 1
            assert orc.sample(x, T, float(u)) == want
