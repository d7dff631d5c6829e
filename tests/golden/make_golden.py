"""Generates the golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

Nothing here comes from running the reference (it cannot run here: Zig + IREE).
The fixtures are:
  reference_kats.json  known-answer tests transcribed from the reference's own test
                       file src/examples/isolated_vjp_tests.zig (inputs, expected
                       values, tolerances, line citations);
  advantages.json      reward vectors of the benchmark configurations and their
                       advantages as f32 bit patterns, from a numpy float32 scalar
                       simulation of rl_shepherd.zig:466-478 (IEEE, no FMA);
  cases.npz            small loss-head problems (edge cases: V=1, ties, +-100 logits,
                       ignore index -100, empty sequences, odd V, bf16, the shifted
                       reference layout, clipped ratios) with expected outputs from
                       torch CPU autograd in float64 of the loss expressions of
                       tools/export_qwen_forward.py:150-163 (REINFORCE) and of the
                       clipped-ratio + k3-KL loss.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from pcp_amd.synth import CONFIGS, per_sequence  # noqa: E402

REINFORCE, CLIP_KL = 0, 1


# ---------------------------------------------------------------------------
# Advantages: numpy float32 scalar simulation of rl_shepherd.zig:466-478.
# ---------------------------------------------------------------------------
def advantages_f32(r: np.ndarray, group: int, eps=np.float32(1e-8)) -> np.ndarray:
    r = np.asarray(r, dtype=np.float32)
    out = np.empty_like(r)
    n = r.size
    for i in range(0, n, group):
        grp = r[i:min(i + group, n)]
        cnt = np.float32(len(grp))
        s = np.float32(0)
        for x in grp:
            s = np.float32(s + x)
        mean = np.float32(s / cnt)
        ssd = np.float32(0)
        for x in grp:
            d = np.float32(x - mean)
            ssd = np.float32(ssd + np.float32(d * d))
        sd = np.float32(np.sqrt(np.float32(ssd / cnt)) + eps)
        for k, x in enumerate(grp):
            out[i + k] = np.float32(np.float32(x - mean) / sd)
    return out


# ---------------------------------------------------------------------------
# Loss head in torch float64 (independent of oracle/grpo_oracle.cpp).
# ---------------------------------------------------------------------------
def bf16_bits(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def widen(x: np.ndarray) -> np.ndarray:
    if x.dtype == np.uint16:
        return (x.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return x.astype(np.float64)


def torch_loss_head(c: dict) -> dict:
    x = torch.tensor(widen(c["logits"]), dtype=torch.float64, requires_grad=True)
    S, LS, V = x.shape
    rows, off = int(c["rows"]), int(c["tok_offset"])
    ids = torch.tensor(c["ids"][:, off:off + rows], dtype=torch.int64)
    m = torch.tensor(c["mask"][:, off:off + rows], dtype=torch.float64)
    live = (m != 0) & (ids != -100) & (ids >= 0) & (ids < V)
    lsm = torch.log_softmax(x[:, :rows, :], dim=-1)
    lp = torch.where(live, lsm.gather(-1, ids.clamp(0, V - 1).unsqueeze(-1)).squeeze(-1), torch.zeros(()))
    lp_leaf = lp.detach().clone().requires_grad_(True)
    G = float(c["loss_norm"]) if c["loss_norm"] > 0 else float(S)
    L = torch.clamp(torch.tensor(c["mask"][:, off:off + rows], dtype=torch.float32).sum(1), min=1.0).double()
    if "advantages" in c:
        A = torch.tensor(c["advantages"], dtype=torch.float64)
    else:
        A = torch.tensor(advantages_f32(c["rewards"], int(c["group_size"])), dtype=torch.float64)
    lr = torch.zeros_like(lp)
    if c.get("ref_logits") is not None:
        r = torch.tensor(widen(c["ref_logits"]), dtype=torch.float64)
        rl = torch.log_softmax(r[:, :rows, :], dim=-1)
        lr = torch.where(live, rl.gather(-1, ids.clamp(0, V - 1).unsqueeze(-1)).squeeze(-1), torch.zeros(()))

    def loss_of(lpv):
        if int(c["loss_mode"]) == REINFORCE:
            tok = torch.where(live, m * (-lpv), torch.zeros(()))
            seq = tok.sum(1) / L
            return (seq * A).sum() / G, tok
        old = torch.tensor(c["old_logp"][:, off:off + rows], dtype=torch.float64) if c.get("old_logp") is not None \
            else lpv.detach()
        # the C ABI carries eps and beta as f32
        eps, beta = float(np.float32(c["clip_eps"])), float(np.float32(c["kl_beta"]))
        ratio = torch.exp(lpv - old)
        Ab = A[:, None]
        surr = torch.minimum(ratio * Ab, torch.clamp(ratio, 1 - eps, 1 + eps) * Ab)
        dlr = lr - lpv
        kl = torch.exp(dlr) - dlr - 1
        tok = torch.where(live, m * (-surr + beta * kl), torch.zeros(()))
        seq = tok.sum(1) / L
        return seq.sum() / G, tok

    loss, tok = loss_of(lp)
    loss.backward()
    loss2, _ = loss_of(lp_leaf)
    loss2.backward()
    dl = x.grad.numpy().copy()

    def place(v):
        out = np.zeros(c["ids"].shape, np.float64)
        out[:, off:off + rows] = v
        return out

    return {
        "exp_loss": np.float64(loss.item()),
        "exp_lp": place(lp.detach().numpy()),
        "exp_lr": place(lr.detach().numpy()),
        "exp_token_loss": place(tok.detach().numpy()),
        "exp_coef": place(torch.where(live, lp_leaf.grad, torch.zeros(())).numpy()),
        "exp_adv": A.numpy().astype(np.float32),
        "exp_dlogits": dl,
    }


def make_cases() -> dict:
    rng = np.random.default_rng(1234)
    cases = {}

    def base(S, T, V, *, rows=None, off=0, LS=None, mode=REINFORCE, dtype="f32", scale=2.0, group=2):
        LS = LS or T
        rows = T - off if rows is None else rows
        pol = (rng.standard_normal((S, LS, V)) * scale).astype(np.float32)
        ref = (pol + rng.standard_normal((S, LS, V)) * 0.1).astype(np.float32)
        if dtype == "bf16":
            pol, ref = bf16_bits(pol), bf16_bits(ref)
        ids = rng.integers(0, V, size=(S, T)).astype(np.int64)
        lengths = rng.integers(1, T + 1, size=S)
        mask = (np.arange(T)[None] < lengths[:, None]).astype(np.float32)
        return {
            "logits": pol, "ref_logits": ref if mode == CLIP_KL else None, "ids": ids, "mask": mask,
            "rewards": rng.integers(0, 2, size=S).astype(np.float32), "old_logp": None,
            "rows": rows, "tok_offset": off, "group_size": group, "loss_norm": 0.0, "loss_mode": mode,
            "clip_eps": 0.2, "kl_beta": 0.04,
        }

    c = base(2, 3, 1, group=2)
    cases["v1"] = c
    c = base(2, 4, 2, group=2)
    c["logits"][0, 0] = [0.0, 0.0]          # tie
    c["logits"][0, 1] = [100.0, -100.0]     # the reference's CE stability input
    c["ids"][0, 1] = 0
    c["logits"][1, 2] = [-100.0, 100.0]
    c["ids"][1, 2] = 0                      # target has p ~ e^-200
    c["mask"][:] = 1
    c["advantages"] = np.array([1.0, -0.5], np.float32)
    cases["v2_ties_large"] = c
    c = base(3, 6, 7, group=3)
    c["ids"][0, 2] = -100                   # ignore index
    c["mask"][1, :] = 0                     # empty sequence
    c["mask"][2, 3] = 0                     # hole
    cases["v7_ignore_empty"] = c
    c = base(4, 8, 1024, mode=CLIP_KL, group=2)
    lp_probe = torch_loss_head({**c, "loss_mode": REINFORCE, "advantages": np.ones(4, np.float32)})["exp_lp"]
    old = lp_probe + rng.standard_normal(lp_probe.shape) * 0.3  # ratios well outside [0.8, 1.2]
    c["old_logp"] = old.astype(np.float32)
    c["rewards"] = np.array([1, 0, 0.25, 0.75], np.float32)
    cases["v1024_clip_kl"] = c
    c = base(2, 5, 130, mode=CLIP_KL, dtype="bf16", scale=3.0, group=2)
    cases["v130_bf16_clip_kl"] = c
    c = base(2, 6, 64, rows=5, off=1, group=2)   # reference shifted layout: logits[:, :-1] vs ids[:, 1:]
    c["advantages"] = np.array([0.7, -1.3], np.float32)
    c["loss_norm"] = 2.0
    cases["v64_shifted"] = c
    for k, c in cases.items():
        c.update(torch_loss_head(c))
    return cases


def main() -> None:
    kats = {
        "source": "src/examples/isolated_vjp_tests.zig",
        "cross_entropy_stability": {
            "lines": "1460-1583",
            "logits": [100.0, -100.0], "target": 0,
            "expect_loss": 0.0, "expect_grad": [0.0, 0.0], "atol": 1e-4,
            "note": "loss = -log_softmax(logits)[0]; gradient with upstream 1.0",
        },
        "reduce_max_grad": {
            "lines": "713-760",
            "x": [1.0, 5.0, 3.0], "upstream": 1.0, "expect_grad": [0.0, 1.0, 0.0], "atol": 1e-6,
        },
    }
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(kats, f, indent=1)

    adv = {"eps": 1e-8, "cases": []}
    for key, cfg in CONFIGS.items():
        _, rewards = per_sequence(cfg)
        a = advantages_f32(rewards, cfg.group)
        adv["cases"].append({"name": f"config{key}", "group": cfg.group,
                             "rewards_bits": rewards.view(np.uint32).tolist(),
                             "adv_bits": a.view(np.uint32).tolist()})
    hand = [
        ("g4_one_hot", [1, 0, 0, 0], 4),
        ("g3_partial_last", [0.5, 0.25, 1.0, 0.125, 0.75], 3),
        ("g8_all_equal_third", [1 / 3] * 8, 8),
        ("g16_all_equal_0p7", [0.7] * 16, 16),
        ("g4_binary_equal", [1, 1, 1, 1, 0, 0, 0, 0], 4),
    ]
    for name, r, g in hand:
        r = np.asarray(r, np.float32)
        a = advantages_f32(r, g)
        adv["cases"].append({"name": name, "group": g, "rewards_bits": r.view(np.uint32).tolist(),
                             "adv_bits": a.view(np.uint32).tolist()})
    with open(os.path.join(HERE, "advantages.json"), "w") as f:
        json.dump(adv, f)

    cases = make_cases()
    flat = {}
    for k, c in cases.items():
        for f, v in c.items():
            if v is None:
                continue
            flat[f"{k}/{f}"] = np.asarray(v)
    np.savez_compressed(os.path.join(HERE, "cases.npz"), **flat)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
