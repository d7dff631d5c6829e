"""Seeded synthetic inputs of the benchmark configurations.

The five configurations are the BASELINE workloads of the GRPO loss head:
  1 toy-qwen:   2 prompts x G=4, T=128, V=1024, f32 logits ~N(0, 2^2), ref = policy
                + N(0, 0.05^2), ids uniform, lengths U[32, 128], rewards Bernoulli(0.5)
  2 qwen2.5-0.5b-vocab: 8 x G=8, T=512, V=151936, bf16 ~N(0, 3^2), ref + N(0, 0.1^2),
                ids drawn from softmax(policy) (Gumbel-max), lengths U[64, 512], rewards {0,1}
  3 qwen3-8b-shape: 4 x G=16, T=1024, as 2, lengths U[64, 1024], rewards U[0,1) with
                all-equal groups (the std + 1e-8 path)
  4 long-rollout: 1 x G=8, T=8192, as 2, lengths lognormal(ln 1024, 1) clipped to
                [1, 8192], rewards Bernoulli(0.3)
  5 fused LM-head: N=16384 tokens, H=4096 (built separately)
Old log-probs are the policy's own log-probs + N(0, 0.01^2); clip eps 0.2, KL beta 0.04.
Rows use the aligned layout: row (s, t) scores ids[s, t]; mask[s, t] = t < length[s].

Big tensors are generated in HBM by the library's Philox kernels (pcp_synth.h);
per-sequence data and config-1 tensors come from numpy's PCG64 so they are the
same on every machine.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from ._lib import DType, check, lib


@dataclass(frozen=True)
class GrpoConfig:
    key: int
    name: str
    prompts: int
    group: int
    T: int
    V: int
    dtype: str                      # "f32" or "bf16"
    std_p: float
    std_r: float
    lengths: tuple                  # ("uniform", lo, hi) | ("lognormal", mu, sigma)
    rewards: tuple                  # ("bernoulli", p) | ("binary",) | ("uniform_degenerate", n_equal_groups)
    ids: str                        # "uniform" | "gumbel"
    old_noise: float = 0.01
    clip_eps: float = 0.2
    kl_beta: float = 0.04
    seed: int = 0
    notes: dict = field(default_factory=dict)

    @property
    def S(self) -> int:
        return self.prompts * self.group

    @property
    def N(self) -> int:
        return self.S * self.T


CONFIGS = {
    1: GrpoConfig(1, "toy-qwen", 2, 4, 128, 1024, "f32", 2.0, 0.05, ("uniform", 32, 128),
                  ("bernoulli", 0.5), "uniform"),
    2: GrpoConfig(2, "qwen2.5-0.5b-vocab", 8, 8, 512, 151936, "bf16", 3.0, 0.1, ("uniform", 64, 512),
                  ("binary",), "gumbel"),
    3: GrpoConfig(3, "qwen3-8b-shape", 4, 16, 1024, 151936, "bf16", 3.0, 0.1, ("uniform", 64, 1024),
                  ("uniform_degenerate", 2), "gumbel"),
    4: GrpoConfig(4, "long-rollout", 1, 8, 8192, 151936, "bf16", 3.0, 0.1, ("lognormal", float(np.log(1024.0)), 1.0),
                  ("bernoulli", 0.3), "gumbel", notes={"lognormal_sigma": "1.0 (builder's choice)"}),
}


@dataclass(frozen=True)
class LmheadConfig:
    """Configuration 5: fused LM-head + GRPO log-prob. hidden [N, H] ~ N(0, 1),
    W [V, H] ~ N(0, 0.02^2), W_ref = W + N(0, 0.002^2), all bf16; tokens drawn from
    softmax(hidden W^T) by Gumbel-max as in configuration 2 (the logits are formed
    once, in token chunks, for the draw only); lengths, rewards and groups as
    configuration 2 (G=8, T=512)."""
    key: int = 5
    name: str = "fused-lm-head"
    prompts: int = 4
    group: int = 8
    T: int = 512
    H: int = 4096
    V: int = 151936
    std_h: float = 1.0
    std_w: float = 0.02
    std_r: float = 0.002
    lengths: tuple = ("uniform", 64, 512)
    rewards: tuple = ("binary",)
    old_noise: float = 0.01
    clip_eps: float = 0.2
    kl_beta: float = 0.04
    seed: int = 0

    @property
    def S(self) -> int:
        return self.prompts * self.group

    @property
    def N(self) -> int:
        return self.S * self.T


LMHEAD = LmheadConfig()


def make_lmhead_inputs(cfg: LmheadConfig, device="cuda"):
    """Inputs of the fused LM-head configuration in HBM (hidden, weight, ref_weight,
    ids, mask, rewards, old_logp offsets)."""
    import torch

    lengths, rewards = per_sequence(cfg)
    S, T, H, V = cfg.S, cfg.T, cfg.H, cfg.V
    stream = torch.cuda.current_stream().cuda_stream or None
    hidden = torch.empty((S * T, H), dtype=torch.bfloat16, device=device)
    check(lib().pcp_synth_logits(hidden.data_ptr(), None, hidden.numel(), int(DType.bf16), ctypes.c_float(cfg.std_h),
                                 ctypes.c_float(0.0), cfg.seed + 10, stream))
    weight = torch.empty((V, H), dtype=torch.bfloat16, device=device)
    ref_weight = torch.empty_like(weight)
    check(lib().pcp_synth_logits(weight.data_ptr(), ref_weight.data_ptr(), weight.numel(), int(DType.bf16),
                                 ctypes.c_float(cfg.std_w), ctypes.c_float(cfg.std_r), cfg.seed + 11, stream))
    rng = np.random.default_rng(cfg.seed + 12)
    ids = sample_lmhead_ids(hidden, weight, cfg.seed + 13, chunk=1024).view(S, T)
    mask = torch.from_numpy(mask_from_lengths(lengths, T)).to(device)
    old_shift = torch.from_numpy((rng.standard_normal((S, T)) * cfg.old_noise).astype(np.float32)).to(device)
    return {"hidden": hidden, "weight": weight, "ref_weight": ref_weight, "ids": ids, "mask": mask,
            "rewards": torch.from_numpy(rewards).to(device), "old_shift": old_shift, "lengths": lengths}


def sample_lmhead_ids(hidden, weight, seed: int, chunk: int = 1024, ctx=None):
    """One token per hidden row drawn from softmax(hidden W^T) by Gumbel-max
    (pcp_synth_lmhead_tokens: f32 logits from the library's MFMA tile kernel, `chunk`
    rows at a time, chunk k drawn with seed + k, as pcp_synth_sample_tokens draws for
    the logits configurations). Returns int64 [N] on the device."""
    import torch

    from .grpo import default_context

    ctx = ctx or default_context(hidden.device.index or 0)
    N, H = hidden.shape
    V = weight.shape[0]
    ids = torch.empty(N, dtype=torch.int64, device=hidden.device)
    stream = torch.cuda.current_stream().cuda_stream or None
    check(lib().pcp_synth_lmhead_tokens(ctx.handle, hidden.data_ptr(), weight.data_ptr(), N, H, V, chunk, seed,
                                        ids.data_ptr(), stream), ctx.handle)
    return ids


def per_sequence(cfg) -> tuple[np.ndarray, np.ndarray]:
    """Response lengths (int64 [S]) and rewards (f32 [S]) from PCG64(seed)."""
    rng = np.random.default_rng(cfg.seed)
    S, T = cfg.S, cfg.T
    kind = cfg.lengths[0]
    if kind == "uniform":
        lengths = rng.integers(cfg.lengths[1], cfg.lengths[2], size=S, endpoint=True)
    elif kind == "lognormal":
        lengths = np.clip(np.round(rng.lognormal(cfg.lengths[1], cfg.lengths[2], size=S)), 1, T).astype(np.int64)
    else:
        raise ValueError(kind)
    rk = cfg.rewards[0]
    if rk == "bernoulli":
        rewards = (rng.random(S) < cfg.rewards[1]).astype(np.float32)
    elif rk == "binary":
        rewards = rng.integers(0, 2, size=S).astype(np.float32)
    elif rk == "uniform_degenerate":
        rewards = rng.random(S).astype(np.float32)
        # The first n groups get all-equal rewards (group std 0: the +1e-8 path).
        for g in range(cfg.rewards[1]):
            rewards[g * cfg.group:(g + 1) * cfg.group] = rewards[g * cfg.group]
    else:
        raise ValueError(rk)
    return lengths.astype(np.int64), rewards


def mask_from_lengths(lengths: np.ndarray, T: int) -> np.ndarray:
    return (np.arange(T)[None, :] < np.asarray(lengths)[:, None]).astype(np.float32)


def host_logits(cfg: GrpoConfig) -> tuple[np.ndarray, np.ndarray]:
    """Config-1-sized policy and ref logits on the host (f32)."""
    rng = np.random.default_rng(cfg.seed + 1)
    shape = (cfg.S, cfg.T, cfg.V)
    pol = (rng.standard_normal(shape, dtype=np.float32) * np.float32(cfg.std_p)).astype(np.float32)
    ref = (pol + rng.standard_normal(shape, dtype=np.float32) * np.float32(cfg.std_r)).astype(np.float32)
    return pol, ref


def philox(ctr, key) -> list[int]:
    c = (ctypes.c_uint32 * 4)(*ctr)
    k = (ctypes.c_uint32 * 2)(*key)
    o = (ctypes.c_uint32 * 4)()
    lib().pcp_synth_philox4x32_10(c, k, o)
    return list(o)


def make_device_inputs(cfg: GrpoConfig, device="cuda", n_seq: int | None = None):
    """All inputs of a configuration as torch tensors in HBM.

    ``n_seq`` keeps only the first n sequences (for tests); per-sequence data is
    still drawn for the full configuration so a subset is a prefix of the whole.
    Returns a dict with logits, ref_logits, ids, mask, rewards, old_logp, lengths.
    """
    import torch

    from .grpo import logprob_fwd

    lengths, rewards = per_sequence(cfg)
    S = cfg.S if n_seq is None else int(n_seq)
    lengths, rewards = lengths[:S], rewards[:S]
    T, V = cfg.T, cfg.V
    if cfg.dtype == "f32":
        pol, ref = host_logits(cfg)
        logits = torch.from_numpy(pol[:S]).to(device)
        ref_logits = torch.from_numpy(ref[:S]).to(device)
    else:
        tdt = {"bf16": torch.bfloat16, "f16": torch.float16}[cfg.dtype]
        code = {"bf16": DType.bf16, "f16": DType.f16}[cfg.dtype]
        logits = torch.empty((S, T, V), dtype=tdt, device=device)
        ref_logits = torch.empty_like(logits)
        check(lib().pcp_synth_logits(logits.data_ptr(), ref_logits.data_ptr(), logits.numel(), int(code),
                                     ctypes.c_float(cfg.std_p), ctypes.c_float(cfg.std_r), cfg.seed,
                                     torch.cuda.current_stream().cuda_stream or None))
    if cfg.ids == "uniform":
        rng = np.random.default_rng(cfg.seed + 2)
        ids = torch.from_numpy(rng.integers(0, V, size=(cfg.S, T))[:S].astype(np.int64)).to(device)
    else:
        ids = torch.empty((S, T), dtype=torch.int64, device=device)
        code = {"bf16": DType.bf16, "f16": DType.f16, "f32": DType.f32}[cfg.dtype]
        check(lib().pcp_synth_sample_tokens(logits.data_ptr(), int(code), S * T, V, cfg.seed + 3,
                                            ids.data_ptr(), torch.cuda.current_stream().cuda_stream or None))
    mask = torch.from_numpy(mask_from_lengths(lengths, T)).to(device)
    lp, _ = logprob_fwd(logits, ids)
    rng = np.random.default_rng(cfg.seed + 4)
    noise = torch.from_numpy((rng.standard_normal((cfg.S, T)).astype(np.float32) * np.float32(cfg.old_noise))[:S])
    old_logp = (lp + noise.to(device)).contiguous()
    return {
        "logits": logits, "ref_logits": ref_logits, "ids": ids, "mask": mask,
        "rewards": torch.from_numpy(rewards).to(device), "old_logp": old_logp,
        "lengths": lengths,
    }
