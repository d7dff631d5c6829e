"""GRPO logprob + loss fwd+bwd benchmark on one MI355X.

A step is one pass of the GRPO loss head over one batch held in HBM: group
advantages from rewards, per-sequence lengths, the fused per-row kernel (policy +
reference log-softmax, token gather, clipped-ratio + k3-KL loss, dlogits =
c*(onehot - softmax) written in bf16, zero rows for masked tokens) and the
deterministic loss reduction. Default workload: configuration 2 (Qwen2.5-0.5B
vocabulary, 64 sequences x 512 tokens, V=151936, bf16).

Prints one JSON line. value = valid (mask=1) tokens per second over the whole
step. roofline: algorithmic bytes of the fused row kernel per launch divided by
its mean duration, timed with HIP events recorded by the library on the launch
stream. cpu_baseline: the CPU oracle (fp32, reference op order, OpenMP) on a
bounded sample of the same rows.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s


def algorithmic_bytes(cfg, lengths, mode_clip_kl: bool, zero_fill: bool = True, s_out: int | None = None) -> dict:
    """Bytes the fused row kernel must move: per live row one read of the policy row,
    one of the reference row (clip-KL mode) and one write of dlogits (s_out bytes per
    element; by default the logits' size); per masked row the zero-fill write; per row
    28 B of token scalars (id 8, mask 4, old logp 4, logp 4, ref logp 4, token loss 4)."""
    import numpy as np

    s_in = 2 if cfg.dtype == "bf16" else 4
    s_out = s_in if s_out is None else s_out
    V = cfg.V
    live = int(np.minimum(lengths, cfg.T).sum())
    rows = cfg.S * cfg.T
    dead = rows - live
    per_live = (2 if mode_clip_kl else 1) * V * s_in + V * s_out
    per_dead = V * s_out if zero_fill else 0
    total = live * per_live + dead * per_dead + rows * 28
    return {"live_rows": live, "rows": rows, "per_live": per_live, "per_dead": per_dead, "bytes": total}


def host_cpu_info() -> dict:
    """The host the CPU baseline runs on: nproc, the CPUs this process may use, the
    OpenMP thread count it was given and the /proc/cpuinfo model name."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    omp = os.environ.get("OMP_NUM_THREADS", "")
    return {"nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "omp_num_threads": int(omp) if omp.isdigit() else None, "cpu_model": model}


def cpu_threads() -> tuple[int, str]:
    """Threads for the multi-threaded CPU baseline: every CPU this process may run on,
    capped by OMP_NUM_THREADS when the host sets it (the GPU box allots each GPU job a
    fixed share of host threads and sets OMP_NUM_THREADS to it; more would oversubscribe
    CPUs that belong to other jobs)."""
    aff = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and 0 < int(omp) < aff:
        return int(omp), f"OMP_NUM_THREADS={omp}: the host's thread allotment for this job ({aff} CPUs visible)"
    return aff, "every CPU this process may run on"


CPU_REPS = 5


def median_timing(fn, reps: int = CPU_REPS) -> tuple[float, list]:
    """One untimed warm-up call, then `reps` timed calls: (median seconds, all times)."""
    import statistics

    fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), times


def protocol_record(value, unit, threads, reason, kind, sample, value_1t=None, times=None, times_1t=None,
                    note_1t="") -> dict:
    """A cpu_baseline record: the median over CPU_REPS timed repetitions after a warm-up
    at `threads` threads, the same on one thread, and the host it ran on."""
    rec = {"value": value, "unit": unit, "cores": threads, "kind": kind, "sample": sample,
           "threads_reason": reason, "warmup": 1, "reps": CPU_REPS, "statistic": "median"}
    if value_1t is not None:
        rec["value_1thread"] = value_1t
    if times is not None:
        rec["rep_seconds"] = [round(t, 6) for t in times]
    if times_1t is not None:
        rec["rep_seconds_1thread"] = [round(t, 6) for t in times_1t]
    if note_1t:
        rec["note_1thread"] = note_1t
    rec.update(host_cpu_info())
    return rec


def cpu_baseline(inp, cfg, mode_clip_kl: bool, rows_mt: int = 2048, rows_1t: int = 256) -> dict:
    """The CPU oracle (fp32 reference op order, OpenMP) on a fixed sample of the same
    rows: rows_mt rows at the job's thread count and the first rows_1t of them on one
    thread, each as a warm-up plus the median of CPU_REPS timed repetitions."""
    import numpy as np
    import torch

    from oracle import oracle as orc

    threads, reason = cpu_threads()
    V, T = cfg.V, cfg.T
    flat = inp["logits"].view(-1, V)
    rflat = inp["ref_logits"].view(-1, V)
    ids = inp["ids"].view(-1).cpu().numpy()
    mask = inp["mask"].cpu().numpy()
    w = mask.reshape(-1)
    adv = orc.advantages(inp["rewards"].cpu().numpy(), cfg.group)
    Ls = orc.seq_lengths(mask, T, 0)
    old = inp["old_logp"].view(-1).cpu().numpy()
    nrows = flat.shape[0]
    # A fixed pseudo-random sample of rows, so it has the workload's live fraction.
    idx = np.sort(np.random.default_rng(0).permutation(nrows)[:min(rows_mt, nrows)])
    ti = torch.as_tensor(idx, device=flat.device)
    L, R = flat.index_select(0, ti), rflat.index_select(0, ti)
    if L.dtype == torch.bfloat16:
        L = L.view(torch.int16).cpu().numpy().view(np.uint16)
        R = R.view(torch.int16).cpu().numpy().view(np.uint16)
        dt = orc.BF16
    else:
        L, R, dt = L.cpu().numpy(), R.cpu().numpy(), orc.F32
    seq = idx // T

    def run(n, nthreads):
        orc.grpo_rows(L[:n], ids[idx[:n]], w[idx[:n]], adv[seq[:n]], Ls[seq[:n]], float(cfg.S),
                      ref_logits=R[:n] if mode_clip_kl else None, old_logp=old[idx[:n]],
                      loss_mode=orc.CLIP_KL if mode_clip_kl else orc.REINFORCE, clip_eps=cfg.clip_eps,
                      kl_beta=cfg.kl_beta, precision=orc.REF_F32, dtype=dt, nthreads=nthreads)

    n_mt, n_1t = len(idx), min(rows_1t, len(idx))
    live_mt, live_1t = int((w[idx] != 0).sum()), int((w[idx[:n_1t]] != 0).sum())
    med, times = median_timing(lambda: run(n_mt, threads))
    med1, times1 = median_timing(lambda: run(n_1t, 1))
    return protocol_record(
        live_mt / med, "valid tokens/s", threads, reason, "port",
        f"{n_mt} of {nrows} rows ({live_mt} valid), a fixed seeded sample; one thread: the first {n_1t} of them "
        f"({live_1t} valid). Oracle fp32 reference-op-order fwd+bwd (grpo_oracle.cpp, OpenMP)",
        value_1t=live_1t / med1, times=times, times_1t=times1)


MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, 2.5 PFLOP/s


def cpu_baseline_lmhead(inp, cfg, mode_clip_kl: bool, tokens_mt: int = 64, tokens_1t: int = 8) -> dict:
    """A CPU port of the fused LM-head step on a fixed token sample of the same inputs:
    fp32 logits hidden.W^T (and W_ref) on BLAS, the oracle's loss rows with dlogits
    (fp32, reference op order), then dhidden = D.W and dW += D^T.hidden on BLAS. As
    cpu_baseline: tokens_mt tokens at the job's thread count, tokens_1t on one thread,
    each a warm-up plus the median of CPU_REPS repetitions."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_limits

    from oracle import oracle as orc

    threads, reason = cpu_threads()
    T = cfg.T
    W = inp["weight"].float().cpu().numpy()
    Wr = inp["ref_weight"].float().cpu().numpy() if mode_clip_kl else None
    h_all = inp["hidden"]
    ids = inp["ids"].view(-1).cpu().numpy()
    mask = inp["mask"].cpu().numpy()
    w = mask.reshape(-1)
    adv = orc.advantages(inp["rewards"].cpu().numpy(), cfg.group)
    Ls = orc.seq_lengths(mask, T, 0)
    old = inp["old_logp"].view(-1).cpu().numpy()
    dW = np.zeros_like(W)
    idx = np.sort(np.random.default_rng(0).permutation(len(ids))[:tokens_mt])
    hc_all = h_all.index_select(0, torch.as_tensor(idx, device=h_all.device)).float().cpu().numpy()
    seq = idx // T

    def run(n, nthreads):
        with threadpool_limits(nthreads):
            hc = hc_all[:n]
            Lc = hc @ W.T
            Rc = hc @ Wr.T if mode_clip_kl else None
            r = orc.grpo_rows(Lc, ids[idx[:n]], w[idx[:n]], adv[seq[:n]], Ls[seq[:n]], float(cfg.S), ref_logits=Rc,
                              old_logp=old[idx[:n]], loss_mode=orc.CLIP_KL if mode_clip_kl else orc.REINFORCE,
                              clip_eps=cfg.clip_eps, kl_beta=cfg.kl_beta, precision=orc.REF_F32, dtype=orc.F32,
                              nthreads=nthreads)
            _dh = r.dlogits @ W
            dW[...] += r.dlogits.T @ hc

    n1 = min(tokens_1t, len(idx))
    live_mt, live_1t = int((w[idx] != 0).sum()), int((w[idx[:n1]] != 0).sum())
    med, times = median_timing(lambda: run(len(idx), threads))
    med1, times1 = median_timing(lambda: run(n1, 1))
    return protocol_record(
        live_mt / med, "valid tokens/s", threads, reason, "port",
        f"{len(idx)} of {len(ids)} tokens ({live_mt} valid), a fixed seeded sample; one thread: the first {n1} "
        f"({live_1t} valid). fp32 BLAS logits + oracle loss rows (reference op order) + fp32 BLAS dhidden/dW",
        value_1t=live_1t / med1, times=times, times_1t=times1)


def bench_lmhead(args) -> None:
    """Configuration 5: the fused LM-head + GRPO loss step (logits never stored)."""
    import ctypes

    import torch

    from pcp_amd import grpo, synth
    from pcp_amd._lib import LossMode, check, lib

    cfg = synth.LMHEAD
    dev = torch.device("cuda:0")
    clip = args.mode == "clip_kl"
    mode = LossMode.GRPO_CLIP_KL if clip else LossMode.REINFORCE
    t_setup = time.perf_counter()
    inp = synth.make_lmhead_inputs(cfg, dev)
    ctx = grpo.default_context(0)
    fwd = grpo.lmhead_fwd_bwd(inp["hidden"], inp["weight"], inp["ids"], inp["mask"], rewards=inp["rewards"],
                              group_size=cfg.group, want_grads=False, ctx=ctx)
    inp["old_logp"] = (fwd.logp + inp["old_shift"]).contiguous()
    torch.cuda.synchronize()
    t_setup = time.perf_counter() - t_setup
    kw = dict(ref_weight=inp["ref_weight"] if clip else None, rewards=inp["rewards"], group_size=cfg.group,
              old_logp=inp["old_logp"], loss_mode=mode, clip_eps=cfg.clip_eps, kl_beta=cfg.kl_beta,
              exact_bf16=args.exact_bf16, vocab_chunk=args.vocab_chunk, ctx=ctx)
    if args.final_norm:
        # The decoder's final RMSNorm fused in: hidden is the last layer's output before it.
        g = torch.Generator(device=dev).manual_seed(5)
        kw["norm_weight"] = (1 + 0.1 * torch.randn(cfg.H, device=dev, generator=g)).bfloat16().float()
        kw["norm_eps"] = 1e-6
    out = grpo.lmhead_fwd_bwd(inp["hidden"], inp["weight"], inp["ids"], inp["mask"], **kw)
    for _ in range(args.warmup):
        grpo.lmhead_fwd_bwd(inp["hidden"], inp["weight"], inp["ids"], inp["mask"], outputs=out, sync=False, **kw)
    ctx.sync()
    torch.cuda.synchronize()
    check(lib().pcp_profile_start(ctx.handle, args.steps), ctx.handle)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        grpo.lmhead_fwd_bwd(inp["hidden"], inp["weight"], inp["ids"], inp["mask"], outputs=out, sync=False, **kw)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ctx.sync()
    n_l = ctypes.c_int(0)
    tot = ctypes.c_double(0)
    check(lib().pcp_profile_stop(ctx.handle, ctypes.byref(n_l), ctypes.byref(tot)), ctx.handle)
    kernel_ms = tot.value / max(n_l.value, 1)

    N, H, V = cfg.N, cfg.H, cfg.V
    live = int(inp["mask"].sum().item())
    ms_step = elapsed * 1e3 / args.steps
    # Dense products per step over the live (compacted) tokens: forward logits per
    # model, dhidden, dW (the backward reads the forward's softmax cache, so no logits
    # are recomputed). Masked tokens carry no loss weight and no gradient, so the
    # algorithm needs 2*H*V flops per live token per product. The timed launch is the
    # dominant kernel: dhidden and dW in one launch of the MFMA tile kernel.
    products = (2 if clip else 1) + 2
    step_flops = products * 2.0 * live * H * V
    # With the chunked backward (--vocab-chunk) the library times the forward launch
    # instead: one product per model.
    chunked = args.vocab_chunk > 0
    tile_flops = (products - 2 if chunked else 2) * 2.0 * live * H * V
    achieved = tile_flops / (kernel_ms / 1e3) / 1e12
    tile_kernel = ("lm_tile_kernel<kLmFwd> (policy and reference logits, one launch)" if chunked
                   else "lm_tile_kernel<kLmGemm> (dhidden + dW products, one launch)")
    line = {
        "metric": "GRPO fused LM-head + loss fwd+bwd tokens/s, H=4096, V=151936 bf16",
        "value": live / (ms_step / 1e3),
        "unit": "valid tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded Philox/PCG64 inputs of the configuration)",
        "config": {"workload": f"config5 {cfg.name}: {cfg.prompts} prompts x G={cfg.group}, T={cfg.T}, "
                               f"hidden {H}, V={V}, bf16 hidden/weights, loss={args.mode}"
                               + (", final RMSNorm fused" if args.final_norm else "")
                               + (", exact bf16 dlogits (f32 softmax terms)" if args.exact_bf16 else "")
                               + (f", recomputing backward in {args.vocab_chunk}-wide vocab chunks"
                                  if args.vocab_chunk else ""),
                   "tokens": N, "valid_tokens": live, "global_batch": cfg.S, "seq_len": cfg.T},
        "step_tflops": step_flops / (ms_step / 1e3) / 1e12,
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / MFMA_BF16_PEAK_TFLOPS, "traffic": None,
                     "kernel": tile_kernel, "kernel_ms": kernel_ms,
                     "algorithmic_flops": tile_flops},
        "setup_s": t_setup,
    }
    tfile = os.path.join(ROOT, "profiles", f"traffic_config5_{args.mode}.json")
    if os.path.exists(tfile) and not args.exact_bf16 and not chunked:   # measured on the default path
        with open(tfile) as f:
            line["roofline"]["traffic"] = json.load(f).get("hbm_bytes_per_launch")
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_lmhead(inp, cfg, clip)
    print(json.dumps(line), flush=True)


def _timed_calls(ctx, steps: int, call):
    """Run call() steps times between pcp_profile_start/stop: returns (mean kernel ms
    from the library's HIP events on the launch stream, wall seconds)."""
    import ctypes

    import torch

    from pcp_amd._lib import check, lib

    check(lib().pcp_profile_start(ctx.handle, steps), ctx.handle)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        call()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    n_l, tot = ctypes.c_int(0), ctypes.c_double(0)
    check(lib().pcp_profile_stop(ctx.handle, ctypes.byref(n_l), ctypes.byref(tot)), ctx.handle)
    return tot.value / max(n_l.value, 1), elapsed


QWEN05_PARAMS = 494_032_768   # Qwen2.5-0.5B, the RL model of the reference's runs (~494M f32 params)


def bench_nesterov(args) -> None:
    """The Nesterov update of RLShepherd's master weights (nesterov.zig:70-98) as one HBM
    pass over a flat f32 parameter buffer, with the bf16 shadow copy for the next bf16
    forward: reads p, v, g (12 B) and writes p, v, bf16 p (10 B) per parameter."""
    import numpy as np
    import torch

    from pcp_amd import step

    dev = torch.device("cuda:0")
    P = QWEN05_PARAMS
    gen = torch.Generator(device=dev).manual_seed(0)
    p = torch.randn(P, device=dev, generator=gen)
    g = torch.randn(P, device=dev, generator=gen) * 1e-3
    shadow = torch.empty(P, dtype=torch.bfloat16, device=dev)
    opt = step.Nesterov([P], 1e-5, 0.9)
    for _ in range(args.warmup):
        opt.update_flat(p, g, shadow)
    torch.cuda.synchronize()
    kernel_ms, elapsed = _timed_calls(opt.ctx, args.steps, lambda: opt.update_flat(p, g, shadow))
    ms_step = elapsed * 1e3 / args.steps
    alg = 22 * P
    line = {
        "metric": "Nesterov update params/s and achieved HBM GB/s, 494M f32 params + bf16 shadow",
        "value": P / (ms_step / 1e3), "unit": "params/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (torch normal init)",
        "config": {"workload": f"Nesterov (Sutskever, nesterov.zig:86-97) over {P} f32 parameters, "
                               "flat buffer, bf16 shadow", "params": P},
        "roofline": {"bound": "hbm", "achieved": alg / (kernel_ms / 1e3) / 1e9, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": alg / (kernel_ms / 1e3) / 1e9 / HBM_PEAK_GBS, "traffic": None,
                     "kernel": "nesterov_kernel<0, true>", "kernel_ms": kernel_ms, "algorithmic_bytes": alg},
    }
    tfile = os.path.join(ROOT, "profiles", "traffic_nesterov.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            line["roofline"]["traffic"] = json.load(f).get("hbm_bytes_per_launch")
    if not args.no_cpu_baseline:
        from oracle import oracle as orc
        n = P
        ps, vs, gs = (np.random.default_rng(0).standard_normal(n).astype(np.float32) for _ in range(3))
        med, times = median_timing(lambda: orc.nesterov(ps, vs, gs, 1e-5, 0.9))
        line["cpu_baseline"] = protocol_record(
            n / med, "params/s", 1, "the reference's host loop (nesterov.zig:86-97) is single-threaded", "port",
            f"{n} params: oracle f32 loop of nesterov.zig:86-97 (step_oracle.cpp), one thread",
            value_1t=n / med, times=times)
    print(json.dumps(line), flush=True)
    opt.close()


def bench_sample(args) -> None:
    """The rollout sampler over f32 logits [R, 151936] in HBM (Sampler.sample,
    math.zig:21-58, at temperature 0.7, the reference's default, generation_engine.zig:163).
    R = 64 (--rows, default) is one decoding step of configuration 2's 64 rollouts; R = 1
    is the reference's own call pattern, one row per generated token. By default every
    call returns with the tokens on the device (the library synchronises), so
    ms_per_step is the latency of one call; with --async-sample calls are only enqueued
    (as a decode loop issues them behind its forward), so ms_per_step is the time per
    call of a stream of them. The CPU baseline is the reference's path for the same rows: copy
    the logits to host memory (600 KB per row, generation_engine.zig:255-268), then the
    sequential sampler loop."""
    import numpy as np
    import torch

    from pcp_amd import step

    dev = torch.device("cuda:0")
    R, V, T = args.rows, 151936, 0.7
    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((R, V), device=dev, generator=gen) * 3
    u = torch.rand(R, device=dev, generator=gen)
    ids = torch.empty(R, dtype=torch.int64, device=dev)
    from pcp_amd.grpo import default_context
    ctx = default_context(0)
    stream = torch.cuda.current_stream().cuda_stream or None
    if args.async_sample:
        # The enqueue-only entry point called through the C ABI with its arguments marshalled
        # once, as a compiled decode loop calls it (the Python wrapper's per-call checks
        # cost more than the kernel at one row).
        import ctypes

        from pcp_amd._lib import DType, PcpError, lib
        fn = lib().pcp_sample_tokens_async
        cargs = (ctx.handle, x.data_ptr(), int(DType.f32), R, V, x.stride(0), ctypes.c_float(T), u.data_ptr(),
                 ids.data_ptr(), stream)

        def call():
            rc = fn(*cargs)
            if rc != 0:
                raise PcpError(rc, lib().pcp_last_error(ctx.handle).decode())
    else:
        call = lambda: step.sample_tokens(x, T, u, ids=ids, stream=stream, ctx=ctx)
    for _ in range(args.warmup):
        call()
    ctx.sync()
    torch.cuda.synchronize()
    # The calls per second from a loop without kernel timing (its two HIP events per call
    # cost host time comparable to a one-row call), then the kernel time from a timed loop.
    t0 = time.perf_counter()
    for _ in range(args.steps):
        call()
    ctx.sync()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kernel_ms, _ = _timed_calls(ctx, args.steps, call)
    ctx.sync()
    ms_step = elapsed * 1e3 / args.steps
    alg = R * V * 4 + R * 4 + R * 8
    line = {
        "metric": f"rollout sampler tokens/s and achieved HBM GB/s, {R} row{'s' if R > 1 else ''} x V=151936 f32",
        "value": R / (ms_step / 1e3), "unit": "sampled tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (torch normal logits, uniform draws)",
        "config": {"workload": f"Sampler.sample at T={T} over {R} rows of {V} f32 logits"
                               + (", enqueued only (pcp_sample_tokens_async through the C ABI; back-to-back "
                                  "calls on one stream, the host waits once at the end)" if args.async_sample else
                                  ", each call synchronous"), "rows": R, "vocab": V,
                   ("us_per_call_enqueued" if args.async_sample else "latency_us_per_call"): ms_step * 1e3},
        "roofline": {"bound": "hbm", "achieved": alg / (kernel_ms / 1e3) / 1e9, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": alg / (kernel_ms / 1e3) / 1e9 / HBM_PEAK_GBS, "traffic": None,
                     "kernel": "sampler kernels (one call)", "kernel_ms": kernel_ms, "algorithmic_bytes": alg},
    }
    tfile = os.path.join(ROOT, "profiles", "traffic_sample.json" if R == 64 else f"traffic_sample_rows{R}.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            line["roofline"]["traffic"] = json.load(f).get("hbm_bytes_per_launch")
    if not args.no_cpu_baseline:
        from oracle import oracle as orc
        uh = u.cpu().numpy()

        def run():
            xh = x.cpu().numpy()                       # the per-step device-to-host copy of the logits
            for r in range(R):
                orc.sample(xh[r], T, float(uh[r]))

        med, times = median_timing(run)
        line["cpu_baseline"] = protocol_record(
            R / med, "sampled tokens/s", 1, "the reference's sampler loop (math.zig:21-58) is single-threaded",
            "port", f"{R} row{'s' if R > 1 else ''}: device-to-host copy of the f32 logits ({R * V * 4} bytes, "
                    "generation_engine.zig:255-268) + oracle f32 loop of math.zig:21-58 (step_oracle.cpp), one "
                    "thread", value_1t=R / med, times=times)
        line["cpu_baseline"]["latency_us_per_call"] = med * 1e6
    print(json.dumps(line), flush=True)


def bench_b64(args) -> None:
    """The UPDATE_WEIGHTS payload (rl_shepherd.zig:691-711 encodes, worker.zig:2631-2667
    decodes): base64 of Qwen2.5-0.5B's flat f32 weights (1.98 GB) on the device. A step
    is one encode and one decode; the roofline entry is the encode kernel (reads the
    weight bytes, writes 4/3 as many characters)."""
    import base64

    import torch

    from pcp_amd import formats
    from pcp_amd.grpo import default_context

    dev = torch.device("cuda:0")
    P = QWEN05_PARAMS
    w = torch.randn(P, device=dev, generator=torch.Generator(device=dev).manual_seed(0))
    raw = w.view(torch.uint8)
    nb = raw.numel()
    enc = torch.empty(nb // 3 * 4 + 4, dtype=torch.uint8, device=dev)
    dec = torch.empty(nb + 3, dtype=torch.uint8, device=dev)   # len / 4 * 3 >= nb: room for the padded quad
    text = formats.b64encode(raw, out=enc)
    nc = text.numel()
    for _ in range(args.warmup):
        formats.b64encode(raw, out=enc)
        formats.b64decode(text, out=dec)
    torch.cuda.synchronize()
    ctx = default_context(0)
    enc_ms, t_enc = _timed_calls(ctx, args.steps, lambda: formats.b64encode(raw, out=enc))
    dec_ms, t_dec = _timed_calls(ctx, args.steps, lambda: formats.b64decode(text, out=dec))
    if not torch.equal(dec[:nb], raw):
        raise SystemExit("base64 round trip differs")
    ms_step = (t_enc + t_dec) * 1e3 / args.steps
    alg = nb + nc   # encode: read the weight bytes, write the characters (decode: the reverse)
    line = {
        "metric": "UPDATE_WEIGHTS payload base64 encode + decode, bytes of weights/s, 494M f32 weights",
        "value": 2 * nb / (ms_step / 1e3), "unit": "bytes/s (weights, encode + decode)", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
        "data": "synthetic (torch normal weights)",
        "config": {"workload": f"base64 of {nb} weight bytes ({P} f32) -> {nc} characters, then back", "bytes": nb},
        "roofline": {"bound": "hbm", "achieved": alg / (enc_ms / 1e3) / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": alg / (enc_ms / 1e3) / 1e9 / HBM_PEAK_GBS, "traffic": None,
                     "kernel": "b64_encode_kernel", "kernel_ms": enc_ms, "algorithmic_bytes": alg,
                     "decode_kernel_ms": dec_ms, "decode_gbs": alg / (dec_ms / 1e3) / 1e9},
    }
    tfile = os.path.join(ROOT, "profiles", "traffic_b64.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            line["roofline"]["traffic"] = json.load(f).get("hbm_bytes_per_launch")
    if not args.no_cpu_baseline:
        host = raw[:3 << 26].cpu().numpy().tobytes()
        med, times = median_timing(lambda: base64.b64encode(host))
        line["cpu_baseline"] = protocol_record(
            len(host) / med, "bytes/s (weights, encode)", 1, "the reference's std.base64 encoder runs on one thread",
            "port", f"{len(host)} weight bytes encoded by Python's base64 (C, one thread), standing for the "
                    "reference's host std.base64 encoder", value_1t=len(host) / med, times=times)
    print(json.dumps(line), flush=True)


def bench_hbm_roof(args) -> None:
    """The practical HBM roof (pcp_hbm_stream): read-only, write-only, copy and the
    row kernel's 2-read : 1-write mix over --roof-gib GiB buffers, plain and with
    nontemporal loads and stores, at 1 and 4 vectors per lane; each kind's best shape is
    its roof. `value` is the mix (the headline kernel's access pattern) in GB/s of bytes
    moved."""
    import torch

    from pcp_amd._lib import check, lib
    from pcp_amd.grpo import default_context

    dev = torch.device("cuda:0")
    nbytes = int(args.roof_gib * (1 << 30)) // 16 * 16
    a = torch.full((nbytes // 4,), 7, dtype=torch.int32, device=dev)
    b = torch.full_like(a, 3)
    c = torch.empty_like(a)
    ctx = default_context(0)
    stream = torch.cuda.current_stream().cuda_stream or None
    moved = {0: 1, 1: 1, 2: 2, 3: 3}
    names = {0: "read", 1: "write", 2: "copy", 3: "mix2r1w"}
    res = {}
    for vpt in (1, 4):
        for nt in (0, 1):
            for kind in range(4):
                call = lambda: check(lib().pcp_hbm_stream(ctx.handle, kind, nt, vpt, a.data_ptr(), b.data_ptr(),
                                                          c.data_ptr(), nbytes, stream), ctx.handle)
                for _ in range(args.warmup):
                    call()
                torch.cuda.synchronize()
                ms, _ = _timed_calls(ctx, args.steps, call)
                res[f"{names[kind]}{'_nt' if nt else ''}_v{vpt}"] = {"kernel_ms": ms,
                                                                    "gbs": moved[kind] * nbytes / (ms / 1e3) / 1e9}
    if not torch.equal(c, a ^ b):
        raise SystemExit("mix stream result differs")
    roof = {n: max((v for k, v in res.items() if k.split("_")[0] == n), key=lambda v: v["gbs"])["gbs"]
            for n in names.values()}
    best = max((k for k in res if k.startswith("mix2r1w")), key=lambda k: res[k]["gbs"])
    mix = res[best]["gbs"]
    line = {
        "metric": "HBM stream bandwidth, 2 reads : 1 write (the row kernel's mix)", "value": mix * 1e9,
        "unit": "bytes/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": sum(r["kernel_ms"] for r in res.values()), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u32", "data": "constant device buffers",
        "config": {"workload": f"pcp_hbm_stream over {nbytes} bytes per buffer", "bytes": nbytes},
        "roofline": {"bound": "hbm", "achieved": mix, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": mix / HBM_PEAK_GBS,
                     "traffic": None, "kernel": f"hbm_stream_kernel ({best})", "kernel_ms": res[best]["kernel_ms"],
                     "algorithmic_bytes": 3 * nbytes},
        "streams": res,
        "roof_gbs": roof,
    }
    print(json.dumps(line), flush=True)


MFMA_FLOPS_PER_CLK_SIMD = 1024   # bf16 dense: 2.5 PFLOP/s = 256 CUs x 4 SIMDs x 2.4 GHz x 1024 (v_mfma_f32_32x32x16_bf16:
                                 # 32768 flops in 32 cycles)


def bench_mfma_roof(args) -> None:
    """The practical MFMA roof (pcp_mfma_peak): register-resident bf16 MFMAs, both shapes
    (v_mfma_f32_32x32x16_bf16 and v_mfma_f32_16x16x32_bf16), on one workgroup of eight
    waves per CU (the LM-head tile kernel's occupancy), no memory traffic. Short and long
    launches per shape (--mfma-iters rounds of 32x32x16 work per wave, and a tenth of
    that), since the clock under sustained MFMA load settles lower. The implied clock is
    the rate over the CUs' 4 SIMDs x 1024 flops per cycle: the shader clock if the MFMA
    pipes never idle, a lower bound on it otherwise. `value` is the best long-launch rate."""
    import torch

    from pcp_amd._lib import check, lib
    from pcp_amd.grpo import default_context

    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    ctx = default_context(0)
    stream = torch.cuda.current_stream().cuda_stream or None
    out = torch.empty(8192, dtype=torch.float32, device=dev)
    res = {}
    # Flops per round and wave: 8 x 32768 (32x32x16) or 32 x 16384 (16x16x32); the
    # 16x16x32 launches run half the rounds, so both shapes do the same work.
    for shape, name, per_round in ((0, "32x32x16", 8 * 32768), (1, "16x16x32", 32 * 16384)):
        long_iters = max(2, args.mfma_iters * 8 * 32768 // per_round // 2 * 2)
        for iters in (max(2, long_iters // 10 // 2 * 2), long_iters):
            call = lambda: check(lib().pcp_mfma_peak(ctx.handle, shape, cus, iters, 1, out.data_ptr(), None, stream),
                                 ctx.handle)
            for _ in range(args.warmup):
                call()
            torch.cuda.synchronize()
            ms, _ = _timed_calls(ctx, args.steps, call)
            tf = cus * 8 * iters * per_round / (ms / 1e3) / 1e12
            res[f"{name}_iters{iters}"] = {"shape": name, "rounds": iters, "kernel_ms": ms, "tflops": tf,
                                           "implied_clock_ghz": tf * 1e12 / (cus * 4 * MFMA_FLOPS_PER_CLK_SIMD) / 1e9,
                                           "long": iters == long_iters}
    best = max((v for v in res.values() if v["long"]), key=lambda v: v["tflops"])
    line = {
        "metric": "bf16 MFMA rate, register-resident, 8 waves per CU (best of v_mfma_f32_32x32x16_bf16 and "
                  "v_mfma_f32_16x16x32_bf16)",
        "value": best["tflops"], "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": best["kernel_ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "pseudo-random bf16 operands in [-1, 1), register-resident",
        "config": {"workload": f"pcp_mfma_peak: {cus} workgroups x 8 waves, {args.mfma_iters} rounds of "
                               f"32x32x16 work per wave (long launches)", "cus": cus},
        "roofline": {"bound": "mfma", "achieved": best["tflops"], "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": best["tflops"] / MFMA_BF16_PEAK_TFLOPS, "traffic": None,
                     "kernel": f"mfma_peak_kernel ({best['shape']})", "kernel_ms": best["kernel_ms"]},
        "launches": res,
    }
    print(json.dumps(line), flush=True)


def bench_logprob(args) -> None:
    """Forward-only log-probs (pcp_grpo_logprob_fwd: log-softmax + sampled-token gather
    of the policy rows, and of the reference rows unless --policy-only) over the
    configuration's rows; masked tokens give 0 without reading their rows. The roofline
    entry is grpo_fwd_kernel: its algorithmic bytes are one read of each live row and
    the token scalars (id 8, mask 4, one 4-byte log-prob per model) of every row."""
    import numpy as np
    import torch

    from pcp_amd import grpo, synth

    dev = torch.device("cuda:0")
    cfg = synth.CONFIGS[args.config]
    inp = synth.make_device_inputs(cfg, dev)
    ref = None if args.policy_only else inp["ref_logits"]
    ctx = grpo.default_context(0)

    def call():
        return grpo.logprob_fwd(inp["logits"], inp["ids"], ref, mask=inp["mask"], sync=False, ctx=ctx)

    for _ in range(args.warmup):
        call()
    ctx.sync()
    torch.cuda.synchronize()
    kernel_ms, elapsed = _timed_calls(ctx, args.steps, call)
    ctx.sync()
    nmod = 1 if args.policy_only else 2
    s_in = 2 if cfg.dtype == "bf16" else 4
    live = int((inp["mask"] != 0).sum())
    rows = cfg.S * cfg.T
    alg = live * nmod * cfg.V * s_in + rows * (12 + 4 * nmod)
    ms_step = elapsed * 1e3 / args.steps
    achieved = alg / (kernel_ms / 1e3) / 1e9
    what = "policy" if args.policy_only else "policy + reference"
    line = {
        "metric": f"GRPO forward-only log-probs ({what}), valid tokens/s, V={cfg.V} {cfg.dtype}",
        "value": live / (ms_step / 1e3), "unit": "valid tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": cfg.dtype, "data": "synthetic (seeded Philox/PCG64 inputs of the configuration)",
        "config": {"workload": f"config{cfg.key} {cfg.name}: log-probs of {what} rows, {cfg.prompts} prompts x "
                               f"G={cfg.group}, T={cfg.T}, V={cfg.V}, {cfg.dtype} logits",
                   "rows": rows, "valid_rows": live},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel": "grpo_fwd_kernel",
                     "kernel_ms": kernel_ms, "algorithmic_bytes": alg},
    }
    tfile = os.path.join(ROOT, "profiles", f"traffic_logprob_config{cfg.key}_{'policy' if args.policy_only else 'ref'}.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            line["roofline"]["traffic"] = json.load(f).get("hbm_bytes_per_launch")
    if not args.no_cpu_baseline:
        from oracle import oracle as orc

        threads, reason = cpu_threads()
        flat = inp["logits"].view(-1, cfg.V)
        ids = inp["ids"].view(-1).cpu().numpy()
        livei = np.nonzero(inp["mask"].view(-1).cpu().numpy() != 0)[0]
        idx = np.sort(np.random.default_rng(0).permutation(livei)[:2048])
        ti = torch.as_tensor(idx, device=dev)
        blocks = []
        for src in ([flat] if args.policy_only else [flat, inp["ref_logits"].view(-1, cfg.V)]):
            blk = src.index_select(0, ti)
            if blk.dtype == torch.bfloat16:
                blocks.append((blk.view(torch.int16).cpu().numpy().view(np.uint16), orc.BF16))
            else:
                blocks.append((blk.cpu().numpy(), orc.F32))

        def run(n, nthreads):
            for host, dt in blocks:
                orc.logprob(host[:n], ids[idx[:n]], dtype=dt, precision=orc.REF_F32, nthreads=nthreads)

        n1 = min(256, len(idx))
        med, times = median_timing(lambda: run(len(idx), threads))
        med1, times1 = median_timing(lambda: run(n1, 1))
        line["cpu_baseline"] = protocol_record(
            len(idx) / med, "valid tokens/s", threads, reason, "port",
            f"{len(idx)} of {live} valid rows, a fixed seeded sample (one thread: the first {n1}): oracle fp32 "
            f"reference-op-order log-softmax + gather of the {what} rows (grpo_oracle.cpp, OpenMP)",
            value_1t=n1 / med1, times=times, times_1t=times1)
    print(json.dumps(line), flush=True)


def bench_execute(args) -> None:
    """The host-bytes boundary: pcp_execute("grpo_clip_kl_fwd_bwd") (the mirror of
    IreeBackend.execute, iree.zig:336-442) on the configuration's inputs held in
    ordinary (pageable) host memory, as the reference's caller passes them. A step is
    one call: upload, the loss head on the device, download of every output. Reported
    for the record of the PCIe-inclusive rate; the device-resident path is the
    headline."""
    import ctypes

    import numpy as np
    import torch

    from pcp_amd import synth
    from pcp_amd._lib import DType, check, lib
    from pcp_amd.backend import HipGrpoBackend, marshal_inputs

    dev = torch.device("cuda:0")
    cfg = synth.CONFIGS[args.config]
    inp = synth.make_device_inputs(cfg, dev)

    def host(t):
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).cpu().numpy().view(np.uint16)
        return t.cpu().numpy()

    ins = [host(inp["logits"]), host(inp["ref_logits"]), inp["ids"].to(torch.int64).cpu().numpy(),
           inp["mask"].float().cpu().numpy(), inp["old_logp"].cpu().numpy(), inp["rewards"].cpu().numpy(),
           np.array([cfg.group, cfg.clip_eps, cfg.kl_beta, 0.0], np.float32)]
    del inp
    torch.cuda.empty_cache()
    ldt = DType.bf16 if cfg.dtype == "bf16" else DType.f32
    dts = [ldt, ldt, DType.i64, DType.f32, DType.f32, DType.f32, DType.f32]
    m = marshal_inputs(ins, [x.shape for x in ins], dts)
    be = HipGrpoBackend.init()
    h = be._h
    in_bytes = sum(x.nbytes for x in ins)

    def call():
        n_out = ctypes.c_int(0)
        od = ctypes.POINTER(ctypes.c_void_p)()
        ob = ctypes.POINTER(ctypes.c_size_t)()
        t0 = time.perf_counter()
        check(lib().pcp_execute(h, b"grpo_clip_kl_fwd_bwd", m.n, m.ptrs, m.nbytes, m.shapes, m.ranks, m.dtypes,
                                ctypes.byref(n_out), ctypes.byref(od), ctypes.byref(ob)), h)
        dt = time.perf_counter() - t0
        out_bytes = sum(ob[i] for i in range(n_out.value))
        lib().pcp_free(h, n_out.value, od, ob)
        return dt, out_bytes

    for _ in range(args.warmup):
        call()
    times, out_bytes = [], 0
    for _ in range(args.steps):
        dt, out_bytes = call()
        times.append(dt)
    be.deinit()
    ms_step = 1e3 * sum(times) / len(times)
    live = int((ins[3][:, 1:] != 0).sum())   # the shifted layout: row t predicts ids[t + 1]
    line = {
        "metric": f"GRPO loss fwd+bwd through the host-bytes execute boundary (PCIe-inclusive), valid tokens/s, "
                  f"V={cfg.V} {cfg.dtype}",
        "value": live / (ms_step / 1e3), "unit": "valid tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": cfg.dtype, "data": "synthetic (seeded Philox/PCG64 inputs, pageable host memory)",
        "config": {"workload": f"config{cfg.key} {cfg.name} via pcp_execute(grpo_clip_kl_fwd_bwd)", "valid_rows": live},
        "host_bytes_in": in_bytes, "host_bytes_out": out_bytes,
        "host_GBs": (in_bytes + out_bytes) / (ms_step / 1e3) / 1e9,
        "step_ms_min": 1e3 * min(times),
    }
    print(json.dumps(line), flush=True)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--workload", choices=["loss", "logprob", "execute", "nesterov", "sample", "b64", "hbm_roof",
                                           "mfma_roof"],
                    default="loss",
                    help="loss: the GRPO loss head of --config (the headline metric); logprob: forward-only "
                         "log-probs of --config's rows; execute: the host-bytes boundary (PCIe-inclusive); nesterov: the "
                         "optimizer step over Qwen2.5-0.5B's parameters; sample: the rollout sampler; "
                         "b64: the UPDATE_WEIGHTS payload codec; hbm_roof: the practical HBM roof (stream probes); "
                         "mfma_roof: the practical bf16 MFMA roof and clock (register-resident probe)")
    ap.add_argument("--roof-gib", type=float, default=4.0, help="hbm_roof workload: bytes per buffer, in GiB")
    ap.add_argument("--mfma-iters", type=int, default=40000,
                    help="mfma_roof workload: rounds of 8 32x32x16 MFMAs (or the same work in 16x16x32 ones) per "
                         "wave in the long launch (the short one runs a tenth)")
    ap.add_argument("--mode", choices=["clip_kl", "reinforce"], default="clip_kl")
    ap.add_argument("--force-streaming", action="store_true")
    ap.add_argument("--no-zero-fill", action="store_true",
                    help="loss workload: leave the dlogits rows of masked and pad tokens unwritten "
                         "(PCP_FLAG_NO_ZERO_FILL); algorithmic bytes then count live rows only")
    ap.add_argument("--exact-bf16", action="store_true",
                    help="loss workload: PCP_FLAG_EXACT_BF16 (no f16 softmax terms in the bf16 dlogits pass); "
                         "config 5: the same flag (the forward keeps f32 softmax terms)")
    ap.add_argument("--dlogits-f32", action="store_true",
                    help="loss workload: f32 dlogits from the configuration's bf16 logits")
    ap.add_argument("--vocab-chunk", type=int, default=0,
                    help="config 5: the recomputing backward's vocab chunk (a multiple of 256; 0: the forward's "
                         "softmax terms)")
    ap.add_argument("--policy-only", action="store_true", help="logprob workload: the policy rows only")
    ap.add_argument("--rows", type=int, default=64,
                    help="sample workload: rows per call (64: a decoding step of config 2; 1: the reference's "
                         "one row per generated token)")
    ap.add_argument("--async-sample", action="store_true",
                    help="sample workload: enqueue each call without waiting (pcp_sample_tokens_async)")
    ap.add_argument("--final-norm", action="store_true",
                    help="config 5: fuse the decoder's final RMSNorm (hidden = the last layer's output)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration-gib", type=float, default=0.0,
                    help="run one device-to-device copy of this many GiB first: under rocprofv3 --pmc its "
                         "FETCH_SIZE / WRITE_SIZE give the counters' scale factors")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the GRPO loss head shards by whole "
                                   "sequence groups, but no multi-GPU path is built; use --gpus 1"}))
        sys.exit(2)

    import ctypes

    import torch

    from pcp_amd import grpo, synth
    from pcp_amd._lib import LossMode, check, lib

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    if args.copy_calibration_gib > 0:
        n = int(args.copy_calibration_gib * (1 << 30)) // 2
        src = torch.ones(n, dtype=torch.bfloat16, device=dev)
        torch.empty_like(src).copy_(src)
        torch.cuda.synchronize()
        del src
    if args.workload == "nesterov":
        bench_nesterov(args)
        return
    if args.workload == "sample":
        bench_sample(args)
        return
    if args.workload == "b64":
        bench_b64(args)
        return
    if args.workload == "hbm_roof":
        bench_hbm_roof(args)
        return
    if args.workload == "mfma_roof":
        bench_mfma_roof(args)
        return
    if args.workload == "logprob":
        bench_logprob(args)
        return
    if args.workload == "execute":
        bench_execute(args)
        return
    if args.config == 5:
        bench_lmhead(args)
        return
    cfg = synth.CONFIGS[args.config]
    clip = args.mode == "clip_kl"
    mode = LossMode.GRPO_CLIP_KL if clip else LossMode.REINFORCE
    t_setup = time.perf_counter()
    inp = synth.make_device_inputs(cfg, dev)
    torch.cuda.synchronize()
    t_setup = time.perf_counter() - t_setup
    ctx = grpo.default_context(0)
    kw = dict(rewards=inp["rewards"], group_size=cfg.group, ref_logits=inp["ref_logits"] if clip else None,
              old_logp=inp["old_logp"], loss_mode=mode, clip_eps=cfg.clip_eps, kl_beta=cfg.kl_beta,
              force_streaming=args.force_streaming, zero_fill=not args.no_zero_fill,
              exact_bf16=args.exact_bf16, ctx=ctx)
    d_dtype = torch.float32 if args.dlogits_f32 else None
    out = grpo.grpo_loss_fwd_bwd(inp["logits"], inp["ids"], inp["mask"], dlogits_dtype=d_dtype,
                                 **kw)  # allocates outputs
    for _ in range(args.warmup):
        grpo.grpo_loss_fwd_bwd(inp["logits"], inp["ids"], inp["mask"], outputs=out, sync=False, **kw)
    ctx.sync()
    torch.cuda.synchronize()

    check(lib().pcp_profile_start(ctx.handle, args.steps), ctx.handle)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        grpo.grpo_loss_fwd_bwd(inp["logits"], inp["ids"], inp["mask"], outputs=out, sync=False, **kw)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ctx.sync()
    n_l = ctypes.c_int(0)
    tot = ctypes.c_double(0)
    check(lib().pcp_profile_stop(ctx.handle, ctypes.byref(n_l), ctypes.byref(tot)), ctx.handle)
    kernel_ms = tot.value / max(n_l.value, 1)

    ab = algorithmic_bytes(cfg, inp["lengths"], clip, zero_fill=not args.no_zero_fill,
                           s_out=4 if args.dlogits_f32 else None)
    ms_step = elapsed * 1e3 / args.steps
    value = ab["live_rows"] / (ms_step / 1e3)
    achieved = ab["bytes"] / (kernel_ms / 1e3) / 1e9
    line = {
        "metric": "GRPO logprob+loss fwd+bwd tokens/s and achieved HBM GB/s, V=151936 bf16",
        "value": value,
        "unit": "valid tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.dtype,
        "data": "synthetic (seeded Philox/PCG64 inputs of the configuration)",
        "config": {"workload": f"config{cfg.key} {cfg.name}: {cfg.prompts} prompts x G={cfg.group}, T={cfg.T}, "
                               f"V={cfg.V}, {cfg.dtype} logits, loss={args.mode}"
                               + (", dlogits of masked rows left unwritten (no zero-fill)" if args.no_zero_fill
                                  else "")
                               + (", bf16 dlogits rounded once from f32 (exact mode)" if args.exact_bf16 else "")
                               + (", f32 dlogits" if args.dlogits_f32 else ""),
                   "rows": ab["rows"], "valid_rows": ab["live_rows"], "global_batch": cfg.S, "seq_len": cfg.T,
                   "zero_fill": not args.no_zero_fill},
        "step_gbs": ab["bytes"] / (ms_step / 1e3) / 1e9,
        "rows_per_s": ab["rows"] / (ms_step / 1e3),
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "kernel": ("grpo_stream_kernel" if args.force_streaming else "grpo_resident_kernel"),
                     "kernel_ms": kernel_ms, "algorithmic_bytes": ab["bytes"]},
        "setup_s": t_setup,
    }
    tfile = os.path.join(ROOT, "profiles", f"traffic_config{cfg.key}_{args.mode}"
                                           f"{'_no_zero_fill' if args.no_zero_fill else ''}"
                                           f"{'_exact' if args.exact_bf16 else ''}"
                                           f"{'_f32_out' if args.dlogits_f32 else ''}"
                                           f"{'_streaming' if args.force_streaming else ''}.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            line["roofline"]["traffic"] = json.load(f).get("hbm_bytes_per_launch")
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(inp, cfg, clip)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
