"""Benchmark of the sqrt(N) attention hot path on one MI355X.

Default workload (BASELINE metric): B=1, H=16, D=128, S=131072, fp16, causal,
q/k/v/dO ~ N(0,1) from an on-device generator (seed 0).  A step is one
forward + backward of the attention op (o = attn(q, k, v); o.backward(dO)).
Prints ONE JSON line:
  value        whole-job effective TFLOP/s of fwd+bwd (14*D*pairs / time)
  fwd_ms / fwdbwd_ms and their effective TFLOP/s
  fwdbwd_per_step  10% trimmed mean, coefficient of variation, min and max of
               the same step timed one call at a time
  roofline     the forward kernel (one launch of cra_fwd = one kernel), timed
               with HIP events on the stream it runs on, against the fp16
               dense MFMA peak; traffic from a committed rocprofv3 --pmc
               summary when present
  cpu_baseline the oracle's chunked CPU port (the reference's cra_cpu_fast
               algorithm, fp32) on the host cores, on a bounded sample of whole
               heads of the same workload, as TFLOP/s, with the CPU model and
               the thread count used

Other modes:
  --config N|all       time BASELINE configurations 2-5 at every listed S (ms,
                       TFLOP/s, roofline fraction, 50% target; config 5 through
                       the hybrid dispatcher with SDPA beside it), one JSON line
                       per point
  --crossover          sweep S against torch's SDPA (forward and fwd+bwd)
  --sdpa-dense         torch's fused SDPA on dense causal attention at long S,
                       as TFLOP/s and fraction of the fp16 MFMA peak (context)
  --profile-workload   short fixed workload for rocprofv3 --pmc passes
  --counter-summary D  markdown summary of rocprofv3 --pmc output directories
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "cron-root-attention_amd"))
sys.path.insert(0, ROOT)

METRIC = "fwd & fwd+bwd ms + eff. TFLOP/s, H=16 D=128 S=128K fp16, 1 MI355X"
PEAK_FP16_TFLOPS = 2500.0      # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0
MFMA_FLOPS = 2 * 16 * 16 * 32   # one v_mfma_f32_16x16x32_{f16,bf16}
CUS = 256                       # MI355X compute units (4 SIMDs each)
TARGET_FRAC = 0.5               # the north star's roofline fraction


def pairs_fast(S: int, top_k: int = 2) -> int:
    import numpy as np
    W = int(math.ceil(math.sqrt(S)))
    i = np.arange(S, dtype=np.int64)
    ls = np.maximum(i - W + 1, 0)
    p = np.minimum(i + 1, W) + (ls + W - 1) // W
    if S > 2048:
        p = p + top_k * (ls // W)
    return int(p.sum())


def phase_pairs(S: int, top_k: int = 2) -> dict:
    """Pairs per (b, h) by phase: local window, strided rows, relay rows."""
    import numpy as np
    W = int(math.ceil(math.sqrt(S)))
    i = np.arange(S, dtype=np.int64)
    ls = np.maximum(i - W + 1, 0)
    return {"local": int(np.minimum(i + 1, W).sum()),
            "strided": int(((ls + W - 1) // W).sum()),
            "relay": int((top_k * (ls // W)).sum()) if S > 2048 else 0}


def row_pairs(rows, S, top_k=2):
    import numpy as np
    W = int(math.ceil(math.sqrt(S)))
    i = np.asarray(rows, dtype=np.int64)
    ls = np.maximum(i - W + 1, 0)
    p = np.minimum(i + 1, W) + (ls + W - 1) // W
    if S > 2048:
        p = p + top_k * (ls // W)
    return int(p.sum())


def timed(fn, steps, warmup, torch):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def per_step_ms(fn, steps, torch):
    """Each of `steps` calls bracketed by its own events (no warmup: call
    after `timed`); returns the list of per-call milliseconds."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    for e0, e1 in ev:
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    return [e0.elapsed_time(e1) for e0, e1 in ev]


def spread(ms):
    """10% trimmed mean and coefficient of variation of per-step times."""
    xs = sorted(ms)
    k = len(xs) // 10
    core = xs[k:len(xs) - k] if len(xs) > 2 * k else xs
    mean = sum(xs) / len(xs)
    var = sum((x - mean) ** 2 for x in xs) / max(1, len(xs) - 1)
    return {"n": len(xs), "trimmed_mean_ms": round(sum(core) / len(core), 4),
            "cov": round(var ** 0.5 / mean, 4), "min_ms": round(xs[0], 4), "max_ms": round(xs[-1], 4)}


def per_launch_ms(fn, steps, warmup, torch):
    """Average duration of single launches, each bracketed by its own pair of
    events on the current stream (the stream the library launches on), so
    that no launch overlaps the next one's start, as in a kernel trace."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    for e0, e1 in ev:
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    return sum(e0.elapsed_time(e1) for e0, e1 in ev) / steps


def host_cpu() -> dict:
    """CPU model, logical CPUs of the machine, CPUs this process may run on,
    physical cores (from /proc/cpuinfo where readable)."""
    model, phys = None, set()
    try:
        with open("/proc/cpuinfo") as f:
            pid = core = None
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    pid = v
                elif k == "core id":
                    core = v
                    phys.add((pid, core))
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = os.cpu_count()
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "cpus_allowed": allowed,
            "physical_cores": len(phys) or None}


def cpu_threads(requested=None) -> int:
    """Threads for the CPU baseline: as requested, else the job's CPU share
    (OMP_NUM_THREADS, which the GPU box sets to its share of the host), else
    every CPU this process may run on."""
    if requested:
        return int(requested)
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    return host_cpu()["cpus_allowed"] or 1


def cpu_baseline(B, H, S, D, budget_s: float, threads: int):
    """Oracle CPU port (fp32 forward, the reference's cra_cpu_fast algorithm)
    on the host cores: pairs of heads of the same workload, each over all S
    queries, until ~budget_s of CPU time (or all H heads); the relay
    selection (fp32 norms + topk, as cra_cpu_fast) is inside the timed
    region. Returns effective TFLOP/s over the heads done."""
    import torch
    from oracle import cra_oracle as O
    from oracle.cpu_port import cra_cpu_chunked
    torch.set_num_threads(threads)
    plan = O.make_plan(S)
    Hs = 2
    t_used, heads_done, flops = 0.0, 0, 0
    g = torch.Generator().manual_seed(0)
    while heads_done < H and t_used < budget_s:
        q, k, v = (torch.randn(1, Hs, S, D, generator=g) for _ in range(3))
        t0 = time.perf_counter()
        cra_cpu_chunked(q, k, v, plan, norm="torch")
        t_used += time.perf_counter() - t0
        heads_done += Hs
        flops += 4 * D * pairs_fast(S) * Hs
    out = {"value": flops / t_used / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
           "sample": f"fp32 forward of {heads_done} of {H} heads (all {S} queries each, relay "
                     f"selection included), D={D}, {t_used:.1f} s on {threads} threads",
           "seconds": round(t_used, 2)}
    out.update(host_cpu())
    return out


def mfma_busy_needed(n_mfma: float, flops: float, clock_ghz: float, frac: float) -> float:
    """Share of cycles every SIMD's matrix core must be busy (16 cycles per
    executed v_mfma_f32_16x16x32) for `flops` of algorithmic work to run at
    `frac` of the nominal fp16 peak, at the clock `clock_ghz`: the step then
    takes flops / (frac * peak) seconds."""
    seconds = flops / (frac * PEAK_FP16_TFLOPS * 1e12)
    return n_mfma * 16 / (seconds * clock_ghz * 1e9 * CUS * 4)


def executed_for(workload: str):
    """Executed MFMA instructions per kernel launch (SQ_INSTS_MFMA) and the
    sustained clock, from the committed counter summary of this workload
    (profiles/executed_<workload>.json, written by --counter-summary
    --json-out from rocprofv3 --pmc passes over --profile-workload)."""
    path = os.path.join(ROOT, "profiles", f"executed_{workload}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


def traffic_for(kernel: str, workload: str):
    path = os.path.join(ROOT, "profiles", f"traffic_{kernel}_{workload}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def forward_phases(B, H, S, D, q, k, v, p, gk, gv, args, torch):
    """Per-phase forward (cra_fwd_phases: the local window alone, the global
    rows alone, and the global rows of a relay-off packing = the strided rows
    alone) and the global-row build (K1, HBM-bound), each timed per launch.
    The relay rows sit in the same packed tiles as the strided rows, so no
    launch computes them alone: their share is reported as the difference of
    the two global launches and labelled so. Counter-backed MFMA-busy shares
    of the same launches come from profiles/phases_counters_<workload>.json
    when present."""
    from cron_root_attention import _native
    dtype = q.dtype
    W = int(math.ceil(math.sqrt(S)))
    pp = phase_pairs(S)
    t_loc = per_launch_ms(lambda: _native.forward(p, q, k, v, gk, gv, phases=_native.PHASE_LOCAL),
                          args.steps, args.warmup, torch)
    t_glob = per_launch_ms(lambda: _native.forward(p, q, k, v, gk, gv,
                                                   phases=_native.PHASE_GLOBAL),
                           args.steps, args.warmup, torch)
    # strided rows alone: the same global-phase kernel over packed rows built
    # without relay (one row per block); the relay rows' share is the
    # difference to the full global phase
    p_s = _native.problem(B, H, H, S, D, W, False, 2, dtype, 1 / math.sqrt(D))
    gk_s, gv_s, _ = _native.build_global(p_s, k, v, None)
    t_str = per_launch_ms(lambda: _native.forward(p_s, q, k, v, gk_s, gv_s,
                                                  phases=_native.PHASE_GLOBAL),
                          args.steps, args.warmup, torch)
    del gk_s, gv_s
    t_bg = per_launch_ms(lambda: _native.build_global(p, k, v, None), args.steps, args.warmup,
                         torch)
    G = int(_native.global_rows(p))
    NB = (S + W - 1) // W
    e = 2
    bg_bytes = B * H * (S * D * e + G * D * e + 2 * G * D * e + 4 * NB * 2)
    f_loc = 4 * D * pp["local"] * B * H
    f_glob = 4 * D * (pp["strided"] + pp["relay"]) * B * H
    f_str = 4 * D * pp["strided"] * B * H
    t_rel = t_glob - t_str
    phases = {
        "local": {"ms": round(t_loc, 4), "pairs_per_head": pp["local"],
                  "tflops": round(f_loc / (t_loc * 1e-3) / 1e12, 2),
                  "mfma_frac": round(f_loc / (t_loc * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4)},
        "global": {"ms": round(t_glob, 4),
                   "pairs_per_head": pp["strided"] + pp["relay"],
                   "strided_pairs_per_head": pp["strided"], "relay_pairs_per_head": pp["relay"],
                   "tflops": round(f_glob / (t_glob * 1e-3) / 1e12, 2),
                   "mfma_frac": round(f_glob / (t_glob * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4)},
        "strided": {"ms": round(t_str, 4), "pairs_per_head": pp["strided"],
                    "tflops": round(f_str / (t_str * 1e-3) / 1e12, 2),
                    "mfma_frac": round(f_str / (t_str * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
                    "how": "global phase over strided rows only (relay off)"},
        "relay": {"ms_difference": round(t_rel, 4), "pairs_per_head": pp["relay"],
                  "how": "global launch minus the strided-only launch: relay rows share the "
                         "packed tiles of the strided rows, no launch computes them alone"},
        "build_global": {"ms": round(t_bg, 4), "bytes": bg_bytes,
                         "GBps": round(bg_bytes / (t_bg * 1e-3) / 1e9, 1),
                         "hbm_frac": round(bg_bytes / (t_bg * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
    }
    wl = f"H{H}_D{D}_S{S}_fp16"
    cpath = os.path.join(ROOT, "profiles", f"phases_counters_{wl}.json")
    if os.path.exists(cpath):
        with open(cpath) as f:
            cnt = json.load(f)
        for name in ("local", "global", "strided"):
            if name in cnt:
                phases[name]["mfma_busy_counter"] = cnt[name]
        phases["counters_source"] = "profiles/" + os.path.basename(cpath)
    return phases


def run_main(args):
    import torch
    import cron_root_attention as cra
    from cron_root_attention import _native
    dev = torch.device("cuda", 0)
    B, H, S, D = 1, 16, 131072, 128
    dtype = torch.float16
    gen = torch.Generator(device=dev).manual_seed(0)
    mk = lambda: torch.randn(B, H, S, D, generator=gen, device=dev, dtype=torch.float32).to(dtype)
    q, k, v, dO = mk(), mk(), mk(), mk()
    P = pairs_fast(S)
    f_fwd = 4 * D * P * B * H
    f_all = 14 * D * P * B * H

    with torch.no_grad():
        fwd_ms = timed(lambda: cra.cron_root_attention(q, k, v), args.steps, args.warmup, torch)
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))

    def step():
        qg.grad = kg.grad = vg.grad = None
        cra.cron_root_attention(qg, kg, vg).backward(dO)

    step_ms = timed(step, args.steps, args.warmup, torch)
    # per-step spread of the same step (reported beside the bracketed mean)
    per_step = per_step_ms(step, max(args.steps, 10), torch)

    # forward kernel alone: cra_fwd launches exactly one kernel
    W = int(math.ceil(math.sqrt(S)))
    p = _native.problem(B, H, H, S, D, W, True, 2, dtype, 1 / math.sqrt(D))
    gk, gv, _ = _native.build_global(p, k, v, None)
    kern_ms = per_launch_ms(lambda: _native.forward(p, q, k, v, gk, gv), args.steps, args.warmup,
                            torch)
    achieved = f_fwd / (kern_ms * 1e-3) / 1e12
    workload = "H16_D128_S131072_fp16"
    roof = {"kernel": "fwd2_kernel<f16,128,4 waves,all phases>", "bound": "mfma", "achieved": round(achieved, 2),
            "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
            "traffic": traffic_for("fwd", workload), "avg_ms": round(kern_ms, 4),
            "algorithmic_flops": f_fwd}

    phases = forward_phases(B, H, S, D, q, k, v, p, gk, gv, args, torch)

    # forward+backward against the same peak, with the executed MFMA work of
    # the kernels (counter summary) beside the algorithmic 14*D*pairs
    ex = executed_for(workload)
    roof_fb = {"bound": "mfma", "achieved": round(f_all / (step_ms * 1e-3) / 1e12, 2),
               "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
               "frac": round(f_all / (step_ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
               "algorithmic_flops": f_all, "ms": round(step_ms, 4)}
    if ex:
        n_mfma = sum(ex["mfma_per_launch"].values())
        flops_ex = n_mfma * MFMA_FLOPS
        roof_fb.update({
            "executed_mfma": n_mfma, "executed_flops": flops_ex,
            "executed_vs_algorithmic": round(flops_ex / f_all, 4),
            "executed_frac": round(flops_ex / (step_ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
            # MFMA-busy share every SIMD would need for half the nominal
            # peak, at the clock these kernels sustain (counter summary)
            "mfma_busy_needed_for_half_peak": round(
                mfma_busy_needed(n_mfma, f_all, ex["clock_ghz"], TARGET_FRAC), 4),
            "clock_ghz": ex["clock_ghz"], "per_kernel": ex["mfma_per_launch"],
            "source": "profiles/executed_" + workload + ".json"})

    cpu = None
    if not args.skip_cpu:
        cpu = cpu_baseline(B, H, S, D, args.cpu_seconds, cpu_threads(args.cpu_threads))

    out = {
        "metric": METRIC, "value": round(f_all / (step_ms * 1e-3) / 1e12, 3), "unit": "TFLOP/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(step_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic: q, k, v, dO ~ N(0,1), on-device generator seed 0",
        "config": {"workload": "fwd+bwd of sqrt(N) attention, B=1 H=16 D=128 S=131072 fp16 "
                               "causal (BASELINE config 3 at the north-star S)",
                   "B": B, "H": H, "S": S, "D": D, "window": W, "relay_top_k": 2},
        "fwd_ms": round(fwd_ms, 4), "fwd_tflops": round(f_fwd / (fwd_ms * 1e-3) / 1e12, 3),
        "fwdbwd_ms": round(step_ms, 4), "fwdbwd_tflops": round(f_all / (step_ms * 1e-3) / 1e12, 3),
        "pairs_per_head": P, "fwdbwd_per_step": spread(per_step),
        "roofline": roof, "roofline_fwdbwd": roof_fb, "phases": phases, "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def run_phases(args):
    """BASELINE config 3 (B=1 H=16 D=128 fp16) at each S of --phases: the
    forward kernel's time and roofline fraction and the per-phase figures of
    forward_phases, one JSON line per S."""
    import torch
    from cron_root_attention import _native
    dev = torch.device("cuda", 0)
    B, H, D = 1, 16, 128
    for S in (int(x) for x in args.phases.split(",")):
        gen = torch.Generator(device=dev).manual_seed(0)
        q, k, v = (torch.randn(B, H, S, D, generator=gen, device=dev, dtype=torch.float32).half()
                   for _ in range(3))
        W = int(math.ceil(math.sqrt(S)))
        p = _native.problem(B, H, H, S, D, W, S > 2048, 2, torch.float16, 1 / math.sqrt(D))
        gk, gv, _ = _native.build_global(p, k, v, None)
        kern_ms = per_launch_ms(lambda: _native.forward(p, q, k, v, gk, gv), args.steps,
                                args.warmup, torch)
        f_fwd = 4 * D * pairs_fast(S) * B * H
        roof, bound, _ = roofline_ms(B, H, S, D, 2, False)
        out = {"config": 3, "B": B, "H": H, "D": D, "S": S, "window": W,
               "fwd_kernel_ms": round(kern_ms, 4),
               "fwd_kernel_tflops": round(f_fwd / (kern_ms * 1e-3) / 1e12, 2),
               "fwd_roofline_frac": round(roof / kern_ms, 4), "bound": bound,
               "phases": forward_phases(B, H, S, D, q, k, v, p, gk, gv, args, torch)}
        print(json.dumps(out), flush=True)
        del q, k, v, gk, gv
        torch.cuda.empty_cache()


# BASELINE configurations 2-5 (config 1 is the CPU reference's plumbing case):
# (B, H, D, dtype, S values, mode). mode "fwd": forward under no_grad;
# "train": forward + backward; "hybrid": CronRootAttention(hybrid=True)'s
# dispatch (cron_root_attention_hybrid) in both modes, with the √N op and
# SDPA timed beside it.
CONFIGS = {
    2: (1, 8, 64, "f16", (2048, 8192, 65536, 262144), "fwd"),
    3: (1, 16, 128, "f16", (16384, 131072, 524288), "fwd"),
    4: (1, 12, 64, "f16", (8192, 32768, 131072), "train"),
    5: (2, 32, 128, "bf16", (512, 1024, 2048, 4096, 65536, 262144), "hybrid"),
}
# The reference's published forward / training ms on an RTX 5070 Ti (context
# only: other hardware; README.md:23-80, 97-107). Config 5 is published at
# B=1 only and config 4 (H=12) has no training figure.
REFERENCE_MS = {
    (2, 2048): 0.048, (2, 8192): 0.102, (2, 65536): 2.35, (2, 262144): 17.3,
    (3, 16384): 1.25, (3, 131072): 27.6, (3, 524288): 191.0,
    (5, 512): 0.052, (5, 1024): 0.070, (5, 2048): 0.132, (5, 4096): 0.242, (5, 65536): 17.0,
    (5, 262144): 125.0,
}


def roofline_ms(B, H, S, D, esize, train: bool):
    """max(F / MFMA peak, compulsory bytes / HBM peak) in ms, and the bound."""
    P = pairs_fast(S)
    F = (14 if train else 4) * D * P * B * H
    nbytes = B * H * ((12 if train else 4) * S * D * esize + (8 if train else 4) * S)
    t_f = F / (PEAK_FP16_TFLOPS * 1e12) * 1e3
    t_b = nbytes / (PEAK_HBM_GBS * 1e9) * 1e3
    return max(t_f, t_b), ("mfma" if t_f >= t_b else "hbm"), F


def run_configs(args):
    """Times every S of the selected BASELINE configurations: ms, effective
    TFLOP/s, the fraction of the MFMA/HBM roofline and the 50% target; one
    JSON line per point."""
    import torch
    import torch.nn.functional as F
    import cron_root_attention as cra
    from cron_root_attention.hybrid import dispatch_backend
    dev = torch.device("cuda", 0)
    sel = sorted(CONFIGS) if args.config == "all" else [int(x) for x in args.config.split(",")]
    for c in sel:
        B, H, D, dts, seqs, mode = CONFIGS[c]
        dtype = {"f16": torch.float16, "bf16": torch.bfloat16}[dts]
        for S in seqs:
            gen = torch.Generator(device=dev).manual_seed(0)
            mk = lambda: torch.randn(B, H, S, D, generator=gen, device=dev,
                                     dtype=torch.float32).to(dtype)
            q, k, v, dO = mk(), mk(), mk(), mk()
            res = {"config": c, "B": B, "H": H, "D": D, "S": S, "dtype": dts, "mode": mode}

            def fwd_ms(fn):
                with torch.no_grad():
                    return timed(lambda: fn(q, k, v), args.steps, args.warmup, torch)

            def train_ms(fn):
                qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))

                def st():
                    qg.grad = kg.grad = vg.grad = None
                    fn(qg, kg, vg).backward(dO)
                return timed(st, args.steps, args.warmup, torch)

            cr = lambda a, b, cc: cra.cron_root_attention(a, b, cc)
            for tr in ((False, True) if mode == "hybrid" else ((mode == "train"),)):
                tag = "train" if tr else "fwd"
                roof, bound, flops = roofline_ms(B, H, S, D, 2, tr)
                t = train_ms(cr) if tr else fwd_ms(cr)
                res[f"{tag}_ms"] = round(t, 4)
                res[f"{tag}_tflops"] = round(flops / (t * 1e-3) / 1e12, 2)
                res[f"{tag}_roofline_frac"] = round(roof / t, 4)
                res[f"{tag}_bound"] = bound
                res[f"{tag}_target_50pct_ms"] = round(2 * roof, 4)
                if mode == "hybrid":
                    backend = dispatch_backend(S, D, tr, B * H)
                    res[f"{tag}_dispatch"] = backend
                    if S <= 65536:
                        sd = lambda a, b, cc: F.scaled_dot_product_attention(a, b, cc, is_causal=True)
                        res[f"{tag}_sdpa_ms"] = round(train_ms(sd) if tr else fwd_ms(sd), 4)
                    hy = lambda a, b, cc: cra.cron_root_attention_hybrid(a, b, cc)
                    res[f"{tag}_hybrid_ms"] = round(train_ms(hy) if tr else fwd_ms(hy), 4)
            ref = REFERENCE_MS.get((c, S))
            if ref is not None:
                res["reference_rtx5070ti_fwd_ms"] = ref
            print(json.dumps(res), flush=True)
            del q, k, v, dO
            torch.cuda.empty_cache()


def run_profile_workload(args):
    """Short fixed workload for counter passes (rocprofv3 --pmc): a 1 GiB
    device copy first (read 1 GiB + write 1 GiB, the calibration of
    FETCH_SIZE / WRITE_SIZE), then the hot path's kernels at the shape
    --pw B,H,S,D (default the north star, 1,16,131072,128; fp16):
      mode "all":   build_global and cra_fwd twice each, the local-only, the
                    global-only and the strided-only (relay-off packing)
                    forwards once each, then one backward;
      mode "train": one training step of the public op (forward + backward);
      mode "fwd":   one forward of the public op."""
    import torch
    import cron_root_attention as cra
    from cron_root_attention import _native
    dev = torch.device("cuda", 0)
    x = torch.empty(512 * 1024 * 1024, dtype=torch.float16, device=dev).fill_(1.0)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    y.copy_(x)
    torch.cuda.synchronize()
    del x, y
    B, H, S, D = (int(t) for t in args.pw.split(","))
    gen = torch.Generator(device=dev).manual_seed(0)
    q, k, v, do = (torch.randn(B, H, S, D, generator=gen, device=dev, dtype=torch.float32).half()
                   for _ in range(4))
    W = int(math.ceil(math.sqrt(S)))
    relay = S > 2048
    if args.pw_mode == "all":
        p = _native.problem(B, H, H, S, D, W, relay, 2, torch.float16, 1 / math.sqrt(D))
        for _ in range(2):
            gk, gv, src = _native.build_global(p, k, v, None)
            o, lse = _native.forward(p, q, k, v, gk, gv)
        # the local-window and global-row phases on their own (their own kernels),
        # then the global phase over a relay-off packing (the strided rows alone)
        _native.forward(p, q, k, v, gk, gv, phases=_native.PHASE_LOCAL)
        _native.forward(p, q, k, v, gk, gv, phases=_native.PHASE_GLOBAL)
        p_s = _native.problem(B, H, H, S, D, W, False, 2, torch.float16, 1 / math.sqrt(D))
        gk_s, gv_s, _ = _native.build_global(p_s, k, v, None)
        _native.forward(p_s, q, k, v, gk_s, gv_s, phases=_native.PHASE_GLOBAL)
        _native.backward(p, q, k, v, o, do, lse, gk, gv, src, None, False)
    elif args.pw_mode == "train":
        qg, kg, vg = (t.requires_grad_(True) for t in (q, k, v))
        cra.cron_root_attention(qg, kg, vg).backward(do)
    else:
        with torch.no_grad():
            cra.cron_root_attention(q, k, v)
    torch.cuda.synchronize()
    print(json.dumps({"profile_workload": "done", "mode": args.pw_mode, "B": B, "H": H, "S": S,
                      "D": D}), flush=True)


def _demangle(name: str) -> str:
    if not name.startswith("_Z"):
        return name
    import re
    # this library's kernels: cra::(anon)::<kernel><template args>(args struct);
    # decoded here because c++filt may not know the _Float16 (DF16_) mangling
    m = re.match(r"_ZN3cra12_GLOBAL__N_1(\d+)(\w+)", name)
    if m:
        n = int(m.group(1))
        kname, rest = m.group(2)[:n], m.group(2)[n:]
        if rest.startswith("I"):
            targs = []
            for t in re.finditer(r"DF16_|DF16b|L[ib](\d+)E|(?<![A-Za-z])f(?=[LE])", rest[1:]):
                tok = t.group(0)
                targs.append({"DF16_": "f16", "DF16b": "bf16", "f": "f32"}.get(
                    tok, "true" if tok == "Lb1E" else "false" if tok == "Lb0E" else t.group(1)))
            return f"{kname}<{', '.join(targs)}>()"
        return kname + "()"
    import subprocess
    try:
        out = subprocess.run(["c++filt", name], capture_output=True, text=True, timeout=10)
        return out.stdout.strip() or name
    except (OSError, subprocess.SubprocessError):
        return name


def _short_kernel(name: str) -> str:
    """'void cra::(anonymous namespace)::fwd2_kernel<_Float16, 128, 4, 3>(cra::FwdArgs)'
    -> 'fwd2_kernel<_Float16, 128, 4, 3>'; torch kernels -> their template head."""
    import re
    name = _demangle(name)
    m = re.search(r"(\w+_kernel)(<[^()]*>)?\(", name)
    if m:
        return m.group(1) + (m.group(2) or "")
    return name[:60]


def counter_summary(dirs, cus: int = 256, xcds: int = 8):
    """Markdown summary of rocprofv3 --pmc passes (run_counter_collection.csv
    under each directory) over --profile-workload: per kernel, the mean of
    every counter over its dispatches and the derived figures."""
    import csv
    import glob
    from collections import defaultdict
    vals = defaultdict(lambda: defaultdict(list))   # kernel -> counter -> [per dispatch]
    dur = defaultdict(list)
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(f) as fh:
                per = defaultdict(float)
                meta = {}
                for r in csv.DictReader(fh):
                    key = (r["Dispatch_Id"], r["Counter_Name"])
                    per[key] += float(r["Counter_Value"])
                    meta[r["Dispatch_Id"]] = (_short_kernel(r["Kernel_Name"]),
                                              int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
                for (disp, cn), v in per.items():
                    kname, ns = meta[disp]
                    vals[kname][cn].append(v)
                    if cn in ("SQ_INSTS_MFMA", "FETCH_SIZE"):
                        dur[kname].append(ns)
    mean = lambda xs: sum(xs) / len(xs) if xs else float("nan")
    rows = []
    copy_fetch = None
    for k, c in vals.items():
        if "copy" in k.lower() or "direct_copy" in k.lower():
            copy_fetch = (mean(c.get("FETCH_SIZE", [])), mean(c.get("WRITE_SIZE", [])))
    lines = ["| kernel | dispatches | MFMA busy | VALU / MFMA | trans / MFMA | SALU / MFMA | LDS / MFMA "
             "| LDS bank-conflict cycles / LDS instr | wave time waiting | clock (GHz) "
             "| read MB | written MB |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for k in sorted(vals, key=lambda x: -mean(dur.get(x, [0]))):
        c = {n: mean(v) for n, v in vals[k].items()}
        mf = c.get("SQ_INSTS_MFMA", 0)
        if not mf:
            continue
        grbm = c.get("GRBM_GUI_ACTIVE")
        busy = c.get("SQ_VALU_MFMA_BUSY_CYCLES")
        util = busy / (grbm / xcds * cus * 4) if (grbm and busy) else float("nan")
        ghz = (grbm / xcds) / mean(dur[k]) if grbm and dur.get(k) else float("nan")
        wait = c.get("SQ_WAIT_ANY", 0) / c["SQ_WAVE_CYCLES"] if c.get("SQ_WAVE_CYCLES") else float("nan")
        rd = c.get("FETCH_SIZE", float("nan")) * 1024 * 2 / 1e6   # FETCH_SIZE counts half the bytes read
        wr = c.get("WRITE_SIZE", float("nan")) * 1024 / 1e6
        lines.append(
            f"| `{k}` | {len(vals[k]['SQ_INSTS_MFMA'])} | {util:.1%} | {c.get('SQ_INSTS_VALU', 0) / mf:.2f} "
            f"| {c.get('SQ_INSTS_VALU_TRANS_F32', 0) / mf:.2f} | {c.get('SQ_INSTS_SALU', 0) / mf:.2f} "
            f"| {c.get('SQ_INSTS_LDS', 0) / mf:.2f} "
            f"| {c.get('SQ_LDS_BANK_CONFLICT', 0) / max(1.0, c.get('SQ_INSTS_LDS', 0)):.2f} "
            f"| {wait:.1%} | {ghz:.2f} | {rd:.1f} | {wr:.1f} |")
    extra = ["", "Raw means per dispatch (every counter of every pass):", "",
             "| kernel | counter | mean per dispatch |", "|---|---|---|"]
    for k in sorted(vals):
        for n in sorted(vals[k]):
            extra.append(f"| `{k}` | {n} | {mean(vals[k][n]):.6g} |")
    cal = ""
    if copy_fetch:
        cal = (f"\nCalibration (1 GiB device copy of the same run): FETCH_SIZE {copy_fetch[0]:.0f} KiB, "
               f"WRITE_SIZE {copy_fetch[1]:.0f} KiB per GiB moved.\n")
    return "\n".join(lines) + "\n" + cal + "\n".join(extra) + "\n"


def counter_dispatches(dirs):
    """Per-dispatch counter records of rocprofv3 --pmc output directories, in
    dispatch order: [(kernel, {counter: value}, duration_ns)] per pass."""
    import csv
    import glob
    from collections import defaultdict
    passes = []
    for d in dirs:
        for f in sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)):
            per = defaultdict(lambda: defaultdict(float))
            meta = {}
            with open(f) as fh:
                for r in csv.DictReader(fh):
                    per[int(r["Dispatch_Id"])][r["Counter_Name"]] += float(r["Counter_Value"])
                    meta[int(r["Dispatch_Id"])] = (_short_kernel(r["Kernel_Name"]),
                                                   int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
            passes.append([(meta[i][0], dict(per[i]), meta[i][1]) for i in sorted(per)])
    return passes


def counter_json(dirs, workload: str, xcds: int = 8):
    """From --pmc passes over `--profile-workload --pw-mode all`: per-launch
    executed MFMA instructions of the forward and backward kernels with the
    clock they ran at (profiles/executed_<workload>.json), and the MFMA-busy
    share of the local-only, global-only and strided-only forward launches
    (profiles/phases_counters_<workload>.json)."""
    passes = counter_dispatches(dirs)
    by_kernel = {}
    for recs in passes:
        seen = {}
        for name, c, ns in recs:
            i = seen.get(name, 0)
            seen[name] = i + 1
            slot = by_kernel.setdefault((name, i), {"ns": []})
            slot.update(c)
            slot["ns"].append(ns)
    def find(prefix, idx=0, suffix=""):
        for (name, i), c in by_kernel.items():
            if name.startswith(prefix) and name.endswith(suffix) and i == idx:
                return c
        return None
    fwd = find("fwd2_kernel", 0, ", 3>")
    dq = find("dq2_kernel")
    glob_k = find("dkdv2_kernel", 0, ", 128>") or find("dkdv2_kernel", 0, "true, 8, 1, 128>")
    loc = None
    for (name, i), c in by_kernel.items():
        if name.startswith("dkdv2_kernel") and ", false," in name:
            loc = c
    mf = {"forward": fwd, "dq": dq, "global_dkdv": glob_k, "local_dkdv": loc}
    mfma = {k: int(v["SQ_INSTS_MFMA"]) for k, v in mf.items() if v and "SQ_INSTS_MFMA" in v}
    tot_ns = sum(sum(v["ns"]) / len(v["ns"]) for v in mf.values() if v)
    clock = sum((v["GRBM_GUI_ACTIVE"] / xcds) for v in mf.values()
                if v and "GRBM_GUI_ACTIVE" in v) / tot_ns if tot_ns else None
    executed = {"workload": workload, "mfma_per_launch": mfma,
                "clock_ghz": round(clock, 3) if clock else None,
                "how": "SQ_INSTS_MFMA per launch of each kernel of one forward + backward; "
                       "clock = sum(GRBM_GUI_ACTIVE / 8 XCDs) / sum(duration) over those kernels"}
    def busy(c):
        if not c or "SQ_VALU_MFMA_BUSY_CYCLES" not in c or "GRBM_GUI_ACTIVE" not in c:
            return None
        return round(c["SQ_VALU_MFMA_BUSY_CYCLES"] / (c["GRBM_GUI_ACTIVE"] / xcds * CUS * 4), 4)
    phases = {"local": busy(find("fwd2_kernel", 0, ", 1>")),
              "global": busy(find("fwd2_kernel", 0, ", 2>")),
              "strided": busy(find("fwd2_kernel", 1, ", 2>")),
              "forward": busy(fwd),
              "how": "SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 256 CUs x 4 SIMDs) "
                     "of the local-only, global-only and strided-only (relay-off packing) "
                     "forward launches of --profile-workload"}
    return executed, phases


def sdpa_backend(q, k, v, torch, F):
    """First fused SDPA backend that runs this shape (flash, then memory
    efficient). The math backend is never used: its batched products on
    transposed bf16 views are unsafe on this platform."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    for b in (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION):
        try:
            with sdpa_kernel([b]):
                F.scaled_dot_product_attention(q, k, v, is_causal=True)
            torch.cuda.synchronize()
            return b
        except RuntimeError:
            continue
    return None


def run_sdpa_dense(args):
    """Context for the MFMA fractions: torch's fused SDPA (flash backend, else
    memory-efficient; never math) on dense causal attention at long S, the
    same shapes' head dims and dtypes as the BASELINE configs. FLOPs: 4·D per
    causal (query, key) pair forward, 14·D forward+backward (the counts the
    sqrt(N) op's figures use); one JSON line per shape."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import sdpa_kernel
    dev = torch.device("cuda", 0)
    for (B, H, S, D, dtype) in ((1, 16, 16384, 128, torch.float16),
                                (1, 16, 32768, 128, torch.float16),
                                (2, 32, 8192, 128, torch.bfloat16),
                                (1, 12, 32768, 64, torch.float16)):
        g = torch.Generator(device=dev).manual_seed(0)
        q, k, v, do = (torch.randn(B, H, S, D, generator=g, device=dev, dtype=dtype)
                       for _ in range(4))
        backend = sdpa_backend(q, k, v, torch, F)
        if backend is None:
            print(json.dumps({"B": B, "H": H, "S": S, "D": D, "sdpa_backend": None}), flush=True)
            continue

        def fwd(a, b_, c):
            with sdpa_kernel([backend]):
                return F.scaled_dot_product_attention(a, b_, c, is_causal=True)

        st = torch.cuda.current_stream()
        with torch.no_grad():
            t_f = timed(lambda: fwd(q, k, v), args.steps, args.warmup, torch)
        qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))

        def step():
            qg.grad = kg.grad = vg.grad = None
            fwd(qg, kg, vg).backward(do)

        t_t = timed(step, args.steps, args.warmup, torch)
        pairs = S * (S + 1) // 2 * B * H
        ff, ft = 4 * D * pairs, 14 * D * pairs
        print(json.dumps({
            "B": B, "H": H, "S": S, "D": D, "dtype": str(dtype).split(".")[-1],
            "sdpa_backend": str(backend).split(".")[-1], "causal": True,
            "fwd_ms": round(t_f, 4), "fwd_tflops": round(ff / (t_f * 1e-3) / 1e12, 1),
            "fwd_frac": round(ff / (t_f * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
            "train_ms": round(t_t, 4), "train_tflops": round(ft / (t_t * 1e-3) / 1e12, 1),
            "train_frac": round(ft / (t_t * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4)}), flush=True)
        del q, k, v, do, qg, kg, vg
        torch.cuda.empty_cache()


def first_win(points, key_a, key_b):
    """Smallest S from which a is faster than b at every larger swept S."""
    win = None
    for pt in sorted(points, key=lambda x: -x["S"]):
        if pt.get(key_b) is None or pt[key_a] < pt[key_b]:
            win = pt["S"]
        else:
            break
    return win


def run_crossover(args):
    """S sweep of the sqrt(N) op against ROCm SDPA (causal), forward and
    forward+backward, for the BASELINE head shapes; one JSON line per point
    and one summary line per shape with the crossover S of each mode."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import sdpa_kernel
    import cron_root_attention as cra
    dev = torch.device("cuda", 0)
    shapes = ((2, 32, 128, torch.bfloat16), (1, 16, 128, torch.float16),
              (1, 8, 64, torch.float16), (1, 12, 64, torch.float16))
    seqs = (1, 2, 4, 8, 16, 32, 48, 64, 96, 128, 192, 256, 384, 512, 768, 1024, 1536, 2048,
            3072, 4096, 6144, 8192, 16384)
    for (B, H, D, dtype) in shapes:
        points = []
        backend = None
        for S in seqs:
            g = torch.Generator(device=dev).manual_seed(0)
            q, k, v, do = (torch.randn(B, H, S, D, generator=g, device=dev, dtype=dtype)
                           for _ in range(4))
            if backend is None:
                backend = sdpa_backend(q, k, v, torch, F)
            res = {"B": B, "H": H, "D": D, "S": S, "dtype": str(dtype).split(".")[-1],
                   "sdpa_backend": str(backend).split(".")[-1] if backend is not None else None}
            impls = [("cra", lambda a, b, c: cra.cron_root_attention(a, b, c))]
            if backend is not None:
                def sd(a, b, c, _b=backend):
                    with sdpa_kernel([_b]):
                        return F.scaled_dot_product_attention(a, b, c, is_causal=True)
                impls.append(("sdpa", sd))
            for name, fn in impls:
                with torch.no_grad():
                    res[f"{name}_fwd_ms"] = round(timed(lambda: fn(q, k, v), 20, 5, torch), 4)
                qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))

                def st():
                    qg.grad = kg.grad = vg.grad = None
                    fn(qg, kg, vg).backward(do)
                res[f"{name}_train_ms"] = round(timed(st, 10, 3, torch), 4)
            points.append(res)
            print(json.dumps(res), flush=True)
        summary = {"crossover": True, "B": B, "H": H, "D": D, "dtype": str(dtype).split(".")[-1],
                   "sdpa_backend": points[0]["sdpa_backend"], "swept_from_S": seqs[0]}
        for mode in ("fwd", "train"):
            w = first_win(points, f"cra_{mode}_ms", f"sdpa_{mode}_ms")
            summary[f"{mode}_crossover_S"] = w
            # a crossover is bracketed when SDPA wins at the swept S just below it
            summary[f"{mode}_kind"] = ("sqrt(N) op faster at every swept S" if w == seqs[0]
                                       else "no win in the sweep" if w is None else "bracketed")
        print(json.dumps(summary), flush=True)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--skip-cpu", action="store_true", help="omit the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--cpu-threads", type=int, default=None,
                    help="CPU baseline threads (default: OMP_NUM_THREADS, else all allowed CPUs)")
    ap.add_argument("--crossover", action="store_true")
    ap.add_argument("--sdpa-dense", action="store_true",
                    help="time torch's fused SDPA on dense causal attention at long S (context)")
    ap.add_argument("--config", default=None, metavar="N[,N]|all",
                    help="time the BASELINE configurations 2-5 at every listed S instead")
    ap.add_argument("--profile-workload", action="store_true",
                    help="copy calibration + hot-path kernels once, for counter passes")
    ap.add_argument("--counter-summary", nargs="+", metavar="DIR",
                    help="print a markdown summary of rocprofv3 --pmc output directories")
    ap.add_argument("--json-out", metavar="WORKLOAD", default=None,
                    help="with --counter-summary: also write profiles/executed_WORKLOAD.json and "
                         "profiles/phases_counters_WORKLOAD.json")
    ap.add_argument("--pw", default="1,16,131072,128", metavar="B,H,S,D",
                    help="shape of --profile-workload (fp16)")
    ap.add_argument("--pw-mode", default="all", choices=("all", "train", "fwd"),
                    help="what --profile-workload runs")
    ap.add_argument("--phases", default=None, metavar="S[,S]",
                    help="per-phase forward figures at B=1 H=16 D=128 fp16 for these S "
                         "(BASELINE config 3), one JSON line each")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "sharding across GPUs is design-only", file=sys.stderr)
        return 2
    if args.counter_summary:
        print(counter_summary(args.counter_summary))
        if args.json_out:
            ex, ph = counter_json(args.counter_summary, args.json_out)
            for name, obj in (("executed", ex), ("phases_counters", ph)):
                with open(os.path.join(ROOT, "profiles", f"{name}_{args.json_out}.json"), "w") as f:
                    json.dump(obj, f, indent=1)
                    f.write("\n")
        return 0
    if args.config:
        run_configs(args)
    elif args.crossover:
        run_crossover(args)
    elif args.sdpa_dense:
        run_sdpa_dense(args)
    elif args.profile_workload:
        run_profile_workload(args)
    elif args.phases:
        run_phases(args)
    else:
        run_main(args)
    return 0


if __name__ == "__main__":
    sys.exit(main())
