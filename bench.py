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
  cpu_baseline the oracle's chunked CPU port on the host cores, on a bounded
               sample of query rows of the same workload, as TFLOP/s

``--crossover`` instead sweeps S against torch's SDPA (forward and fwd+bwd)
and prints one JSON line per point.
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


def cpu_baseline(B, H, S, D, budget_s: float, threads: int):
    """Oracle CPU port (fp32 forward) on the host cores: pairs of heads of the
    same workload, each over all S queries, until ~budget_s of CPU time (or
    all H heads); returns effective TFLOP/s over the rows done."""
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
        src = O.relay_select(k, plan, "lanetree")
        t0 = time.perf_counter()
        cra_cpu_chunked(q, k, v, plan, src=src)
        t_used += time.perf_counter() - t0
        heads_done += Hs
        flops += 4 * D * pairs_fast(S) * Hs
    return {"value": flops / t_used / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"fp32 forward of {heads_done} of {H} heads (all {S} queries each), "
                      f"D={D}, {t_used:.1f} s",
            "seconds": round(t_used, 2)}


def traffic_for(kernel: str, workload: str):
    path = os.path.join(ROOT, "profiles", f"traffic_{kernel}_{workload}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


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

    # per-phase forward (cra_fwd_phases) and the global-row build (K1)
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
    f_rel = 4 * D * pp["relay"] * B * H
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
        "relay": {"ms": round(t_rel, 4), "pairs_per_head": pp["relay"],
                  "tflops": round(f_rel / (t_rel * 1e-3) / 1e12, 2) if t_rel > 0 else None,
                  "mfma_frac": (round(f_rel / (t_rel * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4)
                                if t_rel > 0 else None),
                  "how": "global phase minus strided-only"},
        "build_global": {"ms": round(t_bg, 4), "bytes": bg_bytes,
                         "GBps": round(bg_bytes / (t_bg * 1e-3) / 1e9, 1),
                         "hbm_frac": round(bg_bytes / (t_bg * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
    }

    cpu = None
    if not args.skip_cpu:
        cpu = cpu_baseline(B, H, S, D, args.cpu_seconds, args.cpu_threads)

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
        "roofline": roof, "phases": phases, "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def run_profile_workload(args):
    """Short fixed workload for counter passes (rocprofv3 --pmc): a 1 GiB
    device copy first (read 1 GiB + write 1 GiB, the calibration of
    FETCH_SIZE / WRITE_SIZE), then the hot path's kernels: build_global and
    cra_fwd twice each, then one backward."""
    import torch
    from cron_root_attention import _native
    dev = torch.device("cuda", 0)
    x = torch.empty(512 * 1024 * 1024, dtype=torch.float16, device=dev).fill_(1.0)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    y.copy_(x)
    torch.cuda.synchronize()
    del x, y
    B, H, S, D = 1, 16, 131072, 128
    gen = torch.Generator(device=dev).manual_seed(0)
    q, k, v, do = (torch.randn(B, H, S, D, generator=gen, device=dev, dtype=torch.float32).half()
                   for _ in range(4))
    W = int(math.ceil(math.sqrt(S)))
    p = _native.problem(B, H, H, S, D, W, True, 2, torch.float16, 1 / math.sqrt(D))
    for _ in range(2):
        gk, gv, src = _native.build_global(p, k, v, None)
        o, lse = _native.forward(p, q, k, v, gk, gv)
    _native.backward(p, q, k, v, o, do, lse, gk, gv, src, None, False)
    torch.cuda.synchronize()
    print(json.dumps({"profile_workload": "done", "B": B, "H": H, "S": S, "D": D}), flush=True)


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
    seqs = (256, 384, 512, 768, 1024, 1536, 2048, 3072, 4096, 6144, 8192, 16384)
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
                   "sdpa_backend": points[0]["sdpa_backend"],
                   "fwd_crossover_S": first_win(points, "cra_fwd_ms", "sdpa_fwd_ms"),
                   "train_crossover_S": first_win(points, "cra_train_ms", "sdpa_train_ms")}
        print(json.dumps(summary), flush=True)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--skip-cpu", action="store_true", help="omit the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--crossover", action="store_true")
    ap.add_argument("--profile-workload", action="store_true",
                    help="copy calibration + hot-path kernels once, for counter passes")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "sharding across GPUs is design-only", file=sys.stderr)
        return 2
    if args.crossover:
        run_crossover(args)
    elif args.profile_workload:
        run_profile_workload(args)
    else:
        run_main(args)
    return 0


if __name__ == "__main__":
    sys.exit(main())
