"""Shared checks of the GPU parity tests: seeded inputs, the element-wise
forward check and the gradient spot checks against the fp64 oracle.

Tolerances (the north star's fp16 figures; bf16/fp32 scaled to their
precision):
  forward  fp16: max |o - o_ref| <= 2e-3, asserted as written.
           bf16/fp32: |o - o_ref| <= max(TOL, bound) per element, TOL = 1.6e-2 /
           2e-5 (bf16: 4 unit roundoffs of 2^-8, the fp16 contract's 2e-3 =
           4 x 2^-11 scaled to bf16), and mean |o - o_ref| <= mean(bound) / 2.
  lse      fp16 1e-3, bf16 4e-3, fp32 1e-5 (max-abs; the normaliser sums the
           rounded P, so ln l moves by up to one unit roundoff).
  backward ||g - g_ref|| / ||g_ref||  fp16 1e-2, bf16 3e-2, fp32 1e-4, per
           gradient tensor (full checks) or per row / row range (spot checks).
bound = 1.05 u (P|v| + |o|) + 1e-6 is the first-order error of any kernel that
rounds P to the input dtype before P.V (as the reference does, core.py:1027,
1086, 1141) and rounds O once (core.py:1155); u is the unit roundoff (2^-11
fp16, 2^-8 bf16).  It is printed for every case as a diagnostic.
The oracle runs in fp64 on the inputs already rounded to the test dtype.
"""
import math
import sys

import numpy as np
import torch

from oracle import cra_oracle as O

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32
TOL_FWD = {F16: 2e-3, BF16: 1.6e-2, F32: 2e-5}
TOL_GRAD = {F16: 1e-2, BF16: 3e-2, F32: 1e-4}
# LSE (internal, saved for the backward): the kernels' normaliser sums the
# rounded P that the P.V products use, so ln(l) may differ from the exact
# log-sum-exp by up to one unit roundoff of the type (2^-11 fp16, 2^-8 bf16)
TOL_LSE = {F16: 1e-3, BF16: 4e-3, F32: 1e-5}
UNIT_ROUNDOFF = {F16: 2.0 ** -11, BF16: 2.0 ** -8, F32: 2.0 ** -24}
DEV = "cuda"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def rand(shape, dtype, gen):
    return torch.randn(*shape, generator=gen, dtype=torch.float32).to(dtype)


def inputs(B, Hq, Hkv, S, D, dtype, seed):
    """CPU generator, draws q, k, v, dO in that order (fp32, then rounded)."""
    g = torch.Generator().manual_seed(seed)
    q = rand((B, Hq, S, D), dtype, g)
    k = rand((B, Hkv, S, D), dtype, g)
    v = rand((B, Hkv, S, D), dtype, g)
    do = rand((B, Hq, S, D), dtype, g)
    return q, k, v, do


def device_inputs(B, Hq, Hkv, S, D, dtype, seed=0, with_do=False):
    """Large shapes: on-device generator, same draw order (q, k, v, dO)."""
    gen = torch.Generator(device=DEV).manual_seed(seed)
    mk = lambda H: torch.randn(B, H, S, D, generator=gen, device=DEV,
                               dtype=torch.float32).to(dtype)
    q, k, v = mk(Hq), mk(Hkv), mk(Hkv)
    return (q, k, v, mk(Hq)) if with_do else (q, k, v)


def plan_for(S, top_k=2):
    return O.Plan(S, O.window_size(S), S > 2048, top_k)


def max_abs(a, b):
    return float((a.detach().cpu().double() - b.detach().cpu().double()).abs().max())


def rel_fro(a, b):
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def check_forward(o, q, k, v, plan, dtype, kv_groups=1, rows=None, **kw):
    """Element-wise forward check against the fp64 oracle (see module doc)."""
    ref, ref_lse, _ = O.forward(q, k, v, plan, kv_groups=kv_groups, rows=rows, **kw)
    pv, _, _ = O.forward(q, k, v.abs(), plan, kv_groups=kv_groups, rows=rows, **kw)  # P|v|
    err = (o.detach().cpu().double() - ref).abs()
    bound = 1.05 * UNIT_ROUNDOFF[dtype] * (pv + ref.abs()) + 1e-6
    tol = TOL_FWD[dtype]
    say(f"  max err {float(err.max()):.3e}  mean {float(err.mean()):.3e}  "
        f"rounding-model bound max {float(bound.max()):.3e}  "
        f"> {tol:g}: {int((err > tol).sum())}/{err.numel()}")
    if dtype == F16:
        assert float(err.max()) <= tol, float(err.max())
    else:
        assert bool((err <= torch.clamp(bound, min=tol)).all()), float((err - bound).max())
    assert float(err.mean()) <= 0.5 * float(bound.mean())
    return ref, ref_lse


def spot_ranges(S, n=256):
    """Start, middle and end row ranges of a sequence."""
    n = min(n, S)
    mid = max(0, S // 2 - n // 2)
    return sorted({(0, n), (mid, mid + n), (S - n, S)})


def spot_keys(plan, src_row, doubled=None):
    """Key rows covering every way a key is reached: a local-only row, the
    strided rows r*W at the start, middle and end, several relay source rows,
    and (``doubled``) a strided row that is also its block's top relay row."""
    W, NB = plan.W, plan.num_blocks
    keys = []
    srcs = [int(x) for x in src_row] if src_row is not None else []
    src_set = set(srcs)
    j = W + 5
    while j % W == 0 or j in src_set:
        j += 1
    keys.append(j)                                                   # local only
    keys += [0, W, (NB // 2) * W, (NB - 2) * W, (NB - 1) * W]          # strided
    if srcs:
        picks = [srcs[0], srcs[1], srcs[len(srcs) // 2], srcs[len(srcs) // 2 + 1],
                 srcs[-2 * plan.top_k], srcs[-2 * plan.top_k + 1]]
        keys += [s for s in picks if s % W]                           # relay sources
    if doubled is not None:
        keys.append(doubled)
    return sorted(set(k for k in keys if 0 <= k < plan.S))


def check_grad_rows(q, k, v, do, dq, dk, dv, plan, b, heads, kv_groups=1, doubled=None,
                    src=None, tol=1e-2):
    """Gradient spot check of one batch entry at full size (fp64 oracle):
    dQ on three 256-row ranges of every query head in ``heads`` and dK/dV on
    the rows of :func:`spot_keys` of their kv heads, each row range / row
    within relative error ``tol``.  Inputs are GPU tensors; only the heads
    involved are copied to the host."""
    kvh = sorted({h // kv_groups for h in heads})
    qh = sorted({hq for g in kvh for hq in range(g * kv_groups, (g + 1) * kv_groups)})
    qc = q[b:b + 1, qh].detach().cpu()
    doc = do[b:b + 1, qh].detach().cpu()
    kc = k[b:b + 1, kvh].detach().cpu()
    vc = v[b:b + 1, kvh].detach().cpu()
    if plan.relay:
        src_c = (src[b:b + 1, kvh].detach().cpu().long() if src is not None
                 else O.relay_select(kc, plan))
    else:
        src_c = None
    o, lse, _ = O.forward(qc, kc, vc, plan, kv_groups=kv_groups, src=src_c, chunk=1024)
    delta = (o * doc.double()).sum(-1)
    worst = 0.0
    for h in heads:
        hl = qh.index(h)
        for lo, hi in spot_ranges(plan.S):
            ref = O.query_row_grads(qc[:, hl:hl + 1], kc[:, [kvh.index(h // kv_groups)]],
                                    vc[:, [kvh.index(h // kv_groups)]], doc[:, hl:hl + 1],
                                    plan, (lo, hi),
                                    src=src_c[:, [kvh.index(h // kv_groups)]]
                                    if src_c is not None else None)
            e = rel_fro(dq[b, h, lo:hi], ref[0, 0])
            worst = max(worst, e)
            assert e <= tol, f"dq head {h} rows [{lo},{hi}): rel {e:.3e}"
    for gl, g in enumerate(kvh):
        rows = spot_keys(plan, src_c[0, gl] if src_c is not None else None,
                         doubled=doubled)
        res = O.key_row_grads(qc, kc, vc, doc, plan, [(0, gl, j) for j in rows], lse, delta,
                              src_c, kv_groups)
        for (_, _, j), (rk, rv) in res.items():
            ek = rel_fro(dk[b, g, j], rk)
            ev = rel_fro(dv[b, g, j], rv)
            worst = max(worst, ek, ev)
            assert ek <= tol and ev <= tol, f"kv head {g} key {j}: dk {ek:.3e} dv {ev:.3e}"
    say(f"  grad spot rows: worst relative error {worst:.3e}")
    return worst
