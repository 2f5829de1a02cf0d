"""Head dims above 128 against the fp64 oracle (GPU).

The reference takes any head dim (``BLOCK_D = triton.next_power_of_2(D)``,
core.py:3495). This build compiles D = 256 (every dtype; D in (128, 256] is
zero-padded to 256, scores keeping 1/sqrt(D) of the true D) on its generic
kernels with 16 queries or keys per wave. Forward element-wise and every
gradient against the oracle, as for the other head dims (tolerances in
``tests/parity_util.py``), at small shapes in full and at S = 32768 on
spot rows; GQA, relay top-k, relay_log_scale and use_persistent included.
"""
import math

import pytest
import torch

import cron_root_attention as cra
from oracle import cra_oracle as O
from tests.parity_util import (BF16, DEV, F16, F32, TOL_GRAD, TOL_LSE, check_forward,
                               check_grad_rows, device_inputs, inputs, max_abs, plan_for,
                               rel_fro, say, spot_ranges)

pytestmark = pytest.mark.gpu

CASES = [
    # dtype, B, Hq, Hkv, S, D, top_k, relay_log_scale
    (F16, 1, 2, 2, 700, 256, 2, False),      # no relay
    (BF16, 2, 4, 2, 3000, 256, 2, False),    # relay, GQA 2:1
    (F32, 1, 2, 1, 2500, 256, 3, True),      # fp32, GQA 2:1, learnable relay scale
    (F16, 1, 4, 4, 5000, 200, 1, False),     # padded to 256
    (BF16, 1, 2, 1, 9000, 256, 4, True),     # relay top-4 with scale
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-B{c[1]}-H{c[2]}x{c[3]}-S{c[4]}-D{c[5]}")
def test_wide_head_forward_backward(case):
    dt, B, Hq, Hkv, S, D, top_k, with_alpha = case
    say(f"wide head {case}")
    q, k, v, do = inputs(B, Hq, Hkv, S, D, dt, seed=S + D)
    plan = plan_for(S, top_k)
    alpha = torch.linspace(-0.25, 0.35, Hkv) if with_alpha else None
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    ad = alpha.to(DEV).requires_grad_(True) if alpha is not None else None
    o = cra.cron_root_attention(qd, kd, vd, kv_groups=Hq // Hkv, relay_log_scale=ad,
                                relay_top_k=top_k)
    kw = {}
    if alpha is not None and plan.relay:
        kw = dict(relay_scale=alpha.exp().to(dt).to(F32), relay_dtype=dt)
    check_forward(o, q, k, v, plan, dt, kv_groups=Hq // Hkv, **kw)
    o.backward(do.to(DEV))
    _, _, _, g = O.forward_backward(q, k, v, do, plan, kv_groups=Hq // Hkv,
                                    relay_log_scale=alpha if plan.relay else None)
    for name, got, ref in (("dq", qd.grad, g["dq"]), ("dk", kd.grad, g["dk"]),
                           ("dv", vd.grad, g["dv"])):
        e = rel_fro(got, ref)
        say(f"  {name}: rel {e:.3e}")
        assert e <= TOL_GRAD[dt], name
    if alpha is not None and plan.relay:
        e = rel_fro(ad.grad, g["dalpha"])
        say(f"  dalpha: rel {e:.3e}")
        assert e <= TOL_GRAD[dt]


def test_wide_head_long_sequence_rows():
    """B=1 H=4 S=32768 D=256 fp16: forward rows at the start, middle and end
    (lse too) and gradient rows (dQ ranges; local, strided and relay key
    rows) of two heads against the oracle; the backward is deterministic."""
    say("wide head S=32768 D=256 rows")
    B, H, S, D = 1, 4, 32768, 256
    q, k, v, do = device_inputs(B, H, H, S, D, F16, seed=11, with_do=True)
    plan = plan_for(S)
    res = []
    for _ in range(2):
        qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
        o = cra.cron_root_attention(qd, kd, vd)
        o.backward(do)
        res.append((o.detach(), qd.grad, kd.grad, vd.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)
    o, dq, dk, dv = res[0]
    heads = [0, H - 1]
    qc, kc, vc, oc = (t.cpu()[:, heads] for t in (q, k, v, o))
    for lo, hi in spot_ranges(S):
        say(f"  rows [{lo},{hi})")
        check_forward(oc[:, :, lo:hi], qc, kc, vc, plan, F16, rows=(lo, hi))
    check_grad_rows(q, k, v, do, dq, dk, dv, plan, 0, heads)


def test_wide_head_persistent_request():
    """use_persistent=True at D = 256 (S <= 2048, no relay) computes the same
    function as the tiled call and matches the oracle."""
    q, k, v, _ = inputs(1, 4, 4, 1800, 256, F16, seed=5)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    with torch.no_grad():
        a = cra.cron_root_attention(qd, kd, vd, use_persistent=True)
        b = cra.cron_root_attention(qd, kd, vd)
    assert torch.equal(a, b)
    check_forward(a.cpu(), q, k, v, plan_for(1800), F16)


def test_head_dim_above_256_is_refused():
    q = torch.randn(1, 2, 64, 264, device=DEV, dtype=F16)
    with pytest.raises(NotImplementedError):
        cra.cron_root_attention(q, q, q)
