"""Seeded random sweep of the public op against the fp64 oracle: batch, GQA
group, sequence length (window and relay switch follow), head dim (padded or
not), dtype, relay top-k, relay_log_scale and memory layout all drawn per
case, forward and backward, through whichever path the public op takes (the
C++ operator or the Python Function).  Every draw is printed before it runs."""
import random

import pytest
import torch

import cron_root_attention as cra
from oracle import cra_oracle as O
from parity_util import (BF16, DEV, F16, F32, TOL_GRAD, check_forward, inputs, plan_for,
                         rel_fro, say)

pytestmark = pytest.mark.gpu


def _draw(seed):
    r = random.Random(seed)
    hkv = r.choice([1, 2])
    grp = r.choice([1, 2, 4])
    S = r.choice([r.randint(1, 300), r.randint(300, 2048), r.randint(2049, 4200)])
    return dict(B=r.choice([1, 2]), Hkv=hkv, Hq=hkv * grp, S=S,
                D=r.choice([16, 32, 40, 64, 72, 96, 128]),
                dtype=r.choice([F16, F16, BF16]),
                top_k=r.choice([1, 2, 2, 3, 4]),
                alpha=r.random() < 0.5,
                layout=r.choice(["bhsd", "bshd"]))


@pytest.mark.parametrize("seed", list(range(16)))
def test_random_case_forward_backward(seed):
    c = _draw(seed)
    say(f"random case {seed}: {c}")
    B, Hq, Hkv, S, D, dt = c["B"], c["Hq"], c["Hkv"], c["S"], c["D"], c["dtype"]
    q, k, v, do = inputs(B, Hq, Hkv, S, D, dt, seed=1000 + seed)
    plan = plan_for(S, c["top_k"])
    alpha = (torch.linspace(-0.3, 0.4, Hkv) if c["alpha"] else None)

    def dev(t):
        if c["layout"] == "bshd":   # [B, S, H, D] memory viewed as [B, H, S, D]
            t = t.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
        else:
            t = t.to(DEV)
        return t.requires_grad_(True)

    qd, kd, vd = dev(q), dev(k), dev(v)
    ad = alpha.to(DEV).requires_grad_(True) if alpha is not None else None
    o = cra.cron_root_attention(qd, kd, vd, kv_groups=Hq // Hkv, relay_log_scale=ad,
                                relay_top_k=c["top_k"])
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
        say(f"  {name}: rel = {e:.3e}")
        assert e <= TOL_GRAD[dt], name
    if alpha is not None:
        if plan.relay:
            e = rel_fro(ad.grad, g["dalpha"])
            say(f"  dalpha: rel = {e:.3e}")
            assert e <= TOL_GRAD[dt]
        else:
            assert ad.grad is None or float(ad.grad.abs().max()) == 0.0
