"""BASELINE configurations 2-4 on the GPU against the fp64 oracle, at the
sizes the reference publishes (reference README.md:19-80, 97-107).

* config 2, B=1 H=8 D=64 fp16, forward: full oracle at S=2048 and 8192;
  at S=65536 and 262144 start/middle/end rows of heads 0 and 7 plus the
  relay selection of every head, bit for bit;
* config 3 at S=16384, B=1 H=16 D=128 fp16, forward: full oracle, every head;
* config 4, B=1 H=12 D=64 fp16, forward+backward: full fp64 autograd at
  S=8192; at S=32768 and 131072 forward rows plus the gradient spot rows
  (dQ ranges, dK/dV of local, strided, relay and doubled key rows) of heads
  0 and 11.

Config 5 (through CronRootAttention(hybrid=True)) is in test_module_gpu.py;
config 3 at S=131072 and 524288 in test_parity_gpu.py.
"""
import math

import pytest
import torch

import cron_root_attention as cra
from cron_root_attention import _native
from oracle import cra_oracle as O
from tests.parity_util import (F16, TOL_GRAD, check_forward, check_grad_rows, device_inputs,
                               inputs, plan_for, rel_fro, say, spot_ranges)

pytestmark = pytest.mark.gpu


def _relay_bit_exact(k, plan):
    B, H, S, D = k.shape
    p = _native.problem(B, H, H, S, D, plan.W, True, plan.top_k, k.dtype, 1 / math.sqrt(D))
    _, _, src = _native.build_global(p, k, k, None)
    ref = O.relay_select(k.cpu(), plan, "lanetree").to(torch.int32)
    assert torch.equal(src.cpu(), ref)
    return src


@pytest.mark.parametrize("S", [2048, 8192, 65536, 262144])
def test_config2_forward(S):
    B, H, D = 1, 8, 64
    say(f"config 2 forward B={B} H={H} D={D} S={S} fp16")
    plan = plan_for(S)
    if S <= 8192:
        q, k, v, _ = inputs(B, H, H, S, D, F16, seed=S)
        with torch.no_grad():
            o = cra.cron_root_attention(q.cuda(), k.cuda(), v.cuda())
        check_forward(o, q, k, v, plan, F16)
        return
    q, k, v = device_inputs(B, H, H, S, D, F16, seed=0)
    with torch.no_grad():
        o = cra.cron_root_attention(q, k, v)
    src = _relay_bit_exact(k, plan)
    heads = [0, 7]
    qc, kc, vc, oc = (t[:, heads].cpu() for t in (q, k, v, o))
    for lo, hi in spot_ranges(S):
        say(f"  rows [{lo},{hi})")
        check_forward(oc[:, :, lo:hi], qc, kc, vc, plan, F16, rows=(lo, hi),
                      src=src[:, heads].cpu().long())


def test_config3_forward_16k():
    B, H, S, D = 1, 16, 16384, 128
    say(f"config 3 forward B={B} H={H} D={D} S={S} fp16")
    q, k, v, _ = inputs(B, H, H, S, D, F16, seed=S)
    with torch.no_grad():
        o = cra.cron_root_attention(q.cuda(), k.cuda(), v.cuda())
    _relay_bit_exact(k.cuda(), plan_for(S))
    for h0 in range(0, H, 4):          # four heads per oracle call
        hs = list(range(h0, h0 + 4))
        say(f"  heads {hs}")
        check_forward(o[:, hs], q[:, hs], k[:, hs], v[:, hs], plan_for(S), F16)


def test_config4_training_8k_full_autograd():
    B, H, S, D = 1, 12, 8192, 64
    say(f"config 4 fwd+bwd B={B} H={H} D={D} S={S} fp16 (full fp64 autograd)")
    q, k, v, do = inputs(B, H, H, S, D, F16, seed=S + 4)
    qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
    o = cra.cron_root_attention(qd, kd, vd)
    o.backward(do.cuda())
    check_forward(o, q, k, v, plan_for(S), F16)
    _, _, _, g = O.forward_backward(q, k, v, do, plan_for(S))
    for name, hip, ref in (("dq", qd.grad, g["dq"]), ("dk", kd.grad, g["dk"]),
                           ("dv", vd.grad, g["dv"])):
        e = rel_fro(hip, ref)
        say(f"  {name}: rel = {e:.3e}")
        assert e <= TOL_GRAD[F16], name
        for h in range(H):      # every head on its own, too
            assert rel_fro(hip[:, h], ref[:, h]) <= TOL_GRAD[F16], (name, h)


@pytest.mark.parametrize("S", [32768, 131072])
def test_config4_training_rows(S):
    B, H, D = 1, 12, 64
    say(f"config 4 fwd+bwd B={B} H={H} D={D} S={S} fp16 (spot rows)")
    q, k, v, do = device_inputs(B, H, H, S, D, F16, seed=0, with_do=True)
    plan = plan_for(S)
    doubled = plan.num_blocks // 3 * plan.W
    for h in (0, 11):
        k[:, h, doubled] *= 3
    qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = cra.cron_root_attention(qd, kd, vd)
    o.backward(do)
    for t in (o, qd.grad, kd.grad, vd.grad):
        assert bool(torch.isfinite(t).all())
    heads = [0, 11]
    qc, kc, vc, oc = (t[:, heads].detach().cpu() for t in (q, k, v, o))
    for lo, hi in spot_ranges(S):
        say(f"  forward rows [{lo},{hi})")
        check_forward(oc[:, :, lo:hi], qc, kc, vc, plan, F16, rows=(lo, hi))
    check_grad_rows(q, k, v, do, qd.grad, kd.grad, vd.grad, plan, 0, heads, doubled=doubled)
