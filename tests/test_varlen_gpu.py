"""Packed documents (varlen) on the GPU: one set of launches over every
document against the reference's semantics, one op call per document
(reference core.py:3911-3952).

* forward: bit-identical to the plain op run on each document alone (the
  kernels do the same arithmetic per document), and within the forward
  tolerance of the fp64 oracle (``forward_varlen``);
* backward: dQ bit-identical per document; dK/dV equal to the per-document
  calls up to the fp32 summation order of the global-row partials (the
  packed call cuts queries into a number of chunks chosen over all
  documents): relative Frobenius error <= REL_SPLIT; all gradients within
  the backward tolerance of the oracle; d(relay_log_scale) sums the
  documents.
More than 64 documents run as several launches of each kernel (one per
group of 64); those cases cover the group boundary.
"""
import math
import random
import sys

import pytest
import torch

import cron_root_attention as cra
from cron_root_attention.core import _attention_with_plan, _varlen_with_plan, window_size
from oracle import cra_oracle as O

pytestmark = pytest.mark.gpu

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32
TOL_FWD = {F16: 2e-3, BF16: 1.6e-2, F32: 2e-5}  # bf16: 4 unit roundoffs, as fp16's 2e-3
TOL_GRAD = {F16: 1e-2, BF16: 3e-2, F32: 1e-4}
UNIT_ROUNDOFF = {F16: 2.0 ** -11, BF16: 2.0 ** -8, F32: 2.0 ** -24}
REL_SPLIT = {F16: 2e-3, BF16: 1.5e-2, F32: 1e-5}
DEV = "cuda"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def inputs(B, Hq, Hkv, S, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float32).to(dtype)
    return r(B, Hq, S, D), r(B, Hkv, S, D), r(B, Hkv, S, D), r(B, Hq, S, D)


def rel_fro(a, b):
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def cu_of(lengths):
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return cu


def per_document(q, k, v, cu, kv_groups=1, windows=None, relays=None, alpha=None, do=None,
                 top_k=2):
    """The reference's varlen: the plain op once per document (contiguous
    copies, so that nothing but the document is visible to the kernels)."""
    outs, grads, dalpha = [], [], None
    for d, (s, e) in enumerate(zip(cu, cu[1:])):
        qs, ks, vs = (t[:, :, s:e].contiguous().requires_grad_(do is not None) for t in (q, k, v))
        a = alpha.detach().clone().requires_grad_(True) if alpha is not None else None
        if windows is None:
            o = cra.cron_root_attention(qs, ks, vs, kv_groups=kv_groups, relay_log_scale=a,
                                        relay_top_k=top_k)
        else:
            o = _attention_with_plan(qs, ks, vs, windows[d], relays[d], kv_groups, a, top_k)
        outs.append(o.detach())
        if do is not None:
            o.backward(do[:, :, s:e])
            grads.append((qs.grad, ks.grad, vs.grad))
            if a is not None and a.grad is not None:
                dalpha = a.grad.clone() if dalpha is None else dalpha + a.grad
    return outs, grads, dalpha


def check_oracle_forward(o, q, k, v, cu, dtype, kv_groups, plans=None, alpha=None):
    """``alpha``: the relay_log_scale of the call; the op scales relay rows by
    exp(alpha) rounded to the input dtype and rounds the scaled rows too."""
    kw = {}
    if alpha is not None:
        kw = dict(relay_scale=alpha.exp().to(dtype).to(F32), relay_dtype=dtype)
    ref, _, _ = O.forward_varlen(q.cpu(), k.cpu(), v.cpu(), cu, plans, kv_groups, **kw)
    pv, _, _ = O.forward_varlen(q.cpu(), k.cpu(), v.cpu().abs(), cu, plans, kv_groups, **kw)
    err = (o.detach().cpu().double() - ref).abs()
    bound = 1.05 * UNIT_ROUNDOFF[dtype] * (pv + ref.abs()) + 1e-6
    say(f"  oracle: max err {float(err.max()):.3e}")
    assert bool((err <= torch.clamp(bound, min=TOL_FWD[dtype])).all())


FWD_CASES = [
    # dtype, B, Hq, Hkv, D, document lengths
    (F16, 1, 2, 2, 128, [700, 1, 64, 2500, 65, 129]),
    (BF16, 2, 4, 2, 64, [3000, 63, 2049, 300]),
    (F32, 1, 2, 1, 32, [100, 2100, 17]),
    (F16, 1, 4, 4, 96, [128, 2300, 999]),
    (BF16, 1, 2, 2, 256, [900, 2100, 33]),     # head dim 256 (generic kernels)
]


@pytest.mark.parametrize("case", FWD_CASES, ids=lambda c: f"{c[0]}-D{c[4]}-{len(c[5])}docs")
def test_varlen_forward_equals_per_document_and_oracle(case):
    dtype, B, Hq, Hkv, D, lengths = case
    say(f"varlen forward {case}")
    cu = cu_of(lengths)
    q, k, v, _ = inputs(B, Hq, Hkv, cu[-1], D, dtype, seed=sum(lengths) + D)
    qd, kd, vd = (t.to(DEV) for t in (q, k, v))
    o = cra.cron_root_attention_varlen(qd, kd, vd, torch.tensor(cu), kv_groups=Hq // Hkv)
    assert o.shape == q.shape and o.dtype == dtype
    ref, _, _ = per_document(qd, kd, vd, cu, Hq // Hkv)
    for d, (s, e) in enumerate(zip(cu, cu[1:])):
        assert torch.equal(o[:, :, s:e], ref[d]), f"document {d} ({e - s} rows)"
    check_oracle_forward(o, q, k, v, cu, dtype, Hq // Hkv)


def test_varlen_forward_strided_views():
    """q/k/v as [B, S, H, D] transposes (the layout a projection produces)."""
    say("varlen strided views")
    lengths = [900, 2200, 31]
    cu = cu_of(lengths)
    B, H, D, S = 1, 4, 64, cu[-1]
    g = torch.Generator().manual_seed(3)
    x = [torch.randn(B, S, H, D, generator=g).to(F16).to(DEV) for _ in range(3)]
    q, k, v = (t.transpose(1, 2) for t in x)
    o = cra.cron_root_attention_varlen(q, k, v, cu)
    oc = cra.cron_root_attention_varlen(q.contiguous(), k.contiguous(), v.contiguous(), cu)
    assert torch.equal(o, oc)


BWD_CASES = [
    (F16, 1, 2, 2, 128, [700, 1, 2500, 65]),
    (BF16, 1, 4, 2, 64, [2049, 300, 64, 1000]),
    (F32, 2, 2, 1, 32, [100, 2100, 17]),
    (F16, 1, 2, 1, 256, [1500, 2200, 40]),     # head dim 256 (generic kernels)
]


@pytest.mark.parametrize("case", BWD_CASES, ids=lambda c: f"{c[0]}-D{c[4]}-{len(c[5])}docs")
def test_varlen_backward_matches_per_document_and_oracle(case):
    dtype, B, Hq, Hkv, D, lengths = case
    say(f"varlen backward {case}")
    cu = cu_of(lengths)
    q, k, v, do = inputs(B, Hq, Hkv, cu[-1], D, dtype, seed=sum(lengths) * 3 + D)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    dod = do.to(DEV)
    cra.cron_root_attention_varlen(qd, kd, vd, cu, kv_groups=Hq // Hkv).backward(dod)
    _, grads, _ = per_document(q.to(DEV), k.to(DEV), v.to(DEV), cu, Hq // Hkv, do=dod)
    for d, (s, e) in enumerate(zip(cu, cu[1:])):
        gq, gk, gv = grads[d]
        assert torch.equal(qd.grad[:, :, s:e], gq), f"dq document {d}"
        for name, mine, ref in (("dk", kd.grad, gk), ("dv", vd.grad, gv)):
            err = rel_fro(mine[:, :, s:e], ref)
            assert err <= REL_SPLIT[dtype], (name, d, err)
    _, _, _, g = O.forward_backward_varlen(q, k, v, do, cu, kv_groups=Hq // Hkv)
    for name, mine in (("dq", qd.grad), ("dk", kd.grad), ("dv", vd.grad)):
        e = rel_fro(mine, g[name])
        say(f"  {name}: rel = {e:.3e}")
        assert e <= TOL_GRAD[dtype], name


def test_varlen_relay_log_scale_gradient():
    say("varlen relay_log_scale")
    lengths = [2500, 400, 3100]
    cu = cu_of(lengths)
    B, H, D = 1, 2, 64
    q, k, v, do = inputs(B, H, H, cu[-1], D, F32, seed=21)
    alpha = torch.tensor([0.3, -0.25])
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    ad = alpha.to(DEV).requires_grad_(True)
    cra.cron_root_attention_varlen(qd, kd, vd, cu, relay_log_scale=ad).backward(do.to(DEV))
    _, _, _, g = O.forward_backward_varlen(q, k, v, do, cu, relay_log_scale=alpha)
    for name, mine in (("dq", qd.grad), ("dk", kd.grad), ("dv", vd.grad), ("dalpha", ad.grad)):
        e = rel_fro(mine, g[name])
        say(f"  {name}: rel = {e:.3e}")
        assert e <= 1e-4, name


@pytest.mark.parametrize("dtype", [F16, F32])
def test_varlen_many_documents_span_launch_groups(dtype):
    """150 documents (three launch groups), relay forced on with small
    windows so that every group has relay rows and d(alpha) accumulates
    across groups."""
    say(f"varlen 150 documents {dtype}")
    rng = random.Random(5)
    lengths = [rng.randint(1, 90) for _ in range(148)] + [600, 1500]
    cu = cu_of(lengths)
    W = [max(1, int(math.isqrt(n))) for n in lengths]
    R = [n >= 4 for n in lengths]
    B, H, D = 1, 2, 64
    q, k, v, do = inputs(B, H, H, cu[-1], D, dtype, seed=77)
    alpha = torch.tensor([0.2, -0.1])
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    ad = alpha.to(DEV).requires_grad_(True)
    o = _varlen_with_plan(qd, kd, vd, cu, W, R, relay_log_scale=ad)
    o.backward(do.to(DEV))
    outs, grads, dalpha = per_document(q.to(DEV), k.to(DEV), v.to(DEV), cu, windows=W, relays=R,
                                       alpha=alpha.to(DEV), do=do.to(DEV))
    for d, (s, e) in enumerate(zip(cu, cu[1:])):
        assert torch.equal(o[:, :, s:e].detach(), outs[d]), f"o document {d}"
        assert torch.equal(qd.grad[:, :, s:e], grads[d][0]), f"dq document {d}"
    dk_ref = torch.cat([g[1] for g in grads], 2)
    dv_ref = torch.cat([g[2] for g in grads], 2)
    assert rel_fro(kd.grad, dk_ref) <= REL_SPLIT[dtype]
    assert rel_fro(vd.grad, dv_ref) <= REL_SPLIT[dtype]
    assert rel_fro(ad.grad, dalpha) <= (1e-4 if dtype == F32 else 1e-2)
    plans = [O.Plan(n, w, r, 2) for n, w, r in zip(lengths, W, R)]
    check_oracle_forward(o, q, k, v, cu, dtype, 1, plans, alpha=alpha)


def test_varlen_single_document_is_the_plain_op():
    q, k, v, _ = inputs(1, 2, 2, 3000, 64, F16, seed=8)
    qd, kd, vd = (t.to(DEV) for t in (q, k, v))
    assert torch.equal(cra.cron_root_attention_varlen(qd, kd, vd, [0, 3000]),
                       cra.cron_root_attention(qd, kd, vd))


def test_varlen_deterministic():
    lengths = [3000, 120, 2600]
    cu = cu_of(lengths)
    q, k, v, do = inputs(1, 4, 4, cu[-1], 128, F16, seed=13)
    res = []
    for _ in range(2):
        qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
        cra.cron_root_attention_varlen(qd, kd, vd, cu).backward(do.to(DEV))
        res.append((qd.grad.clone(), kd.grad.clone(), vd.grad.clone()))
    for a, b in zip(*res):
        assert torch.equal(a, b)
