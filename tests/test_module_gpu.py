"""Hybrid dispatch, modules and BASELINE config 5 against the oracle (GPU).

Each module's attention output is captured at the input of its output
projection (a forward hook) and compared with the fp64 oracle fed the
module's own q/k/v projections (above the crossover) or with fp64 causal
attention (below it); the backend the dispatcher reports is asserted, and
the captured tensor must be far from the other backend's result, so the
comparison itself shows which one ran.  Reference: hybrid.py:25-124,
module.py:20-247.
"""
import math

import pytest
import torch
import torch.nn.functional as F

import cron_root_attention as cra
from cron_root_attention.hybrid import crossover, dispatch_backend
from oracle import cra_oracle as O
from tests.parity_util import (BF16, DEV, F16, F32, TOL_GRAD, check_forward, inputs,
                               plan_for, rel_fro, say, spot_ranges)

pytestmark = pytest.mark.gpu


def _capture(linear):
    box = []
    h = linear.register_forward_hook(lambda m, inp, out: box.append(inp[0].detach()))
    return box, h


def _heads(x, B, S, H, D):
    return x.view(B, S, H, D).transpose(1, 2)


def _check_backend(attn, q, k, v, backend, dtype, heads, kv_groups=1):
    """attn/q/k/v: GPU [B, H, S, D]; heads: list of (b, h) to compare."""
    S = q.shape[2]
    plan = plan_for(S)
    for b, h in heads:
        g = h // kv_groups
        qc = q[b:b + 1, h:h + 1].float().cpu().to(dtype)
        kc = k[b:b + 1, g:g + 1].float().cpu().to(dtype)
        vc = v[b:b + 1, g:g + 1].float().cpu().to(dtype)
        ac = attn[b:b + 1, h:h + 1].cpu()
        say(f"  b={b} h={h} backend={backend}")
        if backend == "sdpa":
            ref = O.causal_sdpa_reference(qc, kc, vc)
            tol = {F16: 2e-3, BF16: 3e-2, F32: 1e-4}[dtype]
            assert float((ac.double() - ref).abs().max()) <= tol
            other, _, _ = O.forward(qc, kc, vc, plan)
            assert float((ac.double() - other).abs().max()) > 3 * tol
        else:
            ranges = [(0, S)] if S <= 4096 else spot_ranges(S)
            for lo, hi in ranges:
                check_forward(ac[:, :, lo:hi], qc, kc, vc, plan, dtype, rows=(lo, hi))
            if S <= 4096:
                other = O.causal_sdpa_reference(qc, kc, vc)
                assert float((ac.double() - other).abs().max()) > 0.1


# ------------------------------------------------------------ config 5

CFG5 = [512, 1024, 2048, 4096, 65536, 262144]


@pytest.mark.parametrize("training", [False, True], ids=["eval", "train"])
@pytest.mark.parametrize("S", CFG5)
def test_config5_module_hybrid(S, training):
    """B=2 H=32 D=128 bf16 through CronRootAttention(hybrid=True): the
    dispatcher's choice per S (the gfx950 table's crossover for B*H = 64) and
    the result of whichever backend ran."""
    B, H, D = 2, 32, 128
    E = H * D
    say(f"config 5 module hybrid S={S} {'train' if training else 'eval'}")
    torch.manual_seed(0)
    m = cra.CronRootAttention(E, H, hybrid=True).to(DEV, BF16).train(training)
    gen = torch.Generator(device=DEV).manual_seed(S)
    x = torch.randn(B, S, E, generator=gen, device=DEV).to(BF16).requires_grad_(training)
    box, hook = _capture(m.o_proj)
    grads, ghooks = _capture_grads(m) if training else ({}, [])
    with torch.set_grad_enabled(training):
        y = m(x)
    hook.remove()
    backend = m.backend_for(x)
    with torch.no_grad():
        expect = "cron_root" if S >= crossover(D, training, B * H) else "sdpa"
        assert backend == expect
        assert S < 1024 or backend == "cron_root"
        attn = _heads(box[0], B, S, H, D)
        assert torch.equal(y, m.o_proj(box[0]))
        q = _heads(m.q_proj(x), B, S, H, D)
        k = _heads(m.k_proj(x), B, S, H, D)
        v = _heads(m.v_proj(x), B, S, H, D)
        _check_backend(attn, q, k, v, backend, BF16, [(0, 0), (1, 31)])
    if training:
        gy = torch.randn(y.shape, generator=gen, device=DEV).to(BF16)
        y.backward(gy)
        for h in ghooks:
            h.remove()
        assert bool(torch.isfinite(x.grad).all())
        for p in m.parameters():
            assert bool(torch.isfinite(p.grad).all())
        if backend == "cron_root" and S <= 4096:
            _check_attention_grads(q, k, v, grads, B, S, H, D, [(0, 0), (1, 31)])


def _capture_grads(m):
    """Gradients reaching the attention op: dL/dq, dL/dk, dL/dv (the outputs
    of the three projections) and dL/d(attention output) (the input of the
    output projection)."""
    grads = {}
    hooks = []
    for name, lin in (("dq", m.q_proj), ("dk", m.k_proj), ("dv", m.v_proj)):
        def fwd(mod, inp, out, name=name):
            if out.requires_grad:  # not the test's own recomputation under no_grad
                out.register_hook(lambda g, name=name: grads.__setitem__(name, g.detach()))
        hooks.append(lin.register_forward_hook(fwd))
    hooks.append(m.o_proj.register_full_backward_hook(
        lambda mod, gin, gout: grads.__setitem__("do", gin[0].detach())))
    return grads, hooks


def _check_attention_grads(q, k, v, grads, B, S, H, D, heads):
    """The sqrt(N) op's backward inside the module against the fp64 oracle:
    the q/k/v gradients of each (b, h) in ``heads`` from the attention inputs
    and output gradient the module produced (bf16), relative error within
    the bf16 gradient tolerance."""
    plan = plan_for(S)
    hd = lambda t: t.view(B, S, H, D).transpose(1, 2)
    dq, dk, dv, do = (hd(grads[n]) for n in ("dq", "dk", "dv", "do"))
    for b, h in heads:
        sl = lambda t: t[b:b + 1, h:h + 1].float().cpu().to(BF16)
        _, _, _, g = O.forward_backward(sl(q), sl(k), sl(v), sl(do), plan)
        for name, t in (("dq", dq), ("dk", dk), ("dv", dv)):
            e = rel_fro(t[b:b + 1, h:h + 1], g[name])
            say(f"  b={b} h={h} {name}: rel {e:.2e}")
            assert e <= TOL_GRAD[BF16], (b, h, name, e)


# ------------------------------------------------------------- dispatcher

@pytest.mark.parametrize("S", [48, 512, 1024, 3000])
def test_hybrid_function_dispatch(S):
    """cron_root_attention_hybrid(threshold=None): SDPA below the table's
    crossover (bit-identical to F.sdpa), the sqrt(N) op at or above it
    (bit-identical to cron_root_attention); explicit thresholds and forced
    backends as the reference."""
    B, H, D = 1, 16, 128
    say(f"hybrid function S={S}")
    q, k, v, _ = inputs(B, H, H, S, D, F16, seed=S)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    with torch.no_grad():
        out = cra.cron_root_attention_hybrid(qd, kd, vd)
        backend = dispatch_backend(S, D, False, B * H)
        sd = F.scaled_dot_product_attention(qd, kd, vd, is_causal=True)
        cr = cra.cron_root_attention(qd, kd, vd)
        assert torch.equal(out, sd if backend == "sdpa" else cr)
        assert torch.equal(cra.cron_root_attention_hybrid(qd, kd, vd, backend="sdpa"), sd)
        assert torch.equal(cra.cron_root_attention_hybrid(qd, kd, vd, backend="cron_root"), cr)
        assert torch.equal(cra.cron_root_attention_hybrid(qd, kd, vd, threshold=S), cr)
        assert torch.equal(cra.cron_root_attention_hybrid(qd, kd, vd, threshold=S + 1), sd)
    _check_backend(out, qd, kd, vd, backend, F16, [(0, 0), (0, 15)])
    with pytest.raises(ValueError):
        cra.cron_root_attention_hybrid(qd, kd, vd, backend="flash")


def test_hybrid_training_mode_uses_training_crossover(monkeypatch):
    """Grad mode picks the training row of the table (rows set apart here:
    the measured gfx950 rows are equal)."""
    from cron_root_attention import hybrid
    monkeypatch.setitem(hybrid.CROSSOVER_GFX950, ("train", 128, 1), 2048)
    monkeypatch.setitem(hybrid.CROSSOVER_GFX950, ("fwd", 128, 1), 512)
    B, H, D = 1, 16, 128
    thr_f, thr_t = crossover(D, False, B * H), crossover(D, True, B * H)
    assert thr_f < thr_t
    S = (thr_f + thr_t) // 2    # sqrt(N) for inference, SDPA for training
    q, k, v, do = inputs(B, H, H, S, D, F16, seed=2)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = cra.cron_root_attention_hybrid(qd, kd, vd)
    sd = F.scaled_dot_product_attention(qd.detach(), kd.detach(), vd.detach(), is_causal=True)
    assert dispatch_backend(S, D, True, B * H) == "sdpa"
    assert torch.equal(out.detach(), sd)
    out.backward(do.to(DEV))
    with torch.no_grad():
        assert dispatch_backend(S, D, False, B * H) == "cron_root"
        assert torch.equal(cra.cron_root_attention_hybrid(qd, kd, vd),
                           cra.cron_root_attention(qd, kd, vd))


@pytest.mark.parametrize("S", [48, 4096])
def test_hybrid_module(S):
    """CronRootAttentionHybrid: the default threshold (the gfx950 table, whose
    rows say the sqrt(N) op at every length) and explicit thresholds on
    either side of S, so that both backends run."""
    B, H, D = 1, 8, 64
    E = H * D
    say(f"CronRootAttentionHybrid S={S}")
    torch.manual_seed(1)
    m = cra.CronRootAttentionHybrid(E, H).to(DEV, F16).eval()
    assert m.threshold is None
    x = torch.randn(B, S, E, generator=torch.Generator().manual_seed(S)).to(F16).to(DEV)
    box, hook = _capture(m.o_proj)
    with torch.no_grad():
        y = m(x)
        hook.remove()
        assert torch.equal(y, m.o_proj(box[0]))
        q, k, v = (_heads(p(x), B, S, H, D) for p in (m.q_proj, m.k_proj, m.v_proj))
        backend = dispatch_backend(S, D, False, B * H)
        assert backend == ("sdpa" if S < crossover(D, False, B * H) else "cron_root")
        _check_backend(_heads(box[0], B, S, H, D), q, k, v, backend, F16, [(0, 0), (0, 7)])
        for thr, expect in ((S, "cron_root"), (S + 1, "sdpa")):
            m2 = cra.CronRootAttentionHybrid(E, H, threshold=thr).to(DEV, F16).eval()
            m2.load_state_dict(m.state_dict())
            box2, hook2 = _capture(m2.o_proj)
            m2(x)
            hook2.remove()
            _check_backend(_heads(box2[0], B, S, H, D), q, k, v, expect, F16, [(0, 3)])


# ---------------------------------------------------------------- modules

@pytest.mark.parametrize("kv_heads", [8, 2])
def test_cron_root_attention_module_forward_backward(kv_heads):
    """CronRootAttention (GQA 8/2 native) against an fp64 restatement of the
    module: projections, oracle attention, output projection; forward and
    every gradient (input and weights)."""
    B, S, H, D = 1, 3000, 8, 64
    E = H * D
    say(f"CronRootAttention module kv_heads={kv_heads}")
    torch.manual_seed(3)
    m = cra.CronRootAttention(E, H, n_kv_heads=kv_heads).to(DEV, F16)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, S, E, generator=g).to(F16)
    gy = torch.randn(B, S, E, generator=g).to(F16)
    xd = x.to(DEV).requires_grad_(True)
    y = m(xd)
    y.backward(gy.to(DEV))
    # fp64 restatement on the CPU
    W = {n: p.detach().cpu().double().requires_grad_(True) for n, p in m.named_parameters()}
    x64 = x.double().requires_grad_(True)
    G = H // kv_heads
    q = _heads(x64 @ W["q_proj.weight"].T, B, S, H, D)
    k = _heads(x64 @ W["k_proj.weight"].T, B, S, kv_heads, D)
    v = _heads(x64 @ W["v_proj.weight"].T, B, S, kv_heads, D)
    o, _, _ = O.forward(q, k, v, plan_for(S), kv_groups=G)
    y64 = o.transpose(1, 2).reshape(B, S, E) @ W["o_proj.weight"].T
    y64.backward(gy.double())
    e = rel_fro(y, y64.detach())
    say(f"  y rel {e:.3e}")
    assert e <= 1e-2
    assert rel_fro(xd.grad, x64.grad) <= TOL_GRAD[F16]
    for n, p in m.named_parameters():
        en = rel_fro(p.grad, W[n].grad)
        say(f"  {n}.grad rel {en:.3e}")
        assert en <= TOL_GRAD[F16], n


@pytest.mark.parametrize("batch_first", [True, False])
def test_multihead_attention_matches_oracle(batch_first):
    """CronRootMultiheadAttention: out_proj(oracle(in_proj x)) (reference
    module.py:129-247); returns (out, None)."""
    B, S, E, H = 2, 2500, 512, 8
    D = E // H
    say(f"CronRootMultiheadAttention batch_first={batch_first}")
    torch.manual_seed(5)
    m = cra.CronRootMultiheadAttention(E, H, batch_first=batch_first).to(DEV, F16).eval()
    x = torch.randn(B, S, E, generator=torch.Generator().manual_seed(6)).to(F16).to(DEV)
    xin = x if batch_first else x.transpose(0, 1).contiguous()
    box, hook = _capture(m.out_proj)
    with torch.no_grad():
        out, w = m(xin, xin, xin)
        hook.remove()
        assert w is None
        out_b = out if batch_first else out.transpose(0, 1)
        assert torch.equal(out_b, m.out_proj(box[0]))
        qkv = F.linear(x, m.in_proj_weight, m.in_proj_bias).view(B, S, 3, H, D)
        q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
        _check_backend(_heads(box[0], B, S, H, D), q, k, v, "cron_root", F16, [(0, 0), (1, 7)])
    with pytest.raises(AssertionError):
        m(xin, xin.clone(), xin)


# ------------------------------------------------------ persistent, errors

@pytest.mark.parametrize("S", [1500, 3000])
def test_use_persistent_is_bit_identical(S):
    """use_persistent=True (the reference's persistent forward, core.py:711-900,
    dispatched at core.py:3548-3569): output and gradients against the fp64
    oracle, and bit-identical to the tiled forward's."""
    q, k, v, do = inputs(1, 4, 4, S, 64, F16, seed=S + 9)
    res = []
    for pers in (False, True):
        qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
        o = cra.cron_root_attention(qd, kd, vd, use_persistent=pers)
        o.backward(do.to(DEV))
        res.append((o.detach(), qd.grad, kd.grad, vd.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)
    plan = plan_for(S)
    o_p, dq, dk, dv = res[1]
    check_forward(o_p.cpu(), q, k, v, plan, F16)
    _, _, _, g = O.forward_backward(q, k, v, do, plan)
    for name, t in (("dq", dq), ("dk", dk), ("dv", dv)):
        e = rel_fro(t, g[name])
        say(f"  persistent {name}: rel {e:.2e}")
        assert e <= TOL_GRAD[F16], name


@pytest.mark.parametrize("Hq,Hkv,kw", [(4, 2, {}), (4, 2, {"kv_groups": 3}), (3, 2, {"kv_groups": 1})])
def test_kv_groups_validated_on_gpu(Hq, Hkv, kw):
    """The GPU path takes the grouping from kv_groups (reference core.py:981)
    and rejects shapes that disagree with it."""
    q = torch.randn(1, Hq, 64, 32, device=DEV, dtype=F16)
    k = torch.randn(1, Hkv, 64, 32, device=DEV, dtype=F16)
    with pytest.raises(ValueError):
        cra.cron_root_attention(q, k, k, **kw)


def test_relay_log_scale_on_host_is_rejected():
    """A host relay_log_scale with device q/k/v raises before any launch
    (its pointer would otherwise reach the GPU)."""
    q, k, v, _ = inputs(1, 2, 2, 3000, 64, F16, seed=1)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    alpha = torch.zeros(2)
    with pytest.raises(ValueError, match="relay_log_scale"):
        cra.cron_root_attention(qd, kd, vd, relay_log_scale=alpha)
    with pytest.raises(ValueError, match="relay_log_scale"):
        cra.cron_root_attention_varlen(qd, kd, vd, [0, 2500, 3000], relay_log_scale=alpha)
    with pytest.raises(ValueError, match="relay_log_scale"):
        cra.cron_root_attention(qd, kd, vd, relay_log_scale=torch.zeros(3, device=DEV))
