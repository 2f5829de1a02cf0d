"""HIP vs the CPU oracle on identical seeded inputs (GPU).

Tolerances and the forward check are in ``tests/parity_util.py``: fp16
forward max-abs <= 2e-3 as the north star states it, gradients relative
error <= 1e-2 (fp16); relay selection and the packed global rows are
compared bit for bit.
"""
import math
import os

import numpy as np
import pytest
import torch

import cron_root_attention as cra
from cron_root_attention import _native
from cron_root_attention.core import _attention_with_plan
from oracle import cra_oracle as O
from tests.golden.make_golden import SHAPES, make_inputs
from tests.parity_util import (BF16, DEV, F16, F32, TOL_FWD, TOL_GRAD, TOL_LSE, check_forward,
                               check_grad_rows, device_inputs, inputs, max_abs, plan_for,
                               rel_fro, say, spot_ranges)

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------ relay rows

@pytest.mark.parametrize("dtype,S,D,top_k,scaled", [
    (F16, 2049, 128, 2, False), (F16, 4096, 64, 2, True), (BF16, 3000, 128, 4, False),
    (F32, 2500, 32, 3, True), (F16, 10001, 128, 1, False), (F16, 700, 64, 2, False),
])
def test_global_rows_bit_exact(dtype, S, D, top_k, scaled):
    say(f"global rows {dtype} S={S} D={D} top_k={top_k} scaled={scaled}")
    B, H = 2, 3
    q, k, v, _ = inputs(B, H, H, S, D, dtype, seed=S + D)
    plan = O.Plan(S, O.window_size(S), True, top_k)
    p = _native.problem(B, H, H, S, D, plan.W, True, top_k, dtype, 1 / math.sqrt(D))
    rs = None
    if scaled:
        rs = torch.tensor([0.5, 1.25, 2.0]).to(dtype).to(F32)
    gk, gv, src = _native.build_global(p, k.to(DEV), v.to(DEV), rs.to(DEV) if rs is not None else None)
    torch.cuda.synchronize()
    ref_src = O.relay_select(k, plan, "lanetree").to(torch.int32)
    assert torch.equal(src.cpu(), ref_src)
    for b in range(B):
        for h in range(H):
            rows = O.packed_rows(plan, ref_src[b, h].view(-1, top_k).tolist())
            ek, ev = k[b, h, rows].clone(), v[b, h, rows].clone()
            if scaled:
                relay = torch.tensor([i % (1 + top_k) != 0 for i in range(len(rows))])
                ek[relay] = (ek[relay].float() * rs[h]).to(dtype)
                ev[relay] = (ev[relay].float() * rs[h]).to(dtype)
            assert torch.equal(gk[b, h].cpu(), ek)
            assert torch.equal(gv[b, h].cpu(), ev)


def test_global_rows_no_relay_are_strided_rows():
    S, D = 1500, 64
    q, k, v, _ = inputs(1, 2, 2, S, D, F16, 1)
    W = O.window_size(S)
    p = _native.problem(1, 2, 2, S, D, W, False, 2, F16, 0.125)
    gk, gv, src = _native.build_global(p, k.to(DEV), v.to(DEV), None)
    assert src is None
    idx = torch.arange(0, S, W)
    assert torch.equal(gk.cpu(), k[:, :, idx]) and torch.equal(gv.cpu(), v[:, :, idx])


# --------------------------------------------------------------------- forward

FWD_CASES = [
    # dtype, B, Hq, Hkv, S, D, top_k
    (F16, 1, 2, 2, 1, 128, 2), (F16, 1, 2, 2, 2, 128, 2), (F16, 2, 2, 2, 63, 64, 2),
    (F16, 1, 3, 3, 129, 128, 2), (F16, 1, 2, 2, 300, 32, 2), (F16, 1, 2, 2, 2048, 128, 2),
    (F16, 1, 2, 2, 2049, 128, 2), (F16, 1, 4, 2, 4097, 128, 2), (F16, 1, 4, 1, 3000, 64, 1),
    (F16, 1, 2, 2, 5000, 128, 3), (F16, 1, 2, 2, 2500, 64, 4), (BF16, 1, 2, 2, 4096, 128, 2),
    (BF16, 1, 2, 2, 1000, 64, 2), (F32, 1, 2, 2, 4096, 64, 2), (F32, 1, 2, 2, 777, 128, 2),
    (F32, 1, 2, 2, 3001, 32, 2), (F16, 1, 2, 2, 16, 16, 2), (F16, 1, 2, 2, 2100, 80, 2),
    (BF16, 1, 2, 1, 3333, 96, 2),
    # 10 heads at D = 128 (not a multiple of 8: the XCD-aware block order)
    # over an odd number of query tiles
    (F16, 2, 5, 5, 1300, 128, 2),
]


def hip_fwd_with_lse(q, k, v, plan, kv_groups=1):
    B, Hq, S, D = q.shape
    p = _native.problem(B, Hq, k.shape[1], S, D, plan.W, plan.relay, plan.top_k, q.dtype,
                        1 / math.sqrt(D))
    gk, gv, src = _native.build_global(p, k, v, None)
    return _native.forward(p, q, k, v, gk, gv)


@pytest.mark.parametrize("case", FWD_CASES, ids=lambda c: "-".join(map(str, c)))
def test_forward_matches_oracle(case):
    dtype, B, Hq, Hkv, S, D, top_k = case
    say(f"forward {case}")
    q, k, v, _ = inputs(B, Hq, Hkv, S, D, dtype, seed=S * 7 + D)
    o = cra.cron_root_attention(q.to(DEV), k.to(DEV), v.to(DEV), kv_groups=Hq // Hkv,
                                relay_top_k=top_k)
    assert o.shape == q.shape and o.dtype == dtype
    ref, ref_lse = check_forward(o, q, k, v, plan_for(S, top_k), dtype, kv_groups=Hq // Hkv)
    if D in (32, 64, 128):
        _, lse = hip_fwd_with_lse(q.to(DEV), k.to(DEV), v.to(DEV), plan_for(S, top_k), Hq // Hkv)
        assert max_abs(lse, ref_lse) <= TOL_LSE[dtype]


@pytest.mark.parametrize("dtype,S,D", [(F16, 3000, 128), (BF16, 2500, 64), (F32, 2300, 32),
                                       (F16, 1500, 64)])
def test_forward_phase_subsets(dtype, S, D):
    """cra_fwd_phases (the per-phase measurement entry point): the local-only
    and global-only forwards each match the oracle restricted to that phase."""
    say(f"forward phases {dtype} S={S} D={D}")
    B, H = 1, 2
    q, k, v, _ = inputs(B, H, H, S, D, dtype, seed=S + 3 * D)
    plan = plan_for(S)
    p = _native.problem(B, H, H, S, D, plan.W, plan.relay, plan.top_k, dtype, 1 / math.sqrt(D))
    gk, gv, _ = _native.build_global(p, k.to(DEV), v.to(DEV), None)
    for name, mask in (("local", _native.PHASE_LOCAL), ("global", _native.PHASE_GLOBAL)):
        o, lse = _native.forward(p, q.to(DEV), k.to(DEV), v.to(DEV), gk, gv, phases=mask)
        ref, ref_lse = check_forward(o, q, k, v, plan, dtype, phases=name)
        fin = torch.isfinite(ref_lse)
        assert torch.equal(torch.isfinite(lse.cpu()), fin)
        assert max_abs(lse.cpu()[fin], ref_lse[fin]) <= TOL_LSE[dtype]


def test_forward_strided_views_and_relay_scale():
    say("forward strided views + relay_log_scale")
    B, S, H, D = 1, 3000, 4, 64
    g = torch.Generator().manual_seed(11)
    x = torch.randn(B, S, 3, H, D, generator=g).to(F16)
    q, k, v = (x[:, :, i].transpose(1, 2) for i in range(3))     # [B, H, S, D] views
    alpha = torch.tensor([0.2, -0.1, 0.0, 0.4])
    xd = x.to(DEV)
    o = cra.cron_root_attention(xd[:, :, 0].transpose(1, 2), xd[:, :, 1].transpose(1, 2),
                                xd[:, :, 2].transpose(1, 2), relay_log_scale=alpha.to(DEV))
    rs = alpha.exp().to(F16).to(F32)
    check_forward(o, q, k, v, plan_for(S), F16, relay_scale=rs, relay_dtype=F16)


@pytest.mark.parametrize("shape", SHAPES)
def test_forward_matches_reference_golden(shape):
    """cpu_reference semantics (floor window, relay on) vs the reference's own outputs."""
    say(f"golden {shape}")
    z = np.load(os.path.join(os.path.dirname(__file__), "golden",
                             "cra_cpu_fast_B%d_H%d_S%d_D%d.npz" % shape))
    q, k, v, _ = make_inputs(*shape)
    plan = O.make_plan(shape[2], "cpu_reference")
    o = _attention_with_plan(q.to(DEV), k.to(DEV), v.to(DEV), window=plan.W, relay=True)
    rows = torch.from_numpy(z["rows"])
    err = float((o.cpu()[:, :, rows] - torch.from_numpy(z["o_rows"])).abs().max())
    say(f"  max|o-golden| = {err:.3e}")
    assert err <= 2e-5
    assert np.abs(o.double().sum(dim=(2, 3)).cpu().numpy() - z["o_sum"]).max() < 1e-2


def test_config1_public_api_matches_golden():
    shape = (1, 8, 4096, 64)
    z = np.load(os.path.join(os.path.dirname(__file__), "golden",
                             "cra_cpu_fast_B1_H8_S4096_D64.npz"))
    q, k, v, _ = make_inputs(*shape)
    o = cra.cron_root_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    rows = torch.from_numpy(z["rows"])
    assert float((o.cpu()[:, :, rows] - torch.from_numpy(z["o_rows"])).abs().max()) <= 2e-5


# -------------------------------------------------------------------- backward

BWD_CASES = [
    (F16, 1, 2, 2, 100, 64, 2), (F16, 1, 2, 2, 2049, 128, 2), (F16, 1, 4, 2, 3000, 128, 2),
    (BF16, 1, 2, 2, 2500, 64, 2), (F32, 1, 2, 2, 1500, 32, 2), (F32, 1, 2, 2, 4096, 64, 3),
    (F16, 2, 2, 2, 700, 128, 2), (F16, 1, 2, 2, 2600, 80, 2), (F16, 1, 4, 1, 5000, 64, 2),
    # 2-byte types at D = 32 (and 16, padded to 32): tiles whose fill takes
    # fewer instructions than the kernels have waves
    (F16, 1, 2, 2, 3000, 32, 2), (BF16, 1, 2, 2, 2100, 16, 2),
    # a single query and a sequence shorter than one query tile; relay
    # top-1 and top-3 in the 2-byte kernels; 8 query heads per kv head
    (F16, 1, 2, 2, 1, 64, 2), (F16, 1, 2, 2, 33, 128, 2), (F16, 1, 2, 2, 4500, 128, 1),
    (BF16, 1, 4, 2, 3500, 128, 3), (F16, 1, 8, 1, 2200, 128, 2),
    # 10 heads at D = 128: the XCD-aware block order of the dQ and local
    # dK/dV kernels over odd tile counts
    (F16, 2, 5, 5, 1300, 128, 2),
]


@pytest.mark.parametrize("case", BWD_CASES, ids=lambda c: "-".join(map(str, c)))
def test_backward_matches_oracle(case):
    dtype, B, Hq, Hkv, S, D, top_k = case
    say(f"backward {case}")
    q, k, v, do = inputs(B, Hq, Hkv, S, D, dtype, seed=S * 3 + D)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = cra.cron_root_attention(qd, kd, vd, kv_groups=Hq // Hkv, relay_top_k=top_k)
    o.backward(do.to(DEV))
    _, _, _, g = O.forward_backward(q, k, v, do, plan_for(S, top_k), kv_groups=Hq // Hkv)
    for name, hip, ref in (("dq", qd.grad, g["dq"]), ("dk", kd.grad, g["dk"]),
                           ("dv", vd.grad, g["dv"])):
        if float(ref.norm()) <= 1e-9 * float(do.norm()):
            # A single query with its single key (S = 1): P = 1 and dP equals
            # Delta, so dQ = dK = 0 exactly; the kernels form Delta from the
            # rounded O and return rounding-level values, for which a
            # relative error is undefined.
            m = float(hip.detach().abs().max())
            say(f"  {name}: exact gradient is zero, max-abs = {m:.3e}")
            assert m <= 1e-4, name
            continue
        e = rel_fro(hip, ref)
        say(f"  {name}: rel = {e:.3e}")
        assert e <= TOL_GRAD[dtype], name


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_large_logits_forward_backward(dtype):
    """q and k scaled by 4, so the logits spread over tens of units (standard
    deviation about 16 at D = 64): softmax rows are sharply peaked, and the
    lazily raised running maximum fails its overflow test and rescales the
    accumulators on many tiles, not only on a wave's first."""
    B, H, S, D = 1, 2, 3000, 64
    q, k, v, do = inputs(B, H, H, S, D, F32, seed=11)
    q, k = (q * 4).to(dtype), (k * 4).to(dtype)
    v, do = v.to(dtype), do.to(dtype)
    say(f"large logits {dtype}")
    plan = plan_for(S)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = cra.cron_root_attention(qd, kd, vd)
    check_forward(o, q, k, v, plan, dtype)
    o.backward(do.to(DEV))
    _, _, _, g = O.forward_backward(q, k, v, do, plan)
    for name, hip, ref in (("dq", qd.grad, g["dq"]), ("dk", kd.grad, g["dk"]),
                           ("dv", vd.grad, g["dv"])):
        e = rel_fro(hip, ref)
        say(f"  {name}: rel = {e:.3e}")
        assert e <= TOL_GRAD[dtype], name


def test_backward_relay_log_scale():
    say("backward relay_log_scale")
    B, H, S, D = 1, 2, 3000, 64
    q, k, v, do = inputs(B, H, H, S, D, F32, seed=5)
    alpha = torch.tensor([0.3, -0.25])
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    ad = alpha.to(DEV).requires_grad_(True)
    o = cra.cron_root_attention(qd, kd, vd, relay_log_scale=ad)
    o.backward(do.to(DEV))
    _, _, _, g = O.forward_backward(q, k, v, do, plan_for(S), relay_log_scale=alpha)
    assert rel_fro(qd.grad, g["dq"]) <= 1e-4
    assert rel_fro(kd.grad, g["dk"]) <= 1e-4
    assert rel_fro(vd.grad, g["dv"]) <= 1e-4
    assert rel_fro(ad.grad, g["dalpha"]) <= 1e-4


@pytest.mark.parametrize("dtype,B,H,S,D", [(F16, 1, 2, 1, 128), (F16, 2, 3, 700, 64),
                                           (F16, 1, 16, 2048, 128), (BF16, 1, 4, 5000, 128),
                                           (F16, 1, 2, 9000, 32), (F16, 1, 16, 131072, 128)])
def test_persistent_forward_bit_identical(dtype, B, H, S, D):
    """cra_fwd_persistent (work queue over a CU-sized grid; the reference's
    persistent forward, core.py:711-900, dispatched at core.py:3548-3569)
    against the fp64 oracle: every row of every head up to S = 9000, and at
    the north-star shape three 256-row ranges of heads 0 and 15 (lse too);
    bit for bit equal to cra_fwd, with and without relay, and a second call
    with a fresh counter too."""
    say(f"persistent forward {dtype} B={B} H={H} S={S} D={D}")
    q, k, v = device_inputs(B, H, H, S, D, dtype, seed=S)
    plan = plan_for(S)
    p = _native.problem(B, H, H, S, D, plan.W, plan.relay, 2, dtype, 1 / math.sqrt(D))
    gk, gv, src = _native.build_global(p, k, v, None)
    o, lse = _native.forward(p, q, k, v, gk, gv)
    for _ in range(2):
        op, lsep = _native.forward_persistent(p, q, k, v, gk, gv)
        torch.cuda.synchronize()
        assert torch.equal(op, o) and torch.equal(lsep, lse)
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    if plan.relay:
        assert torch.equal(src.cpu(), O.relay_select(kc, plan, "lanetree").to(torch.int32))
    if S <= 9000:
        _, ref_lse = check_forward(op.cpu(), qc, kc, vc, plan, dtype)
        assert max_abs(lsep, ref_lse) <= TOL_LSE[dtype]
    else:
        heads = [0, H - 1]
        srch = src.cpu()[:, heads].long()
        qh, kh, vh, oh = qc[:, heads], kc[:, heads], vc[:, heads], op.cpu()[:, heads]
        for lo, hi in spot_ranges(S):
            say(f"  rows [{lo},{hi})")
            _, ref_lse = check_forward(oh[:, :, lo:hi], qh, kh, vh, plan, dtype,
                                       rows=(lo, hi), src=srch)
            assert max_abs(lsep.cpu()[:, heads, lo:hi], ref_lse) <= TOL_LSE[dtype]


def test_backward_deterministic():
    B, H, S, D = 1, 4, 6000, 128
    q, k, v, do = inputs(B, H, H, S, D, F16, seed=9)
    grads = []
    for _ in range(2):
        qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
        cra.cron_root_attention(qd, kd, vd).backward(do.to(DEV))
        grads.append((qd.grad.clone(), kd.grad.clone(), vd.grad.clone()))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


# ------------------------------------------------- north-star size (ns) checks

def ns_inputs(dtype=F16):
    return device_inputs(1, 16, 16, 131072, 128, dtype, seed=0)


def test_ns_forward_rows_and_relay_selection():
    say("ns forward spot rows")
    q, k, v = ns_inputs()
    S = q.shape[2]
    plan = plan_for(S)
    o = cra.cron_root_attention(q, k, v)
    p = _native.problem(1, 16, 16, S, 128, plan.W, True, 2, F16, 1 / math.sqrt(128))
    _, _, src = _native.build_global(p, k, v, None)
    kc = k.cpu()
    assert torch.equal(src.cpu(), O.relay_select(kc, plan, "lanetree").to(torch.int32))
    heads = [0, 15]
    qc, vc, oc = q.cpu()[:, heads], v.cpu()[:, heads], o.cpu()[:, heads]
    kh = kc[:, heads]
    srch = src.cpu()[:, heads].long()
    for lo, hi in ((0, 256), (65536, 65792), (S - 256, S)):
        say(f"  rows [{lo},{hi})")
        check_forward(oc[:, :, lo:hi], qc, kh, vc, plan, F16, rows=(lo, hi), src=srch)


def _doubled_block(k, plan, heads, r):
    """Make block r's strided row the top relay row of each head in
    ``heads`` (its key then counts twice for late queries)."""
    j = r * plan.W
    for h in heads:
        k[:, h, j] = k[:, h, j] * 3
    return j


def test_ns_backward_rows_match_oracle():
    """Full north-star shape: dQ on three 256-row ranges and dK/dV of a
    local-only row, strided rows at the start, middle and end, relay source
    rows and a row that is both strided and relay (block 181), for heads 0
    and 15, against the fp64 oracle; plus the two softmax-gradient
    identities and bit-identical reruns."""
    say("ns backward rows")
    q, k, v, do = device_inputs(1, 16, 16, 131072, 128, F16, seed=0, with_do=True)
    plan = plan_for(q.shape[2])
    doubled = _doubled_block(k, plan, [0, 15], plan.num_blocks // 2)
    res = []
    for _ in range(2):
        qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
        cra.cron_root_attention(qd, kd, vd).backward(do)
        res.append((qd.grad, kd.grad, vd.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)
    dq, dk, dv = res[0]
    assert torch.isfinite(dq).all() and torch.isfinite(dk).all() and torch.isfinite(dv).all()
    sdv = dv.double().sum(2)
    sdo = do.double().sum(2)
    assert float((sdv - sdo).abs().max()) <= 1e-3 * float(sdo.abs().max()) + 0.5
    sdk = dk.double().sum(2)
    assert float(sdk.abs().max()) <= 1e-2 * float(dk.double().abs().sum(2).max())
    check_grad_rows(q, k, v, do, dq, dk, dv, plan, 0, [0, 15], doubled=doubled)


@pytest.mark.parametrize("B,H,S,D,chunks", [(1, 1, 65536, 128, 96), (4, 32, 4096, 64, 3)])
def test_backward_rows_at_chunk_count_extremes(B, H, S, D, chunks):
    """The global-row kernel's query-chunk count follows the problem: one
    head of S = 65536 is cut into 96 chunks (each row's gradient then sums up
    to 96 partials), 128 heads of S = 4096 into 3. Gradient spot rows of the
    first and last head against the fp64 oracle in both cases."""
    import ctypes
    say(f"backward rows, {chunks} query chunks: B={B} H={H} S={S} D={D}")
    p = _native.problem(B, H, H, S, D, O.window_size(S), S > 2048, 2, torch.float16,
                        1 / math.sqrt(D))
    lib = _native.load_library()
    per_query = (B * H * S * 4 + 255) // 256 * 256
    per_chunk = B * H * int(_native.global_rows(p)) * 2 * D * 4
    assert (lib.cra_bwd_workspace_bytes(ctypes.byref(p)) - 2 * per_query) // per_chunk == chunks
    q, k, v, do = device_inputs(B, H, H, S, D, F16, seed=3, with_do=True)
    plan = plan_for(S)
    qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
    cra.cron_root_attention(qd, kd, vd).backward(do)
    for t in (qd.grad, kd.grad, vd.grad):
        assert torch.isfinite(t).all()
    check_grad_rows(q, k, v, do, qd.grad, kd.grad, vd.grad, plan, B - 1, sorted({0, H - 1}))


@pytest.mark.parametrize("B,H,S,dtype,bwd", [(1, 16, 524288, F16, True), (2, 32, 262144, BF16, False)])
def test_largest_baseline_shapes(B, H, S, dtype, bwd):
    """BASELINE's largest configurations (config 3 at S=524288 with the
    backward, config 5 at S=262144): finite outputs and gradients, the
    start, middle and end 256-row ranges of the first and last head against
    the oracle (element-wise forward check), and at S=524288 the gradient
    spot rows of head 0."""
    say(f"large shape B={B} H={H} S={S} {dtype} bwd={bwd}")
    D = 128
    g = torch.Generator(device=DEV).manual_seed(0)
    mk = lambda: torch.randn(B, H, S, D, generator=g, device=DEV, dtype=torch.float32).to(dtype)
    q, k, v = mk(), mk(), mk()
    if bwd:
        qg, kg, vg = (t.requires_grad_(True) for t in (q, k, v))
        o = cra.cron_root_attention(qg, kg, vg)
        do = mk()
        o.backward(do)
        for t in (o, qg.grad, kg.grad, vg.grad):
            assert bool(torch.isfinite(t).all())
    else:
        with torch.no_grad():
            o = cra.cron_root_attention(q, k, v)
        assert bool(torch.isfinite(o).all())
    plan = plan_for(S)
    for b, h in ((0, 0), (B - 1, H - 1)):
        qc, kc, vc = (t[b:b + 1, h:h + 1].detach().float().cpu() for t in (q, k, v))
        src = O.relay_select(kc, plan, "lanetree")
        oc = o[b:b + 1, h:h + 1].detach().cpu()
        for lo, hi in spot_ranges(S):
            say(f"  b={b} h={h} rows [{lo},{hi})")
            check_forward(oc[:, :, lo:hi], qc.to(dtype), kc.to(dtype), vc.to(dtype), plan, dtype,
                          rows=(lo, hi), src=src)
    if bwd:  # gradient rows of the first head: dQ ranges; local, strided and relay key rows
        check_grad_rows(q.detach(), k.detach(), v.detach(), do, qg.grad, kg.grad, vg.grad, plan,
                        0, [0])
