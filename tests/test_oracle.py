"""Pins the CPU oracle (CPU only).

Every oracle function is checked against something it does not restate:
brute force over explicit index sets, closed forms, a library routine
(causal SDPA), finite differences, exact identities of softmax gradients,
and the golden vectors written from the reference's own ``cra_cpu_fast``.
Planted mistakes (wrong window, relay dropped) must fail the golden check.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import cra_oracle as O
from oracle import cpu_port
from tests.golden.make_golden import SHAPES, make_inputs

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def fixture(shape):
    B, H, S, D = shape
    return np.load(os.path.join(GOLDEN, f"cra_cpu_fast_B{B}_H{H}_S{S}_D{D}.npz"))


# ---------------------------------------------------------------- planning

@pytest.mark.parametrize("S", [1, 2, 3, 4, 5, 63, 64, 65, 512, 2048, 4096, 8192, 131072, 524288])
def test_window_bounds(S):
    Wc = O.window_size(S, "ceil")
    Wf = O.window_size(S, "floor")
    assert (Wc - 1) ** 2 < S <= Wc ** 2
    assert Wf ** 2 <= S < (Wf + 1) ** 2 or S == 0


def test_window_table():
    # W per S for the GPU (ceil) and CPU (floor) rules at the BASELINE sizes
    table = {512: (23, 22), 1024: (32, 32), 2048: (46, 45), 4096: (64, 64), 8192: (91, 90),
             16384: (128, 128), 32768: (182, 181), 65536: (256, 256), 131072: (363, 362),
             262144: (512, 512), 524288: (725, 724)}
    for S, (c, f) in table.items():
        assert O.window_size(S, "ceil") == c and O.window_size(S, "floor") == f
    assert O.make_plan(2048).relay is False and O.make_plan(2049).relay is True
    assert O.make_plan(64, "cpu_reference").relay is True


# ----------------------------------------------------------- index sets

def _rand_src(plan, rng):
    src = []
    for r in range(plan.num_blocks):
        lo, hi = r * plan.W, min(plan.S, (r + 1) * plan.W)
        src.append(list(rng.integers(lo, hi, size=plan.top_k)))
    return src


@pytest.mark.parametrize("S,relay,top_k", [(1, False, 2), (7, True, 2), (50, True, 2),
                                           (50, False, 2), (81, True, 1), (100, True, 3),
                                           (130, True, 4), (2049, True, 2)])
def test_packed_prefix_equals_bruteforce(S, relay, top_k):
    plan = O.Plan(S, O.window_size(S), relay, top_k)
    src = _rand_src(plan, np.random.default_rng(S))
    packed = O.packed_rows(plan, src)
    step = 1 if S < 300 else 7
    for i in range(0, S, step):
        W = plan.W
        ls = max(0, i - W + 1)
        mine = list(range(ls, i + 1)) + packed[: O.packed_prefix_len(i, plan)]
        assert sorted(mine) == sorted(O.attend_set_bruteforce(i, plan, src)), i


@pytest.mark.parametrize("S,relay", [(10, True), (100, True), (100, False), (1000, True), (2047, False)])
def test_pair_count_bruteforce(S, relay):
    plan = O.Plan(S, O.window_size(S), relay, 2)
    src = _rand_src(plan, np.random.default_rng(0))
    brute = sum(len(O.attend_set_bruteforce(i, plan, src)) for i in range(S))
    assert O.pair_count(plan) == brute
    ph = O.phase_pair_counts(plan)
    assert sum(ph.values()) == brute


def test_pair_count_matches_published_table():
    # per-(b,h) pair counts in millions quoted for the BASELINE configs
    table = {2048: 0.138, 8192: 1.819, 65536: 41.682, 262144: 334.498, 16384: 5.178,
             131072: 118.047, 524288: 946.727, 4096: 0.639, 32768: 14.683}
    for S, m in table.items():
        assert abs(O.pair_count(O.make_plan(S)) / 1e6 - m) < 6e-4, S
    ns = O.make_plan(131072)
    assert abs(O.fwd_flops(ns, 1, 16, 128) / 1e9 - 967.04) < 0.01


# ------------------------------------------------------- relay selection

def test_lanetree_norm_close_to_fp64():
    x = np.random.default_rng(1).standard_normal((64, 128)).astype(np.float16)
    lt = O.relay_norms_lanetree(x)
    ex = (x.astype(np.float64) ** 2).sum(-1)
    assert np.all(np.abs(lt - ex) <= 1e-5 * ex)


def test_lanetree_order_is_the_stated_tree():
    # with powers of two per lane the tree order is observable: tiny values
    # that a left-to-right sum would lose survive the pairwise tree
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 2.0 ** 12           # lane 0 partial = 2^24
    x[0, 8] = 1.0                 # lane 1 partial = 1
    x[0, 24] = 1.0                # lane 3 partial = 1
    # butterfly off=2 then 1: (p0 + p2) + (p1 + p3) = 2^24 + 2 exactly, while a
    # left-to-right sum or adjacent pairs lose both ones to round-to-even
    assert O.relay_norms_lanetree(x)[0] == np.float32(2.0 ** 24 + 2)
    assert np.float32(np.float32(2.0 ** 24) + np.float32(1)) + np.float32(1) == np.float32(2.0 ** 24)


def test_relay_select_bruteforce_and_ties():
    rng = np.random.default_rng(2)
    S, D = 200, 32
    k = torch.from_numpy(rng.standard_normal((1, 2, S, D)).astype(np.float32))
    k[0, 0, 30] = k[0, 0, 20]            # exact tie inside block 1 (W=15)
    k[0, 0, 20:30] *= 0.0
    k[0, 0, 20] = k[0, 0, 30] = 10.0     # equal top norms -> earlier row first
    plan = O.make_plan(S)
    plan = O.Plan(S, plan.W, True, 2)
    src = O.relay_select(k, plan)
    n = (k.double() ** 2).sum(-1)[0]
    for h in range(2):
        for r in range(plan.num_blocks):
            lo, hi = r * plan.W, min(S, (r + 1) * plan.W)
            order = sorted(range(lo, hi), key=lambda j: (-float(n[h, j]), j))[:2]
            order += [lo] * (2 - len(order))
            assert src[0, h, 2 * r: 2 * r + 2].tolist() == order
    r = 20 // plan.W
    assert src[0, 0, 2 * r: 2 * r + 2].tolist()[:1] == [min(20, 30)]


def test_relay_select_partial_block_fills_with_block_start():
    S = 17  # W = 5 -> last block has 2 rows; top_k = 4 leaves 2 slots unfilled
    k = torch.randn(1, 1, S, 8)
    plan = O.Plan(S, O.window_size(S), True, 4)
    src = O.relay_select(k, plan)[0, 0].view(-1, 4)
    last = src[-1].tolist()
    assert sorted(last[:2]) == [15, 16] and last[2:] == [15, 15]


def test_relay_select_matches_torch_topk_rule():
    q, k, v, _ = make_inputs(1, 4, 1024, 64)
    plan = O.make_plan(1024, "cpu_reference")
    a = O.relay_select(k, plan, "torch")
    b = O.relay_select(k, plan, "lanetree")
    full = (plan.S // plan.W) * plan.top_k      # drop the zero-padded last block
    assert torch.equal(a[..., :full], b[..., :full])


# ---------------------------------------------------------------- forward

def test_first_window_rows_equal_causal_sdpa():
    torch.manual_seed(3)
    S, D = 300, 16
    q, k, v = (torch.randn(1, 2, S, D, dtype=torch.float64) for _ in range(3))
    plan = O.make_plan(S)
    o, _, _ = O.forward(q, k, v, plan)
    ref = O.causal_sdpa_reference(q, k, v)
    W = plan.W
    assert torch.allclose(o[:, :, :W], ref[:, :, :W], atol=1e-12, rtol=0)


def test_forward_bruteforce_softmax_tiny():
    torch.manual_seed(4)
    S, D = 60, 4
    plan = O.Plan(S, O.window_size(S), True, 2)
    q, k, v = (torch.randn(1, 1, S, D, dtype=torch.float64) for _ in range(3))
    k[0, 0, 8] *= 5      # make a strided row (8 = W) the block's top relay row too
    o, lse, src = O.forward(q, k, v, plan)
    srcl = src[0, 0].view(-1, 2).tolist()
    assert any(srcl[r][0] == r * plan.W for r in range(len(srcl)))   # a duplicate exists
    scale = 1 / math.sqrt(D)
    for i in range(S):
        rows = O.attend_set_bruteforce(i, plan, srcl)
        s = [float((q[0, 0, i] * k[0, 0, j]).sum()) * scale for j in rows]
        m = max(s)
        w = [math.exp(x - m) for x in s]
        z = sum(w)
        ref = sum(wi * v[0, 0, j] for wi, j in zip(w, rows)) / z
        assert torch.allclose(o[0, 0, i], ref, atol=1e-12)
        assert abs(float(lse[0, 0, i]) - (m + math.log(z))) < 1e-12


def test_forward_constant_values_are_preserved():
    torch.manual_seed(5)
    S, D = 500, 8
    q, k = (torch.randn(1, 2, S, D, dtype=torch.float64) for _ in range(2))
    v = torch.full((1, 2, S, D), 0.75, dtype=torch.float64)
    o, _, _ = O.forward(q, k, v, O.Plan(S, O.window_size(S), True, 2))
    assert torch.allclose(o, v, atol=1e-13)


def test_forward_gqa_equals_repeated_heads():
    torch.manual_seed(6)
    S, D = 400, 16
    q = torch.randn(1, 4, S, D, dtype=torch.float64)
    k, v = (torch.randn(1, 2, S, D, dtype=torch.float64) for _ in range(2))
    plan = O.Plan(S, O.window_size(S), True, 2)
    a, _, _ = O.forward(q, k, v, plan, kv_groups=2)
    b, _, _ = O.forward(q, k.repeat_interleave(2, 1), v.repeat_interleave(2, 1), plan)
    assert torch.allclose(a, b, atol=1e-13)


def test_forward_row_range_matches_full():
    torch.manual_seed(7)
    S, D = 3000, 16
    q, k, v = (torch.randn(1, 1, S, D) for _ in range(3))
    plan = O.make_plan(S)
    full, lf, _ = O.forward(q, k, v, plan)
    part, lp, _ = O.forward(q, k, v, plan, rows=(2500, 2800))
    assert torch.allclose(full[:, :, 2500:2800], part, atol=1e-13)
    assert torch.allclose(lf[:, :, 2500:2800], lp, atol=1e-13)


def test_forward_phase_subsets_merge_to_full():
    """The local-only and global-only restrictions, merged with their
    log-sum-exp weights, give the full forward (softmax over a disjoint
    union); a query before the first global row has an empty global subset."""
    torch.manual_seed(5)
    S, D = 3000, 16
    q, k, v = (torch.randn(1, 2, S, D) for _ in range(3))
    plan = O.make_plan(S)
    o_all, l_all, src = O.forward(q, k, v, plan)
    o_l, l_l, _ = O.forward(q, k, v, plan, src=src, phases="local")
    o_g, l_g, _ = O.forward(q, k, v, plan, src=src, phases="global")
    lse = torch.logaddexp(l_l, l_g)
    fin = torch.isfinite(l_g).unsqueeze(-1)
    merged = torch.exp(l_l - lse).unsqueeze(-1) * o_l + torch.where(
        fin, torch.exp(l_g - lse).unsqueeze(-1) * o_g, torch.zeros_like(o_g))
    assert torch.allclose(merged, o_all, atol=1e-12)
    assert torch.allclose(lse, l_all, atol=1e-12)
    assert bool(torch.isinf(l_g[..., :plan.W]).all()) and bool((o_g[:, :, :plan.W] == 0).all())
    assert bool(torch.isfinite(l_g[..., plan.W:]).all())


@pytest.mark.parametrize("shape", SHAPES)
def test_golden_cpu_reference_mode(shape):
    z = fixture(shape)
    q, k, v, _ = make_inputs(*shape)
    for name, t in (("q", q), ("k", k), ("v", v)):
        assert abs(float(z[f"in_{name}_sum"]) - t.double().sum().item()) < 1e-6
    o, _, _ = O.forward(q, k, v, O.make_plan(shape[2], "cpu_reference"), norm="torch")
    rows = z["rows"]
    assert np.abs(o[:, :, rows].numpy() - z["o_rows"]).max() < 5e-6
    assert np.abs(o.sum(dim=(2, 3)).numpy() - z["o_sum"]).max() < 1e-3
    assert np.abs((o ** 2).sum(dim=(2, 3)).numpy() - z["o_sumsq"]).max() < 1e-3


def test_golden_config1_kernel_mode_coincides():
    # S = 4096: ceil and floor windows agree and relay is on in both paths
    shape = (1, 8, 4096, 64)
    z = fixture(shape)
    q, k, v, _ = make_inputs(*shape)
    o, _, _ = O.forward(q, k, v, O.make_plan(4096, "kernel"))
    assert np.abs(o[:, :, z["rows"]].numpy() - z["o_rows"]).max() < 5e-6


@pytest.mark.parametrize("mutation", ["window+1", "window-1", "no_relay", "top_k=1"])
def test_golden_catches_planted_mistakes(mutation):
    shape = (1, 4, 1024, 64)
    z = fixture(shape)
    q, k, v, _ = make_inputs(*shape)
    p = O.make_plan(1024, "cpu_reference")
    bad = {"window+1": O.Plan(p.S, p.W + 1, True, 2), "window-1": O.Plan(p.S, p.W - 1, True, 2),
           "no_relay": O.Plan(p.S, p.W, False, 2), "top_k=1": O.Plan(p.S, p.W, True, 1)}[mutation]
    o, _, _ = O.forward(q, k, v, bad)
    assert np.abs(o[:, :, z["rows"]].numpy() - z["o_rows"]).max() > 1e-3


# --------------------------------------------------------------- backward

def test_backward_gradcheck_tiny():
    torch.manual_seed(8)
    S, D = 40, 4
    plan = O.Plan(S, O.window_size(S), True, 2)
    q = torch.randn(1, 2, S, D, dtype=torch.float64, requires_grad=True)
    k = torch.randn(1, 1, S, D, dtype=torch.float64, requires_grad=True)
    v = torch.randn(1, 1, S, D, dtype=torch.float64, requires_grad=True)
    a = torch.randn(1, dtype=torch.float64, requires_grad=True)
    src = O.relay_select(k.detach(), plan)   # selection is piecewise constant
    f = lambda q, k, v, a: O.forward(q, k, v, plan, kv_groups=2, src=src,
                                      relay_scale=torch.exp(a))[0]
    assert torch.autograd.gradcheck(f, (q, k, v, a), eps=1e-6, atol=1e-6)


def test_backward_softmax_identities():
    torch.manual_seed(9)
    S, D = 700, 16
    q, k, v, dO = (torch.randn(1, 2, S, D) for _ in range(4))
    _, _, _, g = O.forward_backward(q, k, v, dO, O.make_plan(S))
    # sum_j dV_j = sum_i dO_i (rows of P sum to one); sum_j dK_j = 0
    assert torch.allclose(g["dv"].sum(2), dO.double().sum(2), atol=1e-10)
    assert g["dk"].sum(2).abs().max() < 1e-10


def test_backward_relay_scale_gradient_closed_form():
    torch.manual_seed(10)
    S, D = 300, 8
    q, k, v, dO = (torch.randn(1, 2, S, D) for _ in range(4))
    plan = O.Plan(S, O.window_size(S), True, 2)
    alpha = torch.tensor([0.3, -0.2], dtype=torch.float64)
    _, _, src, g = O.forward_backward(q, k, v, dO, plan, relay_log_scale=alpha)
    # d(alpha) = d/d(eps) L(alpha + eps) at eps = 0, by central difference
    eps = 1e-6
    def L(a):
        o, _, _ = O.forward(q, k, v, plan, src=src, relay_scale=torch.exp(a.double()))
        return float((o * dO.double()).sum())
    for h in range(2):
        e = torch.zeros(2, dtype=torch.float64); e[h] = eps
        fd = (L(alpha + e) - L(alpha - e)) / (2 * eps)
        assert abs(fd - float(g["dalpha"][h])) < 1e-6


# ---------------------------------------------------------------- CPU port

def test_cpu_port_matches_oracle_and_golden():
    shape = (1, 8, 4096, 64)
    z = fixture(shape)
    q, k, v, _ = make_inputs(*shape)
    plan = O.make_plan(4096)
    o = cpu_port.cra_cpu_chunked(q, k, v, plan)
    assert np.abs(o[:, :, z["rows"]].numpy() - z["o_rows"]).max() < 5e-6
    part = cpu_port.cra_cpu_chunked(q, k, v, plan, q_rows=(1000, 1300))
    assert torch.allclose(part, o[:, :, 1000:1300], atol=1e-6)


# ------------------------------------------------------------- varlen (packed)

def test_varlen_single_document_is_forward():
    torch.manual_seed(11)
    S, D = 300, 8
    q, k, v = (torch.randn(1, 2, S, D, dtype=torch.float64) for _ in range(3))
    o1, l1, _ = O.forward_varlen(q, k, v, [0, S])
    o2, l2, _ = O.forward(q, k, v, O.make_plan(S))
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_varlen_plans_follow_each_length():
    plans = O.varlen_plans([0, 100, 2149, 5149])
    assert [(p.S, p.W, p.relay) for p in plans] == [(100, 10, False), (2049, 46, True),
                                                     (3000, 55, True)]


def test_varlen_bruteforce_packed_masks():
    """Every packed query against an explicit softmax over the keys of its own
    document only (offsets, per-document plans, no cross-document keys)."""
    torch.manual_seed(12)
    cu = [0, 1, 41, 101, 130]
    plans = [O.make_plan(1), O.make_plan(40), O.Plan(60, 8, True, 2), O.Plan(29, 5, True, 1)]
    S, D = cu[-1], 4
    q, k, v = (torch.randn(1, 1, S, D, dtype=torch.float64) for _ in range(3))
    o, lse, srcs = O.forward_varlen(q, k, v, cu, plans)
    scale = 1 / math.sqrt(D)
    for d, (s, e) in enumerate(zip(cu, cu[1:])):
        pl = plans[d]
        srcl = (srcs[d][0, 0].view(-1, pl.top_k).tolist() if pl.relay else None)
        for i in range(s, e):
            rows = [s + j for j in O.attend_set_bruteforce(i - s, pl, srcl)]
            assert all(s <= j <= i for j in rows)
            sc = [float((q[0, 0, i] * k[0, 0, j]).sum()) * scale for j in rows]
            m = max(sc)
            w = [math.exp(x - m) for x in sc]
            z = sum(w)
            ref = sum(wi * v[0, 0, j] for wi, j in zip(w, rows)) / z
            assert torch.allclose(o[0, 0, i], ref, atol=1e-12), (d, i)
            assert abs(float(lse[0, 0, i]) - (m + math.log(z))) < 1e-12


def test_varlen_documents_are_isolated():
    torch.manual_seed(13)
    cu = [0, 90, 200]
    q, k, v = (torch.randn(1, 2, 200, 8, dtype=torch.float64) for _ in range(3))
    o, _, _ = O.forward_varlen(q, k, v, cu)
    k2, v2 = k.clone(), v.clone()
    k2[:, :, :90] += 3.0
    v2[:, :, :90] -= 1.0
    o2, _, _ = O.forward_varlen(q, k2, v2, cu)
    assert torch.equal(o[:, :, 90:], o2[:, :, 90:])
    assert not torch.allclose(o[:, :, :90], o2[:, :, :90])


def test_varlen_relay_scale_gradient_sums_documents():
    """d(alpha) of the packed call by central difference, relay in two documents."""
    torch.manual_seed(14)
    cu = [0, 50, 120]
    plans = [O.Plan(50, 7, True, 2), O.Plan(70, 9, True, 2)]
    q, k, v, dO = (torch.randn(1, 2, 120, 8) for _ in range(4))
    alpha = torch.tensor([0.25, -0.4], dtype=torch.float64)
    _, _, srcs, g = O.forward_backward_varlen(q, k, v, dO, cu, plans, relay_log_scale=alpha)
    eps = 1e-6

    def L(a):
        parts = [O.forward(q[:, :, s:e], k[:, :, s:e], v[:, :, s:e], pl, src=src,
                           relay_scale=torch.exp(a))[0]
                 for (s, e), pl, src in zip(zip(cu, cu[1:]), plans, srcs)]
        return float((torch.cat(parts, 2) * dO.double()).sum())

    for h in range(2):
        e = torch.zeros(2, dtype=torch.float64)
        e[h] = eps
        fd = (L(alpha + e) - L(alpha - e)) / (2 * eps)
        assert abs(fd - float(g["dalpha"][h])) < 1e-6


# ------------------------------------------------ gradients of chosen rows

def _grad_case(S, Hq, Hkv, D, seed, top_k=2):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, Hq, S, D, generator=g, dtype=torch.float64)
    k = torch.randn(1, Hkv, S, D, generator=g, dtype=torch.float64)
    v = torch.randn(1, Hkv, S, D, generator=g, dtype=torch.float64)
    do = torch.randn(1, Hq, S, D, generator=g, dtype=torch.float64)
    plan = O.Plan(S, O.window_size(S), True, top_k)
    return q, k, v, do, plan


def _strided_and_relay_keys(plan, src_row):
    """Every key class: local-only, strided, relay source, and both."""
    W = plan.W
    src = set(int(x) for x in src_row)
    strided = [r * W for r in range(plan.num_blocks)]
    both = [j for j in strided if j in src]
    relay_only = [j for j in sorted(src) if j % W]
    local_only = [j for j in range(plan.S) if j % W and j not in src][:5]
    return local_only + strided[:3] + strided[-2:] + relay_only[:6] + both


def test_query_row_grads_equal_full_autograd():
    q, k, v, do, plan = _grad_case(700, 4, 2, 32, seed=3)
    _, _, _, g = O.forward_backward(q, k, v, do, plan, kv_groups=2)
    for lo, hi in ((0, 40), (300, 333), (650, 700)):
        dq = O.query_row_grads(q, k, v, do, plan, (lo, hi), kv_groups=2)
        assert torch.allclose(dq, g["dq"][:, :, lo:hi], rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("kv_groups", [1, 2])
def test_key_row_grads_equal_full_autograd(kv_groups):
    S, Hkv, D = 900, 2, 32
    q, k, v, do, plan = _grad_case(S, Hkv * kv_groups, Hkv, D, seed=5 + kv_groups)
    # make block 7's strided row its top relay row (a key counted twice)
    k[0, 1, 7 * plan.W] *= 4.0
    o, lse, src, g = O.forward_backward(q, k, v, do, plan, kv_groups=kv_groups)
    delta = (o * do).sum(-1)
    assert int(src[0, 1, 7 * plan.top_k]) == 7 * plan.W
    keys = [(0, h, j) for h in range(Hkv) for j in _strided_and_relay_keys(plan, src[0, h])]
    res = O.key_row_grads(q, k, v, do, plan, keys, lse, delta, src, kv_groups)
    for (b, h, j), (dk, dv) in res.items():
        assert torch.allclose(dk, g["dk"][b, h, j], rtol=1e-9, atol=1e-11), (h, j)
        assert torch.allclose(dv, g["dv"][b, h, j], rtol=1e-9, atol=1e-11), (h, j)


@pytest.mark.parametrize("mutation", ["no_strided", "no_relay", "window_off_by_one"])
def test_key_row_grads_catch_planted_mistakes(mutation, monkeypatch):
    """A multiplicity that drops a term or shifts the window must disagree
    with autograd on some key row."""
    S, D = 900, 32
    q, k, v, do, plan = _grad_case(S, 1, 1, D, seed=11)
    k[0, 0, 4 * plan.W] *= 4.0
    o, lse, src, g = O.forward_backward(q, k, v, do, plan)
    delta = (o * do).sum(-1)
    keys = [(0, 0, j) for j in _strided_and_relay_keys(plan, src[0, 0])]
    true_mult = O.key_multiplicity

    def wrong(j, pl, src_row):
        if mutation == "no_strided":
            m = true_mult(j, pl, src_row)
            if j % pl.W == 0:
                i = np.arange(pl.S)
                m = m - (np.maximum(i - pl.W + 1, 0) > j)
            return m
        if mutation == "no_relay":
            return true_mult(j, O.Plan(pl.S, pl.W, False, pl.top_k), None)
        return true_mult(j, O.Plan(pl.S, pl.W + 1, pl.relay, pl.top_k), src_row)

    monkeypatch.setattr(O, "key_multiplicity", wrong)
    res = O.key_row_grads(q, k, v, do, plan, keys, lse, delta, src)
    bad = sum(not torch.allclose(dk, g["dk"][b, h, j], rtol=1e-6, atol=1e-9)
              for (b, h, j), (dk, dv) in res.items())
    assert bad > 0
