"""The C++ operator path (torch.ops.cra.attention, which the public op takes
for its common calls) against the Python autograd Function: the same plan and
the same launches, so outputs and gradients must agree bit for bit."""
import pytest
import torch

from cron_root_attention import _native, core
import cron_root_attention as cra

pytestmark = pytest.mark.gpu
dev = torch.device("cuda", 0)


def _inputs(B, Hq, Hkv, S, D, dtype, seed=0, layout="bhsd"):
    g = torch.Generator(device=dev).manual_seed(seed)
    def mk(H):
        if layout == "bshd":   # [B, S, H, D] memory viewed as [B, H, S, D]
            return torch.randn(B, S, H, D, device=dev, dtype=dtype, generator=g).transpose(1, 2)
        if layout == "bhds":   # D not contiguous: copied before the launches
            return torch.randn(B, H, D, S, device=dev, dtype=dtype, generator=g).transpose(2, 3)
        return torch.randn(B, H, S, D, device=dev, dtype=dtype, generator=g)
    return mk(Hq), mk(Hkv), mk(Hkv), mk(Hq)


def test_operator_is_loaded_on_the_gpu_box():
    assert _native.attention_op() is not None, _native._op_state["error"]


CASES = [
    (1, 4, 4, 1000, 64, torch.float16, "bhsd"),
    (2, 4, 2, 3000, 128, torch.float16, "bhsd"),    # relay, GQA
    (1, 2, 2, 5000, 32, torch.bfloat16, "bshd"),    # relay, strided view
    (1, 2, 1, 2500, 64, torch.float32, "bhsd"),     # fp32 kernels, GQA 2:1
    (1, 3, 3, 1, 128, torch.float16, "bhsd"),       # a single query
    (1, 2, 2, 2300, 64, torch.float16, "bhds"),     # copied layout
    (1, 4, 2, 3000, 256, torch.bfloat16, "bhsd"),   # head dim 256 (generic kernels), GQA
]


@pytest.mark.parametrize("B,Hq,Hkv,S,D,dtype,layout", CASES)
def test_operator_matches_function(B, Hq, Hkv, S, D, dtype, layout):
    print(f"case B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} {dtype} {layout}", flush=True)
    q, k, v, do = _inputs(B, Hq, Hkv, S, D, dtype, layout=layout)
    grp = Hq // Hkv
    plan = core._op_plan(q, k, v, False, grp, 2)
    assert plan is not None
    # C++ operator (through the public entry point)
    qa, ka, va = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    assert qa.stride() == q.stride()
    oa = cra.cron_root_attention(qa, ka, va, kv_groups=grp)
    assert oa.grad_fn is not None and "CraAttention" in oa.grad_fn.name()
    oa.backward(do)
    # Python Function
    qb, kb, vb = (t.detach().clone().requires_grad_(True) for t in (qa, ka, va))
    ob = core.CronRootAttentionV14Function.apply(qb, kb, vb, False, grp, None, 2)
    ob.backward(do)
    torch.cuda.synchronize()
    assert torch.equal(oa, ob)
    for x, y in ((qa, qb), (ka, kb), (va, vb)):
        assert torch.equal(x.grad, y.grad)


def test_operator_without_grad_and_in_inference_mode():
    q, k, v, _ = _inputs(1, 2, 2, 3000, 64, torch.float16, seed=3)
    ref = core.CronRootAttentionV14Function.apply(q, k, v, False, 1, None, 2)
    with torch.no_grad():
        o1 = cra.cron_root_attention(q, k, v)
    with torch.inference_mode():
        o2 = cra.cron_root_attention(q, k, v)
    assert torch.equal(o1, ref) and torch.equal(o2, ref)


def test_operator_upstream_gradient_in_another_layout():
    q, k, v, _ = _inputs(1, 2, 2, 2100, 128, torch.float16, seed=4)
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = cra.cron_root_attention(qa, ka, va)
    do = torch.randn(1, 2100, 2, 128, device=dev, dtype=torch.float16).transpose(1, 2)
    out.backward(do)   # non-contiguous dO: copied inside the operator
    qb, kb, vb = (t.clone().requires_grad_(True) for t in (q, k, v))
    core.CronRootAttentionV14Function.apply(qb, kb, vb, False, 1, None, 2).backward(
        do.contiguous())
    for x, y in ((qa, qb), (ka, kb), (va, vb)):
        assert torch.equal(x.grad, y.grad)


def test_python_path_still_serves_the_rest():
    # padded head dim and relay scale go through the Function
    q, k, v, _ = _inputs(1, 2, 2, 3000, 80, torch.float16, seed=5)
    out = cra.cron_root_attention(q.requires_grad_(True), k, v)
    assert "CronRootAttentionV14Function" in out.grad_fn.name()
    alpha = torch.zeros(2, device=dev, requires_grad=True)
    q2, k2, v2, _ = _inputs(1, 2, 2, 3000, 64, torch.float16, seed=6)
    out2 = cra.cron_root_attention(q2.requires_grad_(True), k2, v2, relay_log_scale=alpha)
    assert "CronRootAttentionV14Function" in out2.grad_fn.name()
