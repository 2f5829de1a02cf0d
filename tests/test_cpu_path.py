"""The CPU-tensor path (CPU only): ``cron_root_attention`` on CPU tensors runs
the library's native host forward with the plan of the reference's CPU path
``cra_cpu_fast`` (W = isqrt(S), relay always on, top 2 rows per block;
reference core.py:3794-3796, cpu_reference.py:198-339).

Pinned by the golden vectors the reference's own ``cra_cpu_fast`` wrote
(tests/golden/, fp32), and by the fp64 oracle in ``cpu_reference`` mode for
the 2-byte types, GQA, odd D and strided inputs. For fp16/bf16 the relay
rows are ranked by norms rounded to the input type, whose exact ties torch's
``topk`` orders in an unspecified way: selection on such ties is parity
unpinned; the test inputs have none among the top two of any block.
"""
import os

import numpy as np
import pytest
import torch

import cron_root_attention as cra
from oracle import cra_oracle as O
from tests.golden.make_golden import SHAPES, make_inputs

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.mark.parametrize("shape", SHAPES)
def test_cpu_path_matches_reference_golden_vectors(shape):
    z = np.load(os.path.join(GOLDEN, "cra_cpu_fast_B%d_H%d_S%d_D%d.npz" % shape))
    q, k, v, _ = make_inputs(*shape)
    o = cra.cron_root_attention(q, k, v)
    rows = torch.from_numpy(z["rows"])
    assert float((o[:, :, rows] - torch.from_numpy(z["o_rows"])).abs().max()) <= 5e-6
    assert np.abs(o.double().sum(dim=(2, 3)).numpy() - z["o_sum"]).max() <= 1e-3


def _stable_src(k, plan):
    """Relay rows by the CPU path's rule: norms as (k * k).sum(-1) in the input
    dtype (the reference's expression, cpu_reference.py:261), descending,
    the earlier row first on equal norms; zero-padded last block."""
    B, H, S, D = k.shape
    W, NB = plan.W, plan.num_blocks
    pad = NB * W - S
    kp = torch.nn.functional.pad(k, (0, 0, 0, pad)) if pad > 0 else k
    nsq = (kp * kp).sum(dim=-1).float().view(B, H, NB, W).numpy()
    order = np.argsort(-nsq, axis=-1, kind="stable")[..., :min(2, W)]
    base = (np.arange(NB) * W).reshape(1, 1, NB, 1)
    return torch.from_numpy((order + base).reshape(B, H, -1))


def _oracle_cpu_mode(q, k, v, kv_groups=1, src_rule="torch"):
    plan = O.make_plan(q.shape[2], "cpu_reference")
    src = O.relay_select(k, plan, "torch") if src_rule == "torch" else _stable_src(k, plan)
    o, _, _ = O.forward(q, k, v, plan, kv_groups=kv_groups, src=src)
    return o


def test_stable_rule_equals_topk_without_ties():
    """On fp32 inputs (no equal norms) the stated rule is torch's topk."""
    g = torch.Generator().manual_seed(0)
    k = torch.randn(1, 3, 2000, 64, generator=g)
    plan = O.make_plan(2000, "cpu_reference")
    assert torch.equal(_stable_src(k, plan), O.relay_select(k, plan, "torch"))


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-5), (torch.float16, 2e-3),
                                       (torch.bfloat16, 3e-2)])
@pytest.mark.parametrize("S,D,Hq,Hkv", [(1500, 64, 2, 2), (700, 48, 4, 2), (5, 16, 1, 1),
                                        (130, 128, 2, 1)])
def test_cpu_path_matches_oracle(dtype, tol, S, D, Hq, Hkv):
    g = torch.Generator().manual_seed(S + D)
    q, k, v = (torch.randn(1, h, S, D, generator=g).to(dtype) for h in (Hq, Hkv, Hkv))
    o = cra.cron_root_attention(q, k, v)
    assert o.dtype == dtype and o.shape == q.shape
    ref = _oracle_cpu_mode(q, k, v, kv_groups=Hq // Hkv,
                           src_rule="torch" if dtype == torch.float32 else "stable")
    assert float((o.double() - ref).abs().max()) <= tol


def test_cpu_path_strided_views_and_ignored_gpu_arguments():
    """Strided [B, H, S, D] views compute the same as contiguous copies; the
    GPU-only arguments are ignored as in the reference's CPU dispatch."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 900, 3, 2, 32, generator=g)
    q, k, v = (x[:, :, i].transpose(1, 2) for i in range(3))
    o = cra.cron_root_attention(q, k, v, use_persistent=True, relay_top_k=3,
                                relay_log_scale=torch.zeros(2))
    assert torch.equal(o, cra.cron_root_attention(q.contiguous(), k.contiguous(), v.contiguous()))
    assert torch.allclose(o.double(), _oracle_cpu_mode(q, k, v), atol=2e-5, rtol=0)


def test_cpu_path_tiny_sequences():
    """S < 4 (window 1, one relay row per block): finite output; row 0 is v_0.
    (The reference's CPU path raises a shape error there: its relay mask
    assumes two rows per block, cpu_reference.py:276-278.)"""
    for S in (1, 2, 3):
        q, k, v = (torch.randn(1, 2, S, 16) for _ in range(3))
        o = cra.cron_root_attention(q, k, v)
        assert bool(torch.isfinite(o).all())
        assert torch.allclose(o[:, :, 0], v[:, :, 0])


def test_cpu_path_has_no_backward():
    q = torch.randn(1, 2, 100, 32, requires_grad=True)
    o = cra.cron_root_attention(q, q.detach(), q.detach())
    with pytest.raises(NotImplementedError, match="CPU"):
        o.sum().backward()


def test_cpu_path_rejects_bad_shapes():
    q = torch.randn(1, 3, 64, 32)
    with pytest.raises(ValueError):
        cra.cron_root_attention(q, torch.randn(1, 2, 64, 32), torch.randn(1, 2, 64, 32))
    with pytest.raises(TypeError):
        cra.cron_root_attention(q.double(), q.double(), q.double())
