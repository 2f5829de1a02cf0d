"""The public op under caller-side HIP graph capture (GPU).

A training step, forward and backward of `cron_root_attention`, is captured
with `torch.cuda.graph` after the usual side-stream warm-up, then replayed
three times on new inputs copied into the captured buffers; between
replays the same step runs eagerly on the same inputs, and every replay's
output and gradients must equal the eager ones bit for bit (the kernels are
deterministic and launch only on the current stream; nothing in the path
records a memset or synchronises). The eager path itself is checked
against the oracle elsewhere (test_parity_gpu.py); the first eager step
here is compared with the oracle as well.
"""
import pytest
import torch

import cron_root_attention as cra
from tests.parity_util import F16, BF16, DEV, check_forward, inputs, plan_for, say

pytestmark = pytest.mark.gpu


def _eager(q, k, v, do, kv_groups):
    qe, ke, ve = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = cra.cron_root_attention(qe, ke, ve, kv_groups=kv_groups)
    o.backward(do)
    return o.detach(), qe.grad, ke.grad, ve.grad


@pytest.mark.parametrize("dtype,B,Hq,Hkv,S,D", [(F16, 1, 4, 4, 3000, 128),
                                              (BF16, 2, 4, 2, 1500, 64)])
def test_training_step_replays_match_eager(dtype, B, Hq, Hkv, S, D):
    say(f"graph capture: {dtype} B={B} Hq={Hq} Hkv={Hkv} S={S} D={D}")
    groups = Hq // Hkv
    q0, k0, v0, do0 = inputs(B, Hq, Hkv, S, D, dtype, seed=11)
    q, k, v = (t.to(DEV).requires_grad_(True) for t in (q0, k0, v0))
    do = do0.to(DEV)

    ref = _eager(q, k, v, do, groups)
    check_forward(ref[0], q0, k0, v0, plan_for(S), dtype, kv_groups=groups)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            q.grad = k.grad = v.grad = None
            cra.cron_root_attention(q, k, v, kv_groups=groups).backward(do)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    q.grad = k.grad = v.grad = None
    with torch.cuda.graph(graph):
        o_static = cra.cron_root_attention(q, k, v, kv_groups=groups)
        o_static.backward(do)
    grads = (q.grad, k.grad, v.grad)

    gen = torch.Generator(device=DEV).manual_seed(5)
    for rep in range(3):
        with torch.no_grad():
            for t in (q, k, v, do):
                t.copy_(torch.randn(t.shape, generator=gen, device=DEV, dtype=torch.float32))
        graph.replay()
        torch.cuda.synchronize()
        want = _eager(q, k, v, do, groups)
        torch.cuda.synchronize()
        for name, got, exp in zip(("o", "dq", "dk", "dv"), (o_static,) + grads, want):
            assert torch.equal(got, exp), f"replay {rep}: {name}"
        say(f"  replay {rep}: o, dq, dk, dv bit-identical to the eager step")
