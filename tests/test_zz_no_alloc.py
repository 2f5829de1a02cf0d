"""cra_bwd_noalloc (the backward without a workspace argument, on the
library's fixed per-device scratch) against cra_bwd through the C ABI.

Two calls in a row, the second smaller, each compared with cra_bwd on the
same inputs: bit-identical where cra_bwd's query-chunk count fits the
scratch; with fewer chunks (a problem whose planned workspace is larger
than the scratch) dQ is still bit-identical and dK/dV agree to the fp16
gradient tolerance (only the fp32 summation order of the chunk partials
differs).  Outputs are filled with NaN first, so a missed write shows.
"""
import math

import pytest
import torch

from cron_root_attention import _native
from tests.parity_util import F16, BF16, inputs, rel_fro, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(B, Hq, Hkv, S, D, dtype, seed, alpha=None):
    q, k, v, do = (t.to(DEV) for t in inputs(B, Hq, Hkv, S, D, dtype, seed))
    W = int(math.ceil(math.sqrt(S)))
    relay = S > 2048
    p = _native.problem(B, Hq, Hkv, S, D, W, relay, 2, dtype, 1 / math.sqrt(D))
    rs = (alpha.exp().to(dtype).float().to(DEV).contiguous() if (alpha is not None and relay)
          else None)
    gk, gv, src = _native.build_global(p, k, v, rs)
    o, lse = _native.forward(p, q, k, v, gk, gv)
    return p, (q, k, v, o, do, lse, gk, gv, src, rs)


def _nan_like(t):
    return torch.full_like(t, float("nan"))


def _compare(p, args, want_dalpha, exact):
    q, k, v = args[:3]
    ref = _native.backward(p, *args, want_dalpha)
    out = (_nan_like(q), _nan_like(k), _nan_like(v))
    got = _native.backward_noalloc(p, *args, want_dalpha, out=out)
    torch.cuda.synchronize()
    assert torch.equal(got[0], ref[0]), "dq"
    for name, a, b in (("dk", got[1], ref[1]), ("dv", got[2], ref[2])):
        assert bool(torch.isfinite(a).all()), name
        if exact:
            assert torch.equal(a, b), name
        else:
            e = rel_fro(a, b)
            say(f"  {name}: rel {e:.3e} against cra_bwd")
            assert e <= 1e-2, name
    if want_dalpha and p.relay:
        if exact:
            assert torch.equal(got[3], ref[3])
        else:
            assert rel_fro(got[3], ref[3]) <= 1e-2


def test_noalloc_matches_cra_bwd_two_calls():
    """Two calls in a row, the second with a smaller input: bit-identical to
    cra_bwd (both fit the scratch with cra_bwd's own chunk count)."""
    say("noalloc call 1: B=1 Hq=4 Hkv=2 S=8192 D=64 fp16, relay scale")
    alpha = torch.tensor([0.3, -0.2])
    p, args = _setup(1, 4, 2, 8192, 64, F16, seed=1, alpha=alpha)
    assert _native.workspace_bytes(p) <= _native.NOALLOC_SCRATCH_BYTES
    _compare(p, args, want_dalpha=True, exact=True)
    say("noalloc call 2 (smaller): B=1 Hq=2 Hkv=2 S=3000 D=128 bf16")
    p2, args2 = _setup(1, 2, 2, 3000, 128, BF16, seed=2)
    _compare(p2, args2, want_dalpha=False, exact=True)


def test_noalloc_fewer_chunks_when_planned_workspace_is_larger():
    """A problem whose planned workspace exceeds the scratch runs with fewer
    query chunks; then a smaller one that fits runs bit-identical again."""
    say("noalloc: B=1 H=16 S=65536 D=128 fp16 (planned workspace > scratch)")
    p, args = _setup(1, 16, 16, 65536, 128, F16, seed=3)
    assert _native.workspace_bytes(p) > _native.NOALLOC_SCRATCH_BYTES
    _compare(p, args, want_dalpha=False, exact=False)
    say("noalloc: then B=1 H=2 S=2500 D=64 fp16")
    p2, args2 = _setup(1, 2, 2, 2500, 64, F16, seed=4)
    _compare(p2, args2, want_dalpha=False, exact=True)


def test_noalloc_allocates_nothing_when_warm():
    """A warm call with caller-provided outputs takes no device memory: the
    torch allocator's count and the device's free memory are unchanged
    across a second call. (Problems beyond the scratch are refused before
    any launch: the CPU test test_abi.py::test_bwd_noalloc_rejects_problems_beyond_its_scratch.)"""
    say("noalloc: allocation check, B=1 H=4 S=4096 D=128 fp16")
    p, args = _setup(1, 4, 4, 4096, 128, F16, seed=6)
    q, k, v = args[:3]
    out = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v))
    _native.backward_noalloc(p, *args, False, out=out)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    alloc0 = torch.cuda.memory_allocated()
    _native.backward_noalloc(p, *args, False, out=out)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert torch.cuda.memory_allocated() == alloc0
    assert free1 == free0, (free0, free1)
    ref = _native.backward(p, *args, False)
    for a, b in zip(out, ref[:3]):
        assert torch.equal(a, b)
