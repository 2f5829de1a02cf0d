"""The C++ operator binding (libcra_torch.so, torch.ops.cra.attention): it
loads, binds the HIP library, registers the schema, and the router sends only
calls it can serve to it (CPU; no kernel launch)."""
import math

import pytest
import torch

from cron_root_attention import _native, core


def test_operator_loads_and_binds():
    op = _native.attention_op()
    assert op is not None, _native._op_state["error"]
    schema = str(torch.ops.cra.attention.default._schema)
    assert schema == ("cra::attention(Tensor q, Tensor k, Tensor v, int window, bool relay, "
                      "int top_k, float scale) -> Tensor")


def test_operator_rejects_a_missing_library():
    with pytest.raises(RuntimeError, match="cannot load"):
        torch.ops.cra.bind("/nonexistent/libcra_hip.so")
    # the binding made at load time is kept
    assert _native.attention_op() is not None


def test_operator_binds_once(tmp_path):
    """Binding the library it is bound to again is a no-op; a different copy of
    the library is refused (a call in flight must not see the table change)."""
    assert _native.attention_op() is not None
    torch.ops.cra.bind(_native.library_path())
    other = tmp_path / "libcra_hip_copy.so"
    other.write_bytes(open(_native.library_path(), "rb").read())
    with pytest.raises(RuntimeError, match="already bound"):
        torch.ops.cra.bind(str(other))
    assert _native.attention_op() is not None


def _meta(shape, dtype=torch.float16, strides=None):
    # a tensor on the meta device stands in for a GPU tensor's shape/layout
    t = torch.empty(shape, dtype=dtype, device="meta")
    return t if strides is None else t.as_strided(shape, strides)


class _FakeCuda:
    """Duck-typed q/k/v with a 'cuda' device for the routing predicate."""

    def __init__(self, t, device="cuda:0", ptr=0):
        self._t, self.device, self._ptr = t, torch.device(device), ptr
        self.shape, self.dtype = t.shape, t.dtype

    def dim(self):
        return self._t.dim()

    def stride(self, i=None):
        return self._t.stride() if i is None else self._t.stride(i)

    def element_size(self):
        return self._t.element_size()

    def data_ptr(self):
        return self._ptr

    def contiguous(self):
        return _FakeCuda(self._t.contiguous(), str(self.device), self._ptr)


def _plan(q, k, v, **kw):
    args = dict(use_persistent=False, kv_groups=1, relay_top_k=2)
    args.update(kw)
    return core._op_plan(q, k, v, args["use_persistent"], args["kv_groups"], args["relay_top_k"])


def test_router_plans():
    f = lambda *s, **kw: _FakeCuda(_meta(s, **kw))
    q, k, v = f(1, 8, 4096, 64), f(1, 8, 4096, 64), f(1, 8, 4096, 64)
    assert _plan(q, k, v) == (64, True, 2, 1.0 / 8.0)
    q2 = f(1, 8, 2048, 128)
    assert _plan(q2, f(1, 8, 2048, 128), f(1, 8, 2048, 128)) == (46, False, 2,
                                                                  1.0 / math.sqrt(128))
    # GQA through the shapes
    assert _plan(f(2, 8, 100, 32), f(2, 2, 100, 32), f(2, 2, 100, 32), kv_groups=4)[:2] == (
        10, False)
    # what stays on the Python path
    assert _plan(f(1, 8, 100, 80), f(1, 8, 100, 80), f(1, 8, 100, 80)) is None       # padded D
    assert _plan(q2, f(1, 8, 2048, 128), f(1, 8, 2048, 128), use_persistent=True) is None
    assert _plan(q, k, v, relay_top_k=5) is None                                    # error path
    assert _plan(f(1, 8, 64, 64), f(1, 4, 64, 64), f(1, 4, 64, 64)) is None         # groups
    assert _plan(f(1, 2, 64, 64, dtype=torch.float64), f(1, 2, 64, 64, dtype=torch.float64),
                 f(1, 2, 64, 64, dtype=torch.float64)) is None
    cpu = _FakeCuda(_meta((1, 2, 64, 64)), device="cpu")
    assert _plan(cpu, cpu, cpu) is None
    # a layout the kernels cannot take as it is (D not contiguous): the
    # operator copies it, as the Function does
    odd = _FakeCuda(_meta((1, 2, 64, 64), strides=(8192, 4096, 1, 64)))
    assert _plan(odd, odd, odd) == (8, False, 2, 1.0 / 8.0)
