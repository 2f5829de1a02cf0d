"""ctypes binding of libcra_hip.so (the C ABI declared in include/cra.h).

PyTorch supplies device memory and the current HIP stream; every buffer is
allocated here with torch and passed to the library as a raw pointer plus
element strides.  The library itself allocates nothing and never
synchronises.

If the library is missing or cannot be loaded every entry point raises
:class:`CraLibraryError`: there is no fallback computation.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

_LIB_NAME = "libcra_hip.so"
_lock = threading.Lock()
_lib = None
_lib_error: Optional[str] = None

F16, BF16, F32 = 0, 1, 2
_DTYPE_CODE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}

# return codes (include/cra.h)
OK, E_INVALID, E_LAYOUT, E_DTYPE, E_UNSUPPORTED, E_HIP, E_WORKSPACE = 0, -1, -2, -3, -4, -5, -6


class CraError(RuntimeError):
    """A libcra_hip call returned an error code."""

    def __init__(self, code: int, func: str, message: str):
        self.code = code
        super().__init__(f"{func}: {message} (code {code})")


class CraLibraryError(RuntimeError):
    """libcra_hip.so is missing or cannot be loaded."""


class CraProblem(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32), ("H_q", ctypes.c_int32), ("H_kv", ctypes.c_int32),
        ("S", ctypes.c_int32), ("D", ctypes.c_int32), ("W", ctypes.c_int32),
        ("relay", ctypes.c_int32), ("top_k", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("scale", ctypes.c_float),
    ]


class CraTensor(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("sb", ctypes.c_int64), ("sh", ctypes.c_int64),
                ("ss", ctypes.c_int64)]


class CraDocs(ctypes.Structure):
    _fields_ = [("n_docs", ctypes.c_int32), ("cu_seqlens", ctypes.POINTER(ctypes.c_int32)),
                ("window", ctypes.POINTER(ctypes.c_int32)),
                ("relay", ctypes.POINTER(ctypes.c_int32))]


class Docs:
    """Host-side document table of a varlen call (keeps the int32 arrays alive)."""

    def __init__(self, cu_seqlens, window, relay):
        n = len(cu_seqlens) - 1
        self._cu = (ctypes.c_int32 * (n + 1))(*cu_seqlens)
        self._w = (ctypes.c_int32 * n)(*window)
        self._r = (ctypes.c_int32 * n)(*(int(x) for x in relay))
        self.cu_seqlens = list(cu_seqlens)
        self.window = list(window)
        self.relay = [bool(x) for x in relay]
        self.struct = CraDocs(n, self._cu, self._w, self._r)

    @property
    def n_docs(self) -> int:
        return len(self.window)


class CraDeviceInfo(ctypes.Structure):
    _fields_ = [("cu_count", ctypes.c_int32), ("lds_bytes_per_cu", ctypes.c_int32),
                ("arch_major", ctypes.c_int32), ("arch_minor", ctypes.c_int32),
                ("arch_name", ctypes.c_char * 64), ("device_name", ctypes.c_char * 128)]


class CraTileConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "fwd_waves", "fwd_queries", "fwd_key_tile", "dq_waves", "dq_queries", "dq_key_tile",
        "dkdv_global_waves", "dkdv_global_rows", "dkdv_global_query_tile",
        "dkdv_local_waves", "dkdv_local_keys", "dkdv_local_query_tile")]


# Exported symbols and their signatures (mirrors include/cra.h).
_P = ctypes.POINTER(CraProblem)
_D = ctypes.POINTER(CraDocs)
_SIGNATURES = {
    "cra_supported_head_dim": (ctypes.c_int, [ctypes.c_int32]),
    "cra_global_rows": (ctypes.c_int64, [_P]),
    "cra_build_global": (ctypes.c_int, [_P, CraTensor, CraTensor, ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "cra_fwd": (ctypes.c_int, [_P, CraTensor, CraTensor, CraTensor, ctypes.c_void_p,
                               ctypes.c_void_p, CraTensor, ctypes.c_void_p, ctypes.c_void_p]),
    "cra_fwd_phases": (ctypes.c_int, [_P, CraTensor, CraTensor, CraTensor, ctypes.c_void_p,
                                      ctypes.c_void_p, CraTensor, ctypes.c_void_p, ctypes.c_int32,
                                      ctypes.c_void_p]),
    "cra_fwd_persistent": (ctypes.c_int, [_P, CraTensor, CraTensor, CraTensor, ctypes.c_void_p,
                                          ctypes.c_void_p, CraTensor, ctypes.c_void_p,
                                          ctypes.c_void_p, ctypes.c_void_p]),
    "cra_bwd_workspace_bytes": (ctypes.c_size_t, [_P]),
    "cra_bwd": (ctypes.c_int, [_P, CraTensor, CraTensor, CraTensor, CraTensor, CraTensor,
                               ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                               ctypes.c_void_p, CraTensor, CraTensor, CraTensor, ctypes.c_void_p,
                               ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "cra_bwd_noalloc": (ctypes.c_int, [_P, CraTensor, CraTensor, CraTensor, CraTensor, CraTensor,
                                       ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_void_p, ctypes.c_void_p, CraTensor, CraTensor,
                                       CraTensor, ctypes.c_void_p, ctypes.c_void_p]),
    "cra_varlen_sizes": (ctypes.c_int, [_P, _D, ctypes.POINTER(ctypes.c_int64),
                                        ctypes.POINTER(ctypes.c_int64)]),
    "cra_build_global_varlen": (ctypes.c_int, [_P, _D, CraTensor, CraTensor, ctypes.c_void_p,
                                               ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_void_p]),
    "cra_fwd_varlen": (ctypes.c_int, [_P, _D, CraTensor, CraTensor, CraTensor, ctypes.c_void_p,
                                      ctypes.c_void_p, CraTensor, ctypes.c_void_p,
                                      ctypes.c_void_p]),
    "cra_bwd_workspace_bytes_varlen": (ctypes.c_size_t, [_P, _D]),
    "cra_bwd_varlen": (ctypes.c_int, [_P, _D, CraTensor, CraTensor, CraTensor, CraTensor,
                                      CraTensor, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                      CraTensor, CraTensor, CraTensor, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "cra_device_info": (ctypes.c_int, [ctypes.c_int32, ctypes.POINTER(CraDeviceInfo)]),
    "cra_tile_config": (ctypes.c_int, [ctypes.c_int32, ctypes.c_int32,
                                       ctypes.POINTER(CraTileConfig)]),
    "cra_fwd_cpu": (ctypes.c_int, [_P, CraTensor, CraTensor, CraTensor, CraTensor,
                                   ctypes.c_int32]),
    "cra_strerror": (ctypes.c_char_p, [ctypes.c_int32]),
    "cra_last_error": (ctypes.c_char_p, []),
    "cra_abi_version": (ctypes.c_int32, []),
}
ABI_VERSION = 1


def library_path() -> str:
    return os.environ.get("CRA_HIP_LIBRARY",
                          os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_NAME))


def load_library():
    """Load (once) and return the ctypes handle; raise CraLibraryError if absent."""
    global _lib, _lib_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise CraLibraryError(
                f"{path} not found: build it with `python cron-root-attention_amd/build.py` "
                "(this package has no non-HIP fallback)")
        try:
            lib = ctypes.CDLL(path)
        except OSError as e:
            raise CraLibraryError(f"cannot load {path}: {e}") from e
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.cra_abi_version() != ABI_VERSION:
            raise CraLibraryError(f"{path}: ABI {lib.cra_abi_version()} != {ABI_VERSION}")
        _lib = lib
        return lib


_TORCH_LIB_NAME = "libcra_torch.so"
_op_state = {"tried": False, "op": None, "error": None}


def torch_op_path() -> str:
    return os.environ.get("CRA_TORCH_LIBRARY",
                          os.path.join(os.path.dirname(os.path.abspath(__file__)), _TORCH_LIB_NAME))


def attention_op():
    """``torch.ops.cra.attention`` bound to the loaded libcra_hip.so, or None
    when libcra_torch.so is absent (then the Python autograd Function serves
    every call; both launch the same kernels through the same C ABI)."""
    if _op_state["tried"]:
        return _op_state["op"]
    load_library()  # raises without the HIP library (takes _lock itself)
    with _lock:
        if not _op_state["tried"]:
            lib_path = library_path()
            path = torch_op_path()
            if os.path.exists(path):
                try:
                    torch.ops.load_library(path)
                    torch.ops.cra.bind(lib_path)
                    _op_state["op"] = torch.ops.cra.attention
                except (OSError, RuntimeError) as e:
                    _op_state["error"] = f"{path}: {e}"
            else:
                _op_state["error"] = f"{path} not found"
            _op_state["tried"] = True
    return _op_state["op"]


def _raise(code: int, func: str):
    lib = load_library()
    msg = (lib.cra_last_error() or b"").decode() or lib.cra_strerror(code).decode()
    if code in (E_INVALID, E_LAYOUT):
        raise ValueError(f"{func}: {msg}")
    if code == E_DTYPE:
        raise TypeError(f"{func}: {msg}")
    if code == E_UNSUPPORTED:
        raise NotImplementedError(f"{func}: {msg}")
    raise CraError(code, func, msg)


def _check(code: int, func: str):
    if code != OK:
        _raise(code, func)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; use float16, bfloat16 or float32") from None


_problems = {}


def problem(B, H_q, H_kv, S, D, W, relay, top_k, dtype, scale) -> CraProblem:
    """The cra_problem of a call; one shared (read-only) instance per
    distinct problem, with its derived sizes cached beside it."""
    key = (B, H_q, H_kv, S, D, W, bool(relay), top_k if relay else 0, dtype, float(scale))
    p = _problems.get(key)
    if p is None:
        p = CraProblem(B, H_q, H_kv, S, D, W, 1 if relay else 0, top_k if relay else 0,
                       dtype_code(dtype), float(scale))
        if len(_problems) > 4096:
            _problems.clear()
        _problems[key] = p
    return p


def _key(p: CraProblem):
    return (p.B, p.H_q, p.H_kv, p.S, p.D, p.W, p.relay, p.top_k, p.dtype, p.scale)


_sizes = {}


def tensor_arg(t: torch.Tensor) -> CraTensor:
    assert t.dim() == 4 and t.stride(3) == 1
    return CraTensor(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def supported_head_dim(D: int) -> bool:
    return bool(load_library().cra_supported_head_dim(D))


def global_rows(p: CraProblem) -> int:
    key = ("G",) + _key(p)
    n = _sizes.get(key)
    if n is None:
        n = load_library().cra_global_rows(ctypes.byref(p))
        if n < 0:
            _raise(E_INVALID, "cra_global_rows")
        n = _sizes[key] = int(n)
    return n


def build_global(p: CraProblem, k: torch.Tensor, v: torch.Tensor,
                 relay_scale: Optional[torch.Tensor], stream: Optional[int] = None):
    """Packed strided+relay rows (glob_k, glob_v) and relay source rows."""
    lib = load_library()
    G = global_rows(p)
    B, Hkv, D = p.B, p.H_kv, p.D
    gkv = torch.empty(2, B, Hkv, G, D, dtype=k.dtype, device=k.device)  # one allocation
    gk, gv = gkv[0], gkv[1]
    nb = (p.S + p.W - 1) // p.W
    src = (torch.empty(B, Hkv, nb * p.top_k, dtype=torch.int32, device=k.device)
           if p.relay else None)
    rs = relay_scale.data_ptr() if (relay_scale is not None and p.relay) else None
    _check(lib.cra_build_global(ctypes.byref(p), tensor_arg(k), tensor_arg(v), gk.data_ptr(),
                                gv.data_ptr(), src.data_ptr() if src is not None else None, rs,
                                _stream(k) if stream is None else stream), "cra_build_global")
    return gk, gv, src


PHASE_LOCAL = 1
PHASE_GLOBAL = 2


def forward(p: CraProblem, q, k, v, gk, gv, phases: int = PHASE_LOCAL | PHASE_GLOBAL,
            stream: Optional[int] = None):
    """cra_fwd (all phases) or cra_fwd_phases (a subset, for measurement)."""
    lib = load_library()
    st = _stream(q) if stream is None else stream
    o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty(p.B, p.H_q, p.S, dtype=torch.float32, device=q.device)
    if phases == PHASE_LOCAL | PHASE_GLOBAL:
        _check(lib.cra_fwd(ctypes.byref(p), tensor_arg(q), tensor_arg(k), tensor_arg(v),
                           gk.data_ptr(), gv.data_ptr(), tensor_arg(o), lse.data_ptr(),
                           st), "cra_fwd")
    else:
        _check(lib.cra_fwd_phases(ctypes.byref(p), tensor_arg(q), tensor_arg(k), tensor_arg(v),
                                  gk.data_ptr(), gv.data_ptr(), tensor_arg(o), lse.data_ptr(),
                                  phases, st), "cra_fwd_phases")
    return o, lse


def forward_persistent(p: CraProblem, q, k, v, gk, gv, stream: Optional[int] = None):
    """cra_fwd_persistent: the work-queue forward (a zeroed counter per call)."""
    lib = load_library()
    o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty(p.B, p.H_q, p.S, dtype=torch.float32, device=q.device)
    counter = torch.zeros(1, dtype=torch.int32, device=q.device)
    _check(lib.cra_fwd_persistent(ctypes.byref(p), tensor_arg(q), tensor_arg(k), tensor_arg(v),
                                  gk.data_ptr(), gv.data_ptr(), tensor_arg(o), lse.data_ptr(),
                                  counter.data_ptr(), _stream(q) if stream is None else stream),
           "cra_fwd_persistent")
    return o, lse


def workspace_bytes(p: CraProblem) -> int:
    key = ("ws",) + _key(p)
    n = _sizes.get(key)
    if n is None:
        n = _sizes[key] = int(load_library().cra_bwd_workspace_bytes(ctypes.byref(p)))
    return n


def backward(p: CraProblem, q, k, v, o, do, lse, gk, gv, src, relay_scale, want_dalpha: bool):
    lib = load_library()
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    nbytes = workspace_bytes(p)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    dalpha = (torch.empty(p.H_kv, dtype=torch.float32, device=q.device)
              if (want_dalpha and p.relay) else None)
    rs = relay_scale.data_ptr() if (relay_scale is not None and p.relay) else None
    _check(lib.cra_bwd(ctypes.byref(p), tensor_arg(q), tensor_arg(k), tensor_arg(v),
                       tensor_arg(o), tensor_arg(do), lse.data_ptr(), gk.data_ptr(),
                       gv.data_ptr(), src.data_ptr() if src is not None else None, rs,
                       tensor_arg(dq), tensor_arg(dk), tensor_arg(dv),
                       dalpha.data_ptr() if dalpha is not None else None, ws.data_ptr(),
                       ws.numel(), _stream(q)), "cra_bwd")
    return dq, dk, dv, dalpha


NOALLOC_SCRATCH_BYTES = 64 << 20   # CRA_NOALLOC_SCRATCH_BYTES


def backward_noalloc(p: CraProblem, q, k, v, o, do, lse, gk, gv, src, relay_scale,
                     want_dalpha: bool, out=None):
    """cra_bwd_noalloc: the backward without a workspace (the library's fixed
    per-device scratch). ``out`` = (dq, dk, dv) preallocated outputs, else
    they are allocated here."""
    lib = load_library()
    if out is None:
        out = (torch.empty(q.shape, dtype=q.dtype, device=q.device),
               torch.empty(k.shape, dtype=k.dtype, device=k.device),
               torch.empty(v.shape, dtype=v.dtype, device=v.device))
    dq, dk, dv = out
    dalpha = (torch.empty(p.H_kv, dtype=torch.float32, device=q.device)
              if (want_dalpha and p.relay) else None)
    rs = relay_scale.data_ptr() if (relay_scale is not None and p.relay) else None
    _check(lib.cra_bwd_noalloc(ctypes.byref(p), tensor_arg(q), tensor_arg(k), tensor_arg(v),
                               tensor_arg(o), tensor_arg(do), lse.data_ptr(), gk.data_ptr(),
                               gv.data_ptr(), src.data_ptr() if src is not None else None, rs,
                               tensor_arg(dq), tensor_arg(dk), tensor_arg(dv),
                               dalpha.data_ptr() if dalpha is not None else None, _stream(q)),
           "cra_bwd_noalloc")
    return dq, dk, dv, dalpha


# ---- varlen: one call over all documents packed along S -------------------

def varlen_sizes(p: CraProblem, docs: Docs):
    """(packed global rows, relay_src entries) per (b, kv head)."""
    g, r = ctypes.c_int64(0), ctypes.c_int64(0)
    _check(load_library().cra_varlen_sizes(ctypes.byref(p), ctypes.byref(docs.struct),
                                           ctypes.byref(g), ctypes.byref(r)), "cra_varlen_sizes")
    return int(g.value), int(r.value)


def build_global_varlen(p: CraProblem, docs: Docs, k: torch.Tensor, v: torch.Tensor,
                        relay_scale: Optional[torch.Tensor]):
    lib = load_library()
    G, nsrc = varlen_sizes(p, docs)
    gk = torch.empty(p.B, p.H_kv, G, p.D, dtype=k.dtype, device=k.device)
    gv = torch.empty_like(gk)
    src = (torch.empty(p.B, p.H_kv, nsrc, dtype=torch.int32, device=k.device)
           if nsrc > 0 else None)
    rs = relay_scale.data_ptr() if (relay_scale is not None and src is not None) else None
    _check(lib.cra_build_global_varlen(ctypes.byref(p), ctypes.byref(docs.struct), tensor_arg(k),
                                       tensor_arg(v), gk.data_ptr(), gv.data_ptr(),
                                       src.data_ptr() if src is not None else None, rs,
                                       _stream(k)), "cra_build_global_varlen")
    return gk, gv, src


def forward_varlen(p: CraProblem, docs: Docs, q, k, v, gk, gv):
    lib = load_library()
    o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty(p.B, p.H_q, p.S, dtype=torch.float32, device=q.device)
    _check(lib.cra_fwd_varlen(ctypes.byref(p), ctypes.byref(docs.struct), tensor_arg(q),
                              tensor_arg(k), tensor_arg(v), gk.data_ptr(), gv.data_ptr(),
                              tensor_arg(o), lse.data_ptr(), _stream(q)), "cra_fwd_varlen")
    return o, lse


def workspace_bytes_varlen(p: CraProblem, docs: Docs) -> int:
    return int(load_library().cra_bwd_workspace_bytes_varlen(ctypes.byref(p),
                                                             ctypes.byref(docs.struct)))


def backward_varlen(p: CraProblem, docs: Docs, q, k, v, o, do, lse, gk, gv, src, relay_scale,
                    want_dalpha: bool):
    lib = load_library()
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    nbytes = workspace_bytes_varlen(p, docs)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    dalpha = (torch.empty(p.H_kv, dtype=torch.float32, device=q.device)
              if (want_dalpha and src is not None) else None)
    rs = relay_scale.data_ptr() if (relay_scale is not None and src is not None) else None
    _check(lib.cra_bwd_varlen(ctypes.byref(p), ctypes.byref(docs.struct), tensor_arg(q),
                              tensor_arg(k), tensor_arg(v), tensor_arg(o), tensor_arg(do),
                              lse.data_ptr(), gk.data_ptr(), gv.data_ptr(),
                              src.data_ptr() if src is not None else None, rs, tensor_arg(dq),
                              tensor_arg(dk), tensor_arg(dv),
                              dalpha.data_ptr() if dalpha is not None else None, ws.data_ptr(),
                              ws.numel(), _stream(q)), "cra_bwd_varlen")
    return dq, dk, dv, dalpha


def forward_cpu(p: CraProblem, q, k, v, threads: int):
    """cra_fwd_cpu: the host forward of CPU tensors (plan in p)."""
    lib = load_library()
    o = torch.empty(q.shape, dtype=q.dtype)
    _check(lib.cra_fwd_cpu(ctypes.byref(p), tensor_arg(q), tensor_arg(k), tensor_arg(v),
                           tensor_arg(o), max(1, int(threads))), "cra_fwd_cpu")
    return o


def tile_config(dtype: torch.dtype, D: int) -> dict:
    """The compiled tile geometry for (dtype, D) (cra_tile_config)."""
    lib = load_library()
    out = CraTileConfig()
    _check(lib.cra_tile_config(dtype_code(dtype), D, ctypes.byref(out)), "cra_tile_config")
    return {n: getattr(out, n) for n, _ in CraTileConfig._fields_}


def device_info(index: int = 0) -> dict:
    lib = load_library()
    info = CraDeviceInfo()
    _check(lib.cra_device_info(index, ctypes.byref(info)), "cra_device_info")
    return {"cu_count": info.cu_count, "lds_bytes_per_cu": info.lds_bytes_per_cu,
            "arch": info.arch_name.decode(), "name": info.device_name.decode(),
            "arch_major": info.arch_major, "arch_minor": info.arch_minor}
