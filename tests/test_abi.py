"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/cra.h declares, and rejects bad arguments with the documented codes
before touching the device."""
import ctypes
import math
import os
import re

import pytest

from cron_root_attention import _native as N

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "cra.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cra_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert set(declared_functions()) == set(N._SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = N.load_library()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.cra_abi_version() == N.ABI_VERSION


def test_strerror_covers_codes():
    lib = N.load_library()
    for code in (0, -1, -2, -3, -4, -5, -6):
        assert lib.cra_strerror(code) and lib.cra_strerror(code) != b"unknown error"
    assert lib.cra_strerror(-99) == b"unknown error"


def test_supported_head_dims():
    lib = N.load_library()
    assert [d for d in range(1, 600) if lib.cra_supported_head_dim(d)] == [32, 64, 128, 256]


def prob(**kw):
    base = dict(B=1, H_q=4, H_kv=2, S=5000, D=128, W=71, relay=1, top_k=2, dtype=0, scale=0.088)
    base.update(kw)
    return N.CraProblem(**base)


def test_global_rows():
    lib = N.load_library()
    nb = (5000 + 70) // 71
    assert lib.cra_global_rows(ctypes.byref(prob())) == nb * 3
    assert lib.cra_global_rows(ctypes.byref(prob(relay=0))) == nb
    assert lib.cra_global_rows(ctypes.byref(prob(top_k=4))) == nb * 5


@pytest.mark.parametrize("kw,code,msg", [
    (dict(dtype=7), N.E_DTYPE, "dtype"),
    (dict(D=48), N.E_UNSUPPORTED, "head dim"),
    (dict(H_kv=3), N.E_INVALID, "multiple"),
    (dict(W=0), N.E_INVALID, "window"),
    (dict(W=6000), N.E_INVALID, "window"),
    (dict(top_k=5), N.E_INVALID, "top_k"),
    (dict(S=0), N.E_INVALID, ">= 1"),
    (dict(scale=0.0), N.E_INVALID, "scale"),
])
def test_fwd_rejects_bad_problem(kw, code, msg):
    lib = N.load_library()
    t = N.CraTensor(0x10000, 1 << 20, 1 << 16, 128)
    rc = lib.cra_fwd(ctypes.byref(prob(**kw)), t, t, t, 0x10000, 0x10000, t, 0x10000, None)
    assert rc == code
    assert msg in lib.cra_last_error().decode()


def test_fwd_rejects_bad_layout():
    lib = N.load_library()
    good = N.CraTensor(0x10000, 1 << 20, 1 << 16, 128)
    odd_ptr = N.CraTensor(0x10002, 1 << 20, 1 << 16, 128)
    odd_stride = N.CraTensor(0x10000, 1 << 20, 1 << 16, 130)
    null = N.CraTensor(None, 1 << 20, 1 << 16, 128)
    p = ctypes.byref(prob())
    assert lib.cra_fwd(p, odd_ptr, good, good, 0x10000, 0x10000, good, 0x10000, None) == N.E_LAYOUT
    assert lib.cra_fwd(p, good, odd_stride, good, 0x10000, 0x10000, good, 0x10000, None) == N.E_LAYOUT
    assert lib.cra_fwd(p, good, good, null, 0x10000, 0x10000, good, 0x10000, None) == N.E_INVALID
    assert lib.cra_fwd(p, good, good, good, 0x10000, 0x10000, good, None, None) == N.E_INVALID


def test_fwd_phases_rejects_bad_mask():
    lib = N.load_library()
    good = N.CraTensor(0x10000, 1 << 20, 1 << 16, 128)
    p = ctypes.byref(prob())
    for mask in (0, 4, -1, 7):
        rc = lib.cra_fwd_phases(p, good, good, good, 0x10000, 0x10000, good, 0x10000, mask, None)
        assert rc == N.E_INVALID, mask
        assert "phase_mask" in lib.cra_last_error().decode()


def test_head_span_limit():
    # k and v are read through buffer resources with 32-bit offsets: a head
    # spanning 2^31 bytes or more is rejected (the Python layer then passes a
    # contiguous copy)
    lib = N.load_library()
    good = N.CraTensor(0x10000, 1 << 20, 1 << 16, 128)
    wide = N.CraTensor(0x10000, 1 << 40, 1 << 35, 1 << 18)  # row stride 512 KiB elements
    p = ctypes.byref(prob())
    assert lib.cra_fwd(p, good, wide, good, 0x10000, 0x10000, good, 0x10000, None) == N.E_LAYOUT
    assert "2^31" in lib.cra_last_error().decode()
    need = lib.cra_bwd_workspace_bytes(p)
    for pos in range(3):
        args = [good] * 3
        args[pos] = wide
        rc = lib.cra_bwd(p, *args, good, good, 0x10000, 0x10000, 0x10000, 0x10000, None, good,
                         good, good, None, 0x10000, need, None)
        assert rc == N.E_LAYOUT and "2^31" in lib.cra_last_error().decode(), pos
    rc = lib.cra_bwd(p, good, good, good, good, wide, 0x10000, 0x10000, 0x10000, 0x10000, None,
                     good, good, good, None, 0x10000, need, None)
    assert rc == N.E_LAYOUT and "dout" in lib.cra_last_error().decode()


def _chunks(lib, **kw):
    """Query chunks of the global-row kernel that cra_bwd_workspace_bytes
    planned: the workspace is -Delta and -lse*log2(e) (fp32 per query, each
    256-byte aligned) followed by nchunk fp32 partials of 2*D per global row."""
    p = prob(**kw)
    need = lib.cra_bwd_workspace_bytes(ctypes.byref(p))
    per_query = (p.B * p.H_q * p.S * 4 + 255) // 256 * 256
    per_chunk = p.B * p.H_kv * lib.cra_global_rows(ctypes.byref(p)) * 2 * p.D * 4
    assert (need - 2 * per_query) % per_chunk == 0
    return (need - 2 * per_query) // per_chunk


def test_global_row_chunk_rule():
    """About 1.5 rounds of the global-row kernel's resident workgroups (256
    CUs; one 192-row workgroup per CU at D = 128, two 128-row ones below), at
    least one chunk per 6144 queries, at most one per 256 (the shapes of the
    measured sweep)."""
    lib = N.load_library()
    w = lambda S: int(math.ceil(math.sqrt(S)))
    assert _chunks(lib, B=1, H_q=16, H_kv=16, S=131072, D=128, W=w(131072)) == 22
    assert _chunks(lib, B=1, H_q=12, H_kv=12, S=8192, D=64, W=w(8192)) == 22
    assert _chunks(lib, B=1, H_q=12, H_kv=12, S=32768, D=64, W=w(32768)) == 13
    assert _chunks(lib, B=2, H_q=32, H_kv=32, S=4096, D=128, W=w(4096)) == 6
    assert _chunks(lib, B=2, H_q=32, H_kv=32, S=65536, D=128, W=w(65536)) == 11
    assert _chunks(lib, B=1, H_q=8, H_kv=8, S=16384, D=64, W=w(16384)) == 32
    # short sequences: at most one chunk per 256 queries
    assert _chunks(lib, B=1, H_q=1, H_kv=1, S=200, D=64, W=w(200), relay=0) == 1


def test_bwd_rejects_small_workspace():
    lib = N.load_library()
    t = N.CraTensor(0x10000, 1 << 20, 1 << 16, 128)
    p = ctypes.byref(prob())
    need = lib.cra_bwd_workspace_bytes(p)
    assert need > 0
    rc = lib.cra_bwd(p, t, t, t, t, t, 0x10000, 0x10000, 0x10000, 0x10000, None, t, t, t, None,
                     0x10000, need - 1, None)
    assert rc == N.E_WORKSPACE and str(need) in lib.cra_last_error().decode()
    rc = lib.cra_bwd(p, t, t, t, t, t, 0x10000, 0x10000, 0x10000, None, None, t, t, t, None,
                     0x10000, need, None)
    assert rc == N.E_INVALID  # relay on needs relay_src


def test_build_global_requires_src_with_relay():
    lib = N.load_library()
    t = N.CraTensor(0x10000, 1 << 20, 1 << 16, 128)
    rc = lib.cra_build_global(ctypes.byref(prob()), t, t, 0x10000, 0x10000, None, None, None)
    assert rc == N.E_INVALID and "relay_src" in lib.cra_last_error().decode()


# ------------------------------------------------------------------ varlen

def vprob(S, **kw):
    base = dict(B=2, H_q=4, H_kv=2, S=S, D=64, W=0, relay=0, top_k=2, dtype=0, scale=0.125)
    base.update(kw)
    return N.CraProblem(**base)


def sizes(p, docs):
    lib = N.load_library()
    g, r = ctypes.c_int64(-1), ctypes.c_int64(-1)
    rc = lib.cra_varlen_sizes(ctypes.byref(p), ctypes.byref(docs.struct), ctypes.byref(g),
                              ctypes.byref(r))
    return rc, g.value, r.value


def test_varlen_sizes():
    docs = N.Docs([0, 100, 2149, 5149], [10, 46, 55], [0, 1, 1])
    rc, g, r = sizes(vprob(5149), docs)
    assert rc == N.OK
    assert g == 10 + 45 * 3 + 55 * 3          # blocks x (1 + top_k) for relay documents
    assert r == (10 + 45 + 55) * 2            # relay_src entries span every document's blocks
    rc, g, r = sizes(vprob(5149, top_k=9), N.Docs([0, 100, 2149, 5149], [10, 46, 55], [0, 0, 0]))
    assert rc == N.OK and g == 110 and r == 0  # top_k is only checked when a document relays


def test_varlen_one_document_matches_plain_sizes():
    lib = N.load_library()
    p = prob()
    docs = N.Docs([0, p.S], [p.W], [p.relay])
    rc, g, _ = sizes(p, docs)
    assert rc == N.OK and g == lib.cra_global_rows(ctypes.byref(p))
    assert (lib.cra_bwd_workspace_bytes_varlen(ctypes.byref(p), ctypes.byref(docs.struct))
            == lib.cra_bwd_workspace_bytes(ctypes.byref(p)))


@pytest.mark.parametrize("cu,W,R,kw,msg", [
    ([1, 50, 100], [5, 5], [0, 0], {}, "from 0"),
    ([0, 50, 99], [5, 5], [0, 0], {}, "from 0"),
    ([0, 60, 60, 100], [5, 5, 5], [0, 0, 0], {}, "rise strictly"),
    ([0, 50, 100], [0, 5], [0, 0], {}, "window"),
    ([0, 50, 100], [5, 51], [0, 0], {}, "window"),
    ([0, 50, 100], [5, 5], [0, 2], {}, "relay"),
    ([0, 50, 100], [5, 5], [0, 1], dict(top_k=5), "top_k"),
])
def test_varlen_rejects_bad_documents(cu, W, R, kw, msg):
    lib = N.load_library()
    rc, _, _ = sizes(vprob(100, **kw), N.Docs(cu, W, R))
    assert rc == N.E_INVALID
    assert msg in lib.cra_last_error().decode()


def test_varlen_rejects_missing_arrays():
    lib = N.load_library()
    p = vprob(100)
    bad = N.CraDocs(2, None, None, None)
    assert lib.cra_varlen_sizes(ctypes.byref(p), ctypes.byref(bad), None, None) == N.E_INVALID
    assert lib.cra_varlen_sizes(ctypes.byref(p), None, None, None) == N.E_INVALID
    zero = N.Docs([0], [], [])
    assert lib.cra_varlen_sizes(ctypes.byref(p), ctypes.byref(zero.struct), None, None) == N.E_INVALID
    assert lib.cra_bwd_workspace_bytes_varlen(ctypes.byref(p), ctypes.byref(bad)) == 0


def test_varlen_entry_points_validate_before_launch():
    lib = N.load_library()
    t = N.CraTensor(0x10000, 1 << 20, 1 << 16, 64)
    p = vprob(100)
    docs = N.Docs([0, 30, 100], [6, 9], [0, 1])
    d = ctypes.byref(docs.struct)
    rc = lib.cra_build_global_varlen(ctypes.byref(p), d, t, t, 0x10000, 0x10000, None, None, None)
    assert rc == N.E_INVALID and "relay_src" in lib.cra_last_error().decode()
    odd = N.CraTensor(0x10002, 1 << 20, 1 << 16, 64)
    rc = lib.cra_fwd_varlen(ctypes.byref(p), d, odd, t, t, 0x10000, 0x10000, t, 0x10000, None)
    assert rc == N.E_LAYOUT
    need = lib.cra_bwd_workspace_bytes_varlen(ctypes.byref(p), d)
    assert need > 0
    rc = lib.cra_bwd_varlen(ctypes.byref(p), d, t, t, t, t, t, 0x10000, 0x10000, 0x10000,
                            0x10000, None, t, t, t, None, 0x10000, need - 1, None)
    assert rc == N.E_WORKSPACE


def test_bwd_noalloc_rejects_problems_beyond_its_scratch():
    """cra_bwd_noalloc refuses, before touching a device, a problem whose
    workspace exceeds the fixed scratch even with one query chunk (here Delta
    alone is 1 GiB), and validates the problem like cra_bwd."""
    lib = N.load_library()
    t = N.CraTensor(0x10000, 1 << 26, 1 << 19, 128)
    big = prob(B=8, H_q=64, H_kv=64, S=524288, W=725)
    rc = lib.cra_bwd_noalloc(ctypes.byref(big), t, t, t, t, t, 0x10000, 0x10000, 0x10000, 0x10000,
                             None, t, t, t, None, None)
    assert rc == N.E_WORKSPACE
    assert "scratch" in lib.cra_last_error().decode()
    rc = lib.cra_bwd_noalloc(ctypes.byref(prob(top_k=9)), t, t, t, t, t, 0x10000, 0x10000,
                             0x10000, 0x10000, None, t, t, t, None, None)
    assert rc == N.E_INVALID


def test_tile_config_reports_compiled_geometry():
    """cra_tile_config (serves calibrate()): the geometry of the kernels as
    built; a workgroup's rows are waves x rows per wave."""
    import torch
    for dt in (torch.float16, torch.bfloat16, torch.float32):
        for D in (32, 64, 128, 256):
            t = N.tile_config(dt, D)
            assert all(v > 0 for v in t.values())
            # 32 queries per wave; 16 at D = 256 (the generic kernels' register budget)
            assert t["fwd_queries"] == (16 if D == 256 else 32) * t["fwd_waves"]
    h256 = N.tile_config(torch.bfloat16, 256)
    assert (h256["fwd_waves"], h256["fwd_queries"], h256["fwd_key_tile"]) == (4, 64, 32)
    assert (h256["dq_queries"], h256["dkdv_global_rows"], h256["dkdv_local_keys"]) == (64, 64, 64)
    assert lib_tc_unsupported(512)
    h = N.tile_config(torch.float16, 128)
    assert (h["fwd_waves"], h["fwd_queries"], h["fwd_key_tile"]) == (4, 128, 64)
    assert (h["dkdv_global_waves"], h["dkdv_global_rows"]) == (12, 192)
    h64 = N.tile_config(torch.float16, 64)   # 4 waves per SIMD below D = 128
    assert (h64["dkdv_global_waves"], h64["dkdv_global_rows"]) == (8, 128)
    assert (h["dkdv_local_waves"], h["dkdv_local_keys"], h["dkdv_local_query_tile"]) == (4, 64, 32)
    # below D = 128 each local wave takes two 16-key blocks
    assert (h64["dkdv_local_waves"], h64["dkdv_local_keys"]) == (4, 128)
    lib = N.load_library()
    out = N.CraTileConfig()
    assert lib.cra_tile_config(0, 48, ctypes.byref(out)) == N.E_UNSUPPORTED
    assert lib.cra_tile_config(9, 64, ctypes.byref(out)) == N.E_DTYPE
    import cron_root_attention as cra
    cfg = cra.calibrate(16, 128, verbose=False)
    assert cfg == {"fwd": (h["fwd_waves"], 2), "bwd": (h["dq_waves"], 2)}   # reference's keys
    # the generic kernels (fp32, D = 256) stage one tile at a time
    assert cra.calibrate(16, 200, dtype=torch.float16, verbose=False) == {"fwd": (4, 1),
                                                                          "bwd": (4, 1)}


def lib_tc_unsupported(D):
    out = N.CraTileConfig()
    return N.load_library().cra_tile_config(0, D, ctypes.byref(out)) == N.E_UNSUPPORTED


def test_fwd_persistent_requires_a_counter():
    lib = N.load_library()
    t = N.CraTensor(0x10000, 1 << 20, 1 << 16, 128)
    rc = lib.cra_fwd_persistent(ctypes.byref(prob(relay=0)), t, t, t, 0x10000, 0x10000, t,
                                0x10000, None, None)
    assert rc == N.E_INVALID and "work_counter" in lib.cra_last_error().decode()
