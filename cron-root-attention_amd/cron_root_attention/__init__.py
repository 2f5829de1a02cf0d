"""sqrt(N) sparse causal attention for MI355X (gfx950), drop-in for the
reference package's public API (reference __init__.py:206-222).

    from cron_root_attention import cron_root_attention, CronRootAttention
    o = cron_root_attention(q, k, v)          # q, k, v: [B, H, S, D] on a ROCm GPU

All compute runs in the hand-written HIP library ``libcra_hip.so`` next to
this file (build: ``python cron-root-attention_amd/build.py``).
"""

__version__ = "0.1.0"

import torch as _torch

from .core import (GPU_SM_MAP, CronRootAttentionV14, CronRootAttentionV14Function,
                   cron_root_attention_v14, cron_root_attention_varlen, get_num_sms,
                   warmup_varlen_shapes)
from .hybrid import CronRootAttentionHybrid, cron_root_attention_hybrid
from .module import CronRootAttention, CronRootMultiheadAttention
from . import _native


def calibrate(H: int = 8, D: int = 64, dtype=None, S: int = 4096, verbose: bool = True) -> dict:
    """Report the kernel configuration for (H, D) (reference __init__.py:84-180).

    The reference benchmarks Triton (num_warps, num_stages) candidates here
    and returns {"fwd": (num_warps, num_stages), "bwd": (...)}. The HIP
    kernels have one tile geometry per (dtype, D), fixed at build time; this
    returns the same shape of dict with (waves per workgroup, LDS pipeline
    stages) of the forward and of the dQ kernel, as the library reports them
    (``cra_tile_config``; the whole geometry: ``_native.tile_config``), and,
    on a GPU, runs one forward+backward at S to load the kernels.
    """
    dtype = dtype or _torch.float16
    Dp = next((d for d in (32, 64, 128, 256) if D <= d), D)
    t = _native.tile_config(dtype, Dp)
    if _torch.cuda.is_available():
        dev = _torch.device("cuda", _torch.cuda.current_device())
        q = _torch.randn(1, H, S, D, device=dev, dtype=dtype, requires_grad=True)
        k = _torch.randn(1, H, S, D, device=dev, dtype=dtype, requires_grad=True)
        v = _torch.randn(1, H, S, D, device=dev, dtype=dtype, requires_grad=True)
        cron_root_attention_v14(q, k, v).sum().backward()
        _torch.cuda.synchronize(dev)
    # the gfx950-tiled kernels (fp16/bf16 up to D = 128) double-buffer their
    # streamed tiles in LDS; the generic ones (fp32, D = 256) stage one tile
    stages = 2 if (dtype != _torch.float32 and Dp <= 128) else 1
    cfg = {"fwd": (t["fwd_waves"], stages), "bwd": (t["dq_waves"], stages)}
    if verbose:
        print(f"  H={H} D={D}: fwd {t['fwd_waves']} waves x {t['fwd_queries']} queries, "
              f"{t['fwd_key_tile']}-key tiles; dQ {t['dq_waves']} waves x {t['dq_queries']} queries; "
              f"global-row dK/dV {t['dkdv_global_waves']} waves x {t['dkdv_global_rows']} rows; "
              f"local dK/dV {t['dkdv_local_waves']} waves x {t['dkdv_local_keys']} keys "
              f"(static gfx950 tiles, {stages} LDS stage{'s' if stages > 1 else ''})")
    return cfg


def get_gpu_info() -> dict:
    """Device name and CU count (reference __init__.py:183-202)."""
    if not _torch.cuda.is_available():
        return {"gpu_name": "No GPU", "sm_count": 0, "is_known_gpu": False}
    name = _torch.cuda.get_device_name()
    info = {"gpu_name": name, "sm_count": get_num_sms(),
            "is_known_gpu": name in GPU_SM_MAP or any(n in name for n in GPU_SM_MAP)}
    try:
        d = _native.device_info(_torch.cuda.current_device())
        info.update({"arch": d["arch"], "lds_bytes_per_cu": d["lds_bytes_per_cu"]})
    except Exception:  # library not built: report torch's view only
        pass
    return info


cron_root_attention = cron_root_attention_v14

__all__ = [
    "cron_root_attention",
    "cron_root_attention_v14",
    "cron_root_attention_varlen",
    "warmup_varlen_shapes",
    "CronRootAttention",
    "CronRootMultiheadAttention",
    "cron_root_attention_hybrid",
    "CronRootAttentionHybrid",
    "calibrate",
    "get_num_sms",
    "get_gpu_info",
    "GPU_SM_MAP",
    "__version__",
]
