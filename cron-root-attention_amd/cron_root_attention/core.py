"""Entry points and autograd of the sqrt(N) sparse attention on MI355X.

Drop-in for the reference's ``core.py`` surface: ``cron_root_attention_v14``
(core.py:3767-3797), ``CronRootAttentionV14Function`` (core.py:2822-3759),
``cron_root_attention_varlen`` / ``warmup_varlen_shapes`` (core.py:3836-4022),
``get_num_sms`` / ``GPU_SM_MAP`` (core.py:58-188).

Planning follows the reference: W = ceil(sqrt(S)) (core.py:3479), relay only
for S > 2048 (core.py:2832, 3507), relay_top_k rows per block (core.py:3771),
logit scale 1/sqrt(D) (core.py:954).  The compute runs in libcra_hip.so:
``cra_build_global`` packs the strided and top-k relay rows, ``cra_fwd`` runs
the three phases, ``cra_bwd`` produces dQ/dK/dV (and the relay-scale
gradient).  Unlike the reference:

* CPU tensors run the library's native host forward ``cra_fwd_cpu`` with the
  plan of the reference's CPU path, ``cra_cpu_fast_compiled`` (core.py:3794-3796):
  W = isqrt(S), relay always on, top 2 rows per block, GQA from the shapes,
  ``kv_groups`` / ``relay_log_scale`` / ``relay_top_k`` / ``use_persistent``
  ignored as there; it has no backward (the reference's CPU autograd fails on
  its own in-place ops), so differentiating through it raises;
* the backward returns fresh tensors (the reference returns static CUDA-graph
  buffers, core.py:3016-3020, 3367-3369) and runs on the caller's current
  stream (the reference replays on the default stream, core.py:3011);
* gradients accumulate in fp32 and round once, deterministically (the
  reference adds fp16 atomics, core.py:1886-1889);
* with ``relay_log_scale`` the gradient reaching the relay source rows
  carries the exp(alpha) factor (the reference's scatter drops it,
  core.py:3541-3544 vs 3274-3290);
* ``use_persistent`` on a sequence without relay (S <= 2048) runs the
  persistent work-queue forward (``cra_fwd_persistent``), as the reference
  does (core.py:3548-3569); the results are the tiled forward's, bit for bit.
"""
from __future__ import annotations

import math
from functools import lru_cache
from typing import Optional, Sequence, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native

RELAY_THRESHOLD = 2048          # core.py:2832
_SUPPORTED_D = (32, 64, 128, 256)

# CU counts for the persistent-grid helpers (reference GPU_SM_MAP, core.py:58-135,
# lists NVIDIA parts only).
GPU_SM_MAP = {
    "AMD Instinct MI355X": 256,
    "AMD Instinct MI350X": 256,
    "AMD Instinct MI325X": 304,
    "AMD Instinct MI300X": 304,
    "AMD Instinct MI300A": 228,
    "AMD Instinct MI250X": 220,
    "AMD Instinct MI210": 104,
}


@lru_cache(maxsize=None)
def _num_sms_for(device_index: int) -> int:
    props = torch.cuda.get_device_properties(device_index)
    n = getattr(props, "multi_processor_count", 0)
    if n > 0:
        return n
    name = torch.cuda.get_device_name(device_index)
    for known, cu in GPU_SM_MAP.items():
        if known in name or name in known:
            return cu
    return 256


def get_num_sms() -> int:
    """Compute units of the current device (reference core.py:137-170)."""
    if not torch.cuda.is_available():
        return 1
    return _num_sms_for(torch.cuda.current_device())


def window_size(S: int) -> int:
    """W = ceil(sqrt(S)) (core.py:3479)."""
    return int(math.ceil(math.sqrt(S)))


def _padded_head_dim(D: int) -> int:
    for d in _SUPPORTED_D:
        if D <= d:
            return d
    raise NotImplementedError(f"head dim {D} > 256 is not built for gfx950 in this release")


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """d contiguous, 16-byte aligned rows, one head within 2 GiB (the kernels
    address a head with 32-bit byte offsets); otherwise a contiguous copy."""
    vec = 16 // t.element_size()
    span = ((t.shape[2] - 1) * t.stride(2) + t.shape[3]) * t.element_size()
    ok = (t.stride(3) == 1 and t.data_ptr() % 16 == 0 and span < (1 << 31)
          and all(s % vec == 0 for s in t.stride()[:3]))
    return t if ok else t.contiguous()


def _pad_d(t: torch.Tensor, Dp: int) -> torch.Tensor:
    D = t.shape[-1]
    return t if D == Dp else F.pad(t, (0, Dp - D))


def _check_inputs(q, k, v, kv_groups):
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be [B, H, S, D]")
    B, Hq, S, D = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[2] != S or k.shape[3] != D:
        raise ValueError(f"k/v shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    Hkv = k.shape[1]
    if kv_groups < 1 or Hkv * kv_groups != Hq:
        raise ValueError(f"H_q={Hq} must equal H_kv={Hkv} * kv_groups={kv_groups}")
    if S < 1 or B < 1 or D < 1:
        raise ValueError("B, S and D must be >= 1")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k, v dtypes differ: {q.dtype}, {k.dtype}, {v.dtype}")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"unsupported dtype {q.dtype}; use float16, bfloat16 or float32")
    if q.device.type != "cuda":
        raise RuntimeError(
            "cron_root_attention runs on ROCm GPU tensors only in this build "
            f"(got device {q.device}); move q, k, v to a HIP device")
    if not (q.device == k.device == v.device):
        raise ValueError("q, k, v must be on the same device")


def _relay_scale(relay_log_scale, relay_on: bool, q: torch.Tensor, Hkv: int):
    """exp(relay_log_scale) rounded to the input dtype (core.py:3541-3544), as
    the fp32 [H_kv] multipliers the kernels read, or None.

    The tensor must live on q's device: the kernels dereference its pointer
    on the GPU, so a host tensor is rejected here, before any launch (the
    reference fails the same call with a device-mismatch error in
    ``relay_k * _relay_scale``).
    """
    if relay_log_scale is None or not relay_on:   # unused without relay (core.py:3541)
        return None
    if not isinstance(relay_log_scale, torch.Tensor):
        raise TypeError("relay_log_scale must be a tensor of shape [H_kv]")
    if relay_log_scale.device != q.device:
        raise ValueError(f"relay_log_scale is on {relay_log_scale.device} but q is on "
                         f"{q.device}; move it to the same device")
    if relay_log_scale.shape != (Hkv,):
        raise ValueError(f"relay_log_scale must have shape [{Hkv}]")
    return relay_log_scale.detach().exp().to(q.dtype).to(torch.float32).contiguous()


class CronRootAttentionV14Function(torch.autograd.Function):
    """Autograd of the three-phase attention (reference core.py:2822-3759).

    ``apply(q, k, v, use_persistent, kv_groups, relay_log_scale, relay_top_k)``
    as in the reference; two trailing optional arguments override the window
    and the relay switch (used by tests to run the CPU-path semantics of
    ``cra_cpu_fast``: floor window, relay always on).
    """

    RELAY_THRESHOLD = RELAY_THRESHOLD
    FUSED_BWD_THRESHOLD = 8192  # inert in the reference too (core.py:2836, 3656)

    @staticmethod
    def forward(ctx, q, k, v, use_persistent: bool = False, kv_groups: int = 1,
                relay_log_scale: Optional[torch.Tensor] = None, relay_top_k: int = 2,
                window: Optional[int] = None, relay: Optional[bool] = None):
        _check_inputs(q, k, v, kv_groups)
        B, Hq, S, D = q.shape
        Hkv = k.shape[1]
        W = window_size(S) if window is None else int(window)
        relay_on = (S > RELAY_THRESHOLD) if relay is None else bool(relay)
        if relay_on and not 1 <= relay_top_k <= 4:
            raise ValueError(f"relay_top_k={relay_top_k} outside [1, 4]")
        Dp = _padded_head_dim(D)
        qp, kp, vp = (_kernel_ready(_pad_d(t, Dp)) for t in (q, k, v))
        p = _native.problem(B, Hq, Hkv, S, Dp, W, relay_on, relay_top_k, q.dtype,
                            1.0 / math.sqrt(D))
        rscale = _relay_scale(relay_log_scale, relay_on, q, Hkv)
        st = torch.cuda.current_stream(q.device).cuda_stream
        gk, gv, src = _native.build_global(p, kp, vp, rscale, stream=st)
        if use_persistent and not relay_on:   # the reference's persistent path (core.py:3548)
            o, lse = _native.forward_persistent(p, qp, kp, vp, gk, gv, stream=st)
        else:
            o, lse = _native.forward(p, qp, kp, vp, gk, gv, stream=st)
        ctx.problem = p
        ctx.D = D
        ctx.has_alpha = relay_log_scale is not None and relay_on
        ctx.alpha_dtype = relay_log_scale.dtype if relay_log_scale is not None else None
        ctx.save_for_backward(qp, kp, vp, o, lse, gk, gv, src, rscale)
        return o if Dp == D else o[..., :D].contiguous()

    @staticmethod
    def backward(ctx, do):
        qp, kp, vp, o, lse, gk, gv, src, rscale = ctx.saved_tensors
        p = ctx.problem
        D = ctx.D
        dop = _kernel_ready(_pad_d(do.to(qp.dtype), p.D))
        dq, dk, dv, dalpha = _native.backward(p, qp, kp, vp, o, dop, lse, gk, gv, src, rscale,
                                              ctx.has_alpha)
        if p.D != D:
            dq, dk, dv = (t[..., :D].contiguous() for t in (dq, dk, dv))
        da = dalpha.to(ctx.alpha_dtype) if (ctx.has_alpha and dalpha is not None) else None
        return dq, dk, dv, None, None, da, None, None, None


class CronRootAttentionCPUFunction(torch.autograd.Function):
    """Forward of CPU tensors (the reference's cra_cpu_fast plan, computed by
    ``cra_fwd_cpu``); its backward raises."""

    @staticmethod
    def forward(ctx, q, k, v):
        return _cpu_forward(q, k, v)

    @staticmethod
    def backward(ctx, do):
        raise NotImplementedError(
            "cron_root_attention has no backward for CPU tensors (neither has the "
            "reference's CPU path); move q, k, v to a ROCm GPU to train")


def _cpu_forward(q, k, v):
    """CPU tensors: cra_cpu_fast's plan (cpu_reference.py:225-268) in native code."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be [B, H, S, D]")
    B, Hq, S, D = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[2] != S or k.shape[3] != D:
        raise ValueError(f"k/v shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    Hkv = k.shape[1]
    if Hq % Hkv:
        raise ValueError(f"H_q={Hq} must be a multiple of H_kv={Hkv}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k, v dtypes differ: {q.dtype}, {k.dtype}, {v.dtype}")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"unsupported dtype {q.dtype}; use float16, bfloat16 or float32")
    if not (k.device.type == v.device.type == "cpu"):
        raise ValueError("q, k, v must be on the same device")
    qc, kc, vc = (t.detach() if t.stride(3) == 1 else t.detach().contiguous()
                  for t in (q, k, v))
    p = _native.problem(B, Hq, Hkv, S, D, max(1, math.isqrt(S)), True, 2, q.dtype,
                        1.0 / math.sqrt(D))
    return _native.forward_cpu(p, qc, kc, vc, torch.get_num_threads())


@torch.compiler.disable
def cron_root_attention_v14(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            use_persistent: bool = False, kv_groups: int = 1,
                            relay_log_scale: Optional[torch.Tensor] = None,
                            relay_top_k: int = 2) -> torch.Tensor:
    """sqrt(N) sparse causal attention (reference core.py:3767-3797).

    Args:
        q: [B, H_q, S, D]; k, v: [B, H_kv, S, D] with H_q = H_kv * kv_groups.
        use_persistent: on sequences without relay (S <= 2048), run the
            persistent work-queue forward (core.py:3548-3569); same results.
        kv_groups: query heads per kv head (query head h reads kv head
            h // kv_groups, core.py:981).
        relay_log_scale: optional [H_kv]; relay rows are scaled by
            exp(relay_log_scale) (core.py:3541-3544); differentiable.
        relay_top_k: relay rows per sqrt(N) block (1..4).

    Returns: [B, H_q, S, D] in the dtype of q.

    CPU tensors take the reference's CPU path (core.py:3794-3796): the plan of
    ``cra_cpu_fast`` (W = isqrt(S), relay always on, top 2), computed by the
    library's host code; forward only.
    """
    if q.device.type == "cpu":
        if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
            return CronRootAttentionCPUFunction.apply(q, k, v)
        return _cpu_forward(q, k, v)
    if relay_log_scale is None:
        op = _native.attention_op()
        if op is not None:
            plan = _op_plan(q, k, v, use_persistent, kv_groups, relay_top_k)
            if plan is not None:
                return op(q, k, v, *plan)
    return CronRootAttentionV14Function.apply(q, k, v, use_persistent, kv_groups,
                                              relay_log_scale, relay_top_k)


_OP_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _op_plan(q, k, v, use_persistent, kv_groups, relay_top_k):
    """(window, relay, top_k, scale) when the call can go to the C++ operator
    ``torch.ops.cra.attention`` (the Function's plan and launches, bit for
    bit, without its Python host cost; it copies layouts the kernels cannot
    take, as the Function does): q, k, v on one GPU, head dim 32/64/128/256, the
    tiled forward. None sends the call to the Python Function, which also
    raises the reference's errors for invalid arguments."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        return None
    B, Hq, S, D = q.shape
    if (D not in _SUPPORTED_D or S < 1 or B < 1 or k.shape != v.shape
            or k.shape[0] != B or k.shape[2] != S or k.shape[3] != D
            or kv_groups < 1 or k.shape[1] * kv_groups != Hq
            or not (q.dtype == k.dtype == v.dtype) or q.dtype not in _OP_DTYPES
            or q.device.type != "cuda" or not (q.device == k.device == v.device)):
        return None
    relay = S > RELAY_THRESHOLD
    if (use_persistent and not relay) or (relay and not 1 <= relay_top_k <= 4):
        return None
    return window_size(S), relay, int(relay_top_k), 1.0 / math.sqrt(D)


def _attention_with_plan(q, k, v, window: int, relay: bool, kv_groups: int = 1,
                         relay_log_scale=None, relay_top_k: int = 2):
    """Same op with an explicit window and relay switch (test hook)."""
    return CronRootAttentionV14Function.apply(q, k, v, False, kv_groups, relay_log_scale,
                                              relay_top_k, window, relay)


def _parse_cu_seqlens(cu_seqlens, S_total: int):
    if isinstance(cu_seqlens, torch.Tensor):
        if cu_seqlens.device.type != "cpu":
            raise ValueError("cu_seqlens must be a CPU tensor (or list); call .cpu() first")
        seqs = [int(x) for x in cu_seqlens.tolist()]
    else:
        seqs = [int(x) for x in cu_seqlens]
    if len(seqs) < 2 or seqs[0] != 0 or seqs[-1] != S_total or any(
            b <= a for a, b in zip(seqs, seqs[1:])):
        raise ValueError(f"cu_seqlens must rise strictly from 0 to {S_total}, got {seqs}")
    return seqs


class CronRootAttentionVarlenFunction(torch.autograd.Function):
    """Autograd of the packed-document op: every document in one set of launches.

    Each document gets the plan of its own length (window ceil(sqrt(len)),
    relay for len > 2048), exactly what the reference's per-document calls
    do (core.py:3911-3952); ``windows`` / ``relays`` override the plan per
    document (test hook).
    """

    @staticmethod
    def forward(ctx, q, k, v, seqs, kv_groups: int = 1,
                relay_log_scale: Optional[torch.Tensor] = None, relay_top_k: int = 2,
                windows: Optional[Sequence[int]] = None, relays: Optional[Sequence[bool]] = None):
        _check_inputs(q, k, v, kv_groups)
        B, Hq, S, D = q.shape
        Hkv = k.shape[1]
        lens = [e - s for s, e in zip(seqs, seqs[1:])]
        W = [window_size(n) for n in lens] if windows is None else [int(w) for w in windows]
        R = [n > RELAY_THRESHOLD for n in lens] if relays is None else [bool(r) for r in relays]
        any_relay = any(R)
        if any_relay and not 1 <= relay_top_k <= 4:
            raise ValueError(f"relay_top_k={relay_top_k} outside [1, 4]")
        docs = _native.Docs(seqs, W, R)
        Dp = _padded_head_dim(D)
        qp, kp, vp = (_kernel_ready(_pad_d(t, Dp)) for t in (q, k, v))
        p = _native.problem(B, Hq, Hkv, S, Dp, 0, any_relay, relay_top_k, q.dtype,
                            1.0 / math.sqrt(D))
        rscale = _relay_scale(relay_log_scale, any_relay, q, Hkv)
        gk, gv, src = _native.build_global_varlen(p, docs, kp, vp, rscale)
        o, lse = _native.forward_varlen(p, docs, qp, kp, vp, gk, gv)
        ctx.problem = p
        ctx.docs = docs
        ctx.D = D
        ctx.has_alpha = relay_log_scale is not None and any_relay
        ctx.alpha_dtype = relay_log_scale.dtype if relay_log_scale is not None else None
        ctx.save_for_backward(qp, kp, vp, o, lse, gk, gv, src, rscale)
        return o if Dp == D else o[..., :D].contiguous()

    @staticmethod
    def backward(ctx, do):
        qp, kp, vp, o, lse, gk, gv, src, rscale = ctx.saved_tensors
        p = ctx.problem
        D = ctx.D
        dop = _kernel_ready(_pad_d(do.to(qp.dtype), p.D))
        dq, dk, dv, dalpha = _native.backward_varlen(p, ctx.docs, qp, kp, vp, o, dop, lse, gk, gv,
                                                     src, rscale, ctx.has_alpha)
        if p.D != D:
            dq, dk, dv = (t[..., :D].contiguous() for t in (dq, dk, dv))
        da = dalpha.to(ctx.alpha_dtype) if (ctx.has_alpha and dalpha is not None) else None
        return dq, dk, dv, None, None, da, None, None, None


@torch.compiler.disable
def cron_root_attention_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                               cu_seqlens: Union[Sequence[int], torch.Tensor],
                               kv_groups: int = 1, use_persistent: bool = False,
                               relay_log_scale: Optional[torch.Tensor] = None,
                               relay_top_k: int = 2) -> torch.Tensor:
    """Packed documents, no attention across boundaries (reference core.py:3836-3954).

    ``cu_seqlens`` (list or CPU tensor, length n_docs + 1, from 0 to S_total)
    splits the sequence axis; each document is attended on its own with the
    window and relay rule of its own length, as the reference's loop of one
    call per document does.  Here all documents go through one set of kernel
    launches (``cra_*_varlen``); differentiable, including
    ``relay_log_scale`` (summed over documents).  ``use_persistent`` has no
    numerical effect, as in ``cron_root_attention_v14``.
    """
    seqs = _parse_cu_seqlens(cu_seqlens, q.shape[2])
    if len(seqs) == 2:  # single document: the plain op (core.py:3913-3921)
        return cron_root_attention_v14(q, k, v, use_persistent, kv_groups, relay_log_scale,
                                       relay_top_k)
    return CronRootAttentionVarlenFunction.apply(q, k, v, seqs, kv_groups, relay_log_scale,
                                                 relay_top_k)


def _varlen_with_plan(q, k, v, cu_seqlens, windows, relays, kv_groups: int = 1,
                      relay_log_scale=None, relay_top_k: int = 2):
    """Varlen op with explicit per-document windows and relay switches (test hook)."""
    seqs = _parse_cu_seqlens(cu_seqlens, q.shape[2])
    return CronRootAttentionVarlenFunction.apply(q, k, v, seqs, kv_groups, relay_log_scale,
                                                 relay_top_k, windows, relays)


def warmup_varlen_shapes(doc_lengths, H: int, D: int, B: int = 1, kv_groups: int = 1,
                         dtype=None, device=None, verbose: bool = False) -> None:
    """Run forward+backward once per distinct length (reference core.py:3957-4022).

    The HIP library has no JIT or graph capture to warm, so this only
    touches the caching allocator for each shape; kept for API compatibility.
    """
    dtype = dtype or torch.float16
    device = device or torch.device("cuda", torch.cuda.current_device())
    Hkv = H // kv_groups
    for S in sorted({int(x) for x in doc_lengths if int(x) > 0}):
        q = torch.randn(B, H, S, D, device=device, dtype=dtype, requires_grad=True)
        k = torch.randn(B, Hkv, S, D, device=device, dtype=dtype, requires_grad=True)
        v = torch.randn(B, Hkv, S, D, device=device, dtype=dtype, requires_grad=True)
        cron_root_attention_v14(q, k, v, kv_groups=kv_groups).sum().backward()
        if verbose:
            print(f"[warmup_varlen_shapes] S={S} done")
    torch.cuda.synchronize(device)


class CronRootAttentionV14(nn.Module):
    """Module wrapper of the functional op (reference core.py:4025-4051)."""

    def __init__(self, use_persistent: bool = False, auto_persistent_threshold: int = 0):
        super().__init__()
        self.use_persistent = use_persistent
        self.auto_persistent_threshold = auto_persistent_threshold

    def forward(self, q, k, v):
        return cron_root_attention_v14(q, k, v, use_persistent=self.use_persistent)
