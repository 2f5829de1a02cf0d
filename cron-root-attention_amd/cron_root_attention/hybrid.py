"""SDPA / sqrt(N) dispatch by sequence length (reference hybrid.py:1-124).

The reference's crossover (1536 tokens, hybrid.py:22) was measured on an RTX
5070 Ti.  Here the crossover is a gfx950 table measured on MI355X boxes with
``bench.py --crossover`` against ROCm's fused (flash) SDPA, causal, for
forward and forward+backward separately: ``CROSSOVER_GFX950``.  Below a few
thousand tokens the sqrt(N) op costs its launch floor (about 15 us forward
and 75-85 us forward+backward through the C++ operator) while SDPA's floor
is 20-25 us and 82-100 us and grows with B*H*S^2.  Swept from S = 1 to 16384
for every BASELINE shape in both modes, the sqrt(N) op was the faster at
every S, so no crossover exists to bracket: every row is 1 (run the sqrt(N)
op for every length) and ``CROSSOVER_BRACKETED`` says so.  The narrowest
margin is at S = 1 in training (0.082 against 0.084 ms at B=2 H=32 D=128).
The table keeps its shape (mode, head dim, B*H) for re-measurement on other
hosts.
``_SDPA_THRESHOLD`` is the forward+backward crossover at D=128 for B*H=16, the
role of the reference's constant.  Both entry points default to
``threshold=None``, which looks the crossover up in the table for the call's
head dim, B*H and grad mode; an integer threshold behaves as the reference's
(S >= threshold runs the sqrt(N) op).
"""
from __future__ import annotations

from typing import Literal, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .core import cron_root_attention_v14

# (mode, head_dim, smallest B*H the row applies to) -> smallest swept S from
# which the sqrt(N) op beats SDPA at every larger swept S.
# Sweep: S in {1, 2, 4, 8, 16, 32, 48, 64, 96, 128, 192, 256, 384, 512, 768,
# 1024, 1536, 2048, 3072, 4096, 6144, 8192, 16384}; shapes (B, H, D, dtype) =
# (1, 16, 128, fp16), (2, 32, 128, bf16), (1, 8, 64, fp16), (1, 12, 64, fp16).
# sqrt(N) op / SDPA ms at S = 1 in each row's comment.
CROSSOVER_GFX950 = {
    ("fwd", 128, 1): 1,        # B=1 H=16 fp16: 0.016 vs 0.021 ms
    ("fwd", 128, 64): 1,       # B=2 H=32 bf16: 0.017 vs 0.020 ms
    ("train", 128, 1): 1,      # B=1 H=16 fp16: 0.081 vs 0.087 ms
    ("train", 128, 64): 1,     # B=2 H=32 bf16: 0.082 vs 0.084 ms
    ("fwd", 64, 1): 1,         # B=1 H=8 and H=12 fp16: 0.015-0.016 vs 0.020 ms
    ("train", 64, 1): 1,       # B=1 H=8 and H=12 fp16: 0.077-0.078 vs 0.082-0.083 ms
}
# Whether SDPA won at a swept S below the row's value (a measured, bracketed
# crossover). False: the sqrt(N) op was faster at every swept S, the row is
# the sweep's lower edge and no crossover exists in the measured range.
CROSSOVER_BRACKETED = {key: False for key in CROSSOVER_GFX950}
_SDPA_THRESHOLD = CROSSOVER_GFX950[("train", 128, 1)]


def _row(head_dim: int, training: bool, batch_heads: int):
    mode = "train" if training else "fwd"
    dims = sorted({d for (m, d, _) in CROSSOVER_GFX950 if m == mode})
    d = min(dims, key=lambda x: abs(x - head_dim))
    rows = sorted(bh for (m, dd, bh) in CROSSOVER_GFX950 if m == mode and dd == d)
    bh = max([r for r in rows if r <= max(1, batch_heads)] or rows[:1])
    return (mode, d, bh)


def crossover(head_dim: int, training: bool, batch_heads: int = 1, detail: bool = False):
    """Measured gfx950 crossover for the nearest tabulated head dim and the
    largest tabulated B*H not above ``batch_heads``: the S from which the
    sqrt(N) op runs.  With ``detail=True`` a dict that also says whether the
    crossover was bracketed by the sweep or the sqrt(N) op was the faster at
    every swept S (then no SDPA range exists)."""
    key = _row(head_dim, training, batch_heads)
    S = CROSSOVER_GFX950[key]
    if not detail:
        return S
    br = CROSSOVER_BRACKETED[key]
    return {"S": S, "bracketed": br, "row": key,
            "meaning": ("measured crossover: SDPA is faster below S" if br else
                        "no crossover: the sqrt(N) op was faster at every swept S (from 1)")}


def dispatch_backend(S: int, head_dim: int, training: bool, batch_heads: int = 1,
                     threshold: Optional[int] = None) -> str:
    """Backend the ``"auto"`` mode picks: ``"cron_root"`` when S >= threshold
    (reference hybrid.py:58-64), else ``"sdpa"``; ``threshold=None`` uses the
    measured gfx950 crossover (:func:`crossover`)."""
    if threshold is None:
        threshold = crossover(head_dim, training, batch_heads)
    return "cron_root" if S >= threshold else "sdpa"


def cron_root_attention_hybrid(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                               backend: Literal["auto", "cron_root", "sdpa"] = "auto",
                               threshold: Optional[int] = None) -> torch.Tensor:
    """SDPA below ``threshold`` tokens, the sqrt(N) kernel at or above it
    (reference hybrid.py:25-64).  ``threshold=None`` picks the measured gfx950
    crossover for this head dim and for training vs inference (grad mode)."""
    S = q.shape[2]
    if backend == "cron_root":
        return cron_root_attention_v14(q, k, v)
    if backend == "sdpa":
        return F.scaled_dot_product_attention(q, k, v, is_causal=True)
    if backend != "auto":
        raise ValueError(f"unknown backend {backend!r}")
    training = torch.is_grad_enabled() and q.requires_grad
    if dispatch_backend(S, q.shape[-1], training, q.shape[0] * q.shape[1],
                        threshold) == "cron_root":
        return cron_root_attention_v14(q, k, v)
    return F.scaled_dot_product_attention(q, k, v, is_causal=True)


class CronRootAttentionHybrid(nn.Module):
    """Projections + hybrid dispatch (reference hybrid.py:67-124)."""

    def __init__(self, d_model: int, n_heads: int, threshold: Optional[int] = None,
                 dropout: float = 0.0, bias: bool = False):
        super().__init__()
        self.d_model = d_model
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.threshold = threshold
        self.dropout = dropout
        self.q_proj = nn.Linear(d_model, d_model, bias=bias)
        self.k_proj = nn.Linear(d_model, d_model, bias=bias)
        self.v_proj = nn.Linear(d_model, d_model, bias=bias)
        self.o_proj = nn.Linear(d_model, d_model, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, S, D = x.shape
        q = self.q_proj(x).view(B, S, self.n_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(x).view(B, S, self.n_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(x).view(B, S, self.n_heads, self.head_dim).transpose(1, 2)
        out = cron_root_attention_hybrid(q, k, v, backend="auto", threshold=self.threshold)
        out = out.transpose(1, 2).contiguous().view(B, S, D)
        out = self.o_proj(out)
        if self.dropout > 0 and self.training:
            out = F.dropout(out, p=self.dropout)
        return out
