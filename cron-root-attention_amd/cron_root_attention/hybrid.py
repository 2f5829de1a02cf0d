"""SDPA / sqrt(N) dispatch by sequence length (reference hybrid.py:1-124).

The reference's crossover (1536 tokens, hybrid.py:22) was measured on an RTX
5070 Ti.  Here the crossover is a gfx950 table, measured on one MI355X with
``bench.py --crossover`` against ROCm's ``scaled_dot_product_attention``
(forward and forward+backward separately, per head dim); see
``CROSSOVER_GFX950``.  ``_SDPA_THRESHOLD`` is the training (fwd+bwd)
crossover at D=128, the reference's role for the constant.
"""
from __future__ import annotations

from typing import Literal, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .core import cron_root_attention_v14

# (mode, head_dim) -> smallest S at which the sqrt(N) kernel beats SDPA on
# MI355X (bf16/fp16, causal). Filled from the measured sweep.
CROSSOVER_GFX950 = {
    ("fwd", 64): 1536,
    ("fwd", 128): 1536,
    ("train", 64): 1536,
    ("train", 128): 1536,
}
_SDPA_THRESHOLD = CROSSOVER_GFX950[("train", 128)]


def crossover(head_dim: int, training: bool) -> int:
    """Measured gfx950 crossover for the nearest tabulated head dim."""
    mode = "train" if training else "fwd"
    dims = sorted({d for (m, d) in CROSSOVER_GFX950 if m == mode})
    d = min(dims, key=lambda x: abs(x - head_dim))
    return CROSSOVER_GFX950[(mode, d)]


def cron_root_attention_hybrid(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                               backend: Literal["auto", "cron_root", "sdpa"] = "auto",
                               threshold: Optional[int] = _SDPA_THRESHOLD) -> torch.Tensor:
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
    if threshold is None:
        threshold = crossover(q.shape[-1], torch.is_grad_enabled() and q.requires_grad)
    if S >= threshold:
        return cron_root_attention_v14(q, k, v)
    return F.scaled_dot_product_attention(q, k, v, is_causal=True)


class CronRootAttentionHybrid(nn.Module):
    """Projections + hybrid dispatch (reference hybrid.py:67-124)."""

    def __init__(self, d_model: int, n_heads: int, threshold: int = _SDPA_THRESHOLD,
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
