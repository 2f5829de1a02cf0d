"""nn.Module wrappers (reference module.py:1-247).

``CronRootAttention`` keeps the reference's constructor and forward
(module.py:20-126) and adds two keyword arguments: ``hybrid`` (dispatch to
SDPA below the gfx950 crossover, as ``CronRootAttentionHybrid`` does) and
``threshold``.  Grouped kv heads go to the kernel natively
(``kv_groups``) instead of being expanded with ``repeat_interleave``
(module.py:111-113); query head h reads kv head h // kv_groups either way, so
the result is the same.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .core import cron_root_attention_v14
from .hybrid import dispatch_backend


class CronRootAttention(nn.Module):
    """sqrt(N) sparse attention layer with q/k/v/o projections."""

    def __init__(self, d_model: int, n_heads: int, n_kv_heads: Optional[int] = None,
                 dropout: float = 0.0, bias: bool = False, hybrid: bool = False,
                 threshold: Optional[int] = None):
        super().__init__()
        self.d_model = d_model
        self.n_heads = n_heads
        self.n_kv_heads = n_kv_heads or n_heads
        self.head_dim = d_model // n_heads
        self.dropout = dropout
        self.hybrid = hybrid
        self.threshold = threshold
        assert d_model % n_heads == 0, "d_model must be divisible by n_heads"
        assert n_heads % self.n_kv_heads == 0, "n_heads must be divisible by n_kv_heads"
        self.kv_groups = n_heads // self.n_kv_heads
        self.drop = nn.Dropout(dropout) if dropout > 0 else nn.Identity()
        self.q_proj = nn.Linear(d_model, d_model, bias=bias)
        self.k_proj = nn.Linear(d_model, self.n_kv_heads * self.head_dim, bias=bias)
        self.v_proj = nn.Linear(d_model, self.n_kv_heads * self.head_dim, bias=bias)
        self.o_proj = nn.Linear(d_model, d_model, bias=bias)
        self._reset_parameters()

    def _reset_parameters(self):
        for lin in (self.q_proj, self.k_proj, self.v_proj, self.o_proj):
            nn.init.xavier_uniform_(lin.weight)
            if lin.bias is not None:
                nn.init.zeros_(lin.bias)

    def backend_for(self, x: torch.Tensor) -> str:
        """``"cron_root"`` or ``"sdpa"``: what forward(x) runs.  Without
        ``hybrid`` always the sqrt(N) op; with it the crossover of
        :func:`dispatch_backend` for this head dim, B*H and train/eval mode."""
        if not self.hybrid:
            return "cron_root"
        return dispatch_backend(x.shape[1], self.head_dim,
                                self.training and torch.is_grad_enabled(),
                                x.shape[0] * self.n_heads, self.threshold)

    def forward(self, x: torch.Tensor, kv: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, S, _ = x.shape
        kv = kv if kv is not None else x
        q = self.q_proj(x).view(B, S, self.n_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(kv).view(B, S, self.n_kv_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(kv).view(B, S, self.n_kv_heads, self.head_dim).transpose(1, 2)
        if self.backend_for(x) == "sdpa":
            out = F.scaled_dot_product_attention(q, k, v, is_causal=True,
                                                 enable_gqa=self.kv_groups > 1)
        else:
            out = cron_root_attention_v14(q, k, v, kv_groups=self.kv_groups)
        out = out.permute(0, 2, 1, 3).reshape(B, S, self.d_model)
        return self.drop(self.o_proj(out))


class CronRootMultiheadAttention(nn.Module):
    """nn.MultiheadAttention-shaped self-attention (reference module.py:129-247).

    As in the reference, attention is always causal sqrt(N) attention:
    ``key_padding_mask``, ``attn_mask`` and ``is_causal`` are ignored, no
    weights are returned, and query, key and value must be the same tensor.
    """

    def __init__(self, embed_dim: int, num_heads: int, dropout: float = 0.0, bias: bool = True,
                 batch_first: bool = True):
        super().__init__()
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.head_dim = embed_dim // num_heads
        self.dropout = dropout
        self.batch_first = batch_first
        assert embed_dim % num_heads == 0, "embed_dim must be divisible by num_heads"
        self.in_proj_weight = nn.Parameter(torch.empty(3 * embed_dim, embed_dim))
        if bias:
            self.in_proj_bias = nn.Parameter(torch.empty(3 * embed_dim))
        else:
            self.register_parameter("in_proj_bias", None)
        self.out_proj = nn.Linear(embed_dim, embed_dim, bias=bias)
        self.drop = nn.Dropout(dropout) if dropout > 0 else nn.Identity()
        self._reset_parameters()

    def _reset_parameters(self):
        nn.init.xavier_uniform_(self.in_proj_weight)
        if self.in_proj_bias is not None:
            nn.init.zeros_(self.in_proj_bias)
        nn.init.xavier_uniform_(self.out_proj.weight)
        if self.out_proj.bias is not None:
            nn.init.zeros_(self.out_proj.bias)

    def forward(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                key_padding_mask: Optional[torch.Tensor] = None, need_weights: bool = False,
                attn_mask: Optional[torch.Tensor] = None, average_attn_weights: bool = True,
                is_causal: bool = True) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        # self-attention only (reference module.py:223); checked before the
        # batch_first transpose, which makes three distinct views of one tensor
        assert query is key and key is value, "Cross-attention not yet supported"
        if not self.batch_first:
            query = query.transpose(0, 1)
        B, S, E = query.shape
        qkv = F.linear(query, self.in_proj_weight, self.in_proj_bias)
        qkv = qkv.view(B, S, 3, self.num_heads, self.head_dim).permute(2, 0, 3, 1, 4)
        out = cron_root_attention_v14(qkv[0], qkv[1], qkv[2])
        out = out.permute(0, 2, 1, 3).reshape(B, S, E)
        out = self.drop(self.out_proj(out))
        if not self.batch_first:
            out = out.transpose(0, 1)
        return out, None
