"""fp64 CPU restatement of the reference's sqrt(N) sparse attention.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): imported by tests,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg, never by the
product package.

Two semantic modes are restated, both parametrised by (W, relay_on, top_k):

* ``mode="kernel"`` -- what ``cron_root_attention()`` computes on a GPU:
  W = ceil(sqrt(S))                               (core.py:3479)
  relay only when S > 2048                        (core.py:2832, 3507)
  relay rows = top-k of fp32 ||k||^2 per W-block, strict '>' so the earlier
  row wins ties, unfilled slots point at the block's first row
                                                  (core.py:2630-2748, 2668-2703)
* ``mode="cpu_reference"`` -- ``cra_cpu_fast`` (the reference's CPU path):
  W = max(1, isqrt(S))                            (cpu_reference.py:233)
  relay always on, norms in the input dtype, torch.topk
                                                  (cpu_reference.py:251-268)

Attention set of query i (ls = max(0, i-W+1), core.py:957):
  local   {j : ls <= j <= i}                      (core.py:993-994)
  strided {s*W : s*W < ls}                        (core.py:1038-1059)
  relay   top-k rows of every block r with (r+1)*W-1 < ls  (core.py:1115-1116)
The softmax runs over the multiset: a relay row that is also a strided row is
counted twice (core.py:1097-1142 loops over both sets independently).
Scores are dot(q,k)/sqrt(D) (core.py:954, 989); O = sum p v / sum p and
LSE = m + ln(sum p) (core.py:1147-1158); the 1e-6 clamps never bind because
every query sees itself.

Each function below is pinned by tests/test_oracle.py against brute force,
closed forms, library routines (causal SDPA on the first W rows), finite
differences, and the golden vectors written from the reference's own
``cra_cpu_fast`` (tests/golden/).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

RELAY_THRESHOLD = 2048  # core.py:2832


# ---------------------------------------------------------------------------
# Planning (core.py:3472-3515, cpu_reference.py:225-268)
# ---------------------------------------------------------------------------

def window_size(S: int, rule: str = "ceil") -> int:
    """sqrt(N) window/stride/block size.

    ``ceil``: ``int(math.ceil(math.sqrt(S)))`` (core.py:3479).
    ``floor``: ``max(1, math.isqrt(S))`` (cpu_reference.py:233).
    """
    if rule == "ceil":
        return int(math.ceil(math.sqrt(S)))
    if rule == "floor":
        return max(1, math.isqrt(S))
    raise ValueError(rule)


@dataclass(frozen=True)
class Plan:
    S: int
    W: int
    relay: bool
    top_k: int

    @property
    def num_blocks(self) -> int:
        """Number of W-blocks, ceil(S/W) (core.py:3519)."""
        return (self.S + self.W - 1) // self.W


def make_plan(S: int, mode: str = "kernel", top_k: int = 2) -> Plan:
    if mode == "kernel":
        return Plan(S, window_size(S, "ceil"), S > RELAY_THRESHOLD, top_k)
    if mode == "cpu_reference":
        return Plan(S, window_size(S, "floor"), True, 2)
    raise ValueError(mode)


def local_start(i, W):
    """ls(i) = max(0, i - W + 1) (core.py:957)."""
    return np.maximum(np.asarray(i) - W + 1, 0)


# ---------------------------------------------------------------------------
# Index sets and the work model
# ---------------------------------------------------------------------------

def attend_set_bruteforce(i: int, plan: Plan, src) -> list:
    """Explicit multiset of key rows query ``i`` attends to (pure Python).

    ``src[r][j]`` is the j-th relay row of block r.  Follows the three masks
    of core.py:1016-1017 (local), :1060-1061 (strided), :1115-1117 (relay).
    """
    W = plan.W
    ls = max(0, i - W + 1)
    rows = list(range(ls, i + 1))
    for s in range(plan.num_blocks):
        if s * W < ls:
            rows.append(s * W)
    if plan.relay:
        for r in range(plan.num_blocks):
            if (r + 1) * W - 1 < ls:
                rows.extend(int(x) for x in src[r][: plan.top_k])
    return rows


def num_strided_visible(i, W):
    """|T(i)| = ceil(ls/W): strided rows s*W < ls (core.py:1038-1040)."""
    ls = local_start(i, W)
    return (ls + W - 1) // W


def num_relay_blocks_visible(i, W):
    """Blocks r with (r+1)*W-1 < ls, i.e. floor(ls/W) (core.py:1115)."""
    return local_start(i, W) // W


def pair_count(plan: Plan) -> int:
    """Algorithmic (query, key) pairs per (b, h), duplicates included.

    P(S) = sum_i [min(i+1, W) + ceil(ls/W) + relay*top_k*floor(ls/W)].
    """
    i = np.arange(plan.S, dtype=np.int64)
    W = plan.W
    loc = np.minimum(i + 1, W)
    strided = num_strided_visible(i, W)
    relay = num_relay_blocks_visible(i, W) * plan.top_k if plan.relay else 0
    return int((loc + strided + relay).sum())


def phase_pair_counts(plan: Plan) -> dict:
    i = np.arange(plan.S, dtype=np.int64)
    W = plan.W
    out = {
        "local": int(np.minimum(i + 1, W).sum()),
        "strided": int(num_strided_visible(i, W).sum()),
        "relay": int((num_relay_blocks_visible(i, W) * plan.top_k).sum()) if plan.relay else 0,
    }
    return out


def fwd_flops(plan: Plan, B: int, H: int, D: int) -> int:
    """4*D per pair: 2*D for q.k plus 2*D for p*v."""
    return 4 * D * pair_count(plan) * B * H


def bwd_flops(plan: Plan, B: int, H: int, D: int) -> int:
    """10*D per pair: recompute q.k, dO.v, p^T dO, dS k, dS^T q."""
    return 10 * D * pair_count(plan) * B * H


# ---------------------------------------------------------------------------
# Relay selection (core.py:2630-2748; cpu_reference.py:251-268)
# ---------------------------------------------------------------------------

def relay_norms_lanetree(rows: np.ndarray) -> np.ndarray:
    """fp32 ||k||^2 with one fixed summation order.

    The reference computes ``tl.sum(k_row.to(f32) ** 2)`` (core.py:2684-2685),
    whose order is Triton's.  This oracle fixes one order so that a kernel
    using it can be checked bit for bit: the row is split into D/8 lanes of 8
    consecutive elements; each lane sums its squares left to right (fp32
    multiply then fp32 add, never fused); the lane partials are then combined
    by a butterfly p[l] += p[l ^ off] for off = D/16, ..., 1.  For fp16/bf16
    inputs the squares are exact in fp32, so only the order matters.
    A row whose length is not 8 times a power of two is zero-padded to one
    (padding lanes add exact zeros first, so e.g. D=16 and its zero-padded
    D=32 give the same bits).
    """
    x = np.asarray(rows, dtype=np.float32)
    D = x.shape[-1]
    L = 1
    while 8 * L < D:
        L *= 2
    if 8 * L != D:
        pad = np.zeros(x.shape[:-1] + (8 * L - D,), dtype=np.float32)
        x = np.concatenate([x, pad], axis=-1)
    x = x.reshape(*x.shape[:-1], L, 8)
    p = np.zeros(x.shape[:-1], dtype=np.float32)
    for e in range(8):
        sq = np.multiply(x[..., e], x[..., e], dtype=np.float32)
        p = np.add(p, sq, dtype=np.float32)
    off = L // 2
    lanes = np.arange(L)
    while off >= 1:
        p = np.add(p, p[..., lanes ^ off], dtype=np.float32)
        off //= 2
    return p[..., 0]


def relay_select(k: torch.Tensor, plan: Plan, norm: str = "lanetree") -> torch.Tensor:
    """Source rows of the relay tokens, int64 [B, H_kv, NB*top_k].

    ``norm="lanetree"`` / ``"fp64"``: the kernel's rule -- per block, rank
    valid rows by fp32 (resp. fp64) norm, descending, earlier row first on
    ties (strict '>' insertion, core.py:2688-2703); a slot with no valid row
    left keeps index 0 of the block (core.py:2668-2669, 2705-2708).
    ``norm="torch"``: cpu_reference.py:251-262 -- zero-pad the last block,
    norms in the input dtype, ``torch.topk``.
    """
    B, H, S, D = k.shape
    W, NB, K = plan.W, plan.num_blocks, plan.top_k
    if norm == "torch":
        pad = NB * W - S
        kp = torch.nn.functional.pad(k, (0, 0, 0, pad)) if pad > 0 else k
        kb = kp.reshape(B, H, NB, W, D)
        nsq = (kb * kb).sum(dim=-1)
        idx = nsq.topk(min(K, W), dim=-1).indices
        base = (torch.arange(NB) * W).view(1, 1, NB, 1)
        return (idx + base).reshape(B, H, NB * min(K, W))
    kk = k.detach().cpu()
    if norm == "lanetree":
        n = relay_norms_lanetree(kk.to(torch.float32).numpy()).astype(np.float64)
    elif norm == "fp64":
        n = (kk.to(torch.float64) ** 2).sum(-1).numpy()
    else:
        raise ValueError(norm)
    src = np.zeros((B, H, NB, K), dtype=np.int64)
    for r in range(NB):
        lo, hi = r * W, min((r + 1) * W, S)
        blk = n[:, :, lo:hi]
        # stable descending sort == strict '>' insertion cascade
        order = np.argsort(-blk, axis=-1, kind="stable")
        take = min(K, hi - lo)
        src[:, :, r, :take] = order[:, :, :take] + lo
        src[:, :, r, take:] = lo
    return torch.from_numpy(src.reshape(B, H, NB * K))


# ---------------------------------------------------------------------------
# Forward (fp64) and backward (autograd of the forward)
# ---------------------------------------------------------------------------

def forward(q, k, v, plan: Plan, kv_groups: int = 1, src: Optional[torch.Tensor] = None,
            relay_scale: Optional[torch.Tensor] = None, chunk: int = 256,
            norm: str = "lanetree", rows: Optional[tuple] = None,
            relay_dtype: Optional[torch.dtype] = None, phases: str = "all"):
    """Exact softmax over each query's multiset, fp64, differentiable.

    q: [B, Hq, S, D]; k, v: [B, Hkv, S, D]; query head h reads kv head
    h // kv_groups (core.py:981).  ``relay_scale`` ([Hkv], already
    exponentiated) multiplies relay k and v rows (core.py:3541-3544); with
    ``relay_dtype`` the scaled rows are rounded to that dtype, as the
    reference's in-dtype multiply does (the rounding is not differentiated).
    ``rows=(lo, hi)`` computes only queries [lo, hi) (outputs then hold those
    rows) so long sequences can be spot-checked.
    ``phases`` = "local" or "global" restricts the multiset to the local
    window or to the strided and relay rows (the subsets the build's
    measurement entry point cra_fwd_phases computes); a query with an empty
    subset gets o = 0 and lse = -inf.
    Returns (o [B,Hq,S,D] fp64, lse [B,Hq,S] fp64, src).
    """
    assert phases in ("all", "local", "global")
    q = q.to(torch.float64)
    k = k.to(torch.float64)
    v = v.to(torch.float64)
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    assert Hq == Hkv * kv_groups
    W = plan.W
    scale = 1.0 / math.sqrt(D)
    if plan.relay and src is None:
        src = relay_select(k, plan, norm)
    NB = plan.num_blocks
    kv_idx = torch.arange(Hq) // kv_groups
    ke = k[:, kv_idx]
    ve = v[:, kv_idx]
    stride_idx = torch.arange(NB) * W
    Ks, Vs = ke[:, :, stride_idx], ve[:, :, stride_idx]
    if plan.relay:
        # cpu_reference mode may name zero-padded rows of the last block;
        # those relay tokens are never visible (their block ends at or after
        # S-1), so any in-range row stands in for them.
        sidx = src[:, kv_idx].clamp(max=S - 1)                  # [B,Hq,NR]
        gi = sidx.unsqueeze(-1).expand(-1, -1, -1, D)
        Kr = torch.gather(ke, 2, gi)
        Vr = torch.gather(ve, 2, gi)
        if relay_scale is not None:
            sc = relay_scale.to(torch.float64)[kv_idx].view(1, Hq, 1, 1)
            Kr = Kr * sc
            Vr = Vr * sc
            if relay_dtype is not None and relay_dtype != torch.float64:
                Kr = Kr + (Kr.detach().to(relay_dtype).to(torch.float64) - Kr.detach())
                Vr = Vr + (Vr.detach().to(relay_dtype).to(torch.float64) - Vr.detach())
        r_end = (torch.arange(NB * plan.top_k) // plan.top_k + 1) * W - 1
    outs, lses = [], []
    lo, hi = (0, S) if rows is None else rows
    for c0 in range(lo, hi, chunk):
        c1 = min(hi, c0 + chunk)
        qi = torch.arange(c0, c1)
        ls = torch.clamp(qi - W + 1, min=0)
        w0 = max(0, c0 - W + 1)
        kj = torch.arange(w0, c1)
        qc = q[:, :, c0:c1]
        s_loc = qc @ ke[:, :, w0:c1].transpose(-1, -2) * scale
        m_loc = (kj[None, :] >= ls[:, None]) & (kj[None, :] <= qi[:, None])
        s_str = qc @ Ks.transpose(-1, -2) * scale
        m_str = stride_idx[None, :] < ls[:, None]
        if phases == "global":
            m_loc = torch.zeros_like(m_loc)
        if phases == "local":
            m_str = torch.zeros_like(m_str)
        parts_s = [s_loc.masked_fill(~m_loc, -math.inf), s_str.masked_fill(~m_str, -math.inf)]
        parts_v = [ve[:, :, w0:c1], Vs]
        if plan.relay:
            s_rel = qc @ Kr.transpose(-1, -2) * scale
            m_rel = r_end[None, :] < ls[:, None]
            if phases == "local":
                m_rel = torch.zeros_like(m_rel)
            parts_s.append(s_rel.masked_fill(~m_rel, -math.inf))
            parts_v.append(Vr)
        s_all = torch.cat(parts_s, dim=-1)
        lse = torch.logsumexp(s_all, dim=-1)
        p = torch.exp(s_all - lse.unsqueeze(-1))
        if phases != "all":  # empty subsets: 0 instead of 0/0
            p = torch.where(torch.isfinite(lse).unsqueeze(-1), p, torch.zeros_like(p))
        o = sum(p[..., off:off + pv.shape[2]] @ pv
                for off, pv in zip(np.cumsum([0] + [x.shape[2] for x in parts_v[:-1]]), parts_v))
        outs.append(o)
        lses.append(lse)
    return torch.cat(outs, dim=2), torch.cat(lses, dim=2), src


def forward_backward(q, k, v, dO, plan: Plan, kv_groups: int = 1,
                     relay_log_scale: Optional[torch.Tensor] = None, norm: str = "lanetree"):
    """Gradients by fp64 autograd of :func:`forward`.

    Relay rows are a gather of k/v, so their gradient lands on the source rows
    (the reference's scatter, core.py:2767-2815); selection itself has zero
    gradient.  With ``relay_log_scale`` the gradient w.r.t. the source rows
    carries the exp(alpha) factor (the reference's scatter omits it,
    core.py:3541-3544 vs :3274-3290), and d(alpha) = sum(dRK*RK + dRV*RV)
    (core.py:3363-3366).
    """
    q64 = q.detach().to(torch.float64).requires_grad_(True)
    k64 = k.detach().to(torch.float64).requires_grad_(True)
    v64 = v.detach().to(torch.float64).requires_grad_(True)
    a64 = None
    scale = None
    if relay_log_scale is not None:
        a64 = relay_log_scale.detach().to(torch.float64).requires_grad_(True)
        scale = torch.exp(a64)
    o, lse, src = forward(q64, k64, v64, plan, kv_groups, relay_scale=scale, norm=norm)
    o.backward(dO.to(torch.float64))
    grads = dict(dq=q64.grad, dk=k64.grad, dv=v64.grad)
    if a64 is not None:
        grads["dalpha"] = a64.grad
    return o.detach(), lse.detach(), src, grads


# ---------------------------------------------------------------------------
# Gradients of chosen rows (spot checks at sizes where full autograd is slow)
# ---------------------------------------------------------------------------

def query_row_grads(q, k, v, dO, plan: Plan, rows: tuple, kv_groups: int = 1,
                    src: Optional[torch.Tensor] = None):
    """dQ of queries [lo, hi) by fp64 autograd of :func:`forward` restricted to
    those rows.  O_i depends on q only through q_i, so differentiating the
    restricted forward with dO[lo:hi] gives exactly rows [lo, hi) of the full
    dQ (the reference's K4, core.py:1165-1316).  Returns [B, Hq, hi-lo, D]."""
    lo, hi = rows
    q64 = q.detach().to(torch.float64).requires_grad_(True)
    o, _, _ = forward(q64, k, v, plan, kv_groups, src=src, rows=rows)
    o.backward(dO[:, :, lo:hi].to(torch.float64))
    return q64.grad[:, :, lo:hi].detach()


def key_multiplicity(j: int, plan: Plan, src_row) -> np.ndarray:
    """How many times key row j occurs in the multiset of every query
    (int64 [S]): once for the queries whose local window holds it
    (i in [j, j+W-1], core.py:1016-1017), once more if j = s*W is a strided
    row and ls(i) > j (core.py:1060-1061), and once per relay token t with
    src[t] = j and (t//top_k + 1)*W - 1 < ls(i) (core.py:1115-1117).
    ``src_row``: the relay source rows of this (b, kv head), [NB*top_k]."""
    S, W = plan.S, plan.W
    i = np.arange(S, dtype=np.int64)
    ls = np.maximum(i - W + 1, 0)
    m = ((i >= j) & (i <= j + W - 1)).astype(np.int64)
    if j % W == 0:
        m += (ls > j)
    if plan.relay:
        for t in np.nonzero(np.asarray(src_row) == j)[0]:
            r = int(t) // plan.top_k
            m += (ls > (r + 1) * W - 1)
    return m


def key_row_grads(q, k, v, dO, plan: Plan, keys, lse, delta, src=None, kv_groups: int = 1):
    """dK and dV of the chosen key rows in closed form, fp64.

    For key row j of kv head g, summed over the query heads h of the group
    and over every query i that sees j (with the multiplicity of
    :func:`key_multiplicity`):
      P_ij = exp(q_i.k_j * scale - lse_i)
      dV_j = sum m_ij P_ij dO_i
      dK_j = scale * sum m_ij P_ij (dO_i.v_j - delta_i) q_i
    with delta_i = O_i.dO_i (the backward of core.py:1165-1316, 1650-1745,
    1755-1889, 2381-2492 plus the relay scatter, core.py:2767-2815, all
    landing on the source row).  ``lse`` and ``delta`` ([B, Hq, S]) must come
    from the exact forward.  No relay scale.  ``keys``: iterable of
    (b, g, j).  Returns {(b, g, j): (dK_j, dV_j)} as fp64 [D] tensors.
    """
    W = plan.W
    D = q.shape[-1]
    scale = 1.0 / math.sqrt(D)
    if plan.relay and src is None:
        src = relay_select(k, plan)
    out = {}
    for (b, g, j) in keys:
        src_row = src[b, g].numpy() if plan.relay else None
        m = key_multiplicity(j, plan, src_row)
        idx = torch.from_numpy(np.nonzero(m)[0])
        mm = torch.from_numpy(m[idx.numpy()]).to(torch.float64)
        kj = k[b, g, j].to(torch.float64)
        vj = v[b, g, j].to(torch.float64)
        dk = torch.zeros(D, dtype=torch.float64)
        dv = torch.zeros(D, dtype=torch.float64)
        for h in range(g * kv_groups, (g + 1) * kv_groups):
            qi = q[b, h, idx].to(torch.float64)
            doi = dO[b, h, idx].to(torch.float64)
            p = torch.exp(qi @ kj * scale - lse[b, h, idx].to(torch.float64)) * mm
            dv += p @ doi
            ds = p * (doi @ vj - delta[b, h, idx].to(torch.float64))
            dk += scale * (ds @ qi)
        out[(b, g, j)] = (dk, dv)
    return out


# ---------------------------------------------------------------------------
# Packed documents (varlen, core.py:3836-3954)
# ---------------------------------------------------------------------------

def varlen_plans(cu_seqlens, mode: str = "kernel", top_k: int = 2) -> list:
    """One plan per document, from the document's own length: the reference
    calls the whole op once per document on a narrow() view
    (core.py:3911-3952), so W and the relay switch follow each length."""
    return [make_plan(e - s, mode, top_k) for s, e in zip(cu_seqlens, cu_seqlens[1:])]


def forward_varlen(q, k, v, cu_seqlens, plans=None, kv_groups: int = 1,
                   relay_scale: Optional[torch.Tensor] = None, top_k: int = 2, **kw):
    """Documents [cu_seqlens[d], cu_seqlens[d+1]) attended on their own and the
    results concatenated along S (core.py:3923-3954: one call per document,
    each written into its slice of the output); differentiable.
    Returns (o, lse, [src of each document])."""
    plans = varlen_plans(cu_seqlens, top_k=top_k) if plans is None else plans
    outs, lses, srcs = [], [], []
    for (s, e), pl in zip(zip(cu_seqlens, cu_seqlens[1:]), plans):
        o, lse, src = forward(q[:, :, s:e], k[:, :, s:e], v[:, :, s:e], pl, kv_groups,
                              relay_scale=relay_scale if pl.relay else None, **kw)
        outs.append(o)
        lses.append(lse)
        srcs.append(src)
    return torch.cat(outs, dim=2), torch.cat(lses, dim=2), srcs


def forward_backward_varlen(q, k, v, dO, cu_seqlens, plans=None, kv_groups: int = 1,
                            relay_log_scale: Optional[torch.Tensor] = None, top_k: int = 2):
    """Gradients of :func:`forward_varlen` by fp64 autograd; d(relay_log_scale)
    sums over every document with relay, the parameter being shared by the
    per-document calls (core.py:3911-3952 pass the same tensor)."""
    q64 = q.detach().to(torch.float64).requires_grad_(True)
    k64 = k.detach().to(torch.float64).requires_grad_(True)
    v64 = v.detach().to(torch.float64).requires_grad_(True)
    a64 = scale = None
    if relay_log_scale is not None:
        a64 = relay_log_scale.detach().to(torch.float64).requires_grad_(True)
        scale = torch.exp(a64)
    o, lse, srcs = forward_varlen(q64, k64, v64, cu_seqlens, plans, kv_groups, relay_scale=scale,
                                  top_k=top_k)
    o.backward(dO.to(torch.float64))
    grads = dict(dq=q64.grad, dk=k64.grad, dv=v64.grad)
    if a64 is not None:
        grads["dalpha"] = a64.grad if a64.grad is not None else torch.zeros_like(a64)
    return o.detach(), lse.detach(), srcs, grads


def causal_sdpa_reference(q, k, v):
    """Dense causal attention in fp64 (the library routine the first W rows
    of every sequence must reduce to: their sets are pure causal prefixes)."""
    q = q.to(torch.float64)
    k = k.to(torch.float64)
    v = v.to(torch.float64)
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)


# ---------------------------------------------------------------------------
# The HIP build's packing of the global rows (checked here against the
# brute-force sets; the kernels rely on it).
# ---------------------------------------------------------------------------

def packed_rows(plan: Plan, src) -> list:
    """Source row of every packed global row: block r contributes its strided
    row r*W, then (relay on) its top_k relay rows in rank order."""
    rows = []
    for r in range(plan.num_blocks):
        rows.append(r * plan.W)
        if plan.relay:
            rows.extend(int(x) for x in src[r][: plan.top_k])
    return rows


def packed_prefix_len(i: int, plan: Plan) -> int:
    """Global rows visible to query i form a prefix of the packed array:
    (1+top_k)*floor(ls/W) + (ls % W != 0) with relay, ceil(ls/W) without."""
    ls = max(0, i - plan.W + 1)
    rpb = 1 + plan.top_k if plan.relay else 1
    return rpb * (ls // plan.W) + (1 if ls % plan.W else 0)
