"""Chunked CPU path of the reference, restated for the timed CPU baseline.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  ``bench.py`` times
this on the GPU box's host cores as ``cpu_baseline`` (kind "port"); tests
check it against :func:`oracle.cra_oracle.forward`.

Follows ``cra_cpu_fast`` (cpu_reference.py:198-339): the strided and relay
rows are gathered once into one "non-local" K/V pair (cpu_reference.py:244-268),
then queries are processed in chunks of 256 with four batched products per
chunk -- local q.k, non-local q.k, local p.v, non-local p.v
(cpu_reference.py:287-337) -- with in-place masks, one global row max over
both score blocks, in-place exp and a final divide.  W, relay and the relay
rows are parameters so the same code times either the reference's CPU
semantics (floor W, relay always on) or the GPU-kernel semantics.
"""
from __future__ import annotations

import math

import torch

from .cra_oracle import Plan, relay_select


def cra_cpu_chunked(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, plan: Plan,
                    src: torch.Tensor | None = None, chunk: int = 256,
                    norm: str = "lanetree", q_rows: tuple | None = None) -> torch.Tensor:
    """Forward only, in the input dtype (fp32 for the baseline).

    ``q_rows=(lo, hi)`` restricts the work to queries [lo, hi) so a bounded
    sample of a long sequence can be timed; the result then holds only
    those rows.
    """
    B, H, S, D = q.shape
    W = plan.W
    BH = B * H
    scale = 1.0 / math.sqrt(D)
    NB = plan.num_blocks
    stride_idx = torch.arange(NB) * W
    K_glob = [k[:, :, stride_idx]]
    V_glob = [v[:, :, stride_idx]]
    ends = [stride_idx]        # strided row s*W visible iff s*W < ls   -> compare s*W
    if plan.relay:
        if src is None:
            src = relay_select(k, plan, norm)
        src = src.clamp(max=S - 1)
        gi = src.unsqueeze(-1).expand(-1, -1, -1, D)
        K_glob.append(torch.gather(k, 2, gi))
        V_glob.append(torch.gather(v, 2, gi))
        # relay token t visible iff (t//top_k + 1)*W - 1 < ls
        ends.append((torch.arange(NB * plan.top_k) // plan.top_k + 1) * W - 1)
    Kg = torch.cat(K_glob, dim=2).reshape(BH, -1, D).contiguous()
    Vg = torch.cat(V_glob, dim=2).reshape(BH, -1, D).contiguous()
    thresh = torch.cat(ends)                                   # visible iff thresh < ls
    lo, hi = (0, S) if q_rows is None else q_rows
    out = torch.empty(B, H, hi - lo, D, dtype=q.dtype)
    qf = q.reshape(BH, S, D)
    kf = k.reshape(BH, S, D)
    vf = v.reshape(BH, S, D)
    for c0 in range(lo, hi, chunk):
        c1 = min(hi, c0 + chunk)
        qi = torch.arange(c0, c1)
        ls = torch.clamp(qi - W + 1, min=0)
        w0 = max(0, c0 - W + 1)
        kj = torch.arange(w0, c1)
        qc = qf[:, c0:c1]
        s_loc = torch.bmm(qc, kf[:, w0:c1].transpose(1, 2)).mul_(scale)
        band = (kj[None, :] >= ls[:, None]) & (kj[None, :] <= qi[:, None])
        s_loc.masked_fill_(~band, float("-inf"))
        s_glb = torch.bmm(qc, Kg.transpose(1, 2)).mul_(scale)
        s_glb.masked_fill_(~(thresh[None, :] < ls[:, None]), float("-inf"))
        m = torch.maximum(s_loc.amax(-1), s_glb.amax(-1)).unsqueeze(-1)
        p_loc = s_loc.sub_(m).exp_()
        p_glb = s_glb.sub_(m).exp_()
        num = torch.bmm(p_loc, vf[:, w0:c1]).add_(torch.bmm(p_glb, Vg))
        den = (p_loc.sum(-1) + p_glb.sum(-1)).unsqueeze(-1)
        out[:, :, c0 - lo:c1 - lo] = num.div_(den).view(B, H, c1 - c0, D)
    return out
