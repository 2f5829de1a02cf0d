"""Write golden vectors from the reference's own CPU implementation.

Runs ONLY in the build container, where the reference tree is mounted
(default ``/root/reference``, override with ``CRA_REFERENCE_ROOT``); it is
never run by the tests.  It loads ``cron_root_attention/cpu_reference.py``
by file path (that module imports only ``math`` and ``torch``) and calls
``cra_cpu_fast`` -- the function the reference dispatches CPU tensors to
(core.py:3794-3796) -- on seeded fp32 inputs drawn q, then k, then v, then
dO from ``torch.Generator().manual_seed(seed)`` (the recipe of
bench_vec_vs_loop.py:25-30).

Each fixture ``cra_cpu_fast_B{B}_H{H}_S{S}_D{D}.npz`` holds:
  * input checksums (fp64 sums and the first values) so a drift of the
    generator is detected instead of silently comparing different inputs;
  * the output rows ``o_rows`` at indices ``rows`` (all rows for S <= 256,
    a strided sample plus the first and last 64 rows otherwise);
  * fp64 sums and sums of squares of the whole output, per head;
  * when the reference's autograd runs, the same for dq/dk/dv.
The inputs themselves are regenerated from the seed by the tests.
"""
from __future__ import annotations

import importlib.util
import json
import os
import sys

import numpy as np
import torch

SHAPES = [(1, 2, 64, 16), (1, 2, 256, 32), (1, 4, 1024, 64), (1, 8, 4096, 64)]
SEED = 0
HERE = os.path.dirname(os.path.abspath(__file__))


def make_inputs(B, H, S, D, seed=SEED):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, S, D, generator=g, dtype=torch.float32)
    k = torch.randn(B, H, S, D, generator=g, dtype=torch.float32)
    v = torch.randn(B, H, S, D, generator=g, dtype=torch.float32)
    dO = torch.randn(B, H, S, D, generator=g, dtype=torch.float32)
    return q, k, v, dO


def sample_rows(S):
    if S <= 256:
        return np.arange(S)
    rows = set(range(0, S, 16)) | set(range(64)) | set(range(S - 64, S))
    return np.array(sorted(rows))


def summarize(prefix, t, rows, out):
    t64 = t.detach().to(torch.float64)
    out[f"{prefix}_rows"] = t.detach()[:, :, rows].numpy().astype(np.float32)
    out[f"{prefix}_sum"] = t64.sum(dim=(2, 3)).numpy()
    out[f"{prefix}_sumsq"] = (t64 ** 2).sum(dim=(2, 3)).numpy()


def main():
    root = os.environ.get("CRA_REFERENCE_ROOT", "/root/reference")
    path = os.path.join(root, "cron_root_attention", "cpu_reference.py")
    spec = importlib.util.spec_from_file_location("_ref_cpu_reference", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    manifest = {}
    for (B, H, S, D) in SHAPES:
        q, k, v, dO = make_inputs(B, H, S, D)
        out = {"shape": np.array([B, H, S, D]), "seed": np.array(SEED)}
        for name, t in (("q", q), ("k", k), ("v", v), ("dO", dO)):
            out[f"in_{name}_sum"] = np.array(t.to(torch.float64).sum().item())
            out[f"in_{name}_head"] = t.reshape(-1)[:8].numpy()
        rows = sample_rows(S)
        out["rows"] = rows
        qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
        o = mod.cra_cpu_fast(qg, kg, vg)
        summarize("o", o, rows, out)
        grad_note = "ok"
        try:
            o.backward(dO)
            summarize("dq", qg.grad, rows, out)
            summarize("dk", kg.grad, rows, out)
            summarize("dv", vg.grad, rows, out)
        except RuntimeError as e:  # in-place ops in the reference may block autograd
            grad_note = f"unavailable: {str(e).splitlines()[0][:160]}"
        name = f"cra_cpu_fast_B{B}_H{H}_S{S}_D{D}.npz"
        np.savez_compressed(os.path.join(HERE, name), **out)
        manifest[name] = {"grad": grad_note, "rows": int(len(rows))}
        print(name, manifest[name], flush=True)
    with open(os.path.join(HERE, "MANIFEST.json"), "w") as f:
        json.dump({"source": "cron_root_attention/cpu_reference.py:198-339 (cra_cpu_fast)",
                   "torch": torch.__version__, "fixtures": manifest}, f, indent=1)


if __name__ == "__main__":
    sys.exit(main())
