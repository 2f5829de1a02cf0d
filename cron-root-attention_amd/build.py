"""Build libcra_hip.so (gfx950) and libcra_torch.so from csrc/.

Usage: ``python cron-root-attention_amd/build.py [--jobs N] [--verbose]``.
Each ``csrc/*.hip`` is compiled with hipcc and each host-only ``csrc/cra_*.cpp``
(the CPU-tensor path) with the system C++ compiler to an object under
``_build/``; the objects are linked into ``cron_root_attention/libcra_hip.so``
next to the Python package that loads it.  ``csrc/cra_torch.cpp`` (the torch
operator ``cra::attention`` with its autograd in C++, bound to libcra_hip.so at
run time) is compiled against the installed torch into
``cron_root_attention/libcra_torch.so``.  Every call recompiles (the build is
the "does it build" check); it takes about a minute.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "cron_root_attention")
LIB_NAME = "libcra_hip.so"
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = os.path.join(rocm, "bin", "hipcc")
    if os.path.exists(cand):
        return cand
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def cxx() -> str:
    return os.environ.get("CXX") or shutil.which("g++") or shutil.which("c++") or "g++"


TORCH_SRC = "cra_torch.cpp"
TORCH_LIB_NAME = "libcra_torch.so"


def torch_ext_cmd(out: str) -> list[str]:
    """Compile and link the torch operator binding (host code only: torch's
    headers, its HIP stream header, the C ABI header; no GPU code)."""
    import torch
    from torch.utils import cpp_extension
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    inc = [f"-I{p}" for p in cpp_extension.include_paths()]
    libdirs = cpp_extension.library_paths()
    return [cxx(), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-function",
            "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM",
            f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
            f"-I{os.path.join(os.path.dirname(HERE), 'include')}", *inc,
            f"-I{os.path.join(rocm, 'include')}", os.path.join(CSRC, TORCH_SRC), "-o", out,
            *[f"-L{d}" for d in libdirs], *[f"-Wl,-rpath,{d}" for d in libdirs],
            "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch", "-ldl"]


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-mcode-object-version=5",
        # Packed fp32 VALU ops stay off: the kernels use scalar/float2 math only.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-function",
        "-Wno-unused-variable",
    ]


def run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-fp32 feature: drop that warning only
    err = "\n".join(l for l in res.stderr.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(jobs: int | None = None, verbose: bool = False, build_dir: str | None = None) -> str:
    t0 = time.time()
    cc = hipcc()
    build_dir = build_dir or os.path.join(os.path.dirname(HERE), "_build")
    os.makedirs(build_dir, exist_ok=True)
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    objs = []
    cmds = []
    for s in srcs:
        obj = os.path.join(build_dir, s.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([cc, *common_flags(), "-c", os.path.join(CSRC, s), "-o", obj])
    # host-only C++ (the CPU-tensor path): the system C++ compiler, no GPU code
    for s in sorted(f for f in os.listdir(CSRC) if f.endswith(".cpp") and f != TORCH_SRC):
        obj = os.path.join(build_dir, s.replace(".cpp", ".cpp.o"))
        objs.append(obj)
        cmds.append([cxx(), "-O3", "-std=c++17", "-fPIC", "-pthread", "-Wall",
                     "-c", os.path.join(CSRC, s), "-o", obj])
    ext_out = os.path.join(OUT_DIR, TORCH_LIB_NAME)
    cmds.append(torch_ext_cmd(ext_out + ".tmp"))
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(run, c, verbose) for c in cmds]:
            f.result()
    os.replace(ext_out + ".tmp", ext_out)
    out = os.path.join(OUT_DIR, LIB_NAME)
    tmp = out + ".tmp"
    run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", "-o", tmp, *objs], verbose)
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} in {time.time() - t0:.1f}s", flush=True)
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    print(build(args.jobs, args.verbose))
    return 0


if __name__ == "__main__":
    sys.exit(main())
