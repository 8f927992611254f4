"""Build libamd_tuned_torch_hip.so (the gfx950 C-ABI kernel library) in-tree.

    python rocm-kernel-select_amd/build_lib.py [--arch gfx950] [-j N] [--incremental]

Every csrc/*.hip file is compiled by hipcc into rocm-kernel-select_amd/_build/*.o and
linked into rocm-kernel-select_amd/amd_tuned_torch/_lib/libamd_tuned_torch_hip.so.  The
library links only against the HIP runtime (no libtorch), so one build serves every
torch/Python version on the machine.  hipcc cross-compiles for gfx950 without a GPU.
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
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "amd_tuned_torch", "_lib")
LIBNAME = "libamd_tuned_torch_hip.so"
LIBPATH = os.path.join(LIBDIR, LIBNAME)

# -packed-fp32-ops: keep the compiler from forming packed fp32 VALU ops (v_pk_*_f32).
COMMON_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(arch: str = "gfx950", jobs: int | None = None, verbose: bool = True,
          incremental: bool = False) -> str:
    """Compile every csrc/*.hip and link the shared library; returns its path.  With
    `incremental`, an object newer than its source, every csrc header and this script is
    reused (the default rebuilds everything)."""
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    cc = hipcc()
    sources = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    if not sources:
        raise RuntimeError("no HIP sources under " + CSRC)
    t0 = time.time()

    deps = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")] + [__file__]
    newest_dep = max(os.path.getmtime(d) for d in deps)

    def compile_one(src: str) -> str:
        obj = os.path.join(BUILD, src[:-4] + ".o")
        if incremental and os.path.exists(obj):
            t_obj = os.path.getmtime(obj)
            if t_obj > os.path.getmtime(os.path.join(CSRC, src)) and t_obj > newest_dep:
                return obj
        _run([cc, f"--offload-arch={arch}", *COMMON_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    jobs = jobs or min(len(sources), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(compile_one, sources))
    tmp = LIBPATH + ".tmp"
    _run([cc, f"--offload-arch={arch}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIBPATH)
    if verbose:
        print(f"built {LIBPATH} from {len(sources)} sources in {time.time() - t0:.1f}s")
    return LIBPATH


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--arch", default=os.environ.get("AMD_TUNED_TORCH_GPU_ARCH", "gfx950"))
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("--incremental", action="store_true",
                    help="reuse objects that are newer than their source and every header")
    args = ap.parse_args()
    build(args.arch, args.jobs, incremental=args.incremental)


if __name__ == "__main__":
    main()
