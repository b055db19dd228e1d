"""Build libh3fp8.so (the HIP kernels + C ABI) for gfx950 with hipcc, in-tree.

    python minimax-h3-2x-dgx-spark-tp2_amd/build.py [--jobs N] [--asm]

Each csrc/*.hip compiles to an object under _build/ (git-ignored); the shared library lands next to the Python
package (h3_tp2_amd/libh3fp8.so), where the loader looks for it.  ``--asm`` also writes the gfx950 assembly of each
source to _build/ (for reading register use and the instruction schedule).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "h3_tp2_amd", "libh3fp8.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 anywhere; denormals kept; no contraction of a*b+c behind the
# reference's back (the epilogue's one fma is explicit).
COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-flush-denormals-to-zero", "-ffp-contract=off",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{INCLUDE}",
]


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str, asm: bool) -> str:
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *COMMON, "-c", src, "-o", obj]
    subprocess.run(cmd, check=True)
    if asm:
        s = os.path.join(BUILD, os.path.basename(src)[:-4] + f"-{ARCH}.s")
        subprocess.run([HIPCC, *COMMON, "--cuda-device-only", "-S", src, "-o", s], check=True)
    return obj


def build(jobs: int = 4, asm: bool = False, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda s: _compile(s, asm), srcs))
    tmp = LIB + ".tmp"
    subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], check=True)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources", file=sys.stderr)
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--asm", action="store_true")
    a = ap.parse_args()
    build(a.jobs, a.asm)


if __name__ == "__main__":
    main()
