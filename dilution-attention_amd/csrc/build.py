"""Build libdilution_hip.so for gfx950 from the HIP sources in this folder.

    python dilution-attention_amd/csrc/build.py [--jobs N]

Each translation unit is compiled with hipcc into _build/ (git-ignored), then
linked into dilution/libdilution_hip.so next to the Python package, in-tree, so
the built library travels with the source tree.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(os.path.dirname(HERE), "dilution")
OUT = os.path.join(PKG, "libdilution_hip.so")
BUILD = os.path.join(HERE, "_build")
SOURCES = ["dil_api.hip", "dil_decode.hip", "dil_forward.hip", "dil_backward.hip", "dil_timing.hip",
           "dil_noalloc.hip", "dil_linear.hip"]
# (object stem, source, extra flags): the ablation variants of each bid
# function are one object each, built from the same source
VARIANT_OBJECTS = [(f"dil_variants_b{b}", "dil_variants.hip", [f"-DDIL_VARIANT_BID={b}"]) for b in range(8)]
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 VALU instructions stay off (device code only; the host pass
    # warns that it does not know the feature, which is harmless)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libdilution_hip.so)")


def _compile(unit) -> str:
    stem, src, extra = unit
    obj = os.path.join(BUILD, stem + ".o")
    cmd = [hipcc(), *FLAGS, *extra, "-c", os.path.join(HERE, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {stem}:\n{proc.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    units = [(os.path.splitext(src)[0], src, []) for src in SOURCES] + VARIANT_OBJECTS
    jobs = jobs or min(len(units), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, units))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    build(args.jobs, verbose=True)
    sys.exit(0)
