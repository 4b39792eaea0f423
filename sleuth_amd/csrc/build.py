"""Builds libforge_attn.so (the HIP kernels + C ABI) in-tree for gfx950 with hipcc.

Usage: python -m sleuth_amd.csrc.build [-v]
The library lands in sleuth_amd/_lib/ so that it travels with the source tree.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
ROOT = PKG.parent
LIB_DIR = PKG / "_lib"
LIB_NAME = "libforge_attn.so"
SOURCES = ["abi.hip", "prep.hip", "decode.hip", "prefill.hip"]
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from emitting packed fp32 VALU ops (v_pk_*_f32).
# atomic optimizer off: the kernels' atomics are single-lane work tickets; the optimizer's
# wave-wide rewrite reads the result at once (a wait for the round trip) where the kernel
# means to read it much later.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is needed to build libforge_attn")
    return exe


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(ROOT / "include"), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stdout}\n{r.stderr}")
    if verbose and r.stderr.strip():
        print(r.stderr, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every source and link the shared library; returns its path."""
    obj_dir = PKG / "_build"
    obj_dir.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    objs = [obj_dir / (Path(s).stem + ".o") for s in SOURCES]
    jobs = min(len(SOURCES), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda so: _compile(CSRC / so[0], so[1], verbose), zip(SOURCES, objs)))
    out = LIB_DIR / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
