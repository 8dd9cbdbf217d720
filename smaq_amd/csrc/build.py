"""Builds libsmaq_hip.so (gfx950) from the HIP sources in this directory.

    python -m smaq_amd.csrc.build          # or smaq_amd.csrc.build.build()

Every .hip file is compiled to an object with hipcc and the objects are linked
into ``smaq_amd/_lib/libsmaq_hip.so`` (in-tree, so the library travels with the
source tree).  It always rebuilds.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
LIB_DIR = PKG / "_lib"
LIB_NAME = "libsmaq_hip.so"
OBJ_DIR = PKG / "_build"

ARCH = os.environ.get("SMAQ_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off: the encoders reproduce torch-CPU rounding, so no implicit
# multiply-add fusion.  Packed FP32 VALU forms are disabled on this pool.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-source extra flags.  The matrix-core decode kernel reduces maxima with
# DPP; without IEEE mode (and with NaN-free arithmetic assumed) each step is one
# fused v_max_f32_dpp instead of a DPP move plus two NaN-quieting maxima.
EXTRA_FLAGS = {
    "attention_mfma.hip": ["-fno-honor-nans", "-mno-amdgpu-ieee"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _compile(src: Path, obj: Path) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile every .hip source and link libsmaq_hip.so; returns its path."""
    sources = sorted(HERE.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no .hip sources in {HERE}")
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    objs = [OBJ_DIR / (s.stem + ".o") for s in sources]
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _compile(*so), zip(sources, objs)))
    out = LIB_DIR / LIB_NAME
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
