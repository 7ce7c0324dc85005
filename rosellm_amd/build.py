"""Build the gfx950 shared library ``librosellm_amd.so`` in-tree with hipcc.

Usage: ``python -m rosellm_amd.build`` (or ``__graft_entry__.build()``).  The
library lands next to this file so it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_NAME = "librosellm_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME

SOURCES = [
    "rrl_host.hip",
    "logprob.hip",
    "logprob_resident.hip",
    "objectives.hip",
    "estimators.hip",
    "sampler.hip",
    "lm_head.hip",
    "layout.hip",
]

ARCH = os.environ.get("ROSELLM_AMD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # Packed FP32 ops are kept out of generated code on this target.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-fvisibility=hidden",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the ROCm toolchain is required to build rosellm_amd")


def _compile(src: str, obj: Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(INCLUDE), "-I", str(CSRC), "-c", str(CSRC / src),
           "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr[-8000:]}")


def build(verbose: bool = True) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""

    with tempfile.TemporaryDirectory(prefix="rosellm_amd_build_") as tmp:
        objs = [Path(tmp) / (Path(s).stem + ".o") for s in SOURCES]
        jobs = min(len(SOURCES), max(1, (os.cpu_count() or 4) // 2))
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            list(pool.map(lambda so: _compile(*so), zip(SOURCES, objs)))
        tmp_lib = Path(tmp) / LIB_NAME
        cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o",
               str(tmp_lib)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"link failed:\n{proc.stderr[-8000:]}")
        # Atomic replace so a concurrently loaded library is never half-written.
        staged = PKG_DIR / (LIB_NAME + ".tmp")
        shutil.copyfile(tmp_lib, staged)
        os.replace(staged, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build()
    sys.exit(0)
