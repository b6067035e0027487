"""Build the gfx950 HIP library ``bayes_ssm/libbssm_hip.so`` in-tree.

Usage: ``python bayes-ssm_amd/build.py`` (also called by ``__graft_entry__.build``).
Each ``csrc/*.hip`` file is compiled separately with hipcc for gfx950 and the
objects are linked into one shared library that exposes the C ABI declared in
``include/bssm.h``.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT = Path(os.environ.get("BSSM_BUILD_OUT", ROOT / "bayes_ssm" / "libbssm_hip.so"))
BUILD = Path(os.environ.get("BSSM_BUILD_DIR", ROOT / "_build"))
# Extra compiler flags (BSSM_EXTRA_FLAGS, space separated).
EXTRA = os.environ.get("BSSM_EXTRA_FLAGS", "").split()
ARCH = os.environ.get("BSSM_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # Packed FP32 (v_pk_*_f32) stays off: ordinary scalar FP32 code only.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    *EXTRA,
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return path


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    noisy = [ln for ln in proc.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if noisy:
        sys.stderr.write("\n".join(noisy) + "\n")
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    OUT.parent.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build()
