"""Build ``libyufhip.so`` in-tree with hipcc for gfx950.

Every ``csrc/*.hip`` and ``csrc/*.cpp`` file is compiled to an object under
``yufmusicgen_amd/_build/`` (in parallel) and linked into
``yufmusicgen_amd/libyufhip.so``.  All device code is built with packed-FP32
instructions disabled (``-Xclang -target-feature -Xclang -packed-fp32-ops``).

    python -m yufmusicgen_amd.build
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libyufhip.so"
ARCH = os.environ.get("YUF_OFFLOAD_ARCH", "gfx950")

COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", f"-I{PKG.parent / 'include'}"]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-munsafe-fp-atomics"]


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return found


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [_hipcc(), *COMMON]
    if src.suffix == ".hip":
        cmd += DEVICE
    cmd += ["-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    workers = min(8, max(1, os.cpu_count() or 1))
    with cf.ThreadPoolExecutor(workers) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
