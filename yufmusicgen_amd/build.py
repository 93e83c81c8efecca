"""Build ``libyufhip.so`` in-tree with hipcc for gfx950.

Every ``csrc/*.hip`` and ``csrc/*.cpp`` file is compiled to an object under
``yufmusicgen_amd/_build/`` (in parallel) and linked into
``yufmusicgen_amd/libyufhip.so``.  All device code is built with packed-FP32
instructions disabled (``-Xclang -target-feature -Xclang -packed-fp32-ops``).
The compiler's per-kernel resource report (registers, scratch, spills, LDS,
occupancy) is kept in ``_build/kernel_resources.json``.

    python -m yufmusicgen_amd.build
"""

from __future__ import annotations

import concurrent.futures as cf
import json
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libyufhip.so"
RESOURCES = BUILD / "kernel_resources.json"
ARCH = os.environ.get("YUF_OFFLOAD_ARCH", "gfx950")

COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", f"-I{PKG.parent / 'include'}"]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-munsafe-fp-atomics"]


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return found


_REMARK = re.compile(r"remark:\s+(Function Name|[A-Za-z ]+?)(?: \[[^\]]*\])?:\s+(\S+) \[-Rpass-analysis=kernel-resource-usage\]")
_FIELDS = {"VGPRs": "vgprs", "AGPRs": "agprs", "TotalSGPRs": "sgprs", "ScratchSize": "scratch_bytes_per_lane",
           "Occupancy": "waves_per_simd", "SGPRs Spill": "sgpr_spills", "VGPRs Spill": "vgpr_spills",
           "LDS Size": "lds_bytes", "Dynamic Stack": "dynamic_stack"}


def _resources(stderr: str, src: Path) -> dict:
    """Per-kernel figures from clang's kernel-resource-usage remarks."""
    out, cur = {}, None
    for m in _REMARK.finditer(stderr):
        key, val = m.group(1).strip(), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {"source": src.name})
        elif cur is not None and key in _FIELDS:
            cur[_FIELDS[key]] = val == "True" if key == "Dynamic Stack" else int(val)
    return out


def _compile(src: Path):
    obj = BUILD / (src.name + ".o")
    cmd = [_hipcc(), *COMMON]
    if src.suffix == ".hip":
        cmd += DEVICE + ["-Rpass-analysis=kernel-resource-usage"]
    cmd += ["-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj, _resources(proc.stderr, src)


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    workers = min(8, max(1, os.cpu_count() or 1))
    with cf.ThreadPoolExecutor(workers) as pool:
        results = list(pool.map(_compile, sources))
    objects = [obj for obj, _ in results]
    resources = {}
    for _, r in results:
        resources.update(r)
    RESOURCES.write_text(json.dumps(resources, indent=1, sort_keys=True))
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
