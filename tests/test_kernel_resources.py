"""Compiler resource report of every device kernel in libyufhip.so.

``yufmusicgen_amd/build.py`` keeps clang's kernel-resource-usage remarks
(registers, scratch, spills, LDS, occupancy) in
``_build/kernel_resources.json``.  A kernel that silently starts using scratch
memory -- a prefetch array the compiler could not keep in registers, a lambda
left as a call whose arguments then live in private memory -- loses most of its
speed with no change in results, so no test of the outputs sees it.  These
checks do: no kernel may use scratch or a dynamic stack except the ones listed
below, each with its measured limit and the reason.
"""

from __future__ import annotations

import json
import re

import pytest

from yufmusicgen_amd import build as yuf_build

# Kernel-name pattern -> largest allowed scratch (bytes per lane) and why.
ALLOWED_SCRATCH = {
    # The unsplit N = 64 chunk scan with fused prep (the C5 shape): its
    # 10-wave workgroup (three waves on some SIMDs) leaves 168 VGPRs per lane,
    # and the compiler spills 4.
    r"wkv7_chunk_kernelILi4ELb1ELb0ELb[01]E": 20,
}


@pytest.fixture(scope="module")
def resources():
    path = yuf_build.RESOURCES
    sources = list(yuf_build.CSRC.glob("*.hip")) + list(yuf_build.CSRC.glob("*.h"))
    if not path.exists() or path.stat().st_mtime < max(s.stat().st_mtime for s in sources):
        yuf_build.build(verbose=False)
    return json.loads(path.read_text())


def test_report_covers_every_kernel_family(resources):
    assert len(resources) > 100
    for family in ("gemm_big_kernel", "gemm_decode_kernel", "wkv7_chunk_kernel", "wkv7_step_kernel",
                   "rosa_scan_kernel", "rosa_carry_kernel", "sample_kernel", "layernorm_kernel"):
        assert any(family in k for k in resources), family
    for name, r in resources.items():
        for field in ("vgprs", "scratch_bytes_per_lane", "waves_per_simd", "lds_bytes", "dynamic_stack"):
            assert field in r, (name, field)


def test_no_scratch_or_dynamic_stack(resources):
    bad = []
    for name, r in resources.items():
        assert not r["dynamic_stack"], name
        scratch = r["scratch_bytes_per_lane"]
        if scratch == 0:
            continue
        limit = next((lim for pat, lim in ALLOWED_SCRATCH.items() if re.search(pat, name)), 0)
        if scratch > limit:
            bad.append((name, scratch, r["vgpr_spills"]))
    assert not bad, f"kernels using scratch memory (name, bytes/lane, VGPR spills): {bad}"


def test_lds_fits_a_compute_unit(resources):
    for name, r in resources.items():
        assert r["lds_bytes"] <= 160 * 1024, (name, r["lds_bytes"])
