"""AddressSanitizer + UndefinedBehaviorSanitizer build of the library's host code.

The .yuf loader (``csrc/checkpoint.cpp``, its own JSON parser) and the host
sampler (``csrc/sampler.cpp``) are compiled with g++ ``-fsanitize=address,
undefined`` together with ``tests/host_sanitize.cpp`` and run on valid
checkpoints, on every class of malformed file (truncations, corrupted header
bytes, lying sizes and offsets) and on random and edge-case sampler inputs.
Any sanitizer report aborts the driver, which fails the test.
"""

from __future__ import annotations

import json
import os
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

from yufmusicgen_amd.checkpoint import write_yuf
from yufmusicgen_amd.config import PRESETS
from yufmusicgen_amd.synth import synth_weights

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "yufmusicgen_amd" / "csrc"
GOLDEN_YUF = ROOT / "tests" / "golden" / "model_state_test.yuf"

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")

ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    out = tmp_path_factory.mktemp("asan") / "host_sanitize"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           str(ROOT / "tests" / "host_sanitize.cpp"), str(CSRC / "checkpoint.cpp"),
           str(CSRC / "sampler.cpp"), str(CSRC / "errors.cpp"), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-4000:]
    return out


def run(driver, *args):
    res = subprocess.run([str(driver), *map(str, args)], capture_output=True, text=True, env=ENV, timeout=120)
    assert res.returncode == 0, f"{args[:2]}: rc {res.returncode}\n{res.stdout[-2000:]}\n{res.stderr[-4000:]}"
    assert "runtime error" not in res.stderr and "Sanitizer" not in res.stderr, res.stderr[-4000:]
    return res.stdout.strip()


def tensor_names(path: Path):
    raw = path.read_bytes()
    hlen = struct.unpack_from("<Q", raw, 8)[0]
    header = json.loads(raw[16:16 + hlen])
    return [t["name"] for t in header["tensors"]]


@pytest.fixture(scope="module")
def checkpoints(tmp_path_factory):
    d = tmp_path_factory.mktemp("yuf")
    cfg = PRESETS["tiny"]
    w = synth_weights(cfg, seed=3)
    v1 = d / "tiny_v1.yuf"
    v2 = d / "tiny_v2.yuf"
    write_yuf(str(v1), cfg, w)
    write_yuf(str(v2), cfg, w, linear_bf16=True)
    return [GOLDEN_YUF, v1, v2]


def test_valid_checkpoints_load_clean(driver, checkpoints):
    for path in checkpoints:
        out = run(driver, "ckpt", path, *tensor_names(path))
        assert out.startswith("ok "), out


def test_malformed_checkpoints_fail_clean(driver, checkpoints, tmp_path):
    rng = np.random.default_rng(0)
    src = checkpoints[2].read_bytes()
    hlen = struct.unpack_from("<Q", src, 8)[0]
    variants, must_fail = [], []
    # Truncations: inside the magic, the length, the header and the payload.
    for cut in sorted({0, 3, 8, 12, 16, 17, 16 + hlen // 2, 16 + hlen - 1, 16 + hlen,
                       16 + hlen + 5, len(src) - 3}):
        must_fail.append(src[:cut])
    # The binary version field (the loader, like checkpoint.rs:103-107, checks it
    # and not the header's "version" key).
    for version in (0, 3, 99):
        must_fail.append(src[:4] + struct.pack("<I", version) + src[8:])
    # A header length beyond the file, zero and absurd.
    for bogus in (len(src), 0, 1 << 40, (1 << 64) - 1):
        must_fail.append(src[:8] + struct.pack("<Q", bogus) + src[16:])
    # Random byte corruptions inside the JSON header (structure, numbers, strings).
    for _ in range(120):
        b = bytearray(src)
        for _ in range(int(rng.integers(1, 4))):
            b[16 + int(rng.integers(0, hlen))] = int(rng.integers(0, 256))
        variants.append(bytes(b))
    # Header rewrites that lie about offsets, counts and shapes.
    header = json.loads(src[16:16 + hlen])
    payload = src[16 + hlen:]
    for mutate in ("offset", "shape", "dtype", "count", "overlap"):
        h = json.loads(json.dumps(header))
        t = h["tensors"][len(h["tensors"]) // 2]
        if mutate == "offset":
            t["offset"] = len(payload) - 4
        elif mutate == "shape":
            t["shape"] = [1 << 31, 1 << 31]
        elif mutate == "dtype":
            t["dtype"] = "f64"
        elif mutate == "version":
            h["version"] = 99
        elif mutate == "count":
            t["count"] = t["count"] + 1
        else:
            t["offset"] = h["tensors"][0]["offset"]
        text = json.dumps(h).encode()
        # Overlapping tensors are readable (checkpoint.rs:149-157 only slices
        # by offset and count), so that lie need not fail.
        (variants if mutate == "overlap" else must_fail).append(
            src[:8] + struct.pack("<Q", len(text)) + text + payload)
    names = tensor_names(checkpoints[2])
    for i, blob in enumerate(must_fail):
        path = tmp_path / f"bad_{i}.yuf"
        path.write_bytes(blob)
        out = run(driver, "ckpt", path, *names)
        assert out.startswith("status "), (i, out)
    # A random corruption may still parse (a changed letter inside a string):
    # it only has to run clean under the sanitizers.
    for i, blob in enumerate(variants):
        path = tmp_path / f"corrupt_{i}.yuf"
        path.write_bytes(blob)
        run(driver, "ckpt", path, *names)


def test_sampler_host_code_is_clean(driver):
    for seed in (1, 2, 3):
        assert run(driver, "sampler", seed, 400) == "ok 400"
