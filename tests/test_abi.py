"""The C-ABI library loads (no GPU needed) and exports every declared entry point."""

import re
from pathlib import Path

from yufmusicgen_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "yuf_engine.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(yuf_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_are_bound():
    declared = declared_functions()
    assert len(declared) >= 25
    assert sorted(_lib.SIGNATURES) == declared


def test_library_exports_every_declared_symbol():
    assert _lib.missing_symbols() == []
    assert _lib.lib().yuf_version().decode().startswith("yufhip")


def test_errors_cross_the_abi_as_status_codes():
    lib = _lib.lib()
    # Unsupported head size: rejected before any GPU work.
    rc = lib.yuf_wkv7_scan_f32(1, 1, 1, 12, *([None] * 10))
    assert rc == -1 and "head size" in lib.yuf_last_error().decode()
    rc = lib.yuf_rosa_scan_f32(1, 1, 2048, *([None] * 9))
    assert rc == -1 and "D must be" in lib.yuf_last_error().decode()


def test_noalloc_rosa_rejects_scratch_beyond_its_static_buffer(monkeypatch):
    """Checked on the host before any HIP call: B = 64, T = 8192, D = 256 needs
    D * D + 2 * B * (T / 64) * D = 65536 + 2 * 64 * 128 * 256 floats, past the
    4,194,304 of the buffer -- also with the operator's sequential switch set,
    which the no-allocation entry point does not read."""
    monkeypatch.setenv("YUF_ROSA_SEGMENTED", "0")
    lib = _lib.lib()
    dummy = 256  # never dereferenced: the call returns before any device work
    rc = lib.yuf_rosa_scan_f32_noalloc(64, 8192, 256, *([dummy] * 8), None)
    assert rc == -1 and "static buffer" in lib.yuf_last_error().decode()
