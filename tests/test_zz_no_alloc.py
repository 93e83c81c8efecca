"""The no-allocation ROSA operator (yuf_rosa_scan_f32_noalloc) against the
allocating one (yuf_rosa_scan_f32) through the C ABI: the same kernels on the
same inputs, so the reads and final memories must be identical, on two calls
in a row (the second smaller, reusing the static scratch) and on a shape that
takes the sequential path (no scratch)."""

import numpy as np
import pytest
import torch

from yufmusicgen_amd._lib import check, lib
from yufmusicgen_amd.synth import rosa_inputs

pytestmark = pytest.mark.gpu


def _run(fn, B, T, D, seed):
    cand, write, read_raw, decay, u = [torch.from_numpy(x).cuda() for x in rosa_inputs(seed, B, T, D)]
    g = torch.Generator().manual_seed(seed)
    mem = (torch.randn(B, D, generator=g) * 0.3).cuda()
    out = torch.full((B, T, D), float("nan"), device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    check(fn(B, T, D, cand.data_ptr(), write.data_ptr(), read_raw.data_ptr(), decay.data_ptr(), u.data_ptr(),
             mem.data_ptr(), mem.data_ptr(), out.data_ptr(), st))
    torch.cuda.synchronize()
    return out.cpu().numpy(), mem.cpu().numpy()


@pytest.mark.parametrize("shapes", [[(8, 2048, 128), (3, 640, 64)], [(2, 256, 256), (1, 128, 256)]])
def test_noalloc_matches_allocating_operator(shapes):
    for i, (B, T, D) in enumerate(shapes):
        print(f"rosa noalloc call {i}: B={B} T={T} D={D}", flush=True)
        ref = _run(lib().yuf_rosa_scan_f32, B, T, D, seed=10 + i)
        got = _run(lib().yuf_rosa_scan_f32_noalloc, B, T, D, seed=10 + i)
        assert np.isfinite(got[0]).all()
        np.testing.assert_array_equal(got[0], ref[0])
        np.testing.assert_array_equal(got[1], ref[1])


def test_noalloc_sequential_shape_and_rejection(monkeypatch):
    # The capacity check must hold whatever the operator's env switch says.
    monkeypatch.setenv("YUF_ROSA_SEGMENTED", "0")
    ref = _run(lib().yuf_rosa_scan_f32, 2, 100, 96, seed=3)  # T % 64 != 0: the sequential scan
    got = _run(lib().yuf_rosa_scan_f32_noalloc, 2, 100, 96, seed=3)
    np.testing.assert_array_equal(got[0], ref[0])
    np.testing.assert_array_equal(got[1], ref[1])
    x = torch.zeros(8, device="cuda")
    # Rejected on the host before any launch: the buffers are never touched,
    # and the stream is the default one (None), never a data pointer.
    rc = lib().yuf_rosa_scan_f32_noalloc(64, 8192, 256, *([x.data_ptr()] * 8), None)
    assert rc == -1 and "static buffer" in lib().yuf_last_error().decode()
