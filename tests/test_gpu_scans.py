"""GPU parity of the WKV-7 and ROSA scan kernels against the CPU oracle.

Tolerances: fp32 outputs and final states within
1e-4 relative / 1e-5 absolute of the float64 oracle.
"""

import os

import numpy as np
import pytest
import torch

from oracle import rosa as orosa
from oracle import wkv7 as owkv
from yufmusicgen_amd.synth import rosa_inputs, wkv_inputs

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-5


def _dev(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()


def _oracle_wkv(arrs, s0=None):
    t = [torch.from_numpy(np.asarray(x, dtype=np.float64)) for x in arrs]
    return owkv.wkv7_scan(*t, None if s0 is None else torch.from_numpy(np.asarray(s0, np.float64)))


KERNELS = ("serial", "chunked")


@pytest.mark.parametrize("wkv_kernel", KERNELS, indirect=True)
@pytest.mark.parametrize("size", [8, 16, 32, 40, 48, 64, 128])
@pytest.mark.parametrize("steps", [1, 16, 17, 50, 100])
def test_wkv7_matches_oracle(size, steps, wkv_kernel):
    from yufmusicgen_amd.ops import rwkv7_scan

    print(f"wkv7 parity N={size} T={steps} kernel={wkv_kernel}", flush=True)
    arrs = wkv_inputs(100 + size + steps, 2, steps, 3, size)
    s0 = np.random.default_rng(size).standard_normal((2, 3, size, size)).astype(np.float32) * 0.3
    y, s = rwkv7_scan(*(_dev(x) for x in arrs), state=_dev(s0))
    ye, se = _oracle_wkv(arrs, s0)
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy(), ye.numpy(), rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(s.cpu().numpy(), se.numpy(), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("wkv_kernel", ["chunked"], indirect=True)
@pytest.mark.parametrize("size", [8, 40])
def test_wkv7_many_heads_one_workgroup_each(size, wkv_kernel):
    """More than 128 heads (here 9 x 16 = 144) run one workgroup per head
    instead of two; with N = 40 (and N = 8) the last 16-key tile is half
    padding and takes the permuted half-tile form."""
    from yufmusicgen_amd.ops import rwkv7_scan

    print(f"wkv7 unsplit N={size}", flush=True)
    arrs = wkv_inputs(300 + size, 9, 37, 16, size)
    s0 = np.random.default_rng(size + 1).standard_normal((9, 16, size, size)).astype(np.float32) * 0.3
    y, s = rwkv7_scan(*(_dev(x) for x in arrs), state=_dev(s0))
    ye, se = _oracle_wkv(arrs, s0)
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy(), ye.numpy(), rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(s.cpu().numpy(), se.numpy(), rtol=RTOL, atol=ATOL)


def test_wkv7_reference_golden(golden_dir):
    from yufmusicgen_amd.ops import rwkv7_scan

    z = np.load(os.path.join(golden_dir, "wkv7_ref.npz"))
    y, s = rwkv7_scan(*(_dev(z[n]) for n in ("r", "w_raw", "k", "v", "a", "b")), state=_dev(z["s0"]))
    np.testing.assert_allclose(y.cpu().numpy(), z["y"], rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(s.cpu().numpy(), z["s"], rtol=RTOL, atol=ATOL)


def test_wkv7_zero_state_matches_reference_entry():
    """rwkv7_cuda (zero start) equals the stateful call with an explicit zero state."""
    from yufmusicgen_amd.ops import rwkv7_cuda, rwkv7_scan

    arrs = [_dev(x) for x in wkv_inputs(7, 2, 33, 2, 40)]
    y0, s0 = rwkv7_cuda(*arrs)
    y1, s1 = rwkv7_scan(*arrs, state=torch.zeros(2, 2, 40, 40, device="cuda"))
    assert torch.equal(y0, y1) and torch.equal(s0, s1)


@pytest.mark.parametrize("wkv_kernel", KERNELS, indirect=True)
def test_wkv7_c2_full_size_parity_and_linearity(wkv_kernel):
    """C2 at its full size (B=8, T=2048, H=16, N=40) against the float64 oracle,
    plus linearity in v (a size-independent property)."""
    from yufmusicgen_amd.ops import rwkv7_scan

    print(f"wkv7 C2 full size kernel={wkv_kernel}", flush=True)
    arrs = wkv_inputs(0, 8, 2048, 16, 40)
    dev = [_dev(x) for x in arrs]
    y, s = rwkv7_scan(*dev)
    ye, se = _oracle_wkv(arrs)
    np.testing.assert_allclose(y.cpu().numpy(), ye.numpy(), rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(s.cpu().numpy(), se.numpy(), rtol=RTOL, atol=ATOL)
    v2 = torch.randn_like(dev[3])
    y2, s2 = rwkv7_scan(dev[0], dev[1], dev[2], v2, dev[4], dev[5])
    y3, s3 = rwkv7_scan(dev[0], dev[1], dev[2], dev[3] + v2, dev[4], dev[5])
    torch.testing.assert_close(y3, y + y2, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(s3, s + s2, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("wkv_kernel", KERNELS, indirect=True)
def test_wkv7_chunked_continuation_equals_one_pass(wkv_kernel):
    """Splitting T across calls that carry the state (stateful prefill) equals one pass."""
    from yufmusicgen_amd.ops import rwkv7_scan

    dev = [_dev(x) for x in wkv_inputs(3, 2, 100, 4, 40)]
    y, s = rwkv7_scan(*dev)
    ya, sa = rwkv7_scan(*(x[:, :37].contiguous() for x in dev))
    yb, sb = rwkv7_scan(*(x[:, 37:].contiguous() for x in dev), state=sa)
    torch.testing.assert_close(torch.cat([ya, yb], 1), y, rtol=RTOL, atol=ATOL)
    torch.testing.assert_close(sb, s, rtol=RTOL, atol=ATOL)


def test_wkv7_delta_rule_write_property():
    """Unit decay, a = -kappa, b = k = kappa: after each token S kappa = v."""
    from yufmusicgen_amd.ops import rwkv7_scan

    r, _, _, v, a, _ = wkv_inputs(9, 2, 12, 2, 40)
    kappa = -a
    w = np.full_like(r, -80.0)
    state = None
    for t in range(12):
        sl = slice(t, t + 1)
        args = [_dev(x[:, sl]) for x in (r, w, kappa, v, a, kappa)]
        _, state = rwkv7_scan(*args, state=state)
        mapped = torch.einsum("bhij,bhj->bhi", state, _dev(kappa[:, t]))
        torch.testing.assert_close(mapped, _dev(v[:, t]), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dim", [12, 32, 128, 256, 512, 1000])
@pytest.mark.parametrize("steps", [1, 19, 64])
@pytest.mark.parametrize("gated", [False, True])
def test_rosa_matches_oracle(dim, steps, gated):
    from yufmusicgen_amd.ops import rosa_householder_scan

    print(f"rosa parity D={dim} T={steps} gated={gated}", flush=True)
    cand, write, read_raw, decay, u = rosa_inputs(dim + steps, 3, steps, dim)
    m0 = np.random.default_rng(dim).standard_normal((3, dim)).astype(np.float32)
    read, m = rosa_householder_scan(*(_dev(x) for x in (cand, write, read_raw, decay, u, m0)), gated=gated)
    t64 = [torch.from_numpy(x.astype(np.float64)) for x in (cand, write, read_raw, decay, u, m0)]
    re, me = orosa.rosa_scan(*t64, gated=gated)
    np.testing.assert_allclose(read.cpu().numpy(), re.numpy(), rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(m.cpu().numpy(), me.numpy(), rtol=RTOL, atol=ATOL)


def test_rosa_reference_golden(golden_dir):
    from yufmusicgen_amd.ops import rosa_householder_scan

    z = np.load(os.path.join(golden_dir, "rosa_ref.npz"))
    args = [_dev(z[n]) for n in ("cand", "write", "read_raw", "decay", "direction", "m0")]
    read, m = rosa_householder_scan(*args, gated=True)
    np.testing.assert_allclose(read.cpu().numpy(), z["read"], rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(m.cpu().numpy(), z["m"], rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("decay_value", [None, 0.99, 0.05])
def test_rosa_full_size(decay_value):
    """C3 shape (B=8, T=2048, D=128, gated), with the drawn decays and with
    every decay pinned at 0.99 (slow memory) and 0.05 (fast memory).  At 0.999
    even an exact-order float32 recurrence leaves elements outside 1e-4/1e-5."""
    from yufmusicgen_amd.ops import rosa_householder_scan

    print(f"rosa full size decay={decay_value}", flush=True)
    cand, write, read_raw, decay, u = rosa_inputs(11, 8, 2048, 128)
    if decay_value is not None:
        decay = np.full_like(decay, decay_value)
    m0 = np.random.default_rng(5).standard_normal((8, 128)).astype(np.float32)
    arrs = (cand, write, read_raw, decay, u, m0)
    read, m = rosa_householder_scan(*(_dev(x) for x in arrs), gated=True)
    re, me = orosa.rosa_scan(*(torch.from_numpy(x.astype(np.float64)) for x in arrs), gated=True)
    np.testing.assert_allclose(read.cpu().numpy(), re.numpy(), rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(m.cpu().numpy(), me.numpy(), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("dim,steps,gated", [(64, 128, True), (128, 640, False), (256, 256, True), (128, 2048, True)])
def test_rosa_segmented_operator(dim, steps, gated, monkeypatch):
    """The operator's segmented form (T a multiple of 64, T >= 128, D in {64,
    128, 256}: A^64 built on the device in double, segments from zero, the
    carry chain, segments from their starts) against the float64 oracle and
    against the sequential scan (YUF_ROSA_SEGMENTED=0), from a non-zero memory."""
    from yufmusicgen_amd.ops import rosa_householder_scan

    print(f"rosa segmented D={dim} T={steps} gated={gated}", flush=True)
    cand, write, read_raw, decay, u = rosa_inputs(12 + dim, 3, steps, dim)
    m0 = np.random.default_rng(6).standard_normal((3, dim)).astype(np.float32)
    arrs = (cand, write, read_raw, decay, u, m0)
    read, m = rosa_householder_scan(*(_dev(x) for x in arrs), gated=gated)
    re, me = orosa.rosa_scan(*(torch.from_numpy(x.astype(np.float64)) for x in arrs), gated=gated)
    np.testing.assert_allclose(read.cpu().numpy(), re.numpy(), rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(m.cpu().numpy(), me.numpy(), rtol=RTOL, atol=ATOL)
    monkeypatch.setenv("YUF_ROSA_SEGMENTED", "0")
    read_s, m_s = rosa_householder_scan(*(_dev(x) for x in arrs), gated=gated)
    np.testing.assert_allclose(read.cpu().numpy(), read_s.cpu().numpy(), rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(m.cpu().numpy(), m_s.cpu().numpy(), rtol=RTOL, atol=ATOL)


def test_rosa_chunked_continuation():
    """Scanning T tokens in ragged pieces, carrying the memory, equals one scan."""
    from yufmusicgen_amd.ops import rosa_householder_scan

    cand, write, read_raw, decay, u = rosa_inputs(4, 2, 100, 128)
    m = torch.zeros(2, 128, device="cuda")
    full, m_full = rosa_householder_scan(*(_dev(x) for x in (cand, write, read_raw, decay, u)), m, gated=True)
    outs = []
    for lo, hi in ((0, 7), (7, 40), (40, 41), (41, 100)):
        piece = [_dev(x[:, lo:hi]) for x in (cand, write, read_raw)]
        r, m = rosa_householder_scan(*piece, _dev(decay), _dev(u), m, gated=True)
        outs.append(r)
    torch.testing.assert_close(torch.cat(outs, dim=1), full, rtol=RTOL, atol=ATOL)
    torch.testing.assert_close(m, m_full, rtol=RTOL, atol=ATOL)
