"""GPU parity of the bf16-weight linear layers (yuf_linear_bf16w, yuf_ln_linear_bf16w).

The reference rounds A and W to bf16 (torch's float32 -> bfloat16 cast, round to
nearest even) and multiplies in float64.  A product of two bf16 values is exact
in fp32, so the kernels differ from it only by fp32 accumulation order and the
fp32 tolerances of test_gpu_linear apply unchanged; an A operand left in fp32
or rounded another way would miss them by an order of magnitude.
"""

import numpy as np
import pytest
import torch

from yufmusicgen_amd._lib import YufError, check, lib

pytestmark = pytest.mark.gpu


def bf16_round(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


def bf16_device(x: np.ndarray) -> torch.Tensor:
    """Raw bf16 bit patterns on the device (int16 storage)."""
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).cuda()


def run_linear_bf16w(a, w, bias=None, act=0, residual=None):
    m, k = a.shape
    n = w.shape[0]
    A, W = torch.from_numpy(a).cuda(), bf16_device(w)
    B = None if bias is None else torch.from_numpy(bias).cuda()
    R = None if residual is None else torch.from_numpy(residual).cuda()
    C = torch.empty(m, n, device="cuda")
    check(lib().yuf_linear_bf16w(m, n, k, A.data_ptr(), W.data_ptr(), None if B is None else B.data_ptr(), act,
                                 None if R is None else R.data_ptr(), C.data_ptr(),
                                 torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return C.cpu().numpy()


@pytest.mark.parametrize("m,n,k", [
    # decode kernel (M <= 64): 32-k steps, column tails, the 64-row tiles of wide products
    (1, 1024, 1024), (64, 1024, 1024), (37, 100, 64), (64, 1024, 4096), (16, 64, 1024), (64, 20480, 1024),
    (5, 768, 256), (64, 8192, 1024),
    # large-tile kernel (M > 64): BN = 256 / 160 / 128 / 64, row tails, short and long K
    (256, 1024, 1024), (300, 1024, 1024), (512, 768, 1024), (1000, 640, 1024), (700, 64, 1024),
    (300, 1024, 64), (65, 1024, 1024), (520, 384, 2048), (1024, 4096, 1024), (256, 1024, 4096)])
def test_linear_bf16w_matches_float64(m, n, k):
    print(f"linear_bf16w {m}x{n}x{k}", flush=True)
    rng = np.random.default_rng(m * 3 + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    got = run_linear_bf16w(a, w)
    expect = bf16_round(a).astype(np.float64) @ bf16_round(w).astype(np.float64).T
    np.testing.assert_allclose(got, expect, rtol=1e-4, atol=1e-4 * np.sqrt(k) * 0.05)
    # The bf16 rounding is visible: fp32 operands give a clearly different result.
    exact = a.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(exact - expect).max() > 10 * np.abs(got - expect).max()


@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("m,n", [(300, 512), (48, 1024), (257, 640)])
def test_linear_bf16w_epilogues(act, m, n):
    rng = np.random.default_rng(act + m)
    a = rng.standard_normal((m, 256)).astype(np.float32)
    w = (rng.standard_normal((n, 256)) * 0.1).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    z = bf16_round(a).astype(np.float64) @ bf16_round(w).astype(np.float64).T + bias
    z = {0: z, 1: np.tanh(z), 2: 1.0 / (1.0 + np.exp(-z))}[act] + res
    np.testing.assert_allclose(run_linear_bf16w(a, w, bias, act, res), z, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("m,n,k,gated", [(64, 1024, 1024, False), (64, 1024, 1024, True), (37, 768, 256, False),
                                         (64, 64, 1024, True), (2, 8192, 1024, False), (64, 4096, 1024, False)])
def test_ln_linear_bf16w_matches_float64(m, n, k, gated):
    """LayerNorm (-> gate) -> bf16 Linear in one decode kernel.  The reference
    normalises in float32 like the kernel, so an A element whose float32 value
    sits within an ulp of a bf16 rounding midpoint may round the other way:
    at most a few rows may exceed the tight bound, and none by more than such
    a flip can move them."""
    print(f"ln_linear_bf16w {m}x{n}x{k} gate={gated}", flush=True)
    rng = np.random.default_rng(m * 7 + n + k + 1)
    a = (rng.standard_normal((m, k)) * 2.0 + 0.5).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(k)).astype(np.float32)
    gate = rng.uniform(0.0, 1.0, (m, k)).astype(np.float32) if gated else None
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    mean = a.mean(1, keepdims=True, dtype=np.float32)
    var = ((a - mean) ** 2).mean(1, keepdims=True, dtype=np.float32)
    xn = ((a - mean) / np.sqrt(var + np.float32(1e-5)) * gamma + beta).astype(np.float32)
    if gated:
        xn = (xn * gate).astype(np.float32)
    expect = bf16_round(xn).astype(np.float64) @ bf16_round(w).astype(np.float64).T + bias + res
    dev = {name: torch.from_numpy(x).cuda() for name, x in
           dict(a=a, gamma=gamma, beta=beta, bias=bias, res=res).items()}
    W = bf16_device(w)
    G = torch.from_numpy(gate).cuda() if gated else None
    C = torch.empty(m, n, device="cuda")
    check(lib().yuf_ln_linear_bf16w(m, n, k, dev["a"].data_ptr(), dev["gamma"].data_ptr(), dev["beta"].data_ptr(),
                                    None if G is None else G.data_ptr(), W.data_ptr(), dev["bias"].data_ptr(),
                                    dev["res"].data_ptr(), C.data_ptr(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    err = np.abs(C.cpu().numpy() - expect)
    tight = 1e-4 * np.abs(expect) + 2e-4 * np.sqrt(k) * 0.05
    assert int((err > tight).any(axis=1).sum()) <= 2
    flip = 2.0 ** -8 * float(np.abs(xn).max()) * float(np.abs(w).max())
    assert float(err.max()) <= 2 * flip + 2e-4 * np.sqrt(k) * 0.05


def test_bf16w_rejects_unaligned_k():
    A = torch.zeros(300, 36, device="cuda")
    W = torch.zeros(64, 36, dtype=torch.int16, device="cuda")
    with pytest.raises(YufError):
        check(lib().yuf_linear_bf16w(300, 64, 36, A.data_ptr(), W.data_ptr(), None, 0, None, A.data_ptr(), None))
    with pytest.raises(YufError):  # M > 64 with N neither % 64 nor % 160
        check(lib().yuf_linear_bf16w(300, 100, 64, A.data_ptr(), W.data_ptr(), None, 0, None, A.data_ptr(), None))
