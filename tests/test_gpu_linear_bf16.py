"""GPU parity of the bf16-weight linear layers (yuf_linear_bf16w, yuf_ln_linear_bf16w).

The reference rounds W to bf16 (torch's float32 -> bfloat16 cast, round to
nearest even) and multiplies the fp32 activations by it in float64.  The
kernels split each activation into two bf16 parts (hi + lo, within 2^-16 of
the fp32 value) whose products with a bf16 weight are exact in fp32, so they
differ from the reference by fp32 accumulation order plus at most
2^-16 (|A| x |bf16(W)|^T): the fp32 tolerances of test_gpu_linear apply with
that term added; an A operand rounded to a single bf16 (2^-8) would miss them
by an order of magnitude.
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


def split_bound(a, w) -> np.ndarray:
    """Largest error the hi + lo split of the activations can add to A x bf16(W):
    |a - hi - lo| <= 2^-16 |a| per element, so 2^-16 (|A| x |bf16(W)|^T)."""
    return 2.0 ** -16 * (np.abs(a).astype(np.float64) @ np.abs(bf16_round(w)).astype(np.float64).T)


def assert_split_close(got, expect, bound, rtol=1e-5, atol=1e-5):
    """fp32-accumulation tolerance plus the split's bound, element by element."""
    err = np.abs(got - expect)
    lim = bound + atol + rtol * np.abs(expect)
    assert np.all(err <= lim), (float(err.max()), float((err - lim).max()))


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
    expect = a.astype(np.float64) @ bf16_round(w).astype(np.float64).T
    assert_split_close(got, expect, split_bound(a, w), rtol=1e-4, atol=1e-4 * np.sqrt(k) * 0.05)
    # The weight rounding is visible (fp32 weights give a clearly different
    # result) and so would a single bf16 rounding of the activations be.
    exact = a.astype(np.float64) @ w.astype(np.float64).T
    one_part = bf16_round(a).astype(np.float64) @ bf16_round(w).astype(np.float64).T
    assert np.abs(exact - expect).max() > 10 * np.abs(got - expect).max()
    assert np.abs(one_part - expect).max() > 10 * np.abs(got - expect).max()


@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("m,n", [(300, 512), (48, 1024), (257, 640)])
def test_linear_bf16w_epilogues(act, m, n):
    rng = np.random.default_rng(act + m)
    a = rng.standard_normal((m, 256)).astype(np.float32)
    w = (rng.standard_normal((n, 256)) * 0.1).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    z = a.astype(np.float64) @ bf16_round(w).astype(np.float64).T + bias
    z = {0: z, 1: np.tanh(z), 2: 1.0 / (1.0 + np.exp(-z))}[act] + res
    # tanh and sigmoid have slope <= 1, so the split's bound carries through.
    assert_split_close(run_linear_bf16w(a, w, bias, act, res), z, split_bound(a, w))


@pytest.mark.parametrize("m,n,k,gated", [(64, 1024, 1024, False), (64, 1024, 1024, True), (37, 768, 256, False),
                                         (64, 64, 1024, True), (2, 8192, 1024, False), (64, 4096, 1024, False)])
def test_ln_linear_bf16w_matches_float64(m, n, k, gated):
    """LayerNorm (-> gate) -> bf16 Linear in one decode kernel, against the
    float64 LayerNorm times the bf16-rounded weights: the normalised rows keep
    fp32 precision through the hi + lo split, so the fp32 bound of
    test_gpu_linear's LayerNorm test applies."""
    print(f"ln_linear_bf16w {m}x{n}x{k} gate={gated}", flush=True)
    rng = np.random.default_rng(m * 7 + n + k + 1)
    a = (rng.standard_normal((m, k)) * 2.0 + 0.5).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(k)).astype(np.float32)
    gate = rng.uniform(0.0, 1.0, (m, k)).astype(np.float32) if gated else None
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    a64 = a.astype(np.float64)
    xn = (a64 - a64.mean(1, keepdims=True)) / np.sqrt(a64.var(1, keepdims=True) + 1e-5) * gamma + beta
    if gated:
        xn = xn * gate
    expect = xn @ bf16_round(w).astype(np.float64).T + bias + res
    dev = {name: torch.from_numpy(x).cuda() for name, x in
           dict(a=a, gamma=gamma, beta=beta, bias=bias, res=res).items()}
    W = bf16_device(w)
    G = torch.from_numpy(gate).cuda() if gated else None
    C = torch.empty(m, n, device="cuda")
    check(lib().yuf_ln_linear_bf16w(m, n, k, dev["a"].data_ptr(), dev["gamma"].data_ptr(), dev["beta"].data_ptr(),
                                    None if G is None else G.data_ptr(), W.data_ptr(), dev["bias"].data_ptr(),
                                    dev["res"].data_ptr(), C.data_ptr(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert_split_close(C.cpu().numpy(), expect, split_bound(xn, w), rtol=1e-4, atol=2e-4 * np.sqrt(k) * 0.05)


def test_bf16w_rejects_unaligned_k():
    A = torch.zeros(300, 36, device="cuda")
    W = torch.zeros(64, 36, dtype=torch.int16, device="cuda")
    with pytest.raises(YufError):
        check(lib().yuf_linear_bf16w(300, 64, 36, A.data_ptr(), W.data_ptr(), None, 0, None, A.data_ptr(), None))
    with pytest.raises(YufError):  # M > 64 with N neither % 64 nor % 160
        check(lib().yuf_linear_bf16w(300, 100, 64, A.data_ptr(), W.data_ptr(), None, 0, None, A.data_ptr(), None))
