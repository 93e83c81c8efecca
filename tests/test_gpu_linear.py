"""GPU parity of the MFMA linear layer (yuf_linear_f32) against float64 torch on the CPU."""

import numpy as np
import pytest
import torch

from yufmusicgen_amd._lib import check, lib

pytestmark = pytest.mark.gpu


def run_linear(a, w, bias=None, act=0, residual=None):
    m, k = a.shape
    n = w.shape[0]
    A, W = torch.from_numpy(a).cuda(), torch.from_numpy(w).cuda()
    B = None if bias is None else torch.from_numpy(bias).cuda()
    R = None if residual is None else torch.from_numpy(residual).cuda()
    C = torch.empty(m, n, device="cuda")
    check(lib().yuf_linear_f32(m, n, k, A.data_ptr(), W.data_ptr(), None if B is None else B.data_ptr(), act,
                               None if R is None else R.data_ptr(), C.data_ptr(),
                               torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return C.cpu().numpy()


@pytest.mark.parametrize("m,n,k", [(1, 640, 640), (64, 640, 640), (300, 200, 12), (129, 130, 33),
                                   (16384, 64, 640), (256, 2560, 640), (77, 20480, 640), (200, 640, 2560),
                                   # 256-row tile path (N % 256 == 0 or N % 160 == 0, M >= 256), with
                                   # row tails and K tails
                                   (300, 640, 100), (512, 512, 36), (1000, 160, 640), (700, 1280, 64),
                                   (2048, 640, 2560), (640, 384, 640), (512, 64, 640), (300, 192, 100),
                                   # decode path (M <= 64): column tails, short K, long K
                                   (64, 5120, 640), (37, 100, 36), (64, 640, 2560), (1, 20480, 640), (16, 64, 64)])
def test_linear_matches_float64(m, n, k):
    print(f"linear {m}x{n}x{k}", flush=True)
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    got = run_linear(a, w)
    expect = a.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(got, expect, rtol=1e-4, atol=1e-4 * np.sqrt(k) * 0.05)


@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("m,n", [(150, 70), (384, 320), (260, 512), (300, 384), (257, 64), (48, 70), (64, 640)])
def test_linear_epilogues(act, m, n):
    rng = np.random.default_rng(act)
    a = rng.standard_normal((m, 96)).astype(np.float32)
    w = (rng.standard_normal((n, 96)) * 0.1).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    z = a.astype(np.float64) @ w.astype(np.float64).T + bias
    z = {0: z, 1: np.tanh(z), 2: 1.0 / (1.0 + np.exp(-z))}[act] + res
    np.testing.assert_allclose(run_linear(a, w, bias, act, res), z, rtol=1e-5, atol=1e-5)
