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
                                   (64, 5120, 640), (37, 100, 36), (64, 640, 2560), (1, 20480, 640), (16, 64, 64),
                                   # wide decode products (A held in registers across >= 512 slices): the
                                   # LM head shape, row tails, a column tail, short K
                                   (64, 20480, 640), (33, 20480, 640), (40, 8200, 36), (48, 10000, 100)])
def test_linear_matches_float64(m, n, k):
    print(f"linear {m}x{n}x{k}", flush=True)
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    got = run_linear(a, w)
    expect = a.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(got, expect, rtol=1e-4, atol=1e-4 * np.sqrt(k) * 0.05)


@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("m,n", [(150, 70), (384, 320), (260, 512), (300, 384), (257, 64), (48, 70), (64, 640),
                                 (48, 8200)])
def test_linear_epilogues(act, m, n):
    rng = np.random.default_rng(act)
    a = rng.standard_normal((m, 96)).astype(np.float32)
    w = (rng.standard_normal((n, 96)) * 0.1).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    z = a.astype(np.float64) @ w.astype(np.float64).T + bias
    z = {0: z, 1: np.tanh(z), 2: 1.0 / (1.0 + np.exp(-z))}[act] + res
    np.testing.assert_allclose(run_linear(a, w, bias, act, res), z, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("m,n,k,gated", [(64, 640, 640, False), (64, 640, 640, True), (37, 384, 640, False),
                                         (5, 100, 36, True), (64, 1280, 1024, False), (64, 640, 1024, True),
                                         (64, 9000, 640, False), (20, 48, 1024, True), (33, 20480, 640, False),
                                         (20, 9000, 640, False)])
def test_ln_linear_matches_float64(m, n, k, gated):
    """LayerNorm (-> gate) -> Linear in one decode kernel.  K = 1024 with a gate,
    and the 9000-wide product at 20 rows (64-row tiles), take the statistics
    pass that re-reads the rows; the 9000- and 20480-wide products at 33-64
    rows run the wide kernel (LayerNorm applied once to the A rows held in
    registers); the others reuse the A values already loaded."""
    print(f"ln_linear {m}x{n}x{k} gate={gated}", flush=True)
    rng = np.random.default_rng(m * 7 + n + k)
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
    expect = xn @ w.astype(np.float64).T + bias + res
    dev = {name: torch.from_numpy(x).cuda() for name, x in
           dict(a=a, gamma=gamma, beta=beta, w=w, bias=bias, res=res).items()}
    G = torch.from_numpy(gate).cuda() if gated else None
    C = torch.empty(m, n, device="cuda")
    check(lib().yuf_ln_linear_f32(m, n, k, dev["a"].data_ptr(), dev["gamma"].data_ptr(), dev["beta"].data_ptr(),
                                  None if G is None else G.data_ptr(), dev["w"].data_ptr(), dev["bias"].data_ptr(),
                                  dev["res"].data_ptr(), C.data_ptr(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    np.testing.assert_allclose(C.cpu().numpy(), expect, rtol=1e-4, atol=2e-4 * np.sqrt(k) * 0.05)


def test_ln_linear_rejects_long_batches():
    from yufmusicgen_amd._lib import YufError
    A = torch.zeros(65, 64, device="cuda")
    with pytest.raises(YufError):
        check(lib().yuf_ln_linear_f32(65, 8, 64, A.data_ptr(), A.data_ptr(), A.data_ptr(), None, A.data_ptr(), None,
                                      None, A.data_ptr(), None))


@pytest.mark.parametrize("m,n,k", [(16384, 5120, 640), (2048, 640, 2560), (512, 20480, 640), (300, 384, 64),
                                   (1000, 160, 128), (256, 256, 32)])
def test_large_tile_products_hold_fp32_accuracy(m, n, k):
    """The large-tile path (M >= 256, K % 32 == 0) runs fp32 products as six bf16
    MFMAs over three-part splits of both operands.  Element by element its error
    against float64 must stay within what fp32 arithmetic itself allows: the
    split and the dropped parts (<= 3 * 2^-24 of |a| |w| per term) plus the
    fp32 accumulation of K terms (K * 2^-24 of sum |a| |w|, a worst-case
    bound), i.e. <= (K + 3) 2^-24 (|A| |W|^T); a single bf16 rounding of either
    operand (2^-9 relative) would break it by orders of magnitude."""
    print(f"x3 linear {m}x{n}x{k}", flush=True)
    rng = np.random.default_rng(m * 3 + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    got = run_linear(a, w)
    a64, w64 = a.astype(np.float64), w.astype(np.float64)
    expect = a64 @ w64.T
    mag = np.abs(a64) @ np.abs(w64).T
    err = np.abs(got - expect)
    assert np.all(err <= (k + 3) * 2.0 ** -24 * mag), float((err / mag).max())
    # Typical error stays at fp32's level (relative to the magnitude sum).
    assert float(np.median(err / mag)) < 4 * 2.0 ** -24


@pytest.mark.parametrize("m,n,k,extras", [
    (256, 5120, 640, "none"), (300, 5120, 640, "bias_tanh"), (4096, 5120, 640, "none"),   # 256-wide tiles
    (1000, 640, 2560, "residual"), (2048, 640, 640, "bias_sigmoid"),                      # 160-wide tiles
    (700, 384, 640, "alias"), (512, 128, 64, "none"),                                     # 128-wide tiles
    (300, 192, 640, "bias"), (257, 64, 32, "none"),                                       # 64-wide tiles
    (1000, 640, 64, "bias"), (700, 640, 128, "residual"),                                 # 64-row tiles (K <= 128)
    (512, 512, 96, "bias_tanh"), (300, 256, 128, "alias"),       # K <= 128 at 256 wide: 256-row tiles
    (1000, 48, 64, "none"),   # no large-tile width fits: the planes are not used
    (64, 640, 640, "none"),   # decode path: the planes are not used
    (999, 640, 640, "offset"),   # A rows not 16-byte aligned: W is split by the kernel as before
])
def test_linear_with_weight_planes_is_bit_identical(m, n, k, extras):
    """The pre-split-plane X3 kernel (yuf_linear_f32_planes, W's three bf16
    parts prepared once by yuf_x3_split_planes and streamed into LDS with
    direct loads) against yuf_linear_f32, whose large-tile kernel splits W
    itself: the same splits and product order, so every output must be
    bit-identical, on every tile width, row tail, epilogue (bias, tanh /
    sigmoid, residual, residual aliasing C) and on the shapes where the planes
    are bypassed.  Also checks that the planes path is actually taken where it
    applies (the kernel trace is not visible here, so the check is that a
    corrupted plane buffer changes the result exactly there)."""
    print(f"linear planes {m}x{n}x{k} {extras}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(m * 7 + n + k)
    off = 1 if extras == "offset" else 0
    a_store = torch.randn(m * k + off, generator=g).cuda()
    a = a_store[off:].view(m, k)
    w = (torch.randn(n, k, generator=g) * 0.05).cuda()
    bias = (torch.randn(n, generator=g) * 0.1).cuda() if "bias" in extras else None
    act = 1 if "tanh" in extras else 2 if "sigmoid" in extras else 0
    res = torch.randn(m, n, generator=g).cuda() if extras in ("residual", "alias") else None
    st = torch.cuda.current_stream().cuda_stream
    elems = lib().yuf_x3_planes_elems(n, k)
    assert elems == n * k * 3
    planes = torch.empty(elems, dtype=torch.int16, device="cuda")
    check(lib().yuf_x3_split_planes(n, k, w.data_ptr(), planes.data_ptr(), st))

    def run(use_planes, wp=None):
        c = res.clone() if extras == "alias" else torch.full((m, n), float("nan"), device="cuda")
        r = c if extras == "alias" else res
        args = (a.data_ptr(), w.data_ptr())
        tail = (None if bias is None else bias.data_ptr(), act, None if r is None else r.data_ptr(), c.data_ptr(), st)
        if use_planes:
            check(lib().yuf_linear_f32_planes(m, n, k, *args, (planes if wp is None else wp).data_ptr(), *tail))
        else:
            check(lib().yuf_linear_f32(m, n, k, *args, *tail))
        torch.cuda.synchronize()
        return c

    ref, got = run(False), run(True)
    assert not torch.isnan(ref).any()
    assert torch.equal(ref, got), f"max diff {float((ref - got).abs().max())}"
    # Zeroed planes change the result exactly where the planes path runs.
    applies = m > 64 and n % 64 == 0 and k % 32 == 0 and extras != "offset"
    zeroed = run(True, torch.zeros_like(planes))
    assert torch.equal(zeroed, ref) != applies


def test_weight_planes_layout():
    """yuf_x3_split_planes against the layout written out on the host: part p
    of W[n, k] (x1 = bf16(w), x2 = bf16(w - x1), x3 = bf16(w - x1 - x2), each
    rounded to nearest even) at element ((n // 16 * (K // 32) + k // 32) * 3 +
    p) * 512 + (n % 16) * 32 + 8 * ((k % 32 // 8) ^ s(n % 16)) + k % 8, with
    s(r) = ((r >> 1) ^ (r >> 3)) & 3; and the parts sum back to w within
    2^-24 relative."""
    n, k = 48, 96
    g = torch.Generator(device="cpu").manual_seed(5)
    w = torch.randn(n, k, generator=g)
    planes = torch.empty(lib().yuf_x3_planes_elems(n, k), dtype=torch.int16, device="cuda")
    check(lib().yuf_x3_split_planes(n, k, w.cuda().data_ptr(), planes.data_ptr(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    got = planes.cpu().view(torch.bfloat16).float()
    x1 = w.to(torch.bfloat16).float()
    x2 = (w - x1).to(torch.bfloat16).float()
    x3 = (w - x1 - x2).to(torch.bfloat16).float()
    parts = [x1, x2, x3]
    want = torch.empty_like(got)
    for row in range(n):
        for col in range(k):
            r = row % 16
            s = ((r >> 1) ^ (r >> 3)) & 3
            for p in range(3):
                o = ((row // 16 * (k // 32) + col // 32) * 3 + p) * 512 + r * 32 + 8 * (((col % 32) // 8) ^ s) + col % 8
                want[o] = parts[p][row, col]
    assert torch.equal(got, want)
    err = (x1.double() + x2.double() + x3.double() - w.double()).abs()
    assert bool((err <= 2.0 ** -24 * w.double().abs()).all())
