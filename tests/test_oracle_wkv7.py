"""Pins for the CPU oracle's WKV-7 scan (oracle/wkv7.py).

Each check reaches the scan by a route other than the oracle's own loop:
reference golden vectors, the O(T^2) closed form, hand-expanded small cases,
the delta-rule write property, linearity, padding and the chunked algebra.
"""

import os

import numpy as np
import pytest
import torch

from oracle import wkv7

DT = torch.float64


def rand_inputs(seed, batch, steps, heads, size, state=True):
    g = torch.Generator().manual_seed(seed)
    shape = (batch, steps, heads, size)
    r, k, v = (torch.randn(shape, generator=g, dtype=DT) for _ in range(3))
    w = torch.randn(shape, generator=g, dtype=DT) * 2.0
    kappa = torch.nn.functional.normalize(torch.randn(shape, generator=g, dtype=DT), dim=-1)
    a = -kappa
    b = kappa * torch.sigmoid(torch.randn(shape, generator=g, dtype=DT))
    s0 = torch.randn(batch, heads, size, size, generator=g, dtype=DT) * 0.5 if state else None
    return r, w, k, v, a, b, s0


def test_matches_reference_golden(golden_dir):
    z = np.load(os.path.join(golden_dir, "wkv7_ref.npz"))
    args = [torch.from_numpy(z[n]).to(DT) for n in ("r", "w_raw", "k", "v", "a", "b")]
    y, s = wkv7.wkv7_scan(*args, torch.from_numpy(z["s0"]).to(DT))
    np.testing.assert_allclose(y.numpy(), z["y"], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(s.numpy(), z["s"], rtol=1e-4, atol=1e-5)


def test_closed_form_without_state_coupling():
    """a = b = 0: S_ij(t) = S0_ij prod_{u<=t} d_j(u) + sum_{s<=t} v_i(s) k_j(s) prod_{s<u<=t} d_j(u)."""
    r, w, k, v, _, _, s0 = rand_inputs(1, 2, 9, 2, 5)
    zero = torch.zeros_like(r)
    y, s = wkv7.wkv7_scan(r, w, k, v, zero, zero, s0)
    d = np.exp(-wkv7.W_SCALE / (1.0 + np.exp(-w.numpy())))
    rn, kn, vn, s0n = r.numpy(), k.numpy(), v.numpy(), s0.numpy()
    steps = r.shape[1]
    for t in range(steps):
        expect = s0n * np.prod(d[:, : t + 1], axis=1)[:, :, None, :]
        for src in range(t + 1):
            decay = np.prod(d[:, src + 1 : t + 1], axis=1)  # [B,H,N] over j
            expect = expect + vn[:, src, :, :, None] * (kn[:, src] * decay)[:, :, None, :]
        y_t = np.einsum("bhij,bhj->bhi", expect, rn[:, t])
        np.testing.assert_allclose(y[:, t].numpy(), y_t, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(s.numpy(), expect, rtol=1e-12, atol=1e-12)


def test_one_and_two_steps_by_hand():
    r, w, k, v, a, b, _ = rand_inputs(2, 1, 2, 1, 6, state=False)
    y, s = wkv7.wkv7_scan(r[:, :1], w[:, :1], k[:, :1], v[:, :1], a[:, :1], b[:, :1])
    v1, k1, r1 = v[0, 0, 0], k[0, 0, 0], r[0, 0, 0]
    np.testing.assert_allclose(s[0, 0].numpy(), torch.outer(v1, k1).numpy(), rtol=1e-14)
    np.testing.assert_allclose(y[0, 0, 0].numpy(), (v1 * torch.dot(k1, r1)).numpy(), rtol=1e-12)
    y, s = wkv7.wkv7_scan(r, w, k, v, a, b)
    v2, k2, r2, a2, b2 = v[0, 1, 0], k[0, 1, 0], r[0, 1, 0], a[0, 1, 0], b[0, 1, 0]
    d2 = torch.exp(-wkv7.W_SCALE * torch.sigmoid(w[0, 1, 0]))
    s2 = torch.outer(v1, k1 * d2) + torch.dot(k1, a2) * torch.outer(v1, b2) + torch.outer(v2, k2)
    np.testing.assert_allclose(s[0, 0].numpy(), s2.numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(y[0, 1, 0].numpy(), (s2 @ r2).numpy(), rtol=1e-12, atol=1e-14)


def test_delta_rule_write_property():
    """With unit decay, a = -kappa and b = k = kappa the update is
    S <- S (I - kappa kappa^T) + v kappa^T, so the new state maps kappa to v exactly."""
    r, _, _, v, a, _, s0 = rand_inputs(3, 2, 6, 2, 7)
    kappa = -a
    w = torch.full_like(r, wkv7.PAD_W_RAW)
    state = s0
    for t in range(r.shape[1]):
        sl = slice(t, t + 1)
        _, state = wkv7.wkv7_scan(r[:, sl], w[:, sl], kappa[:, sl], v[:, sl], a[:, sl], kappa[:, sl], state)
        mapped = torch.einsum("bhij,bhj->bhi", state, kappa[:, t])
        np.testing.assert_allclose(mapped.numpy(), v[:, t].numpy(), rtol=1e-12, atol=1e-12)


def test_linear_in_v_from_zero_state():
    r, w, k, v, a, b, _ = rand_inputs(4, 2, 11, 2, 5, state=False)
    v2 = torch.randn_like(v)
    y1, s1 = wkv7.wkv7_scan(r, w, k, v, a, b)
    y2, s2 = wkv7.wkv7_scan(r, w, k, v2, a, b)
    y3, s3 = wkv7.wkv7_scan(r, w, k, v - 3.0 * v2, a, b)
    np.testing.assert_allclose(y3.numpy(), (y1 - 3.0 * y2).numpy(), rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(s3.numpy(), (s1 - 3.0 * s2).numpy(), rtol=1e-10, atol=1e-10)


def test_reference_padding_preserves_state():
    r, w, k, v, a, b, s0 = rand_inputs(5, 2, 21, 2, 6)
    y, s = wkv7.wkv7_scan(r, w, k, v, a, b, s0)
    padded, length = wkv7.pad_inputs(r, w, k, v, a, b)
    assert padded[0].shape[1] == 32 and length == 21
    # The padded steps alone leave the state bit-identical.
    _, s_after = wkv7.wkv7_scan(*(x[:, length:] for x in padded), s)
    np.testing.assert_array_equal(s_after.numpy(), s.numpy())
    yp, sp = wkv7.wkv7_scan(*padded, s0)
    np.testing.assert_allclose(sp.numpy(), s.numpy(), rtol=1e-14, atol=1e-14)
    np.testing.assert_allclose(yp[:, :length].numpy(), y.numpy(), rtol=1e-14, atol=1e-14)


@pytest.mark.parametrize("steps", [1, 15, 16, 37])
def test_chunked_form_equals_sequential(steps):
    r, w, k, v, a, b, s0 = rand_inputs(6, 2, steps, 3, 8)
    y, s = wkv7.wkv7_scan(r, w, k, v, a, b, s0)
    yc, sc = wkv7.wkv7_scan_chunked(r, w, k, v, a, b, s0)
    np.testing.assert_allclose(yc.numpy(), y.numpy(), rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(sc.numpy(), s.numpy(), rtol=1e-9, atol=1e-10)


def test_float32_restatement_within_tolerance():
    """The fp32 restatement (the timed CPU baseline) stays within the stated
    1e-4 relative / 1e-5 absolute of the float64 oracle on C2-style inputs."""
    from yufmusicgen_amd.synth import wkv_inputs

    arrs = wkv_inputs(0, 2, 256, 4, 40)
    y64, s64 = wkv7.wkv7_scan(*(torch.from_numpy(x).to(DT) for x in arrs))
    y32, s32 = wkv7.wkv7_scan(*(torch.from_numpy(x) for x in arrs))
    np.testing.assert_allclose(y32.numpy(), y64.numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(s32.numpy(), s64.numpy(), rtol=1e-4, atol=1e-5)
