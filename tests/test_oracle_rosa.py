"""Pins for the CPU oracle's ROSA scan (oracle/rosa.py)."""

import os

import numpy as np
import torch

from oracle import rosa

DT = torch.float64


def rand_inputs(seed, batch, steps, dim):
    g = torch.Generator().manual_seed(seed)
    cand, write, read_raw = (torch.randn(batch, steps, dim, generator=g, dtype=DT) for _ in range(3))
    decay = torch.sigmoid(torch.randn(dim, generator=g, dtype=DT) + 2.0)
    u = torch.nn.functional.normalize(torch.randn(dim, generator=g, dtype=DT), dim=0)
    m0 = torch.randn(batch, dim, generator=g, dtype=DT)
    return cand, write, read_raw, decay, u, m0


def test_matches_reference_golden(golden_dir):
    z = np.load(os.path.join(golden_dir, "rosa_ref.npz"))
    args = [torch.from_numpy(z[n]).to(DT) for n in ("cand", "write", "read_raw", "decay", "direction", "m0")]
    read, m = rosa.rosa_scan(*args, gated=True)
    np.testing.assert_allclose(read.numpy(), z["read"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(m.numpy(), z["m"], rtol=1e-5, atol=1e-6)


def test_householder_is_an_involution_and_isometry():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 33, generator=g, dtype=DT)
    u = torch.nn.functional.normalize(torch.randn(33, generator=g, dtype=DT), dim=0)
    hx = rosa.householder(x, u)
    np.testing.assert_allclose(rosa.householder(hx, u).numpy(), x.numpy(), rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(hx.norm(dim=-1).numpy(), x.norm(dim=-1).numpy(), rtol=1e-13)
    # H u = -u, and H fixes the orthogonal complement of u.
    np.testing.assert_allclose(rosa.householder(u, u).numpy(), (-u).numpy(), atol=1e-14)


def test_lti_unrolling_with_dense_matrix_powers():
    """m_t = A m_{t-1} + e_t with A = diag(lambda)(I - 2 u u^T) (time-invariant), so
    m_T = A^T m_0 + sum_s A^{T-1-s} e_s and read_t = (I - 2uu^T) m_t * sigmoid(rho_t)."""
    cand, write, read_raw, decay, u, m0 = rand_inputs(1, 2, 13, 9)
    read, m = rosa.rosa_scan(cand, write, read_raw, decay, u, m0)
    un, lam = u.numpy(), decay.numpy()
    house = np.eye(9) - 2.0 * np.outer(un, un)
    A = np.diag(lam) @ house
    e = (1.0 / (1.0 + np.exp(-write.numpy()))) * np.tanh(cand.numpy())
    gate = 1.0 / (1.0 + np.exp(-read_raw.numpy()))
    for bi in range(2):
        for t in range(13):
            mt = np.linalg.matrix_power(A, t + 1) @ m0.numpy()[bi]
            for s in range(t + 1):
                mt = mt + np.linalg.matrix_power(A, t - s) @ e[bi, s]
            np.testing.assert_allclose(read.numpy()[bi, t], (house @ mt) * gate[bi, t], rtol=1e-11, atol=1e-12)
        np.testing.assert_allclose(m.numpy()[bi], mt, rtol=1e-11, atol=1e-12)


def test_unit_decay_without_writes_alternates():
    cand, _, read_raw, _, u, m0 = rand_inputs(2, 3, 4, 10)
    write = torch.full_like(cand, -1e4)  # sigmoid -> 0, no write
    read, m = rosa.rosa_scan(cand, write, read_raw, torch.ones(10, dtype=DT), u, m0, gated=False)
    np.testing.assert_allclose(read[:, 0].numpy(), m0.numpy(), atol=1e-13)  # H(H m0)
    np.testing.assert_allclose(read[:, 1].numpy(), rosa.householder(m0, u).numpy(), atol=1e-13)
    np.testing.assert_allclose(m.numpy(), m0.numpy(), atol=1e-13)  # four reflections


def test_step_form_equals_scan_form():
    cand, write, read_raw, decay, u, m0 = rand_inputs(3, 2, 8, 16)
    read, m = rosa.rosa_scan(cand, write, read_raw, decay, u, m0)
    state, outs = m0, []
    for t in range(8):
        r_t, state = rosa.rosa_scan(cand[:, t:t + 1], write[:, t:t + 1], read_raw[:, t:t + 1], decay, u, state)
        outs.append(r_t)
    np.testing.assert_allclose(torch.cat(outs, 1).numpy(), read.numpy(), rtol=1e-14, atol=1e-14)
    np.testing.assert_allclose(state.numpy(), m.numpy(), rtol=1e-14, atol=1e-14)
