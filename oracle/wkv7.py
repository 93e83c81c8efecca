"""WKV-7 TimeMix scan -- CPU restatement (test infrastructure only).

Reference: ``yufmusicgen/model.py:145-165`` (``RWKV7TimeMix._torch_recurrence``),
the semantics the fused kernel ``yufmusicgen/cuda/rwkv7_clampw.cu:20-75`` also
implements (decay form ``rwkv7_clampw.cu:16,42``).

Layout: every per-token tensor is ``[B, T, H, N]``; the state is
``[B, H, N, N]`` with axis -2 the value (row) index ``i`` and axis -1 the key
(column) index ``j`` -- the orientation the PyTorch stateful path carries
(``model.py:158-164``; ``cuda_ops.py:226-231`` transposes the CUDA kernel's
checkpoint back to it).
"""

from __future__ import annotations

import torch

# exp(-0.5), the constant of model.py:156 and rwkv7_clampw.cu:16.
W_SCALE = 0.6065306597
# Reference chunk length (cuda_ops.py:18) and the padding value of
# cuda_ops.py:176-186: w_raw = -80 gives retention 1 exactly.
CHUNK_LENGTH = 16
PAD_W_RAW = -80.0


def retention(w_raw: torch.Tensor) -> torch.Tensor:
    """Per-channel decay exp(-e^{-0.5} * sigmoid(w_raw)) (model.py:156)."""
    return torch.exp(-W_SCALE * torch.sigmoid(w_raw))


def wkv7_scan(r, w_raw, k, v, a, b, state=None):
    """Sequential WKV-7 scan, op for op as ``model.py:155-165``.

    Per (batch, head) with S in R^{N x N}:
        sa = S a_t;  S <- S diag(d_t) + sa b_t^T + v_t k_t^T;  y_t = S r_t.
    Returns ``(y [B,T,H,N], final_state [B,H,N,N])``.  Computes in the dtype
    of ``r`` (use float64 for parity, float32 for the CPU baseline).
    """
    batch, steps, heads, size = r.shape
    if state is None:
        memory = torch.zeros(batch, heads, size, size, dtype=r.dtype)
    else:
        memory = state.to(r.dtype).clone()
    decay = retention(w_raw)
    outputs = []
    for t in range(steps):
        state_a = torch.einsum("bhj,bhij->bhi", a[:, t], memory)
        memory = (
            memory * decay[:, t].unsqueeze(-2)
            + state_a.unsqueeze(-1) * b[:, t].unsqueeze(-2)
            + v[:, t].unsqueeze(-1) * k[:, t].unsqueeze(-2)
        )
        outputs.append(torch.einsum("bhij,bhj->bhi", memory, r[:, t]))
    if steps == 0:
        return torch.zeros_like(r), memory
    return torch.stack(outputs, dim=1), memory


def pad_inputs(r, w_raw, k, v, a, b, multiple: int = CHUNK_LENGTH):
    """The reference's T-padding (``cuda_ops.py:160-186``): w_raw = -80 and
    r = k = v = a = b = 0, so padded steps keep the state unchanged."""
    length = r.shape[1]
    padded = ((length + multiple - 1) // multiple) * multiple
    extra = padded - length
    if extra == 0:
        return (r, w_raw, k, v, a, b), length
    shape = (r.shape[0], extra, r.shape[2], r.shape[3])
    zeros = torch.zeros(shape, dtype=r.dtype)
    pad_w = torch.full(shape, PAD_W_RAW, dtype=r.dtype)
    return (
        torch.cat((r, zeros), 1),
        torch.cat((w_raw, pad_w), 1),
        torch.cat((k, zeros), 1),
        torch.cat((v, zeros), 1),
        torch.cat((a, zeros), 1),
        torch.cat((b, zeros), 1),
    ), length


def wkv7_scan_chunked(r, w_raw, k, v, a, b, state=None, chunk: int = CHUNK_LENGTH):
    """Chunk-parallel form of the same scan (the algebra the HIP kernels may use).

    Inside a chunk, with cumulative log-decays L_t = sum_{u<=t} log d_u
    (per column j) and the rescaled vectors
        a~_t = a_t e^{L_{t-1}},  r~_t = r_t e^{L_t},  b~_t = b_t e^{-L_t},  k~_t = k_t e^{-L_t},
    the row-vectors sa_t solve a unit lower-triangular system
        SA = S0 A~^T + SA Lb^T + V Lk^T,  Lb[t,s] = a~_t.b~_s, Lk[t,s] = a~_t.k~_s (s < t)
    and then
        Y  = S0 R~^T + SA Mb^T + V Mk^T,  Mb[t,s] = r~_t.b~_s, Mk[t,s] = r~_t.k~_s (s <= t)
        S_C = S0 diag(e^{L_C}) + SA B^ + V K^,  B^_s = b_s e^{L_C - L_s}, K^_s = k_s e^{L_C - L_s}.
    It is an independent route to the sequential result, so agreement pins both.
    """
    batch, steps, heads, size = r.shape
    dtype = r.dtype
    memory = torch.zeros(batch, heads, size, size, dtype=dtype) if state is None else state.to(dtype).clone()
    log_decay = -W_SCALE * torch.sigmoid(w_raw)
    y = torch.zeros_like(r)
    for c0 in range(0, steps, chunk):
        c1 = min(steps, c0 + chunk)
        n = c1 - c0
        # [B,H,n,N] views of this chunk.
        rc, kc, vc, ac, bc = (x[:, c0:c1].permute(0, 2, 1, 3) for x in (r, k, v, a, b))
        lc = log_decay[:, c0:c1].permute(0, 2, 1, 3)
        cum = torch.cumsum(lc, dim=2)  # L_t, inclusive
        cum_prev = cum - lc  # L_{t-1}
        total = cum[:, :, -1:, :]  # L_C
        a_t = ac * torch.exp(cum_prev)
        r_t = rc * torch.exp(cum)
        b_t = bc * torch.exp(-cum)
        k_t = kc * torch.exp(-cum)
        strict = torch.tril(torch.ones(n, n, dtype=dtype), diagonal=-1)
        incl = torch.tril(torch.ones(n, n, dtype=dtype), diagonal=0)
        lb = (a_t @ b_t.transpose(-1, -2)) * strict
        lk = (a_t @ k_t.transpose(-1, -2)) * strict
        mb = (r_t @ b_t.transpose(-1, -2)) * incl
        mk = (r_t @ k_t.transpose(-1, -2)) * incl
        # Row-vector form: SA is [B,H,N(rows i),n]; SA (I - Lb^T) = S0 A~^T + V^T Lk^T.
        vt = vc.transpose(-1, -2)  # [B,H,N,n]
        rhs = memory @ a_t.transpose(-1, -2) + vt @ lk.transpose(-1, -2)
        eye = torch.eye(n, dtype=dtype)
        system = (eye - lb.transpose(-1, -2)).expand(batch, heads, n, n)
        sa = torch.linalg.solve_triangular(system, rhs, upper=True, left=False)
        out = memory @ r_t.transpose(-1, -2) + sa @ mb.transpose(-1, -2) + vt @ mk.transpose(-1, -2)
        y[:, c0:c1] = out.permute(0, 3, 1, 2)
        b_hat = bc * torch.exp(total - cum)
        k_hat = kc * torch.exp(total - cum)
        memory = memory * torch.exp(total) + sa @ b_hat + vt @ k_hat
    return y, memory
