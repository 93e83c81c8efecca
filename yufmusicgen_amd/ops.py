"""Python mirror of the reference's operator interface for the recurrent scans.

``rwkv7_cuda`` (yufmusicgen/cuda_ops.py:256-266) and ``rosa_householder_scan``
(yufmusicgen/rosa_cuda.py:157-180) keep their names, argument meaning and
validation errors; they run the gfx950 kernels of ``libyufhip.so`` through the
C ABI on torch's current HIP stream.  Tensors are torch plumbing (device
memory and streams); there is no CPU fallback.
"""

from __future__ import annotations

import torch

from ._lib import check, lib

SUPPORTED_HEAD_SIZES = (8, 16, 32, 40, 48, 64, 128)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def rwkv7_scan(r, w, k, v, a, b, state=None):
    """WKV-7 forward scan; returns ``(y [B,T,H,N], final_state [B,H,N,N])``.

    ``state`` (optional, [B,H,N,N], row = value index) is the initial state;
    ``None`` starts from zero like the reference kernel.  Validation follows
    ``cuda_ops.py:200-209``.
    """
    tensors = (r, w, k, v, a, b)
    if r.ndim != 4:
        raise ValueError("RWKV-7 inputs must have shape [B, T, H, N]")
    if not all(x.is_cuda for x in tensors):
        raise ValueError("RWKV-7 inputs must be on the GPU")
    if not all(x.dtype == torch.float32 for x in tensors):
        raise TypeError("the gfx950 scan computes in float32")
    if not all(x.is_contiguous() for x in tensors):
        raise ValueError("RWKV-7 inputs must be contiguous")
    if len({tuple(x.shape) for x in tensors}) != 1:
        raise ValueError("RWKV-7 inputs must have identical shapes")
    batch, steps, heads, size = r.shape
    if size not in SUPPORTED_HEAD_SIZES:
        raise ValueError(f"head size {size} not supported (supported: {SUPPORTED_HEAD_SIZES})")
    if state is not None:
        if state.shape != (batch, heads, size, size) or state.dtype != torch.float32 or not state.is_cuda:
            raise ValueError("state must be a float32 GPU tensor of shape [B, H, N, N]")
        state = state.contiguous()
    y = torch.empty_like(r)
    final = torch.empty(batch, heads, size, size, device=r.device, dtype=torch.float32)
    check(lib().yuf_wkv7_scan_f32(batch, steps, heads, size, *(x.data_ptr() for x in tensors),
                                  _ptr(state), final.data_ptr(), y.data_ptr(), _stream()))
    return y, final


def rwkv7_cuda(r, w, k, v, a, b):
    """Drop-in for the reference ``rwkv7_cuda`` (zero initial state)."""
    return rwkv7_scan(r, w, k, v, a, b)


def rosa_householder_scan(cand, write, read_raw, decay, direction, memory, gated: bool = False):
    """ROSA scan; returns ``(read [B,T,D], final_memory [B,D])``.

    As the reference operator, ``read`` is H(m_t) and the caller applies the
    sigmoid read gate (model.py:311); ``gated=True`` fuses that gate in.
    ``decay`` is post-sigmoid, ``direction`` a unit vector.
    """
    if cand.ndim != 3:
        raise ValueError("ROSA per-step inputs must have shape [B, T, D]")
    if len({tuple(x.shape) for x in (cand, write, read_raw)}) != 1:
        raise ValueError("ROSA per-step inputs must have identical shapes")
    tensors = [x.float().contiguous() for x in (cand, write, read_raw, decay, direction, memory)]
    if not all(x.is_cuda for x in tensors):
        raise ValueError("ROSA inputs must be on the GPU")
    cand, write, read_raw, decay, direction, memory = tensors
    batch, steps, dim = cand.shape
    read = torch.empty_like(cand)
    final = torch.empty(batch, dim, device=cand.device, dtype=torch.float32)
    check(lib().yuf_rosa_scan_f32(batch, steps, dim, cand.data_ptr(), write.data_ptr(),
                                  read_raw.data_ptr() if gated else None, decay.data_ptr(),
                                  direction.data_ptr(), memory.data_ptr(), final.data_ptr(),
                                  read.data_ptr(), _stream()))
    return read, final
