"""ROSA Householder memory scan -- CPU restatement (test infrastructure only).

Reference: ``yufmusicgen/model.py:260-288`` (``ROSAMemory._reference_recurrence``)
and the read/gate placement of ``model.py:303-342``; the fused CUDA op
``yufmusicgen/cuda/rosa_householder.cu:30-101`` returns the *ungated* read
H(m_t) and ``model.py:311`` multiplies by sigmoid(read_gate) afterwards.

Shapes: per-step tensors ``[B, T, D]``; ``decay`` is the post-sigmoid
per-channel vector lambda ``[D]``; ``direction`` the unit Householder vector
u ``[D]``; memory ``[B, D]``.
"""

from __future__ import annotations

import torch
from torch.nn import functional as F


def householder(value: torch.Tensor, direction: torch.Tensor) -> torch.Tensor:
    """H(x) = x - 2 (x.u) u   (model.py:220-222, 282-285)."""
    return value - 2.0 * torch.sum(value * direction, dim=-1, keepdim=True) * direction


def rosa_params(decay_param: torch.Tensor, householder_param: torch.Tensor):
    """lambda = sigmoid(decay), u = normalize(householder)   (model.py:300-301)."""
    return torch.sigmoid(decay_param), F.normalize(householder_param, dim=0)


def rosa_scan(cand, write, read_raw, decay, direction, memory=None, gated: bool = True):
    """m_t = lambda * H(m_{t-1}) + sigmoid(write_t) * tanh(cand_t);
    read_t = H(m_t) [* sigmoid(read_raw_t) when ``gated``]   (model.py:281-287).

    Returns ``(read [B,T,D], final_memory [B,D])``.
    """
    batch, steps, dim = cand.shape
    m = torch.zeros(batch, dim, dtype=cand.dtype) if memory is None else memory.to(cand.dtype).clone()
    outputs = []
    for t in range(steps):
        rotated = householder(m, direction)
        m = decay * rotated + torch.sigmoid(write[:, t]) * torch.tanh(cand[:, t])
        read = householder(m, direction)
        if gated:
            read = read * torch.sigmoid(read_raw[:, t])
        outputs.append(read)
    if steps == 0:
        return torch.zeros_like(cand), m
    return torch.stack(outputs, dim=1), m
