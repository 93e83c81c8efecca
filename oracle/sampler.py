"""Token sampling -- CPU restatement (test infrastructure only).

Reference: ``yufmusicgen/cli/generate.py:45-56`` (``sample_token``) and the
generation-loop mask of ``cli/generate.py:139-148`` / ``vulkan/src/generation.rs:195-203``.
The reference has no top-k; this build defines ``top_k > 0`` as "keep the
``top_k`` largest scaled logits,
set the rest to -inf", applied before the unchanged top-p / multinomial steps.

Randomness is torch's own CPU generator (``torch.manual_seed``), the stream
the reference's Rust sampler (``vulkan/src/sampler.rs:1-17``) claims to
replicate; the build's C++ sampler is checked against this function.
"""

from __future__ import annotations

import torch

PAD, BOS, EOS, SEP = 0, 1, 2, 3  # tokenizer.py:10-13
TEXT_OFFSET = 4  # tokenizer.py:14
MIDI_OFFSET = 260  # tokenizer.py:16
MIN_MIDI_TOKENS_BEFORE_EOS = 16  # cli/generate.py, generation.rs


def sample_token(logits: torch.Tensor, temperature: float, top_p: float, top_k: int = 0) -> torch.Tensor:
    """cli/generate.py:45-56 (+ the build's top-k)."""
    if temperature <= 0:
        return torch.argmax(logits, dim=-1)
    logits = logits / temperature
    if top_k > 0 and top_k < logits.shape[-1]:
        keep = torch.topk(logits, top_k, dim=-1, sorted=False).indices
        masked = torch.full_like(logits, float("-inf"))
        masked.scatter_(-1, keep, logits.gather(-1, keep))
        logits = masked
    sorted_logits, sorted_indices = torch.sort(logits, descending=True, dim=-1)
    probabilities = torch.softmax(sorted_logits, dim=-1)
    cumulative = torch.cumsum(probabilities, dim=-1)
    remove = cumulative - probabilities > top_p
    sorted_logits = sorted_logits.masked_fill(remove, float("-inf"))
    return sorted_indices.gather(-1, torch.multinomial(torch.softmax(sorted_logits, -1), 1)).squeeze(-1)


def generation_mask(logits: torch.Tensor, index: int, blocked_raw_ids=()) -> torch.Tensor:
    """Only MIDI ids (>= 260) are selectable, plus EOS after 16 tokens
    (cli/generate.py:142-148)."""
    allowed = torch.full_like(logits, float("-inf"))
    allowed[..., MIDI_OFFSET:] = logits[..., MIDI_OFFSET:]
    for raw in blocked_raw_ids:
        allowed[..., MIDI_OFFSET + raw] = float("-inf")
    if index >= MIN_MIDI_TOKENS_BEFORE_EOS:
        allowed[..., EOS] = logits[..., EOS]
    return allowed
