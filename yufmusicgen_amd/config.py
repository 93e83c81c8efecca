"""Model configuration: the shapes the engine needs.

Mirrors the inference-relevant part of the reference ``ModelConfig``
(``yufmusicgen/config.py:73-93``) and the Rust ``ModelConfig``
(``vulkan/src/checkpoint.rs:14-48``), with the low-rank width computed the
Python way (``model.py:59``: round-half-even).  The engine itself derives the
low-rank width from the ``w1`` tensor's shape, so a checkpoint is never
mis-read when the two roundings disagree (d_model = 1024: Python 64, Rust 96).
"""

from __future__ import annotations

from dataclasses import asdict, dataclass


@dataclass(frozen=True)
class ModelConfig:
    vocab_size: int = 673
    d_model: int = 640
    n_layers: int = 14
    n_heads: int = 16
    head_size: int = 40
    rosa_size: int = 128
    dropout: float = 0.0
    tie_embeddings: bool = True

    @property
    def low_rank(self) -> int:
        return max(32, int(round(2.5 * (self.d_model ** 0.5) / 32) * 32))

    @property
    def ffn_hidden(self) -> int:
        return 4 * self.d_model

    def validate(self) -> None:
        """``config.py:87-93`` plus ``checkpoint.rs:32-47``."""
        if self.d_model != self.n_heads * self.head_size:
            raise ValueError("d_model must equal n_heads * head_size")
        if self.d_model < 32 or self.n_layers < 1:
            raise ValueError("model is too small to be useful")
        if self.rosa_size < 1 or self.vocab_size < 1:
            raise ValueError("rosa_size and vocab_size must be positive")

    def state_floats_per_layer(self) -> int:
        """prev [d] + WKV state [H*N*N] + ROSA memory [D] (``model.py:29-38``)."""
        return self.d_model + self.n_heads * self.head_size ** 2 + self.rosa_size

    def to_dict(self) -> dict:
        return asdict(self)


# Named shapes used by the tests and the benchmark.
PRESETS = {
    # tests/test_model_state.py:9-20 of the reference.
    "state_test": ModelConfig(vocab_size=300, d_model=32, n_layers=2, n_heads=2, head_size=16, rosa_size=12),
    # C1: tiny plumbing model.
    "tiny": ModelConfig(vocab_size=512, d_model=128, n_layers=2, n_heads=4, head_size=32, rosa_size=32),
    # C3 / C4: the default ~0.1B model with a 20 480-token vocabulary.
    "0.1b": ModelConfig(vocab_size=20480, d_model=640, n_layers=14, n_heads=16, head_size=40, rosa_size=128),
    # C5: the wide model.
    "wide": ModelConfig(vocab_size=20480, d_model=1024, n_layers=24, n_heads=16, head_size=64, rosa_size=256),
}
