"""Seeded synthetic weights and inputs for the benchmark configurations.

No trained checkpoint ships with the reference, so every weight here is drawn
from numpy's PCG64 generator with a fixed draw order.  The deterministic
vectors follow the reference initialisation (``yufmusicgen/model.py:50-83``;
every layer gets the layer-0 token-shift ramps because ``YufBlock`` builds
``RWKV7TimeMix(config)`` without a layer id, ``model.py:349``).  Every matrix
-- Linear weights, embedding, the low-rank w1/w2/a1/a2/g1/g2 pairs and the
Householder vector -- is N(0, std) (std 0.02 by default), and so are the
ROSA biases, so that no path is degenerate (the reference's own init leaves
w1/a1/g1 at zero).
"""

from __future__ import annotations

import numpy as np

from .config import ModelConfig

TEXT_OFFSET = 4  # tokenizer.py:14
MIDI_OFFSET = 260  # tokenizer.py:16


def tensor_specs(cfg: ModelConfig) -> list:
    """(name, shape) in the ``.yuf`` export order.

    ``vulkan/scripts/export_checkpoint.py:77-88`` sorts the state_dict by
    (embedding, layer, final norm) and keeps the module registration order
    inside a layer (``model.py:42-76, 204-214, 345-356``); the six ``mix_*``
    vectors end up contiguous, which the Vulkan engine relies on.
    """
    d, lr, dr, hid = cfg.d_model, cfg.low_rank, cfg.rosa_size, cfg.ffn_hidden
    specs = [("token_embedding.weight", (cfg.vocab_size, d))]
    for layer in range(cfg.n_layers):
        p = f"blocks.{layer}."
        specs += [
            (p + "norm_time.weight", (d,)), (p + "norm_time.bias", (d,)),
            (p + "time_mix.mix_r", (d,)), (p + "time_mix.mix_w", (d,)), (p + "time_mix.mix_k", (d,)),
            (p + "time_mix.mix_v", (d,)), (p + "time_mix.mix_a", (d,)), (p + "time_mix.mix_g", (d,)),
            (p + "time_mix.w0", (d,)), (p + "time_mix.w1", (d, lr)), (p + "time_mix.w2", (lr, d)),
            (p + "time_mix.a0", (d,)), (p + "time_mix.a1", (d, lr)), (p + "time_mix.a2", (lr, d)),
            (p + "time_mix.g1", (d, lr)), (p + "time_mix.g2", (lr, d)),
            (p + "time_mix.k_k", (d,)), (p + "time_mix.k_a", (d,)),
            (p + "time_mix.receptance.weight", (d, d)), (p + "time_mix.key.weight", (d, d)),
            (p + "time_mix.value.weight", (d, d)), (p + "time_mix.output.weight", (d, d)),
            (p + "time_mix.out_norm.weight", (d,)), (p + "time_mix.out_norm.bias", (d,)),
            (p + "norm_rosa.weight", (d,)), (p + "norm_rosa.bias", (d,)),
            (p + "rosa.householder", (dr,)), (p + "rosa.decay", (dr,)),
            (p + "rosa.input.weight", (dr, d)), (p + "rosa.input.bias", (dr,)),
            (p + "rosa.write_gate.weight", (dr, d)), (p + "rosa.write_gate.bias", (dr,)),
            (p + "rosa.read_gate.weight", (dr, d)), (p + "rosa.read_gate.bias", (dr,)),
            (p + "rosa.output.weight", (d, dr)),
            (p + "norm_ffn.weight", (d,)), (p + "norm_ffn.bias", (d,)),
            (p + "ffn_in.weight", (hid, d)), (p + "ffn_gate.weight", (hid, d)), (p + "ffn_out.weight", (d, hid)),
        ]
    specs += [("final_norm.weight", (d,)), ("final_norm.bias", (d,))]
    return specs


_MIX_EXPONENTS = {"mix_r": 0.2, "mix_w": 0.9, "mix_k": 0.7, "mix_v": 0.7, "mix_a": 0.9, "mix_g": 0.2}


def _fixed_value(name: str, shape: tuple):
    """Reference init of the non-matrix parameters, or None for random ones.

    model.py:50-57 (mix ramps, ratio 1), :59 w0, :62 a0, :71-72 k_k/k_a,
    :213 ROSA decay, nn.LayerNorm (1, 0).
    """
    leaf = name.split(".")[-1]
    owner = name.split(".")[-2] if "." in name else ""
    if "norm" in owner and leaf == "weight":
        return np.ones(shape, np.float32)
    if "norm" in owner and leaf == "bias":
        return np.zeros(shape, np.float32)
    if name.endswith("rosa.decay"):
        return np.full(shape, 2.0, np.float32)
    d = shape[0]
    if leaf in _MIX_EXPONENTS:
        ramp = np.linspace(0.0, 1.0, d, dtype=np.float64)
        return (1.0 - ramp ** _MIX_EXPONENTS[leaf]).astype(np.float32)
    if leaf == "w0":
        return np.linspace(-5.5, 0.0, d, dtype=np.float64).astype(np.float32)
    constants = {"a0": -0.19, "k_k": 0.71, "k_a": 1.02}
    if leaf in constants:
        return np.full(shape, constants[leaf], np.float32)
    return None


def synth_weights(cfg: ModelConfig, seed: int = 0, std: float = 0.02) -> dict:
    """All tensors of ``tensor_specs`` as float32 arrays, random ones drawn in that order."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in tensor_specs(cfg):
        fixed = _fixed_value(name, shape)
        if fixed is None:
            fixed = rng.standard_normal(shape, dtype=np.float32) * np.float32(std)
        out[name] = np.ascontiguousarray(fixed, dtype=np.float32)
    return out


def wkv_inputs(seed: int, batch: int, steps: int, heads: int, size: int):
    """C2 isolated-scan inputs, draw order r, k, v, kappa, z, x (all float32).

    a = -kappa, b = kappa * sigmoid(z) with kappa L2-normalised per head, and
    w_raw chosen so that the reference decay exp(-e^{-0.5} sigmoid(w_raw))
    equals exp(-exp(x_c)) with x ~ N(-0.5, 1) clamped to x_c <= -0.5 - 1e-6
    (the clamp ``rwkv7_clampw`` is named for).
    """
    rng = np.random.default_rng(seed)
    shape = (batch, steps, heads, size)
    r = rng.standard_normal(shape, dtype=np.float32)
    k = rng.standard_normal(shape, dtype=np.float32)
    v = rng.standard_normal(shape, dtype=np.float32)
    kappa = rng.standard_normal(shape, dtype=np.float32)
    kappa /= np.maximum(np.linalg.norm(kappa, axis=-1, keepdims=True), 1e-12)
    z = rng.standard_normal(shape, dtype=np.float32)
    x = rng.standard_normal(shape, dtype=np.float32).astype(np.float64) - 0.5
    x_c = np.minimum(x, -0.5 - 1e-6)
    w_raw = (-np.log(np.expm1(-0.5 - x_c))).astype(np.float32)
    a = -kappa
    b = (kappa * (1.0 / (1.0 + np.exp(-z.astype(np.float64))))).astype(np.float32)
    return r, w_raw, k, v, a.astype(np.float32), b


def rosa_inputs(seed: int, batch: int, steps: int, dim: int):
    """ROSA scan inputs: pre-activations N(0,1), lambda = sigmoid(N(2,0.5)), unit u."""
    rng = np.random.default_rng(seed)
    shape = (batch, steps, dim)
    cand = rng.standard_normal(shape, dtype=np.float32)
    write = rng.standard_normal(shape, dtype=np.float32)
    read_raw = rng.standard_normal(shape, dtype=np.float32)
    decay = (1.0 / (1.0 + np.exp(-(2.0 + 0.5 * rng.standard_normal(dim))))).astype(np.float32)
    u = rng.standard_normal(dim)
    u = (u / np.linalg.norm(u)).astype(np.float32)
    return cand, write, read_raw, decay, u


def prompt_tokens(seed: int, batch: int, steps: int, vocab: int, caption: int = 64) -> np.ndarray:
    """C3 ids: the first ``caption`` of each row are caption bytes mapped to
    TEXT_OFFSET + byte (tokenizer.py:50-51), the rest uniform on [0, vocab)."""
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, vocab, size=(batch, steps), dtype=np.int64)
    n = min(caption, steps)
    ids[:, :n] = TEXT_OFFSET + rng.integers(0, 256, size=(batch, n), dtype=np.int64)
    return ids.astype(np.int32)


def uniform_tokens(seed: int, batch: int, steps: int, vocab: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.integers(0, vocab, size=(batch, steps), dtype=np.int64).astype(np.int32)
