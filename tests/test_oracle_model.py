"""Pins for the CPU oracle's full model (oracle/model.py)."""

import os

import numpy as np
import pytest
import torch

from oracle.model import OracleModel, blob_to_state, state_to_blob
from yufmusicgen_amd.checkpoint import config_from_header, read_yuf
from yufmusicgen_amd.config import PRESETS
from yufmusicgen_amd.synth import synth_weights


@pytest.fixture(scope="module")
def state_test(golden_dir):
    header, weights = read_yuf(os.path.join(golden_dir, "model_state_test.yuf"))
    cfg = config_from_header(header)
    return cfg, weights, np.load(os.path.join(golden_dir, "model_state_test.npz"))


def test_full_sequence_matches_reference(state_test):
    cfg, weights, z = state_test
    model = OracleModel(cfg.to_dict(), weights)
    logits, state = model.forward(z["tokens"])
    np.testing.assert_allclose(logits.numpy(), z["logits"], rtol=1e-4, atol=2e-5)
    for layer, st in enumerate(state):
        np.testing.assert_allclose(st.previous.numpy(), z[f"full.state.{layer}.previous"], rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(st.memory.numpy(), z[f"full.state.{layer}.memory"], rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(st.rosa.numpy(), z[f"full.state.{layer}.rosa"], rtol=1e-4, atol=1e-5)


def test_continuation_from_carried_state_matches_reference(state_test):
    cfg, weights, z = state_test
    model = OracleModel(cfg.to_dict(), weights)
    tokens = z["tokens"]
    head, state = model.forward(tokens[:, :5])
    # Round-trip the state through the engine's blob layout on the way.
    state = blob_to_state(state_to_blob(state).astype(np.float64), cfg.to_dict())
    tail, state = model.forward(tokens[:, 5:], state)
    np.testing.assert_allclose(head.numpy(), z["head_logits"], rtol=1e-4, atol=2e-5)
    np.testing.assert_allclose(tail.numpy(), z["tail_logits"], rtol=1e-4, atol=2e-5)
    for layer, st in enumerate(state):
        np.testing.assert_allclose(st.memory.numpy(), z[f"tail.state.{layer}.memory"], rtol=1e-4, atol=1e-5)


def test_step_loop_equals_full_forward(state_test):
    """The reference's own invariant, tests/test_model_state.py:9-28."""
    cfg, weights, z = state_test
    model = OracleModel(cfg.to_dict(), weights)
    tokens = z["tokens"]
    full, _ = model.forward(tokens)
    state, steps = None, []
    for t in range(tokens.shape[1]):
        logits, state = model.step(tokens[:, t], state)
        steps.append(logits)
    np.testing.assert_allclose(torch.stack(steps, 1).numpy(), full.numpy(), rtol=1e-10, atol=1e-10)


def test_tiny_model_prompt_and_greedy_match_reference(golden_dir):
    z = np.load(os.path.join(golden_dir, "model_tiny.npz"))
    cfg = PRESETS["tiny"]
    weights = synth_weights(cfg, seed=int(z["seed"]), std=float(z["std"]))
    checksum = np.array([float(np.sum(v.astype(np.float64))) for v in weights.values()])
    np.testing.assert_array_equal(checksum, z["weight_checksum"])  # generator unchanged
    model = OracleModel(cfg.to_dict(), weights)
    logits, state = model.forward(z["prompt"])
    np.testing.assert_allclose(logits.numpy(), z["prompt_logits"], rtol=1e-4, atol=1e-5)
    last = logits[:, -1]
    for i, expect in enumerate(z["greedy"]):
        top2 = torch.topk(last[0], 2).values
        if float(top2[0] - top2[1]) > 1e-3:
            assert int(torch.argmax(last[0])) == int(expect)
        token = torch.tensor([int(expect)])
        last, state = model.step(token, state)
        np.testing.assert_allclose(last.numpy()[0], z["greedy_logits"][i], rtol=1e-4, atol=1e-5)


def _bf16_rne_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 from the bit patterns (the
    IEEE rule, written independently of torch), returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def test_bf16_rounding_of_the_bf16_oracle():
    """The bf16 configuration's rounding (torch's float32 -> bfloat16 cast) is
    round-to-nearest-even: checked against the bit-level rule on random values,
    exact ties (both directions) and values just off a tie."""
    from oracle.model import _bf16
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0,
                        # ties: low 16 bits exactly 0x8000, even and odd upper halves
                        np.array([0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000], dtype=np.uint32).view(np.float32),
                        # one ulp either side of a tie
                        np.array([0x3F808001, 0x3F807FFF], dtype=np.uint32).view(np.float32)])
    got = _bf16(torch.from_numpy(x.astype(np.float64))).numpy().astype(np.float32)
    np.testing.assert_array_equal(got, _bf16_rne_bits(x))
    ties = np.array([0x3F808000, 0x3F818000], dtype=np.uint32).view(np.float32)
    np.testing.assert_array_equal(_bf16(torch.from_numpy(ties.astype(np.float64))).numpy().astype(np.float32).view(np.uint32),
                                  np.array([0x3F800000, 0x3F820000], dtype=np.uint32))


def test_bf16_oracle_rounds_projection_operands_only():
    """bf16_linear rounds the nn.Linear weights and the LM head, never the
    embedding gather, the norms, the recurrence parameters or the biases, and
    then computes exactly as the fp32 model does on those weights."""
    cfg = PRESETS["tiny"]
    weights = synth_weights(cfg, seed=3)
    model = OracleModel(cfg.to_dict(), weights, bf16_linear=True)
    plain = OracleModel(cfg.to_dict(), weights)
    for name, value in model.w.items():
        same = torch.equal(value, plain.w[name])
        rounded = name == "lm_head.weight" or any(name.endswith(s) for s in
                                                  ("receptance.weight", "key.weight", "value.weight",
                                                   "output.weight", "w1", "w2", "a1", "a2", "g1", "g2",
                                                   "input.weight", "write_gate.weight", "read_gate.weight",
                                                   "ffn_in.weight", "ffn_gate.weight", "ffn_out.weight"))
        if rounded:
            np.testing.assert_array_equal(value.numpy().astype(np.float32),
                                          _bf16_rne_bits(plain.w[name].numpy().astype(np.float32)))
        else:
            assert same, name
    # The two configurations differ, by a bf16-sized amount.
    ids = np.array([[1, 5, 9, 200]])
    a, _ = model.forward(ids)
    b, _ = plain.forward(ids)
    rel = float((a - b).abs().max() / b.abs().max())
    assert 1e-4 < rel < 5e-2, rel
    # Activations are not rounded: the plain model run on the rounded weights
    # is the same program.
    rounded = OracleModel(cfg.to_dict(), {n: v.numpy() for n, v in model.w.items()})  # incl. the rounded head
    c, _ = rounded.forward(ids)
    assert torch.equal(a, c)


def test_split16_is_the_two_part_bf16_split():
    """split16(x) = hi + lo with hi = bf16(x), lo = bf16(x - hi): within 2^-16
    relative of x, both parts exact bf16 values, and x itself when x is a
    bf16 value (lo = 0)."""
    import torch

    from oracle.model import split16

    g = torch.Generator().manual_seed(3)
    x = (torch.randn(20000, generator=g, dtype=torch.float64) * torch.exp(torch.randn(20000, generator=g))).to(torch.float32).double()
    s = split16(x)
    assert torch.all((s - x).abs() <= 2.0 ** -16 * x.abs())
    hi = x.float().bfloat16().double()
    lo = s - hi
    assert torch.equal(lo, lo.float().bfloat16().double())
    assert torch.equal(split16(hi), hi)
    # A plain bf16 rounding (one part) misses the same bound.
    assert torch.any((hi - x).abs() > 2.0 ** -16 * x.abs())
