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
