"""The host sampler against torch's own generator and multinomial (CPU only).

torch.manual_seed's MT19937 stream is the third-party behaviour the reference's
Rust sampler (vulkan/src/sampler.rs:1-17) claims to reproduce; here the C++
sampler is checked against torch directly.
"""

import numpy as np
import pytest
import torch

from oracle.sampler import generation_mask, sample_token as torch_sample
from yufmusicgen_amd.engine import Mt19937, argmax, sample_token


def test_uniform_stream_matches_torch_double_rand():
    for seed in (0, 1, 1337, 2**32 + 5):
        torch.manual_seed(seed)
        expect = torch.rand(2000, dtype=torch.float64).numpy()
        rng = Mt19937(seed)
        got = np.array([rng.next_uniform() for _ in range(2000)])
        np.testing.assert_array_equal(got, expect)


def test_argmax_is_first_maximum():
    x = np.array([1.0, 3.0, 3.0, -1.0], np.float32)
    assert argmax(x) == 1 == int(torch.argmax(torch.from_numpy(x)))


@pytest.mark.parametrize("vocab,temperature,top_p,top_k", [
    (512, 1.0, 0.95, 0), (512, 0.7, 1.0, 0), (20480, 0.9, 0.95, 0), (20480, 1.0, 1.0, 32),
    (673, 1.3, 0.5, 0), (300, 0.8, 0.9, 10),
])
def test_sample_token_matches_torch(vocab, temperature, top_p, top_k):
    rng_np = np.random.default_rng(vocab + top_k)
    agree = 0
    trials = 40
    for trial in range(trials):
        logits = (rng_np.standard_normal(vocab) * 3.0).astype(np.float32)
        seed = 1000 + trial
        torch.manual_seed(seed)
        expect = int(torch_sample(torch.from_numpy(logits), temperature, top_p, top_k))
        got = sample_token(logits, temperature, top_p, Mt19937(seed), top_k=top_k)
        agree += got == expect
    assert agree == trials


def test_sequence_of_draws_shares_one_stream():
    """Consecutive samples consume the generator like successive torch calls."""
    rng_np = np.random.default_rng(0)
    logits = [rng_np.standard_normal(400).astype(np.float32) for _ in range(6)]
    torch.manual_seed(77)
    expect = [int(torch_sample(torch.from_numpy(x), 1.0, 0.9)) for x in logits]
    rng = Mt19937(77)
    assert [sample_token(x, 1.0, 0.9, rng) for x in logits] == expect


def test_generation_mask_then_sample():
    """The reference loop masks ids < 260 (and EOS before 16 tokens) before sampling."""
    rng_np = np.random.default_rng(5)
    x = torch.from_numpy(rng_np.standard_normal(700).astype(np.float32))
    masked = generation_mask(x, index=3)
    torch.manual_seed(9)
    expect = int(torch_sample(masked, 0.9, 0.95))
    got = sample_token(masked.numpy(), 0.9, 0.95, Mt19937(9))
    assert got == expect and got >= 260


@pytest.mark.parametrize("index", [0, 15, 16, 40])
@pytest.mark.parametrize("blocked", [(), (0, 5, 127)])
def test_native_generation_mask_matches_oracle(index, blocked):
    from yufmusicgen_amd.engine import generation_mask as native_mask

    x = np.random.default_rng(index).standard_normal(1000).astype(np.float32)
    expect = generation_mask(torch.from_numpy(x), index=index, blocked_raw_ids=blocked).numpy()
    np.testing.assert_array_equal(native_mask(x, index, blocked), expect)


def test_native_generation_mask_rejects_bad_ids():
    from yufmusicgen_amd._lib import YufError
    from yufmusicgen_amd.engine import generation_mask as native_mask

    x = np.zeros(300, np.float32)
    with pytest.raises(YufError):
        native_mask(x, 0, (40,))  # 260 + 40 >= V
    with pytest.raises(YufError):
        native_mask(x, 20, (), eos_id=300)


def test_greedy_when_temperature_not_positive():
    x = np.array([0.1, 5.0, 2.0], np.float32)
    assert sample_token(x, 0.0, 0.95, Mt19937(1)) == 1
