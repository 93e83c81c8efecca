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


def test_generation_mask_hand_derived_vectors():
    """Expected vectors written out by hand from cli/generate.py:139-148 (and
    generation.rs:195-203), not from any restatement: with V = 270, ids 0..259
    are -inf, ids 260..269 keep their logit; EOS (id 2) is -inf at index 15 and
    keeps its logit from index 16 on; blocked raw id 5 means token 265."""
    from yufmusicgen_amd.engine import generation_mask as native_mask

    V = 270
    x = np.arange(V, dtype=np.float32) * 0.5 - 7.0  # distinct finite logits
    ninf = -np.inf
    for index, eos_kept in ((0, False), (15, False), (16, True), (17, True)):
        expect = np.full(V, ninf, np.float32)
        expect[260:] = x[260:]
        if eos_kept:
            expect[2] = x[2]  # -6.0
        expect_blocked = expect.copy()
        expect_blocked[265] = ninf
        for got in (generation_mask(torch.from_numpy(x), index=index).numpy(), native_mask(x, index)):
            np.testing.assert_array_equal(got, expect)
        for got in (generation_mask(torch.from_numpy(x), index=index, blocked_raw_ids=(5,)).numpy(),
                    native_mask(x, index, (5,))):
            np.testing.assert_array_equal(got, expect_blocked)
    # Spot values, independent of the loop above.
    m15, m16 = native_mask(x, 15), native_mask(x, 16)
    assert m15[259] == ninf and m15[260] == x[260] == 123.0 and m15[2] == ninf
    assert m16[2] == -6.0 and m16[3] == ninf and m16[1] == ninf
    assert native_mask(x, 40, (5,))[265] == ninf and native_mask(x, 40, (5,))[264] == x[264]


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


@pytest.mark.parametrize("vocab,k", [(20480, 32), (300, 64), (40, 40), (7, 3)])
def test_exp_draws_consume_what_a_sample_consumes(vocab, k):
    """yuf_rng_exp_draws takes exactly the V uniforms of one host sample (the
    generators agree afterwards) and its q are -log1p(-u) of torch's stream."""
    rng_a, rng_b = Mt19937(5), Mt19937(5)
    q, first_zero = rng_a.exp_draws(vocab, k)
    sample_token(np.zeros(vocab, np.float32), 1.0, 0.9, rng_b, top_k=min(k, vocab))
    assert [rng_a.next_u32() for _ in range(5)] == [rng_b.next_u32() for _ in range(5)]
    torch.manual_seed(5)
    u = torch.rand(vocab, dtype=torch.float64)
    np.testing.assert_array_equal(q, (-torch.log1p(-u[:k])).to(torch.float32).numpy())
    assert first_zero == -1


def test_rng_copy_is_independent():
    rng = Mt19937(11)
    rng.next_u32()
    twin = rng.copy()
    assert [rng.next_u32() for _ in range(700)] == [twin.next_u32() for _ in range(700)]


def _host_probs(x):
    """The host sampler's first softmax over a sorted row (float exps of the
    double exponential, the 16-lane sum, one reciprocal)."""
    mx = x[0]
    e = np.exp((x - mx).astype(np.float64)).astype(np.float32)
    acc = np.zeros(16, np.float32)
    for i in range(0, e.size, 16):
        chunk = e[i:i + 16]
        acc[:chunk.size] = (acc[:chunk.size] + chunk).astype(np.float32)
    for half in (8, 4, 2, 1):
        acc[:half] = (acc[:half] + acc[half:2 * half]).astype(np.float32)
    return (e * (np.float32(1.0) / acc[0])).astype(np.float32)


@pytest.mark.parametrize("scale,top_p", [(3.0, 0.95), (0.05, 0.95), (1.0, 0.5), (8.0, 0.99), (0.5, 1.0),
                                         (20.0, 0.9)])
def test_full_vocab_cut_by_exact_prefix_equals_sequential_double_sum(scale, top_p):
    """The device's full-vocabulary top-p cut (yuf_sample_device_masked with
    top_k = 0) replaces the host's sequential double cumulative sum by an
    integer prefix sum of p * 2^53 wherever every p so far is a multiple of
    2^-53 and the sum is at most 1 -- there each double addition is exact --
    and decides other positions by a 2^-20 bound on an approximate prefix.
    Checked here against the sequential loop of yuf_sample itself: the exact
    region's sums are bit-equal, and every decision the kernel takes without
    its sequential fallback equals the host's."""
    rng = np.random.default_rng(int(scale * 100) + int(top_p * 1000))
    for trial in range(20):
        x = -np.sort(-(rng.standard_normal(20480) * scale).astype(np.float32))
        p = _host_probs(x)
        cum = np.cumsum(p.astype(np.float64))  # sequential, as the host loop
        host_drop = (cum.astype(np.float32) - p) > np.float32(top_p)
        t = p.astype(np.float64) * 2.0**53
        exact = (t == np.floor(t)) & (t <= 2.0**62)
        fb = int(np.argmin(exact)) if not exact.all() else p.size
        nsum = np.cumsum(np.where(exact, t, 0).astype(np.uint64))
        ok = (np.arange(p.size) < fb) & (nsum <= np.uint64(2**53))
        assert ok[:100].all() or scale >= 8.0  # the exact region covers the head of the order
        np.testing.assert_array_equal(cum[ok], nsum[ok].astype(np.float64) * 2.0**-53)
        dev_drop = (nsum.astype(np.float64) * 2.0**-53).astype(np.float32) - p > np.float32(top_p)
        # The kernel's approximate prefix (a block scan, another summation
        # order): the sequential sum moved by up to 2^-37.
        aprev = np.concatenate([[0.0], cum[:-1]]) + rng.uniform(-2.0**-37, 2.0**-37, p.size)
        certain_drop = aprev > top_p + 2.0**-20
        certain_keep = aprev < top_p - 2.0**-20
        decided = ok | certain_drop | certain_keep
        dev_drop = np.where(ok, dev_drop, certain_drop)
        np.testing.assert_array_equal(dev_drop[decided], host_drop[decided])
        if top_p < 1.0:
            assert decided.all(), "fallback needed below top_p = 1"
