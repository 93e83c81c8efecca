"""GPU parity of the device sampler with the generation mask
(yuf_sample_device_masked) against the host sampler (yuf_sample, itself
checked against torch's CPU sampling in test_sampler.py) and the host mask
(yuf_generation_mask, pinned by hand-derived vectors in test_sampler.py).

Exact mode: each stream's MT19937 generator supplies the Exp(1) draws of one
host sample (yuf_rng_exp_draws), so the device token must equal yuf_sample's
on the masked logits for the same generator state -- bit for bit, every row.
"""

import numpy as np
import pytest
import torch

from yufmusicgen_amd.engine import Mt19937, argmax, generation_mask, sample_device_masked, sample_token

pytestmark = pytest.mark.gpu

MASK = dict(midi_offset=260, eos_id=2, min_before_eos=16, blocked=(0, 5, 17, 127, 128, 900))


def _rows(n, vocab, seed, scale=3.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((n, vocab)) * scale).astype(np.float32)
    # Make EOS competitive so the index rule matters.
    x[:, 2] = x.max(axis=1) + 0.5
    return x


def _exact_draws(gens, vocab, k):
    qs, fzs = zip(*(g.exp_draws(vocab, k) for g in gens))
    return (torch.from_numpy(np.stack(qs)).cuda(), torch.from_numpy(np.array(fzs, np.int32)).cuda())


@pytest.mark.parametrize("temperature,top_p,top_k", [(1.0, 1.0, 32), (0.8, 0.9, 64), (1.3, 0.5, 16), (1.0, 0.0, 8)])
@pytest.mark.parametrize("masked", [True, False])
def test_exact_mode_equals_host_sampler(temperature, top_p, top_k, masked):
    """64 rows of 20480 logits, three consecutive draws per row from its own
    generator: the device token equals yuf_sample's on the masked logits."""
    print(f"exact T={temperature} top_p={top_p} k={top_k} mask={masked}", flush=True)
    n, vocab = 64, 20480
    x = _rows(n, vocab, seed=top_k + int(masked))
    logits = torch.from_numpy(x).cuda()
    tokens = torch.empty(n, dtype=torch.int32, device="cuda")
    index = np.where(np.arange(n) % 2 == 0, 3, 20).astype(np.int32)  # EOS allowed on odd rows only
    index_dev = torch.from_numpy(index).cuda()
    host = [Mt19937(1000 + s) for s in range(n)]
    dev = [g.copy() for g in host]
    for step in range(3):
        q, fz = _exact_draws(dev, vocab, top_k)
        sample_device_masked(logits, tokens, temperature, top_p, top_k, mask=MASK if masked else None,
                             index=index_dev, exp_draws=q, first_zero=fz)
        torch.cuda.synchronize()
        got = tokens.cpu().numpy()
        expect = []
        for s in range(n):
            row = generation_mask(x[s], int(index[s]), MASK["blocked"]) if masked else x[s]
            expect.append(sample_token(row, temperature, top_p, host[s], top_k=top_k))
        np.testing.assert_array_equal(got, np.array(expect), err_msg=f"step {step}")
        if masked:
            assert np.all((got >= 260) | ((got == 2) & (index >= 16)))
            assert not np.isin(got - 260, MASK["blocked"]).any()
        x = np.roll(x, 7, axis=1)  # new logits for the next step
        logits.copy_(torch.from_numpy(x))


def test_exact_mode_fewer_allowed_than_top_k():
    """V = 300 with the mask leaves 40 allowed ids (-inf candidates fill the
    top 64), and a row whose first-zero position wins; against yuf_sample."""
    n, vocab, k = 8, 300, 64
    x = _rows(n, vocab, seed=3)
    logits = torch.from_numpy(x).cuda()
    tokens = torch.empty(n, dtype=torch.int32, device="cuda")
    mask = dict(midi_offset=260, eos_id=2, min_before_eos=16, blocked=(1, 2, 39))
    host = [Mt19937(7 + s) for s in range(n)]
    dev = [g.copy() for g in host]
    q, fz = _exact_draws(dev, vocab, k)
    sample_device_masked(logits, tokens, 0.9, 0.95, k, mask=mask, index=30, exp_draws=q, first_zero=fz)
    torch.cuda.synchronize()
    expect = [sample_token(generation_mask(x[s], 30, mask["blocked"]), 0.9, 0.95, host[s], top_k=k) for s in range(n)]
    np.testing.assert_array_equal(tokens.cpu().numpy(), np.array(expect))
    # A zero draw past the candidates gives a NaN score on the host, which wins:
    # position 70 of the host's order is the 6th smallest id outside the top 64.
    q2 = q.clone()
    fz2 = torch.full((n,), 70, dtype=torch.int32, device="cuda")
    sample_device_masked(logits, tokens, 0.9, 0.95, k, mask=mask, index=30, exp_draws=q2, first_zero=fz2)
    torch.cuda.synchronize()
    for s in range(n):
        allowed = generation_mask(x[s], 30, mask["blocked"]) / np.float32(0.9)
        order = sorted(range(vocab), key=lambda i: (-allowed[i], i))
        assert int(tokens[s]) == order[70]


@pytest.mark.parametrize("index", [0, 15, 16, 40])
def test_greedy_with_mask_is_argmax_of_masked_logits(index):
    n, vocab = 16, 20480
    x = _rows(n, vocab, seed=index)
    logits = torch.from_numpy(x).cuda()
    tokens = torch.empty(n, dtype=torch.int32, device="cuda")
    sample_device_masked(logits, tokens, 0.0, 1.0, 32, mask=MASK, index=index)
    torch.cuda.synchronize()
    expect = [argmax(generation_mask(x[s], index, MASK["blocked"])) for s in range(n)]
    np.testing.assert_array_equal(tokens.cpu().numpy(), np.array(expect))
    assert (tokens.cpu().numpy() == 2).all() == (index >= 16)  # EOS is the largest logit of every row


def test_counter_mode_with_mask_stays_in_the_allowed_top_k():
    n, vocab, k = 32, 20480, 32
    x = _rows(n, vocab, seed=9)
    logits = torch.from_numpy(x).cuda()
    tokens = torch.empty(n, dtype=torch.int32, device="cuda")
    masked = np.stack([generation_mask(x[s], 4, MASK["blocked"]) for s in range(n)])
    top = np.argsort(-masked, axis=1, kind="stable")[:, :k]
    seen = set()
    for c in range(40):
        sample_device_masked(logits, tokens, 1.0, 1.0, k, mask=MASK, index=4, seed=3, counter=c)
        torch.cuda.synchronize()
        got = tokens.cpu().numpy()
        for s in range(n):
            assert got[s] in top[s], (s, got[s])
        seen.add(int(got[0]))
    assert len(seen) > 4
    # top_p = 0 keeps only the first candidate: the masked argmax.
    sample_device_masked(logits, tokens, 1.0, 0.0, k, mask=MASK, index=4, seed=3, counter=0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(tokens.cpu().numpy(), top[:, 0])


def test_exact_mode_with_heavy_ties_takes_the_radix_path():
    """Rows where more than 1024 values sit at the selection bound (the radix
    fallback): the candidate order (value, then id) still equals the host's."""
    n, vocab, k = 4, 20480, 32
    x = np.zeros((n, vocab), np.float32)
    x[0, [7, 300, 4096, 9999, 20479]] = 1.0  # five winners over a sea of ties
    x[1, ::3] = 0.5
    x[2] = np.round(np.random.default_rng(1).standard_normal(vocab), 1)  # many exact ties
    logits = torch.from_numpy(x).cuda()
    tokens = torch.empty(n, dtype=torch.int32, device="cuda")
    host = [Mt19937(40 + s) for s in range(n)]
    dev = [g.copy() for g in host]
    for step in range(4):
        q, fz = _exact_draws(dev, vocab, k)
        sample_device_masked(logits, tokens, 1.0, 0.9, k, exp_draws=q, first_zero=fz)
        torch.cuda.synchronize()
        expect = [sample_token(x[s], 1.0, 0.9, host[s], top_k=k) for s in range(n)]
        np.testing.assert_array_equal(tokens.cpu().numpy(), np.array(expect), err_msg=f"step {step}")


@pytest.mark.parametrize("temperature,top_p,scale", [(1.0, 0.95, 3.0), (1.0, 0.95, 0.05), (0.7, 0.5, 1.0),
                                                     (1.5, 0.99, 8.0), (1.0, 1.0, 0.5), (1.0, 0.0, 1.0)])
@pytest.mark.parametrize("masked", [True, False])
def test_full_vocab_exact_mode_equals_host_sampler(temperature, top_p, scale, masked):
    """The reference's own parameters (temperature 1, top_p 0.95, no top-k:
    cli/generate.py:39-56, sampler.rs:131-256) on the device: top_k = 0 sorts
    all V logits.  64 rows of 20480, three draws per row from its own
    generator (all V Exp(1) draws of one host sample as the exact-mode input):
    the device token equals yuf_sample's, top_k 0, on the masked logits.
    Scale 0.05 is the near-flat case of the random-init model, whose nucleus
    holds most of the vocabulary."""
    print(f"full exact T={temperature} top_p={top_p} scale={scale} mask={masked}", flush=True)
    n, vocab = 64, 20480
    x = _rows(n, vocab, seed=int(scale * 10) + int(masked), scale=scale)
    logits = torch.from_numpy(x).cuda()
    tokens = torch.empty(n, dtype=torch.int32, device="cuda")
    index = np.where(np.arange(n) % 2 == 0, 3, 20).astype(np.int32)
    index_dev = torch.from_numpy(index).cuda()
    host = [Mt19937(500 + s) for s in range(n)]
    dev = [g.copy() for g in host]
    for step in range(3):
        q, _ = _exact_draws(dev, vocab, vocab)
        sample_device_masked(logits, tokens, temperature, top_p, 0, mask=MASK if masked else None,
                             index=index_dev, exp_draws=q)
        torch.cuda.synchronize()
        got = tokens.cpu().numpy()
        expect = []
        for s in range(n):
            row = generation_mask(x[s], int(index[s]), MASK["blocked"]) if masked else x[s]
            expect.append(sample_token(row, temperature, top_p, host[s], top_k=0))
        np.testing.assert_array_equal(got, np.array(expect), err_msg=f"step {step}")
        x = np.roll(x, 7, axis=1)
        logits.copy_(torch.from_numpy(x))


@pytest.mark.parametrize("vocab", [300, 1000, 24576])
def test_full_vocab_edge_rows(vocab):
    """Ties (values rounded to 0.1), -0.0 beside +0.0, a fully -inf row, rows
    with a single allowed id, V not a multiple of 16 or of 1024, the largest
    V, and top_k >= V (the same path): against yuf_sample, two draws each."""
    rng = np.random.default_rng(vocab)
    n = 8
    x = np.round(rng.standard_normal((n, vocab)), 1).astype(np.float32)
    x[1, ::2] = -0.0
    x[1, 1::2] = 0.0
    x[2] = -np.inf
    x[3] = -np.inf
    x[3, vocab // 3] = 1.0
    x[4] = (rng.standard_normal(vocab) * 40.0).astype(np.float32)  # tiny tail probabilities
    x[5] = 0.0  # all equal
    logits = torch.from_numpy(x).cuda()
    tokens = torch.empty(n, dtype=torch.int32, device="cuda")
    for top_k, top_p in ((0, 0.95), (vocab, 0.8), (0, 1.0), (vocab + 5, 0.3)):
        host = [Mt19937(90 + s) for s in range(n)]
        dev = [g.copy() for g in host]
        for step in range(2):
            q, _ = _exact_draws(dev, vocab, vocab)
            sample_device_masked(logits, tokens, 0.9, top_p, top_k, exp_draws=q)
            torch.cuda.synchronize()
            expect = [sample_token(x[s], 0.9, top_p, host[s], top_k=top_k) for s in range(n)]
            np.testing.assert_array_equal(tokens.cpu().numpy(), np.array(expect),
                                          err_msg=f"top_k={top_k} top_p={top_p} step {step}")


def test_full_vocab_counter_mode_stays_in_the_nucleus():
    """Counter draws (no host work): every token lies in the host's nucleus of
    the masked row, and a near-flat row spreads over many ids."""
    n, vocab = 16, 20480
    x = _rows(n, vocab, seed=21, scale=1.0)
    x[0] = np.random.default_rng(5).standard_normal(vocab).astype(np.float32) * 0.05
    logits = torch.from_numpy(x).cuda()
    tokens = torch.empty(n, dtype=torch.int32, device="cuda")
    nuclei = []
    for s in range(n):
        row = generation_mask(x[s], 20, MASK["blocked"]).astype(np.float64)
        order = sorted(range(vocab), key=lambda i: (-row[i], i))
        pr = np.exp(row[order] - row[order[0]])
        pr /= pr.sum()
        cum = np.cumsum(pr)
        nuclei.append(set(np.array(order)[(cum - pr) <= 0.95 + 1e-6].tolist()))
    seen = set()
    for c in range(30):
        sample_device_masked(logits, tokens, 1.0, 0.95, 0, mask=MASK, index=20, seed=11, counter=c)
        torch.cuda.synchronize()
        got = tokens.cpu().numpy()
        for s in range(n):
            assert int(got[s]) in nuclei[s], (s, int(got[s]))
        seen.add(int(got[0]))
    assert len(seen) > 20


def test_masked_sampler_rejects_bad_arguments():
    from yufmusicgen_amd._lib import YufError

    logits = torch.zeros(2, 300, device="cuda")
    tokens = torch.empty(2, dtype=torch.int32, device="cuda")
    with pytest.raises(YufError):  # blocked id past the vocabulary
        sample_device_masked(logits, tokens, 1.0, 1.0, 8, mask=dict(blocked=(40,)))
    with pytest.raises(YufError):  # EOS outside the vocabulary once allowed
        sample_device_masked(logits, tokens, 1.0, 1.0, 8, mask=dict(eos_id=300), index=20)
    with pytest.raises(YufError):
        sample_device_masked(logits, tokens, 1.0, 1.0, 65)
    wide = torch.zeros(1, 24577, device="cuda")  # past the full-vocabulary path's limit
    with pytest.raises(YufError):
        sample_device_masked(wide, tokens[:1], 1.0, 0.95, 0)
