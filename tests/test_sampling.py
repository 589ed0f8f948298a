"""The sampling oracle (oracle/sampling.py, restating reference engine/generate.py:36-55) on the
CPU, pinned by: Philox4x32-10's published known-answer vectors (Random123), the moments and
distribution of the exponential noise, a second restatement through torch's own bf16 ops,
closed-form special cases (top_k = 1, constant noise, ties at the top-k pivot) and the sampling
distribution itself (chi-square against the softmax probabilities)."""
import numpy as np
import pytest
import torch

from oracle.sampling import (bf16_round, exponential_noise, logits_to_probs, logits_to_probs_torch,
                             philox4x32_10, sample_with_noise, uniform01)


@pytest.mark.parametrize("ctr,key,expect", [
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
])
def test_philox_known_answers(ctr, key, expect):
    out = philox4x32_10([np.uint64(c) for c in ctr], key)
    assert [int(v) for v in out] == expect


def test_uniform_and_exponential_noise():
    x = np.array([0, 255, 256, 0xFFFFFFFF], dtype=np.uint64)
    u = uniform01(x)
    assert u[0] == u[1] == 0.5 * 2.0 ** -24 and u[2] == 1.5 * 2.0 ** -24
    assert u[3] == 1.0 - 0.5 * 2.0 ** -24
    q = exponential_noise(seed=1234, offset=7, vocab=200000, row=3)
    assert np.all(q > 0)
    assert abs(q.mean() - 1.0) < 0.01 and abs(q.var() - 1.0) < 0.03
    # Kolmogorov-Smirnov distance to Exp(1) (bf16 rounding moves values by < 0.4 %)
    s = np.sort(q.astype(np.float64))
    cdf = 1.0 - np.exp(-s)
    ks = np.max(np.abs(cdf - np.arange(1, s.size + 1) / s.size))
    assert ks < 0.01
    # counters differ per row, offset and seed
    a = exponential_noise(1, 0, 64, 0)
    assert not np.array_equal(a, exponential_noise(1, 0, 64, 1))
    assert not np.array_equal(a, exponential_noise(1, 1, 64, 0))
    assert not np.array_equal(a, exponential_noise(2, 0, 64, 0))
    assert np.array_equal(a, exponential_noise(1, 0, 64, 0))


def _bf16_logits(rng, v, scale=2.0):
    return bf16_round(rng.standard_normal(v).astype(np.float32) * scale)


@pytest.mark.parametrize("t,k", [(1.0, None), (0.8, 200), (1.3, 5), (0.05, 50), (1.0, 1)])
def test_oracle_matches_torch_restatement(t, k):
    rng = np.random.default_rng(0)
    lg = _bf16_logits(rng, 4096)
    p, _ = logits_to_probs(lg, t, k)
    pt = logits_to_probs_torch(lg, t, k).float().numpy()
    ulp = np.maximum(np.abs(pt), 2.0 ** -126) * 2.0 ** -7
    diff = np.abs(p - pt)
    assert np.all(diff <= ulp + 1e-45)               # at most one bf16 ulp apart
    assert np.mean(diff == 0) > 0.97                 # and nearly always identical
    assert abs(p.sum(dtype=np.float64) - 1.0) < 0.02


def test_top_k_keeps_ties_at_pivot_and_top1_is_argmax():
    lg = np.array([1.0, 3.0, 2.0, 3.0, 2.0, 2.0, -1.0], dtype=np.float32)
    _, x = logits_to_probs(lg, 1.0, 3)
    assert np.isfinite(x).tolist() == [False, True, True, True, True, True, False]   # 2.0 ties kept
    rng = np.random.default_rng(1)
    for _ in range(50):
        lg = _bf16_logits(rng, 300)
        q = exponential_noise(int(rng.integers(1 << 30)), 0, 300)
        assert sample_with_noise(lg, q, 1.0, 1)[0] == int(np.argmax(lg))


def test_constant_noise_gives_argmax():
    rng = np.random.default_rng(2)
    for _ in range(50):
        lg = _bf16_logits(rng, 500)
        idx, r = sample_with_noise(lg, np.ones(500, dtype=np.float32), 0.7, None)
        assert idx == int(np.argmax(lg))


def test_sampling_distribution_chi_square():
    rng = np.random.default_rng(3)
    lg = bf16_round(np.array([2.0, 1.0, 0.5, 0.0, -0.5, -1.0, -2.0, 3.0], dtype=np.float32))
    for t, k in ((1.0, None), (0.7, 4)):
        p, _ = logits_to_probs(lg, t, k)
        n = 20000
        counts = np.zeros(lg.size)
        for i in range(n):
            counts[sample_with_noise(lg, exponential_noise(99, i, lg.size), t, k)[0]] += 1
        keep = p > 0
        assert counts[~keep].sum() == 0
        exp = p[keep] / p[keep].sum() * n
        chi2 = float(((counts[keep] - exp) ** 2 / exp).sum())
        assert chi2 < 30.0, (t, k, chi2, counts, exp)    # dof <= 7: p(chi2 > 30) < 1e-4
