"""CPU tests pinning the sampling oracle (oracle/sampling_ref.py).

* SplitMix64 against its published outputs for state 0 (the first two outputs
  of the generator seeded with 0: 0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4).
* The kept sets against HF transformers' own warpers (TemperatureLogitsWarper,
  TopKLogitsWarper, TopPLogitsWarper, applied in HF's order) on random rows and
  on rows with ties at the k-th value: the fixtures tests/golden/
  hf_sampling_kept.npz, written by tests/golden/make_sampling_golden.py.
* The Gumbel-max draw against the softmax of the kept scores: frequencies over
  many counters within 5 standard deviations, and never a removed token.
"""

import os

import numpy as np
import pytest

from oracle import sampling_ref as S


def test_splitmix64_known_outputs():
    z = S.mix64(np.array([0, 0x9E3779B97F4A7C15], dtype=np.uint64))
    assert [hex(int(v)) for v in z] == ["0xe220a8397b1dcdaf", "0x6e789e6aa1b965f4"]


def test_uniforms_in_open_interval_and_flat():
    u = S.uniforms(seed=7, counter=3, n=200000)
    assert u.dtype == np.float32 and u.min() > 0 and u.max() < 1
    assert abs(float(u.mean()) - 0.5) < 0.005
    hist = np.histogram(u, bins=20, range=(0, 1))[0]
    assert hist.min() > 0.9 * 10000 and hist.max() < 1.1 * 10000
    assert not np.array_equal(u[:100], S.uniforms(seed=7, counter=4, n=100))


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hf_sampling_kept.npz")


@pytest.fixture(scope="module")
def hf_golden():
    return np.load(GOLDEN)


def test_kept_sets_match_hf_warpers(hf_golden):
    """30 random rows (default_rng(seed), N(0, 3^2), 2000 entries) x (T, top-k, top-p) settings."""
    cases = hf_golden["random_cases"]
    kept = np.unpackbits(hf_golden["random_kept"], axis=1)[:, :2000].astype(bool)
    for (seed, t, k, p), want in zip(cases, kept):
        logits = (np.random.default_rng(int(seed)).standard_normal(2000) * 3.0).astype(np.float32)
        _, keep = S.kept_mask(logits, float(t), int(k), float(p))
        assert np.array_equal(keep, want), f"seed {seed} T {t} k {k} p {p}: kept {keep.sum()} vs HF {want.sum()}"


def test_top_k_keeps_ties_like_hf(hf_golden):
    _, keep = S.kept_mask(hf_golden["tie_row"], 1.0, 3, 1.0)
    assert keep.tolist() == hf_golden["tie_kept"].tolist()
    assert keep.sum() == 5  # the three 4s tied at the 3rd value are all kept, as HF does


def test_top_p_keeps_the_top_token_at_tiny_p(hf_golden):
    _, keep = S.kept_mask(hf_golden["tiny_p_row"], 1.0, 0, 1e-9)
    assert keep.tolist() == [False, False, False, True] == hf_golden["tiny_p_kept"].tolist()


def test_greedy_at_zero_temperature():
    logits = np.array([0.5, 2.0, 2.0, -1.0], dtype=np.float32)
    assert S.sample_row(logits, 0.0, 0, 1.0, 1, 0)[0] == 1  # first index of the maximum


def test_gumbel_max_draws_follow_softmax():
    logits = np.array([1.0, 0.2, -0.5, 2.0, 0.0, -3.0, 1.5, 0.7], dtype=np.float32)
    T = 0.8
    n = 20000
    counts = np.zeros(logits.size)
    for c in range(n):
        counts[S.sample_row(logits, T, 0, 1.0, 12345, c)[0]] += 1
    s = logits.astype(np.float64) / T
    p = np.exp(s - s.max())
    p /= p.sum()
    sd = np.sqrt(n * p * (1 - p))
    assert np.all(np.abs(counts - n * p) <= 5 * sd + 1), (counts, n * p)


def test_draws_stay_in_the_kept_set():
    rng = np.random.default_rng(3)
    logits = (rng.standard_normal(300) * 2).astype(np.float32)
    _, keep = S.kept_mask(logits, 1.0, 20, 0.7)
    for c in range(300):
        assert keep[S.sample_row(logits, 1.0, 20, 0.7, 99, c)[0]]
