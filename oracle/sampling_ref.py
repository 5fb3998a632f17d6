"""CPU oracle for the sampling kernels (temperature, top-k, top-p, Gumbel-max draw).

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` as the checker; the product
path (``qmk_sample_rows`` / ``qmk_generate_sample`` in
qwen_megakernel/csrc/qmk_sample.hip) never calls it.

The reference decodes greedily only (csrc/kernel.cu:1020-1183); sampling follows
HF transformers' logits warpers, applied in HF's order (generation/utils.py
builds TemperatureLogitsWarper, TopKLogitsWarper, TopPLogitsWarper;
generation/logits_process.py):

* temperature: ``scores / T`` in fp32;
* top-k: remove ``scores < topk(scores, k)[-1]`` (ties at the k-th value kept);
* top-p: sort ascending, ``cumsum(softmax)``, remove where ``<= 1 - p``, keep
  at least one (the top) token; stated here as: keep v iff the probability mass
  of the kept scores strictly above ``s_v`` is ``< p``.

The draw is a Gumbel-max draw from the softmax of the kept scores,
``argmax(s_v + G_v)`` with ``G_v = -log(-log(U_v))`` and ``U_v`` from
SplitMix64 (Steele, Lea, Flood, OOPSLA 2014) over (seed, counter, v); HF's
``torch.multinomial`` stream cannot be matched, so parity is with this
restatement, which tests/test_sampling.py pins against HF's warpers (kept
sets) and against softmax frequencies (the draw).  Masses are the kernel's:
``floor(exp(s - max) * 2^40 + 0.5)`` as integers, so every sum is exact.
"""

from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1
FIX = float(1 << 40)


def mix64(z: np.ndarray) -> np.ndarray:
    """SplitMix64 finaliser (with its golden-ratio increment) on uint64 arrays, wrapping."""
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = z + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def uniforms(seed: int, counter: int, n: int) -> np.ndarray:
    """U_v in (0, 1) for v < n, float32: the top 24 bits of mix64(base + v), centred."""
    base = mix64(np.array([np.uint64(seed & M64) ^ mix64(np.array([counter & M64], dtype=np.uint64))[0]],
                          dtype=np.uint64))[0]
    with np.errstate(over="ignore"):
        h = mix64(base + np.arange(n, dtype=np.uint64))
    top = (h >> np.uint64(40)).astype(np.uint32).astype(np.float32)
    return (top + np.float32(0.5)) * np.float32(1.0 / 16777216.0)


def key32(x: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 key of float32 values."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32)
    return np.where(u & np.uint32(0x80000000), ~u, u | np.uint32(0x80000000)).astype(np.uint32)


def kept_mask(logits: np.ndarray, temperature: float, top_k: int, top_p: float):
    """(scores, kept) for one row: the temperature-scaled scores and the top-k / top-p filter."""
    x = np.asarray(logits, dtype=np.float32)
    s = x / np.float32(temperature)
    k = key32(s)
    V = s.size
    kmin = np.uint32(0)
    if 0 < top_k < V:
        kmin = np.sort(k)[V - top_k]
    keep = k >= kmin
    if 0.0 < top_p < 1.0:
        mx = s.max()
        m = np.floor(np.exp(s - mx).astype(np.float64) * FIX + 0.5).astype(np.uint64)
        m = np.where(keep, m, np.uint64(0))
        z = int(m.sum(dtype=np.uint64))
        target = max(1, int(float(np.float32(top_p)) * float(z)))
        order = np.argsort(-k.astype(np.int64), kind="stable")  # descending keys
        ks, ms = k[order], m[order]
        cum = np.cumsum(ms, dtype=np.uint64)
        # mass strictly above each key = cumulative mass before its first occurrence
        first = np.searchsorted(-ks.astype(np.int64), -ks.astype(np.int64), side="left")
        above = np.where(first > 0, cum[np.maximum(first - 1, 0)], np.uint64(0))
        keep_sorted = above < np.uint64(target)
        keep_p = np.zeros(V, dtype=bool)
        keep_p[order] = keep_sorted
        keep = keep & keep_p
    return s, keep


def sample_row(logits: np.ndarray, temperature: float, top_k: int, top_p: float, seed: int, counter: int):
    """Token of one row and the gap between the two best perturbed scores (for near-tie checks)."""
    x = np.asarray(logits, dtype=np.float32)
    if not temperature > 0:
        return int(np.argmax(x)), float("inf")
    s, keep = kept_mask(x, temperature, top_k, top_p)
    u = uniforms(seed, counter, s.size)
    g = -np.log(-np.log(u))
    score = (s + g.astype(np.float32)).astype(np.float32)
    score = np.where(keep, score, np.float32(-np.inf))
    tok = int(np.argmax(score))
    top2 = np.sort(score[keep])[-2:] if keep.sum() > 1 else np.array([score[tok], -np.inf])
    return tok, float(top2[-1] - top2[0])
