"""Write the kept-set fixtures of the sampling oracle's tests from HF transformers' warpers.

HF's ``TemperatureLogitsWarper``, ``TopKLogitsWarper`` and ``TopPLogitsWarper``
(transformers 5.15.0, generation/logits_process.py; a third-party package, not
part of the reference) define which tokens a sampled step may draw.  This
script applies them, in HF's order, to the logits rows that
tests/test_sampling.py regenerates (numpy ``default_rng(seed)``, N(0, 3^2),
2000 entries; and two hand-made rows with ties), and records the kept mask of
each case in ``hf_sampling_kept.npz``.

Run:  python tests/golden/make_sampling_golden.py
"""

from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "hf_sampling_kept.npz")

# (seed, temperature, top_k, top_p) of the random rows; each row is
# default_rng(seed).standard_normal(2000) * 3 as float32
RANDOM_CASES = [(seed, t, k, p) for seed in range(6)
                for (t, k, p) in [(0.7, 0, 0.9), (1.0, 50, 1.0), (1.3, 40, 0.8), (0.5, 0, 0.5), (1.0, 7, 0.95)]]
TIE_ROW = [5, 4, 4, 4, 3, 2, 1, 4, 0]          # top-k 3 at T 1: the tied 4s
TINY_P_ROW = [1.0, 3.0, 2.0, 3.5]              # top-p 1e-9 at T 1: the top token alone


def random_row(seed: int) -> np.ndarray:
    return (np.random.default_rng(seed).standard_normal(2000) * 3.0).astype(np.float32)


def hf_kept(logits, temperature, top_k, top_p) -> np.ndarray:
    from transformers.generation.logits_process import (TemperatureLogitsWarper, TopKLogitsWarper,
                                                        TopPLogitsWarper)

    scores = torch.from_numpy(np.asarray(logits, dtype=np.float32))[None, :].clone()
    scores = TemperatureLogitsWarper(temperature)(None, scores)
    if 0 < top_k < scores.shape[-1]:
        scores = TopKLogitsWarper(top_k)(None, scores)
    if 0.0 < top_p < 1.0:
        scores = TopPLogitsWarper(top_p)(None, scores)
    return torch.isfinite(scores[0]).numpy()


def main():
    import transformers

    cases = np.array(RANDOM_CASES, dtype=np.float64)
    kept = np.stack([hf_kept(random_row(int(s)), t, int(k), p) for s, t, k, p in RANDOM_CASES])
    np.savez_compressed(OUT, random_cases=cases, random_kept=np.packbits(kept, axis=1),
                        tie_row=np.array(TIE_ROW, dtype=np.float32),
                        tie_kept=hf_kept(np.array(TIE_ROW, dtype=np.float32), 1.0, 3, 1.0),
                        tiny_p_row=np.array(TINY_P_ROW, dtype=np.float32),
                        tiny_p_kept=hf_kept(np.array(TINY_P_ROW, dtype=np.float32), 1.0, 0, 1e-9),
                        transformers_version=np.array(transformers.__version__))
    print("wrote", OUT, kept.shape, "kept per row", kept.sum(1).tolist())


if __name__ == "__main__":
    main()
