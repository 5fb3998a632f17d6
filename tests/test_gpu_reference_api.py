"""The reference's benchmark entry points on the GPU (reference qwen_megakernel/bench.py:58-133)."""

import pytest

pytestmark = pytest.mark.gpu


def test_correctness_check_matches_hf_tokens():
    """The megakernel's first 8 greedy tokens for the seeded prompt, fed one step at a time as the
    reference's check does, equal HF transformers' (golden data) up to a near-tie."""
    from qwen_megakernel.bench import correctness_check

    res = correctness_check(verbose=True)
    assert len(res["mk"]) == 8 and res["match"], res


def test_bench_megakernel_runs():
    """bench_megakernel() times Decoder.generate of 100 tokens (3 warm-up, 5 timed runs)."""
    from qwen_megakernel.bench import bench_megakernel

    tok_s, ms = bench_megakernel()
    print(f"bench_megakernel: {tok_s:.1f} tok/s, {ms:.3f} ms/token")
    assert tok_s > 100 and abs(tok_s * ms - 1000.0) < 1e-6 * 1000 * tok_s
