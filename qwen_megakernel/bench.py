"""Benchmark and correctness check with the reference's entry points.

Mirrors the reference's qwen_megakernel/bench.py:11-152: the same constants,
``bench_megakernel()`` (3 warm-up and 5 timed ``Decoder.generate`` runs of 100
tokens, returning tok/s and ms/token) and ``correctness_check()`` (the
megakernel's greedy tokens printed beside HF transformers' for the same
weights and prompt), and ``python -m qwen_megakernel.bench``.

Without network there is no ``Qwen/Qwen3-0.6B`` checkpoint and no tokenizer,
so both use the seeded synthetic Qwen3-0.6B weights that ``Decoder()`` draws
(seed 0) and, for the text prompt ``"Hello"``, the 16 seeded prompt ids of the
golden data instead.  HF's tokens come from that golden data
(``data/hf_greedy_qwen3_0p6b.json``: HF ``Qwen3ForCausalLM`` in bf16 eager on
the CPU, fed the same weights one token at a time, written by
tests/golden/make_hf_golden.py), so the check needs neither HF nor a
checkpoint at run time.  With a local checkpoint directory (``model_name``)
and its tokenizer, the text prompt is used as in the reference.  The
reference's ``bench_pytorch_hf`` (HF ``generate`` on the GPU from the hub
checkpoint) is not provided: it needs the network.
"""

from __future__ import annotations

import json
import math
import os
import time

import torch

TOKENS = 100
WARMUP = 3
RUNS = 5
PROMPT = "Hello"
CHECK_TOKENS = 8
RUN_CORRECTNESS = True

_DATA = os.path.join(os.path.dirname(os.path.abspath(__file__)), "data", "hf_greedy_qwen3_0p6b.json")


def golden():
    """HF's greedy continuation of the seeded prompt (prompt ids, tokens, top-2 gaps)."""
    with open(_DATA) as f:
        return json.load(f)


def _prompt(dec):
    if dec.tokenizer is not None:
        return PROMPT
    return golden()["prompt"]


def bench_megakernel(model_name: str = "Qwen/Qwen3-0.6B"):
    """tok/s and ms/token of ``Decoder.generate`` (reference bench.py:58-80)."""
    from qwen_megakernel.model import Decoder

    dec = Decoder(model_name=model_name, verbose=False)
    prompt = _prompt(dec)

    def run():
        dec.reset()
        dec.generate(prompt, max_tokens=TOKENS)

    for _ in range(WARMUP):
        run()
    torch.cuda.synchronize()

    times = []
    for _ in range(RUNS):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        run()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)

    avg = sum(times) / len(times)
    return TOKENS / avg, avg * 1000 / TOKENS


def correctness_check(verbose: bool = True):
    """The megakernel's first CHECK_TOKENS greedy tokens beside HF's (reference bench.py:83-133).

    The prompt is fed one ``Decoder.step`` at a time, as the reference does.
    Returns ``dict(hf=..., mk=..., gaps=..., match=...)``; ``match`` is True
    when the streams agree up to their first difference, if any, and that
    difference is at a near-tie of HF's logits (a top-2 gap below 1e-2 or of
    at most one bf16 ulp of the top logit, i.e. two adjacent bf16 values),
    after which they legitimately continue from different tokens.
    """
    from qwen_megakernel.model import Decoder

    g = golden()
    dec = Decoder(weights=None, verbose=False)
    prompt_ids = list(g["prompt"])
    hf_ids = g["greedy_tokens"][:CHECK_TOKENS]
    gaps = g["top2_gaps"][:CHECK_TOKENS]

    dec.reset()
    for tid in prompt_ids[:-1]:
        dec.step(tid)
    mk_ids = []
    tok = prompt_ids[-1]
    for _ in range(CHECK_TOKENS):
        tok = dec.step(tok)
        mk_ids.append(tok)

    match = True
    for i in range(CHECK_TOKENS):
        if mk_ids[i] == hf_ids[i]:
            continue
        top = abs(g["top_logits"][i])
        ulp = 2.0 ** (math.floor(math.log2(top)) - 7) if top > 0 else 0.0
        # a different token at a near-tie is allowed; the streams then continue from different tokens
        match = gaps[i] < 1e-2 or gaps[i] <= ulp
        break
    if verbose:
        print("Correctness check")
        print(f"HF tokens: {hf_ids}")
        print(f"MK tokens: {mk_ids}")
        print(f"HF top-2 gaps: {[round(x, 4) for x in gaps]}")
        print("match" if match else "MISMATCH")
    return dict(hf=hf_ids, mk=mk_ids, gaps=gaps, match=match)


if __name__ == "__main__":
    print("=" * 55)
    print("Qwen Megakernel Benchmark")
    print("=" * 55)
    print()

    print("Megakernel")
    if RUN_CORRECTNESS:
        correctness_check()
        print()
    mk_tok, mk_ms = bench_megakernel()

    print()
    print("=" * 55)
    print(f"{'Backend':<25} {'tok/s':>8} {'ms/tok':>8}")
    print("-" * 55)
    print(f"{'Megakernel':<25} {mk_tok:>8.1f} {mk_ms:>8.2f}")
