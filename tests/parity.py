"""The parity rule of the GPU tests, and helpers that run the exact oracle (not a test module).

Centre: oracle/qwen3_exact.py, the reference's PyTorch bf16 path (HF Qwen3's
bf16 eager semantics) with exact arithmetic between its bf16 rounding points,
so nothing depends on the CPU the test runs on.

Two fixed bars, per step:

* ``LITERAL`` (the north star's): logits cosine >= 0.999 and max abs <= 0.1
  over the whole vocabulary; the greedy token equal to the oracle's argmax
  except at a near-tie, where the token's oracle logit is within max(1e-2, one
  bf16 ulp of the top logit) of the top.  Logits are bf16: in [2, 4), where
  these models' top logits sit, distinct logits are at least 0.0156 apart, so
  a gap below 1e-2 is an exact tie there and one ulp is the closest two
  distinct logits can be.
* ``DEEP``: cosine >= 0.999, max abs <= 0.15, token within two bf16 ulps of the
  top.  For the workloads on which no fp32 implementation holds ``LITERAL``,
  the reference's own path included: 28 layers over an N(0, 1) long-context
  cache, Qwen3-1.7B, and greedy streams past the north star's 256 steps.  The
  random-weight model amplifies any bf16 rounding difference: computing a
  single op class in fp32 instead of exactly (only RMSNorm, or only the
  projections, or only attention) moves the 28-layer logits by 0.08-0.13;
  HF-semantics fp32 decoding itself sits 0.10-0.125 from the exact centre on
  Qwen3-1.7B and on 0.6B at 1500 positions, and its own 1024-step greedy
  stream departs from the centre's argmax at 2-ulp gaps (steps 114, 209, 299,
  539 of the benchmark workload).  tests/test_oracle_exact.py pins the 1.7B
  distance on the CPU.  0.15 is that 0.125 plus a margin below one ulp at the
  top logits; 2 ulps is the largest gap at which the reference path departs.

Token streams are checked teacher-forced on the decoder's own tokens: the
oracle runs the prompt and the tokens the decoder produced in one pass, and at
every step the decoder's token must be the oracle's argmax given the same
prefix, up to the near-tie rule.  That is the same as requiring the two free-
running streams to be identical, with a near-tie as the only place they may
part.
"""

from __future__ import annotations

import math

import torch

COS_MIN = 0.999
ABS_MAX = 0.1
TIE_GAP = 1e-2


class Bar:
    def __init__(self, name: str, abs_max: float, tie_ulps: int):
        self.name, self.abs_max, self.tie_ulps = name, abs_max, tie_ulps


LITERAL = Bar("literal", ABS_MAX, 1)
DEEP = Bar("deep", 0.15, 2)


def bf16_ulp(x: float) -> float:
    """Spacing of bf16 values at |x| (8 significant bits)."""
    return 2.0 ** (math.floor(math.log2(abs(x))) - 7) if x != 0 else 2.0 ** -133


def tie_tolerance(top: float, ulps: int = 1) -> float:
    return max(TIE_GAP, ulps * bf16_ulp(top))


class Tally:
    """Worst cosine / max abs over the checked rows, the near-tie flips met (with their gaps in
    ulps), and whether the literal bar held on every row."""

    def __init__(self, what: str):
        self.what = what
        self.rows = 0
        self.cos = 1.0
        self.mab = 0.0
        self.flips = []
        self.literal = True

    def __str__(self):
        return (f"{self.what}: {self.rows} rows, worst cos {self.cos:.6f}, max abs {self.mab:.4f}, "
                f"near-tie flips (step, gap in ulps) {self.flips}; literal bar "
                f"{'held' if self.literal else 'missed'}")


def check_row(t: Tally, label, ref: torch.Tensor, tok: int, got: torch.Tensor | None = None, bar: Bar = LITERAL):
    """One step: ``ref`` the oracle's fp32 logits row, ``tok`` the decoder's token, ``got`` its logits."""
    ref = ref.float()
    t.rows += 1
    if got is not None:
        got = got.float().cpu()
        cos = torch.nn.functional.cosine_similarity(got.double(), ref.double(), dim=0).item()
        mab = (got - ref).abs().max().item()
        t.cos, t.mab = min(t.cos, cos), max(t.mab, mab)
        t.literal &= mab <= ABS_MAX
        assert cos >= COS_MIN, f"{t.what} {label}: cos {cos}"
        assert mab <= bar.abs_max, f"{t.what} {label}: max abs {mab} > {bar.abs_max} ({bar.name} bar)"
    want = int(torch.argmax(ref))
    if tok != want:
        top = float(ref[want])
        assert 0 <= tok < ref.numel(), f"{t.what} {label}: token {tok} outside the vocabulary"
        gap = top - float(ref[tok])
        t.literal &= gap <= tie_tolerance(top, 1)
        assert gap <= tie_tolerance(top, bar.tie_ulps), (
            f"{t.what} {label}: token {tok} (oracle logit {float(ref[tok])}) != oracle argmax {want} "
            f"(top {top}, gap {gap}, {bar.name} bar)")
        t.flips.append((label, round(gap / bf16_ulp(top), 2)))


def check_rows(t: Tally, ref: torch.Tensor, toks, got: torch.Tensor | None = None, labels=None, bar: Bar = LITERAL):
    for i in range(len(toks)):
        check_row(t, labels[i] if labels is not None else i, ref[i], int(toks[i]),
                  None if got is None else got[i], bar)
    return t


def exact_oracle(ew, shape, max_seq_len: int, num_layers: int | None = None, kv=None, cache_len: int = 0):
    """A fresh exact oracle on shared float64 weights ``ew``, RoPE tables long enough for
    ``max_seq_len``, optionally with injected cache contents ``kv = (k, v)`` of ``cache_len``."""
    from oracle.qwen3_exact import ExactOracle
    from qwen_megakernel.weights import rope_tables

    cos, sin = (None, None)
    if ew.cos.shape[0] < max_seq_len:
        cos, sin = rope_tables(max_seq_len, shape.head_dim, shape.rope_theta)
    orc = ExactOracle(ew, shape, max_seq_len=max_seq_len, num_layers=num_layers, cos=cos, sin=sin)
    if kv is not None:
        orc.load_kv(kv[0], kv[1], cache_len)
    return orc


def stream_rows(orc, prompt, generated):
    """Oracle logits of the rows that produced ``generated`` (a decoder's tokens after ``prompt``)."""
    seq = list(prompt) + list(generated[:-1])
    n0 = len(prompt) - 1
    return orc.forward(seq, emit=list(range(n0, len(seq))))


def decoder(weights, **kw):
    """A ``Decoder`` on ``weights`` (default max_seq_len 2048)."""
    from qwen_megakernel.model import Decoder

    return Decoder(weights=weights, verbose=False, max_seq_len=kw.pop("max_seq_len", 2048), **kw)


def with_rope(weights, max_seq_len, device):
    """The same weights with RoPE tables long enough for ``max_seq_len`` positions."""
    from qwen_megakernel.weights import rope_tables

    cos, sin = rope_tables(max_seq_len, 128, 1e6)
    w = dict(weights)
    w["cos_table"], w["sin_table"] = cos.to(device), sin.to(device)
    return w


def kernel_stream(dec, prompt, steps):
    """Feed ``prompt`` one ``step_logits`` at a time, then ``steps`` of the decoder's own tokens.

    Returns (inputs fed, tokens out, logits out [N, V] on the CPU); tokens[i] follows inputs[i].
    """
    feed = list(prompt)
    toks, lgs = [], []
    total = len(prompt) - 1 + steps
    for i in range(total):
        tok, lg = dec.step_logits(feed[i])
        toks.append(tok)
        lgs.append(lg.cpu())
        if i + 1 >= len(feed) and i + 1 < total:
            feed.append(tok)
    return feed[:total], toks, torch.stack(lgs)
