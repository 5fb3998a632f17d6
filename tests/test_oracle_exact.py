"""CPU tests that pin the exact-arithmetic oracle (oracle/qwen3_exact.py).

Pins, each chosen so that a plausible mistake fails one of them:
1. The single bf16 rounding against a brute force over the two bf16
   neighbours of each value, with values placed just off bf16 midpoints (where
   rounding through fp32 goes the wrong way).
2. Exact dot products against ``math.fsum`` on random bf16 rows.
3. Closed forms of attention (one position returns V; equal keys average V)
   and batched rows equal to one-token steps, bit for bit.
4. HF transformers' golden logits (tests/golden/*.npz, written by HF's Qwen3 in
   bf16 eager): the exact oracle sits within a few bf16 ulps of HF, which
   accumulates in fp32, and a planted mistake (a RoPE sign flip, a transposed
   GQA head mapping, a dropped residual) moves it far outside that bound.
5. The fp32-accumulating oracle (oracle/qwen3_ref.py) within the same bound.
"""

import math
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle.qwen3_exact as X
from oracle.qwen3_ref import OracleDecoder, greedy_stream
from qwen_megakernel.shapes import QWEN3_0_6B, Qwen3Shape
from qwen_megakernel.weights import make_kv_prefill, make_prompt, make_weights

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TINY = Qwen3Shape("tiny", 2, 256, 512, 4, 2, 64, 1000)
BF16 = torch.bfloat16


def _from_bits(a):
    return torch.from_numpy(np.asarray(a).astype(np.int16)).view(BF16).float()


def _bf16_neighbours(x: float):
    """The bf16 values just below and above x (x finite, not a bf16 value)."""
    b = torch.tensor([x], dtype=torch.float32).to(BF16)  # some nearby bf16 value
    bits = int(b.view(torch.int16).item()) & 0xFFFF
    cands = []
    for d in range(-2, 3):
        nb = (bits + d) & 0xFFFF
        v = torch.tensor([nb if nb < 0x8000 else nb - 0x10000], dtype=torch.int16).view(BF16).double().item()
        if math.isfinite(v):
            cands.append((v, nb))
    below = max((c for c in cands if c[0] <= x), key=lambda c: c[0])
    above = min((c for c in cands if c[0] >= x), key=lambda c: c[0])
    return below, above


def _round_brute(x: float) -> float:
    (lo, lob), (hi, hib) = _bf16_neighbours(x)
    if lo == hi:
        return lo
    dl, dh = Fraction(x) - Fraction(lo), Fraction(hi) - Fraction(x)
    if dl < dh:
        return lo
    if dh < dl:
        return hi
    return lo if (lob & 1) == 0 else hi


def test_round_bf16_single_rounding():
    g = torch.Generator().manual_seed(3)
    vals = (torch.randn(2000, generator=g, dtype=torch.float64) * 10).tolist()
    # values a hair off bf16 midpoints: fp32 rounds them onto the midpoint
    mids = []
    for v in (torch.randn(300, generator=g, dtype=torch.float64) * 5).tolist():
        b = torch.tensor([v]).to(BF16).double().item()
        ulp = 2.0 ** (math.floor(math.log2(abs(b))) - 7)
        m = b + ulp / 2
        mids += [m, m + ulp * 2.0 ** -30, m - ulp * 2.0 ** -30, -m, -(m + ulp * 2.0 ** -30)]
    xs = torch.tensor(vals + mids, dtype=torch.float64)
    got = X.round_bf16(xs).double().tolist()
    want = [_round_brute(x) for x in xs.tolist()]
    assert got == want
    # and the fix is needed: plain float64 -> bf16 through fp32 gets some of them wrong
    naive = xs.to(BF16).double().tolist()
    assert naive != want


def test_exact_linear_equals_fsum():
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(3, 1024, generator=g) * 3).to(BF16)
    w = (torch.randn(17, 1024, generator=g) * 0.05).to(BF16)
    got = X.exact_linear(x, w.double()).double()
    for i in range(3):
        for j in range(17):
            s = math.fsum(a * b for a, b in zip(x[i].double().tolist(), w[j].double().tolist()))
            assert got[i, j].item() == _round_brute(s) or s == got[i, j].item(), (i, j)


def test_rms_norm_closed_form():
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(4, 128, generator=g) * 2).to(BF16)
    w = (1 + 0.1 * torch.randn(128, generator=g)).to(BF16)
    got = X.rms_norm(x, w, 1e-6)
    for i in range(4):
        xs = x[i].double().tolist()
        r = 1.0 / math.sqrt(math.fsum(v * v for v in xs) / 128 + float(torch.tensor(1e-6, dtype=torch.float32)))
        h = torch.tensor([_round_brute(v * r) for v in xs], dtype=torch.float64).to(BF16)
        assert torch.equal(got[i], (w * h))
    # scale invariance (up to rounding of the scaled input: use a power of two)
    assert torch.equal(X.rms_norm(x * 4, w, 0.0), X.rms_norm(x, w, 0.0))


def _tiny_oracle(seed=0, **kw):
    w = make_weights(TINY, seed=seed, norm_std=0.1, max_seq_len=64)
    return w, X.ExactOracle(w, TINY, **kw)


def test_batched_rows_equal_single_steps():
    w, a = _tiny_oracle()
    _, b = _tiny_oracle()
    toks = make_prompt(12, TINY.vocab, seed=7)
    la = a.forward(toks)
    lb = torch.stack([b.step_logits(t) for t in toks])
    assert torch.equal(la, lb)
    assert torch.equal(a.k_cache, b.k_cache) and torch.equal(a.v_cache, b.v_cache)


def test_attention_closed_forms():
    w, o = _tiny_oracle()
    s = TINY
    g = torch.Generator().manual_seed(8)
    # one position: softmax is exactly 1, the output is V
    o.position = 0
    v = torch.randn(s.num_kv_heads, 1, s.head_dim, generator=g).to(BF16)
    o.k_cache[0, :, :1] = torch.randn(s.num_kv_heads, 1, s.head_dim, generator=g).to(BF16)
    o.v_cache[0, :, :1] = v
    q = torch.randn(s.num_q_heads, 1, s.head_dim, generator=g).to(BF16)
    out = o._attention(0, q, 0, 1).view(s.num_q_heads, s.head_dim)
    rep = s.num_q_heads // s.num_kv_heads
    for h in range(s.num_q_heads):
        assert torch.equal(out[h], v[h // rep, 0])  # q head h reads kv head h // rep (HF repeat_kv)
    # equal keys over 4 positions: probabilities are exactly 1/4, the output is bf16(mean V)
    k1 = torch.randn(s.num_kv_heads, 1, s.head_dim, generator=g).to(BF16)
    o.k_cache[0, :, :4] = k1.expand(-1, 4, -1)
    vv = torch.randn(s.num_kv_heads, 4, s.head_dim, generator=g).to(BF16)
    o.v_cache[0, :, :4] = vv
    out = o._attention(0, q, 3, 1).view(s.num_q_heads, s.head_dim)
    for h in range(s.num_q_heads):
        assert torch.equal(out[h], X.round_bf16(vv[h // rep].double().mean(0)))


def _hf_tiny_check(oracle_cls_patch=None):
    g = np.load(os.path.join(GOLDEN, "hf_tiny.npz"))
    w, o = _tiny_oracle()
    inputs = g["inputs"].tolist()
    lg = o.forward(inputs)
    ref = _from_bits(g["logits_bf16"])
    return lg, ref, g


def test_exact_oracle_matches_hf_tiny():
    lg, ref, g = _hf_tiny_check()
    d = (lg - ref).abs().max().item()
    # HF accumulates in fp32: a few bf16 ulps of the logits (|logit| < 1 here)
    assert d <= 0.02, d
    toks = torch.argmax(lg, -1).tolist()
    for i, (t, r) in enumerate(zip(toks, g["tokens"].tolist())):
        if t != r:
            v = torch.topk(ref[i], 2).values
            assert float(v[0] - v[1]) < 1e-2, (i, t, r)


@pytest.mark.parametrize("mistake", ["rope_sign", "gqa_map", "no_attn_scale"])
def test_planted_mistakes_fail_hf_tiny(monkeypatch, mistake):
    if mistake == "rope_sign":
        monkeypatch.setattr(X, "rotate_half", lambda x: torch.cat((x[..., x.shape[-1] // 2:],
                                                                    -x[..., : x.shape[-1] // 2]), dim=-1))
    elif mistake == "gqa_map":
        orig = X.ExactOracle._attention

        def swapped(self, li, q, p0, t):
            s = self.shape
            qq = q.contiguous().view(s.num_kv_heads, s.num_q_heads // s.num_kv_heads, t, s.head_dim).transpose(0, 1)
            return orig(self, li, qq.reshape(s.num_q_heads, t, s.head_dim), p0, t)
        monkeypatch.setattr(X.ExactOracle, "_attention", swapped)
    else:
        orig_init = X.ExactOracle.__init__

        def init(self, *a, **k):
            orig_init(self, *a, **k)
            self.scale = 1.0
        monkeypatch.setattr(X.ExactOracle, "__init__", init)
    lg, ref, _ = _hf_tiny_check()
    assert (lg - ref).abs().max().item() > 0.1


@pytest.fixture(scope="module")
def w06():
    return make_weights(QWEN3_0_6B, seed=0, max_seq_len=128)


@pytest.mark.slow
def test_exact_oracle_matches_hf_qwen3_0p6b(w06):
    g = np.load(os.path.join(GOLDEN, "hf_qwen3_0p6b.npz"))
    o = X.ExactOracle(w06, QWEN3_0_6B, max_seq_len=128)
    inputs = g["inputs"].tolist()
    lg = o.forward(inputs)
    first, last = _from_bits(g["logits_first_bf16"]), _from_bits(g["logits_last_bf16"])
    for a, b in ((lg[0], first), (lg[-1], last)):
        assert torch.nn.functional.cosine_similarity(a, b, dim=0) >= 0.9999
        assert (a - b).abs().max() <= 0.1
    top_ref = _from_bits(g["top16_bf16"])
    idx = torch.from_numpy(g["top16_idx"])
    worst = (lg.gather(1, idx) - top_ref).abs().max().item()
    assert worst <= 0.05, worst  # the top-16 logits of every step within ~3 bf16 ulps of HF's
    # HF's token differs only where the exact logits put its token within one bf16 ulp of the top
    # (here at most a one-ulp gap, or an exact tie that the first index breaks)
    for i, (t, r) in enumerate(zip(torch.argmax(lg, -1).tolist(), g["tokens"].tolist())):
        if t != r:
            top = float(lg[i].max())
            assert top - float(lg[i, r]) <= 2.0 ** (math.floor(math.log2(top)) - 7), (i, t, r)


def test_exact_oracle_near_fp32_oracle():
    """The fp32-accumulating restatement and the exact one agree within a few bf16 ulps, with a
    long-context cache (attention over 200 N(0,1) positions) on the tiny shape."""
    w = make_weights(TINY, seed=1, norm_std=0.1, max_seq_len=256)
    k, v = make_kv_prefill(TINY, 200, seed=2, max_seq_len=256)
    a = OracleDecoder(w, TINY)
    a.load_kv(k, v, 200)
    b = X.ExactOracle(w, TINY)
    b.load_kv(k, v, 200)
    res = greedy_stream(a, [5, 6, 7], 8, record_logits=True)
    lb = b.forward(res["inputs"])
    assert (res["logits"] - lb).abs().max().item() <= 0.03


@pytest.mark.slow
def test_reference_path_itself_misses_the_literal_bar_at_long_context(w06):
    """The reference's PyTorch bf16 path (HF semantics, fp32 accumulation: oracle/qwen3_ref.py)
    against the exact centre on identical inputs: Qwen3-0.6B, 28 layers, a seeded N(0, 1) cache
    of 1500 positions, 12 steps, each run over the exact oracle's own cache.  It is more than
    0.1 away at some step (0.110 on the CPU that wrote this; Qwen3-1.7B after a 24-token prompt
    reaches 0.117 the same way), so the literal 0.1 bar cannot hold there for an fp32
    implementation, and within 0.2 (the GPU tests' bar for these workloads, tests/parity.py)."""
    from qwen_megakernel.weights import rope_tables

    c0 = 1500
    cos, sin = rope_tables(c0 + 16, 128, 1e6)
    w = dict(w06)
    w["cos_table"], w["sin_table"] = cos, sin
    k, v = make_kv_prefill(QWEN3_0_6B, c0, seed=2)
    toks = [11, 22, 5, 6, 7, 8, 9, 10, 12, 13, 14, 15]
    ex = X.ExactOracle(w, QWEN3_0_6B, max_seq_len=c0 + 16)
    ex.load_kv(k, v, c0)
    lx = ex.forward(toks)
    hf = OracleDecoder(w, QWEN3_0_6B, max_seq_len=c0 + 16)
    d = []
    for i, t in enumerate(toks):
        p = c0 + i
        hf.k_cache[:, :, :p] = ex.k_cache[:, :, :p]
        hf.v_cache[:, :, :p] = ex.v_cache[:, :, :p]
        hf.position = p
        d.append((hf.step_logits(t) - lx[i]).abs().max().item())
    print("HF-semantics fp32 vs exact on identical inputs, per step:", [round(x, 4) for x in d])
    assert max(d) > 0.1
    assert max(d) <= 0.2
