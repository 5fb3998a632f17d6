"""CPU tests that pin the fp32 restatement (oracle/qwen3_fp32.c, oracle/qwen3_fp32.py).

Pins, each chosen so that a plausible mistake fails one of them:
1. Each summation order against a sum built by hand in numpy float32 adds, on
   inputs whose result depends on the order (cancellation), so a tree built
   the wrong way round or a missed term fails.
2. HF transformers' golden logits (tests/golden/*.npz, HF Qwen3 bf16 eager,
   which accumulates in fp32): every order within a few bf16 ulps, and planted
   mistakes (a RoPE sign, a transposed GQA head mapping, a missing attention
   scale), made through the inputs, far outside that.
3. The exact oracle (oracle/qwen3_exact.py): within fp32 noise, tiny shape
   with a long N(0,1) cache.
4. Rows over a given cache equal to ordinary rows on the restatement's own
   cache, bit for bit, and the K/V rows it reports equal to the ones it wrote.
5. The per-step bound built from it (tests/parity.py) admits the reference's
   own fp32 path (oracle/qwen3_ref.py, HF semantics) on identical inputs, at
   1500 positions over 28 layers, where HF is more than 0.1 from the centre.
"""

import math
import os

import numpy as np
import pytest
import torch

import oracle.qwen3_exact as X
from oracle.qwen3_fp32 import ORDERS, Fp32Oracle, tree_sum
from qwen_megakernel.shapes import QWEN3_0_6B, Qwen3Shape
from qwen_megakernel.weights import make_kv_prefill, make_prompt, make_weights

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TINY = Qwen3Shape("tiny", 2, 256, 512, 4, 2, 64, 1000)
BF16 = torch.bfloat16


def _from_bits(a):
    return torch.from_numpy(np.asarray(a).astype(np.int16)).view(BF16).float()


def _hand_sum(x: np.ndarray, order: int) -> np.float32:
    x = x.astype(np.float32)
    n = x.size
    if order == 1:
        a = np.float32(0)
        for v in x:
            a = np.float32(a + v)
        return a
    if order == 3:
        a = np.float32(0)
        for v in x[::-1]:
            a = np.float32(a + v)
        return a
    if order == 2:
        lanes = [np.float32(0)] * 8
        for i, v in enumerate(x):
            lanes[i % 8] = np.float32(lanes[i % 8] + v)
        x, n = np.array(lanes, dtype=np.float32), 8
    p = 1
    while p < n:
        p *= 2
    buf = np.zeros(p, dtype=np.float32)
    buf[:n] = x
    while p > 1:
        h = p // 2
        buf[:h] = buf[:h] + buf[h:p]
        p = h
    return buf[0]


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("n", [1, 7, 8, 100, 1024, 1500])
def test_summation_orders_match_hand_built(order, n):
    g = np.random.default_rng(n * 10 + order)
    # large terms that cancel, so that the result depends on the order
    x = (g.standard_normal(n) * 10.0 ** g.integers(-3, 6, n)).astype(np.float32)
    got = tree_sum(torch.from_numpy(x), order)
    want = float(_hand_sum(x, order))
    assert got == want, (order, n, got, want)


def test_summation_orders_differ():
    """The four orders are four different sums (otherwise the envelope measures one order)."""
    g = np.random.default_rng(1)
    x = (g.standard_normal(1000) * 10.0 ** g.integers(-3, 6, 1000)).astype(np.float32)
    sums = {tree_sum(torch.from_numpy(x), o) for o in ORDERS}
    assert len(sums) == 4


def _tiny(seed=0):
    return make_weights(TINY, seed=seed, norm_std=0.1, max_seq_len=64)


def _hf_tiny():
    g = np.load(os.path.join(GOLDEN, "hf_tiny.npz"))
    return g["inputs"].tolist(), _from_bits(g["logits_bf16"]), g["tokens"].tolist()


@pytest.mark.parametrize("order", ORDERS)
def test_fp32_restatement_matches_hf_tiny(order):
    inputs, ref, toks = _hf_tiny()
    lg = Fp32Oracle(_tiny(), TINY).forward(inputs, order=order)
    d = (lg - ref).abs().max().item()
    assert d <= 0.02, d  # a few bf16 ulps of logits below 1
    for i, (t, r) in enumerate(zip(torch.argmax(lg, -1).tolist(), toks)):
        if t != r:
            v = torch.topk(ref[i], 2).values
            assert float(v[0] - v[1]) < 1e-2, (i, t, r)


def _planted(mistake):
    """Tiny weights with a mistake made through the inputs: what the restatement would compute with
    that mistake in its code."""
    w = _tiny()
    s = TINY
    if mistake == "rope_sign":  # x*cos - rotate_half(x)*sin
        w["sin_table"] = -w["sin_table"]
    elif mistake == "gqa_map":  # q head h read KV head h % NKV instead of h // (NQ / NKV)
        rep = s.num_q_heads // s.num_kv_heads
        lw = list(w["layer_weights"])
        for li in range(s.num_layers):
            wq = lw[11 * li + 1].view(s.num_kv_heads, rep, s.head_dim, s.hidden)
            lw[11 * li + 1] = wq.transpose(0, 1).reshape(s.num_q_heads * s.head_dim, s.hidden).contiguous()
            wo = lw[11 * li + 6].view(s.hidden, s.num_kv_heads, rep, s.head_dim)
            lw[11 * li + 6] = wo.transpose(1, 2).reshape(s.hidden, s.num_q_heads * s.head_dim).contiguous()
        w["layer_weights"] = lw
    return w


@pytest.mark.parametrize("mistake", ["rope_sign", "gqa_map", "no_attn_scale"])
def test_planted_mistakes_fail_hf_tiny(mistake):
    inputs, ref, _ = _hf_tiny()
    o = Fp32Oracle(_planted(mistake), TINY)
    if mistake == "no_attn_scale":
        o.scale = 1.0
    lg = o.forward(inputs)
    assert (lg - ref).abs().max().item() > 0.1


def test_gqa_planted_mistake_is_a_different_mapping():
    """The GQA plant moves q heads between KV groups: the exact oracle with the same planted weights
    disagrees with the unplanted one (so the plant is not a relabelling the model undoes)."""
    inputs, _, _ = _hf_tiny()
    a = X.ExactOracle(_tiny(), TINY).forward(inputs)
    b = X.ExactOracle(_planted("gqa_map"), TINY).forward(inputs)
    assert (a - b).abs().max().item() > 0.1


@pytest.mark.slow
@pytest.mark.parametrize("order", ORDERS)
def test_fp32_restatement_matches_hf_qwen3_0p6b(order):
    """HF's 79 steps on its own cache (16-token prompt + 64 greedy steps): the first and last full
    logits rows and every step's top-16 logits within a few bf16 ulps.  (The sequential orders sit
    at cosine 0.99984-0.99988 on the first row, the pairwise one and the exact oracle at 0.99994.)"""
    g = np.load(os.path.join(GOLDEN, "hf_qwen3_0p6b.npz"))
    w = make_weights(QWEN3_0_6B, seed=0, max_seq_len=128)
    lg = Fp32Oracle(w, QWEN3_0_6B, max_seq_len=128).forward(g["inputs"].tolist(), order=order)
    first, last = _from_bits(g["logits_first_bf16"]), _from_bits(g["logits_last_bf16"])
    for a, b in ((lg[0], first), (lg[-1], last)):
        assert torch.nn.functional.cosine_similarity(a, b, dim=0) >= 0.9998
        assert (a - b).abs().max() <= 0.1
    worst = (lg.gather(1, torch.from_numpy(g["top16_idx"])) - _from_bits(g["top16_bf16"])).abs().max().item()
    assert worst <= 0.05, worst


@pytest.mark.parametrize("order", ORDERS)
def test_fp32_restatement_near_exact_oracle_long_cache(order):
    """Attention over 200 N(0,1) positions on the tiny shape: within a few bf16 ulps of the exact
    oracle on the same inputs."""
    w = make_weights(TINY, seed=1, norm_std=0.1, max_seq_len=256)
    k, v = make_kv_prefill(TINY, 200, seed=2, max_seq_len=256)
    toks = make_prompt(10, TINY.vocab, seed=3)
    ex = X.ExactOracle(w, TINY)
    ex.load_kv(k, v, 200)
    lx = ex.forward(toks)
    f = Fp32Oracle(w, TINY)
    f.load_kv(k, v, 200)
    lf = f.forward(toks, order=order)
    assert (lf - lx).abs().max().item() <= 0.03
    # the cache rows it wrote are the exact oracle's up to rounding
    assert (f.k_cache[:, :, 200:210].float() - ex.k_cache[:, :, 200:210].float()).abs().max().item() <= 0.0625


@pytest.mark.parametrize("order", ORDERS)
def test_given_cache_rows_equal_own_rows(order):
    w = _tiny(seed=2)
    toks = make_prompt(12, TINY.vocab, seed=4)
    a = Fp32Oracle(w, TINY)
    la = a.forward(toks, order=order)
    b = Fp32Oracle(w, TINY)
    b.k_cache.copy_(a.k_cache)
    b.v_cache.copy_(a.v_cache)
    lb = b.forward(toks, given_cache=True, order=order, emit=[0, 5, 11])
    assert torch.equal(lb, la[[0, 5, 11]])
    assert torch.equal(b.own_k, a.k_cache[:, :, :12]) and torch.equal(b.own_v, a.v_cache[:, :, :12])
    # and one token at a time equals the batched rows
    c = Fp32Oracle(w, TINY)
    lc = torch.stack([c.forward([t], order=order)[0] for t in toks])
    assert torch.equal(lc, la)


def test_rejects_bad_arguments():
    o = Fp32Oracle(_tiny(), TINY)
    with pytest.raises(ValueError):
        o.forward([TINY.vocab])
    with pytest.raises(ValueError):
        o.forward([1], order=4)
    o.position = 64
    with pytest.raises(ValueError):
        o.forward([1])


@pytest.mark.slow
def test_bound_admits_the_reference_path_at_long_context():
    """The per-step bound of the GPU tests (tests/parity.py, ``envelope`` and ``check_row`` with
    it), applied to the reference's own fp32 path (HF semantics, oracle/qwen3_ref.py) on identical
    inputs: Qwen3-0.6B, 28 layers, a seeded N(0, 1) cache of 1500 positions, 12 steps, each over the
    exact oracle's cache.  HF is more than 0.1 from the centre there, and within the bound at every
    step; a single summation order does not bound it (HF's error exceeds the pairwise tree's by
    more than 1.25 times at some step), which is why the bound takes the largest over four."""
    from oracle.qwen3_ref import OracleDecoder
    from parity import ENVELOPE, Tally, check_row, envelope
    from qwen_megakernel.weights import rope_tables

    c0 = 1500
    w = make_weights(QWEN3_0_6B, seed=0, max_seq_len=128)
    cos, sin = rope_tables(c0 + 16, 128, 1e6)
    w["cos_table"], w["sin_table"] = cos, sin
    k, v = make_kv_prefill(QWEN3_0_6B, c0, seed=2)
    toks = [11, 22, 5, 6, 7, 8, 9, 10, 12, 13, 14, 15]
    ex = X.ExactOracle(w, QWEN3_0_6B, max_seq_len=c0 + 16)
    ex.load_kv(k, v, c0)
    lx = ex.forward(toks)
    f = Fp32Oracle(w, QWEN3_0_6B, max_seq_len=c0 + 16)
    hf = OracleDecoder(w, QWEN3_0_6B, max_seq_len=c0 + 16)
    t = Tally("HF fp32 path, 1500 positions")
    hf_err, tree_err = [], []
    for i, tok in enumerate(toks):
        p = c0 + i
        hf.k_cache[:, :, :p] = ex.k_cache[:, :, :p]
        hf.v_cache[:, :, :p] = ex.v_cache[:, :, :p]
        hf.position = p
        lh = hf.step_logits(tok)
        env = envelope(f, ex.k_cache, ex.v_cache, p, [tok], lx[i:i + 1])[0]
        check_row(t, i, lx[i], int(torch.argmax(lh)), lh, bar=ENVELOPE, env=env)
        hf_err.append((lh - lx[i]).abs().max().item())
        tree_err.append(env.errs[0])
    print(t, [round(a / b, 2) for a, b in zip(hf_err, tree_err)])
    assert max(hf_err) > 0.1
    assert max(a / b for a, b in zip(hf_err, tree_err)) > 1.2
