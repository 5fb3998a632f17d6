"""CPU tests that pin the oracle (oracle/qwen3_ref.py).

Three kinds of pin:
1. Golden vectors written by HF transformers' Qwen3 (tests/golden/make_hf_golden.py):
   the oracle must reproduce HF's bf16 logits -- bit for bit on the CPU that
   wrote them, within bf16 rounding elsewhere.
2. Closed forms and invariants of each op, chosen so that a plausible mistake
   (a dropped norm weight, a wrong rotate-half sign or pairing, a transposed GQA
   mapping, a last-index argmax) fails.
3. Brute force in float64 on tiny inputs.
"""

import math
import os

import numpy as np
import pytest
import torch

from oracle.qwen3_ref import OracleDecoder, apply_rope, attention, greedy_stream, rms_norm, rotate_half, top2_gap
from qwen_megakernel.shapes import QWEN3_0_6B, Qwen3Shape
from qwen_megakernel.weights import make_kv_prefill, make_prompt, make_weights, rope_tables

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TINY = Qwen3Shape("tiny", 2, 256, 512, 4, 2, 64, 1000)
BF16 = torch.bfloat16


def _cpu_signature():
    import importlib.util
    spec = importlib.util.spec_from_file_location("mkg", os.path.join(GOLDEN, "make_hf_golden.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.cpu_signature()


def _from_bits(a):
    return torch.from_numpy(np.asarray(a).astype(np.int16)).view(BF16).float()


@pytest.fixture(scope="module")
def same_cpu():
    g = np.load(os.path.join(GOLDEN, "hf_tiny.npz"))
    return str(g["cpu"]) == _cpu_signature()


# ---------------------------------------------------------------- golden: HF

def test_oracle_matches_hf_tiny(same_cpu):
    g = np.load(os.path.join(GOLDEN, "hf_tiny.npz"))
    w = make_weights(TINY, seed=0, norm_std=0.1, max_seq_len=64)
    dec = OracleDecoder(w, TINY)
    prompt = g["inputs"][: int(g["prompt_len"])].tolist()
    res = greedy_stream(dec, prompt, 16, record_logits=True)
    assert res["inputs"] == g["inputs"].tolist()
    assert res["tokens"] == g["tokens"].tolist()
    ref = _from_bits(g["logits_bf16"])
    diff = (res["logits"] - ref).abs().max().item()
    if same_cpu:
        assert diff == 0.0, diff
    else:
        assert diff <= 0.05, diff


@pytest.fixture(scope="module")
def w06():
    return make_weights(QWEN3_0_6B, seed=0, max_seq_len=128)


def test_weight_fingerprint(w06):
    g = np.load(os.path.join(GOLDEN, "hf_qwen3_0p6b.npz"))
    fp = [w06["embed_weight"].double().sum(), w06["embed_weight"][12345].double().sum()]
    fp += [t.double().sum() for t in w06["layer_weights"]]
    fp.append(w06["final_norm_weight"].double().sum())
    np.testing.assert_array_equal(torch.stack(fp).numpy(), g["weight_fingerprint"])
    assert w06["lm_head_weight"] is w06["embed_weight"]  # tied (qwen_megakernel/model.py:87)


def test_prompt_is_seeded():
    g = np.load(os.path.join(GOLDEN, "hf_qwen3_0p6b.npz"))
    assert make_prompt(16, QWEN3_0_6B.vocab, seed=1) == g["prompt"].tolist()


@pytest.mark.slow
def test_oracle_matches_hf_qwen3_0p6b(w06, same_cpu):
    g = np.load(os.path.join(GOLDEN, "hf_qwen3_0p6b.npz"))
    dec = OracleDecoder(w06, QWEN3_0_6B)
    res = greedy_stream(dec, g["prompt"].tolist(), 64, record_logits=True)
    lg = res["logits"]
    assert res["inputs"] == g["inputs"].tolist()
    top = torch.topk(lg, 16, dim=-1)
    first = _from_bits(g["logits_first_bf16"])
    last = _from_bits(g["logits_last_bf16"])
    if same_cpu:
        assert res["tokens"] == g["tokens"].tolist()
        np.testing.assert_array_equal(top.indices.numpy(), g["top16_idx"])
        np.testing.assert_array_equal(top.values.numpy(), _from_bits(g["top16_bf16"]).numpy())
        assert torch.equal(lg[0], first) and torch.equal(lg[-1], last)
    else:
        # different CPU kernels: same tolerance the GPU parity tests use
        for a, b in ((lg[0], first), (lg[-1], last)):
            assert torch.nn.functional.cosine_similarity(a, b, dim=0) >= 0.999
            assert (a - b).abs().max() <= 0.1
        gaps = g["gaps"]
        for i, (t, r) in enumerate(zip(res["tokens"], g["tokens"].tolist())):
            if t != r:
                assert gaps[i] < 1e-2, (i, t, r, gaps[i])
                break


def test_rope_table_matches_hf_rotary():
    g = np.load(os.path.join(GOLDEN, "hf_rope.npz"))
    pos = g["positions"]
    cos, sin = rope_tables(int(pos.max()) + 1, 128, 1e6)
    np.testing.assert_array_equal(cos[pos].float().numpy(), _from_bits(g["cos_bf16"]).numpy())
    np.testing.assert_array_equal(sin[pos].float().numpy(), _from_bits(g["sin_bf16"]).numpy())


def test_rope_theta_is_qwen3_not_reference_default():
    # The reference hard-codes theta=10000 (qwen_megakernel/model.py:54-56); Qwen3 uses 1e6.
    cos6, _ = rope_tables(8, 128, 1e6)
    cos4, _ = rope_tables(8, 128, 1e4)
    assert not torch.equal(cos6, cos4)
    # highest-frequency pair is theta-independent: cos(p * 1)
    assert torch.equal(cos6[:, 0], cos4[:, 0])


# ------------------------------------------------------- closed forms: ops

def test_rmsnorm_closed_form_and_weight():
    torch.manual_seed(0)
    x = torch.randn(1024).to(BF16)
    w = (1 + 0.1 * torch.randn(1024)).to(BF16)
    ones = torch.ones(1024, dtype=BF16)
    y1 = rms_norm(x, ones, 1e-6).float()
    # unit weights: output RMS is 1 up to bf16 rounding
    assert abs(y1.pow(2).mean().sqrt().item() - 1.0) < 4e-3
    # fp64 brute force
    xd = x.double()
    ref = (xd / torch.sqrt((xd * xd).mean() + 1e-6)).float().to(BF16).float()
    assert torch.equal(y1, ref)
    # the weight multiplies elementwise after the bf16 rounding
    yw = rms_norm(x, w, 1e-6).float()
    assert torch.equal(yw, (w.float() * y1).to(BF16).float())
    assert not torch.equal(yw, y1)
    # scale invariance (power-of-two scale keeps bf16 values exact)
    assert torch.equal(rms_norm((x.float() * 4).to(BF16), ones, 1e-6), rms_norm(x, ones, 1e-6))


def test_rope_identity_at_position_zero_and_pairing():
    cos, sin = rope_tables(16, 128, 1e6)
    torch.manual_seed(1)
    x = torch.randn(1, 16, 1, 128).to(BF16)
    assert torch.equal(apply_rope(x, cos[0], sin[0]), x)  # p = 0: cos 1, sin 0
    # rotate-half pairs d with d+64 and negates the second half
    r = rotate_half(x)
    assert torch.equal(r[..., :64], -x[..., 64:]) and torch.equal(r[..., 64:], x[..., :64])
    # explicit pair formula in fp64 vs the op (differs only by bf16 roundings)
    p = 7
    y = apply_rope(x, cos[p], sin[p]).double()
    c, s = cos[p].double(), sin[p].double()
    xd = x.double()
    ref = torch.cat([xd[..., :64] * c[:64] - xd[..., 64:] * s[:64], xd[..., 64:] * c[64:] + xd[..., :64] * s[64:]], -1)
    assert (y - ref).abs().max() < 0.05
    # pair norm preserved (rotation) up to bf16 rounding
    n0 = xd[..., :64] ** 2 + xd[..., 64:] ** 2
    n1 = y[..., :64] ** 2 + y[..., 64:] ** 2
    assert ((n1 - n0).abs() / (n0 + 1e-3)).max() < 0.03


def test_attention_single_position_returns_v():
    torch.manual_seed(2)
    q = torch.randn(1, 16, 1, 128).to(BF16)
    k = torch.randn(1, 8, 1, 128).to(BF16)
    v = torch.randn(1, 8, 1, 128).to(BF16)
    out = attention(q, k, v, 128 ** -0.5)
    # GQA: q head h reads kv head h // 2
    for h in range(16):
        assert torch.equal(out[0, h, 0], v[0, h // 2, 0])


def test_attention_equal_keys_give_mean_of_v_and_brute_force():
    torch.manual_seed(3)
    q = torch.randn(1, 4, 1, 64).to(BF16)
    k1 = torch.randn(1, 2, 1, 64).to(BF16)
    k = k1.expand(1, 2, 8, 64).contiguous()
    v = torch.randn(1, 2, 8, 64).to(BF16)
    out = attention(q, k, v, 64 ** -0.5).double()
    for h in range(4):
        mean = v[0, h // 2].double().mean(0)
        assert (out[0, h, 0] - mean).abs().max() < 0.02
    # fp64 brute force on random keys (tolerance covers bf16 roundings)
    k = torch.randn(1, 2, 8, 64).to(BF16)
    out = attention(q, k, v, 64 ** -0.5).double()
    for h in range(4):
        s = (k[0, h // 2].double() @ q[0, h, 0].double()) * 64 ** -0.5
        pr = torch.softmax(s, 0)
        assert abs(pr.sum().item() - 1) < 1e-12
        ref = pr @ v[0, h // 2].double()
        assert (out[0, h, 0] - ref).abs().max() < 0.03


def test_silu_mul_closed_form():
    x = torch.tensor([-3.0, -1.0, 0.0, 0.5, 2.0]).to(BF16)
    got = torch.nn.functional.silu(x).float()
    ref = (x.double() / (1 + torch.exp(-x.double()))).float().to(BF16).float()
    assert torch.equal(got, ref)


def test_argmax_takes_first_index_on_ties():
    lg = torch.tensor([0.5, 2.0, -1.0, 2.0, 2.0])
    assert int(torch.argmax(lg)) == 1
    assert top2_gap(lg) == 0.0


# ------------------------------------------------- decoder state behaviour

def test_position_advances_and_cache_written():
    w = make_weights(TINY, seed=0, norm_std=0.1, max_seq_len=16)
    dec = OracleDecoder(w, TINY)
    assert dec.position == 0
    dec.step(5)
    dec.step(6)
    assert dec.position == 2
    assert dec.k_cache[:, :, :2].abs().sum() > 0 and dec.k_cache[:, :, 2:].abs().sum() == 0
    dec.reset()
    assert dec.position == 0 and dec.k_cache.abs().sum() == 0


def test_position_bound_is_enforced():
    w = make_weights(TINY, seed=0, max_seq_len=4)
    dec = OracleDecoder(w, TINY)
    for t in range(4):
        dec.step(t)
    with pytest.raises(ValueError):
        dec.step(1)


def test_kv_injection_equals_decoding_the_same_cache():
    """Continuing from an injected cache equals continuing after real decode steps."""
    w = make_weights(TINY, seed=0, norm_std=0.1, max_seq_len=32)
    a = OracleDecoder(w, TINY)
    for t in (3, 14, 15):
        a.step(t)
    b = OracleDecoder(w, TINY)
    b.load_kv(a.k_cache.clone(), a.v_cache.clone(), 3)
    assert torch.equal(a.step_logits(92), b.step_logits(92))


def test_kv_prefill_is_seeded():
    k1, v1 = make_kv_prefill(TINY, 8, seed=2, max_seq_len=16)
    k2, v2 = make_kv_prefill(TINY, 8, seed=2, max_seq_len=16)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    assert k1[:, :, 8:].abs().sum() == 0 and not torch.equal(k1, v1)
    assert abs(k1[:, :, :8].float().std().item() - 1.0) < 0.1
