"""GPU parity tests of the batched forward (prompt prefill and batched decode).

The batched path (qwen_megakernel_amd/csrc/qmk_batch.hip, MFMA GEMMs) is checked
against the CPU oracle fed one token at a time: HF's eager prefill computes
each row exactly as a decode step at that position does (causal mask, same
per-row linears), so the oracle's per-step logits are the expected logits of
every prefilled row.  Same bar as the decode kernel: cosine >= 0.999 and max
abs <= 0.1 per row, greedy tokens identical except at near-ties (gap < 1e-2 or
one bf16 ulp), with one addition: a token may also differ where the oracle's
top-2 gap is two ulps and our logits of both tokens are each within one ulp of
the oracle's.  Two bf16 logits two ulps apart become equal when each rounds
one ulp toward the other, which fp32 summation order alone does (the decode
kernel and this path differ from the oracle by 0.04-0.07 max abs over the
vocabulary); the check holds the two tokens themselves to one ulp.
"""

import pytest
import torch

from test_gpu_decode import (ABS_MAX, COS_MIN, _decoder, _with_rope, bf16_ulp, is_tie,  # noqa: F401
                             shape, weights_cpu, weights_gpu)

pytestmark = pytest.mark.gpu

V = 151936


def _check_step(i, g, r, tok, ref_tok, gap):
    """Cosine and max-abs bar on the logits; greedy token equal up to near-ties (module docstring)."""
    cos = torch.nn.functional.cosine_similarity(g.double(), r.double(), dim=0).item()
    mab = (g - r).abs().max().item()
    assert cos >= COS_MIN, f"row {i}: cos {cos}"
    assert mab <= ABS_MAX, f"row {i}: max abs {mab}"
    if tok != ref_tok:
        top = float(r.max())
        u = bf16_ulp(top)
        two_ulp = (gap <= 2 * u and abs(float(g[tok] - r[tok])) <= u
                   and abs(float(g[ref_tok] - r[ref_tok])) <= u)
        assert is_tie(gap, top) or two_ulp, (
            f"row {i}: token {tok} != {ref_tok} with top-2 gap {gap} (top {top}); ours "
            f"{float(g[tok])}/{float(g[ref_tok])}, oracle {float(r[tok])}/{float(r[ref_tok])}")
    return cos, mab


def _i32(values):
    return torch.tensor([int(v) for v in values], dtype=torch.int32, device="cuda")


def _oracle_feed(orc, ids):
    """Feed ``ids`` to the oracle; per-token logits, greedy tokens and top-2 gaps."""
    from oracle.qwen3_ref import top2_gap

    logits, tokens, gaps = [], [], []
    for t in ids:
        lg = orc.step_logits(int(t))
        logits.append(lg)
        tokens.append(int(torch.argmax(lg)))
        gaps.append(top2_gap(lg))
    return dict(logits=logits, tokens=tokens, gaps=gaps)


def _forward_rows(fwd, ids, start, k_cache, v_cache, seq=0):
    """All rows of a one-sequence forward at positions start..; returns (tokens, logits [T, V])."""
    n = len(ids)
    out = torch.empty(n, dtype=torch.int32, device="cuda")
    logits = torch.empty(n, V, dtype=torch.float32, device="cuda")
    fwd(_i32(ids), torch.full((n,), seq, dtype=torch.int32, device="cuda"),
        torch.arange(start, start + n, dtype=torch.int32, device="cuda"),
        torch.arange(n, dtype=torch.int32, device="cuda"), out, logits, k_cache, v_cache, start + n)
    return out.cpu().tolist(), logits.cpu()


def _check_rows(toks, logits, ref, offset=0):
    worst = (1.0, 0.0)
    for i in range(len(toks)):
        c, m = _check_step(offset + i, logits[i], ref["logits"][offset + i], toks[i], ref["tokens"][offset + i],
                           ref["gaps"][offset + i])
        worst = (min(worst[0], c), max(worst[1], m))
    return worst


def test_mfma_operand_layout():
    """One v_mfma_f32_16x16x32_bf16 with the GEMM's lane layout equals A @ B^T."""
    from qwen_megakernel_amd.build import get_extension

    ops = get_extension()
    g = torch.Generator().manual_seed(0)
    a = torch.randn(16, 32, generator=g).to(torch.bfloat16)
    b = torch.randn(16, 32, generator=g).to(torch.bfloat16)
    c = torch.empty(16, 16, dtype=torch.float32, device="cuda")
    ops.selftest_mfma(a.cuda(), b.cuda(), c)
    ref = a.double() @ b.double().t()
    err = (c.cpu().double() - ref).abs().max().item()
    assert err <= 1e-4, f"MFMA layout/result mismatch: max abs {err}"


@pytest.mark.parametrize("n", [12, 40], ids=["12tok-split-attention", "40tok-rowwise-attention"])
def test_prefill_all_rows_match_oracle(shape, weights_cpu, weights_gpu, n):
    """Every row of a 28-layer prefill against the oracle's step at that position; K/V written alike."""
    from oracle.qwen3_ref import OracleDecoder
    from qwen_megakernel_amd.weights import make_prompt

    ids = make_prompt(n, shape.vocab, seed=3)
    orc = OracleDecoder(weights_cpu, shape, max_seq_len=2048)
    ref = _oracle_feed(orc, ids)
    dec = _decoder(weights_gpu)
    toks, logits = _forward_rows(dec._forward, ids, 0, dec._k_cache, dec._v_cache)
    worst = _check_rows(toks, logits, ref)
    for name, got, exp in (("K", dec._k_cache, orc.k_cache), ("V", dec._v_cache, orc.v_cache)):
        d = (got[:1, :, :n].float().cpu() - exp[:1, :, :n].float()).abs().max().item()
        assert d <= 0.05, f"layer-0 {name} cache rows differ by {d}"
        cos = torch.nn.functional.cosine_similarity(got[:, :, :n].float().cpu().flatten().double(),
                                                    exp[:, :, :n].float().flatten().double(), dim=0).item()
        assert cos >= 0.999, f"{name} cache cosine {cos}"
    print(f"prefill {n} rows: worst cos {worst[0]:.6f}, max abs {worst[1]:.4f}")


def test_prefill_then_decode_kernel(shape, weights_cpu, weights_gpu):
    """Decoder.prefill writes a cache the decode megakernel continues from."""
    from oracle.qwen3_ref import OracleDecoder, greedy_stream
    from qwen_megakernel_amd.weights import make_prompt

    prompt = make_prompt(24, shape.vocab, seed=5)
    ref = greedy_stream(OracleDecoder(weights_cpu, shape, max_seq_len=2048), prompt, 12, record_logits=True)
    dec = _decoder(weights_gpu)
    tok, lg = dec.prefill(prompt, return_logits=True)
    n0 = len(prompt) - 1
    _check_step(n0, lg.cpu(), ref["logits"][n0], tok, ref["tokens"][n0], ref["gaps"][n0])
    assert dec.position == len(prompt)
    for i in range(len(prompt), len(ref["inputs"])):
        tok, lg = dec.step_logits(ref["inputs"][i])
        _check_step(i, lg.cpu(), ref["logits"][i], tok, ref["tokens"][i], ref["gaps"][i])


def _stream_matches(out, ref, n0, what):
    """A free-running greedy stream equals the oracle's until its first near-tie (gap < 1e-2 or at
    most two ulps; there the streams may part, and nothing after it is compared)."""
    for i, got in enumerate(out):
        want = ref["tokens"][n0 + i]
        if got != want:
            gap, top = ref["gaps"][n0 + i], float(ref["logits"][n0 + i].max())
            assert is_tie(gap, top) or gap <= 2 * bf16_ulp(top), f"{what} step {i}: {got} != {want} (gap {gap})"
            return i
    return len(out)


def test_generate_with_prefill_matches_oracle_stream(shape, weights_cpu, weights_gpu):
    """generate() feeds the prompt through prefill by default (use_prefill=False: one decode step per
    prompt token, as the reference); both streams equal the oracle's up to its first near-tie."""
    from oracle.qwen3_ref import OracleDecoder, greedy_stream
    from qwen_megakernel_amd.weights import make_prompt

    prompt = make_prompt(20, V, seed=6)
    ref = greedy_stream(OracleDecoder(weights_cpu, shape, max_seq_len=2048), prompt, 24, record_logits=True)
    for use_prefill in (True, False):
        out = _decoder(weights_gpu, use_prefill=use_prefill).generate(prompt, 24)
        n = _stream_matches(out, ref, len(prompt) - 1, f"use_prefill={use_prefill}")
        print(f"use_prefill={use_prefill}: {n} of 24 tokens compared")


@pytest.fixture(scope="module")
def batch_case(shape, weights_cpu):
    """Four sequences with prompts of different lengths; oracle logits for the prompts and 10 more steps."""
    from oracle.qwen3_ref import OracleDecoder
    from qwen_megakernel_amd.weights import make_prompt

    lens = [5, 17, 33, 9]
    prompts = [make_prompt(n, shape.vocab, seed=10 + b) for b, n in enumerate(lens)]
    refs = []
    for p in prompts:
        orc = OracleDecoder(weights_cpu, shape, max_seq_len=2048)
        r = _oracle_feed(orc, p)
        # continue greedily: the next inputs are the oracle's own tokens
        feed = [r["tokens"][-1]]
        for _ in range(10):
            step = _oracle_feed(orc, feed[-1:])
            for k in ("logits", "tokens", "gaps"):
                r[k] += step[k]
            feed.append(step["tokens"][0])
        r["inputs"] = list(p) + feed[:-1]
        refs.append(r)
    return prompts, refs


def test_batch_decode_matches_oracle(shape, weights_gpu, batch_case):
    """BatchDecoder: per-sequence prefill, then 10 batched steps (teacher-forced), each sequence at
    its own position, every row against its own oracle."""
    from qwen_megakernel_amd.model import BatchDecoder

    prompts, refs = batch_case
    bd = BatchDecoder(weights=weights_gpu, batch_size=4, max_seq_len=2048, verbose=False)
    for b, p in enumerate(prompts):
        tok, lg = bd.prefill(b, p, return_logits=True)
        i = len(p) - 1
        _check_step(i, lg.cpu(), refs[b]["logits"][i], tok, refs[b]["tokens"][i], refs[b]["gaps"][i])
    assert bd.positions == [len(p) for p in prompts]
    for s in range(10):
        inputs = [refs[b]["inputs"][len(prompts[b]) + s] for b in range(4)]
        toks, logits = bd.step_logits(inputs)
        for b in range(4):
            i = len(prompts[b]) + s
            _check_step(i, logits[b].cpu(), refs[b]["logits"][i], toks[b], refs[b]["tokens"][i], refs[b]["gaps"][i])


def test_batch_generate_matches_oracle_streams(weights_gpu, batch_case):
    """Device-fed batched generation equals each oracle's free-running stream until its first near-tie."""
    from qwen_megakernel_amd.model import BatchDecoder

    prompts, refs = batch_case
    bd = BatchDecoder(weights=weights_gpu, batch_size=4, max_seq_len=2048, verbose=False)
    out = bd.generate_ids(prompts, 11)
    for b in range(4):
        _stream_matches(out[b], refs[b], len(prompts[b]) - 1, f"sequence {b}")
    assert bd.positions == [len(p) + 10 for p in prompts]


def test_long_two_sequence_prefill_mfma_attention(shape, weights_cpu, weights_gpu):
    """1100 tokens of two sequences (600 + 500) in one forward, 2 layers: the MFMA attention
    (1024+ tokens) over 64-token tiles, a partial last tile and the tile holding the end of
    sequence 0 and the start of sequence 1 (row-by-row fallback); every 50th row of each
    sequence and each sequence's last row against its own oracle, and a repeat bit-exact."""
    from oracle.qwen3_ref import OracleDecoder
    from qwen_megakernel_amd.model import BatchDecoder
    from qwen_megakernel_amd.weights import make_prompt

    layers, lens = 2, (600, 500)
    prompts = [make_prompt(n, shape.vocab, seed=70 + i) for i, n in enumerate(lens)]
    refs = [_oracle_feed(OracleDecoder(weights_cpu, shape, num_layers=layers, max_seq_len=1024), p) for p in prompts]
    bd = BatchDecoder(weights=weights_gpu, batch_size=2, max_seq_len=1024, num_layers=layers, verbose=False)
    toks = prompts[0] + prompts[1]
    seqs = [0] * lens[0] + [1] * lens[1]
    pos = list(range(lens[0])) + list(range(lens[1]))
    rows = [(0, i) for i in list(range(0, lens[0], 50)) + [lens[0] - 1]]
    rows += [(1, i) for i in list(range(0, lens[1], 50)) + [lens[1] - 1]]
    emit = [i if s == 0 else lens[0] + i for s, i in rows]
    runs = []
    for _ in range(2):
        out = torch.empty(len(emit), dtype=torch.int32, device="cuda")
        logits = torch.empty(len(emit), V, dtype=torch.float32, device="cuda")
        bd._forward(_i32(toks), _i32(seqs), _i32(pos), _i32(emit), out, logits, bd._k_cache, bd._v_cache, max(lens))
        runs.append((out.cpu().tolist(), logits.cpu()))
    got, lg = runs[0]
    assert runs[1][0] == got and torch.equal(runs[1][1], lg), "second forward differs"
    for r, (sq, i) in enumerate(rows):
        ref = refs[sq]
        _check_step(i, lg[r], ref["logits"][i], got[r], ref["tokens"][i], ref["gaps"][i])


def test_prefill_all_matches_per_sequence_prefill(shape, weights_gpu):
    """Three prompts of different lengths in one forward (tokens of three sequences interleaved in
    one batch, each attending only to its own cache) against one prefill per sequence: the same
    logits to the decode bar, the same positions, and the next batched step continues alike."""
    from qwen_megakernel_amd.model import BatchDecoder
    from qwen_megakernel_amd.weights import make_prompt

    prompts = [make_prompt(m, shape.vocab, seed=50 + m) for m in (5, 17, 33)]
    one = BatchDecoder(weights=weights_gpu, batch_size=3, max_seq_len=128, verbose=False)
    each = BatchDecoder(weights=weights_gpu, batch_size=3, max_seq_len=128, verbose=False)
    toks, lg = one.prefill_all(prompts, return_logits=True)
    ref = [each.prefill(b, p, return_logits=True) for b, p in enumerate(prompts)]
    assert one.positions == each.positions == [5, 17, 33]
    for b in range(3):
        r = ref[b][1].cpu()
        top2 = torch.topk(r, 2).values
        _check_step(b, lg[b].cpu(), r, toks[b], ref[b][0], float(top2[0] - top2[1]))
    feed = [ref[b][0] for b in range(3)]  # the same inputs to both
    s1, l1 = one.step_logits(feed)
    s2, l2 = each.step_logits(feed)
    for b in range(3):
        r = l2[b].cpu()
        top2 = torch.topk(r, 2).values
        _check_step(b, l1[b].cpu(), r, s1[b], s2[b], float(top2[0] - top2[1]))


@pytest.mark.parametrize("n", [8, 40], ids=["8tok-split", "40tok-rowwise"])
def test_long_context_prefill(shape, weights_cpu, weights_gpu, n):
    """Prefill after an injected N(0,1) cache of 2100 positions: the row-wise attention takes two
    2048-position chunks (scores recomputed per pass), the split attention 34 workgroups per head."""
    from oracle.qwen3_ref import OracleDecoder
    from qwen_megakernel_amd.weights import make_kv_prefill, make_prompt

    c0, layers = 2100, 2
    max_seq = c0 + 64
    wc = _with_rope(weights_cpu, max_seq, "cpu")
    wg = _with_rope(weights_gpu, max_seq, "cuda")
    k, v = make_kv_prefill(shape, c0, seed=2)
    orc = OracleDecoder(wc, shape, num_layers=layers, max_seq_len=max_seq)
    orc.load_kv(k, v, c0)
    ids = make_prompt(n, shape.vocab, seed=7)
    ref = _oracle_feed(orc, ids)
    dec = _decoder(wg, num_layers=layers, max_seq_len=max_seq)
    dec.load_kv(k.cuda(), v.cuda(), c0)
    toks, logits = _forward_rows(dec._forward, ids, c0, dec._k_cache, dec._v_cache)
    worst = _check_rows(toks, logits, ref)
    print(f"long-context prefill {n} rows after {c0}: worst cos {worst[0]:.6f}, max abs {worst[1]:.4f}")


def test_random_norm_weights_prefill(shape):
    """Non-unit norm weights (q/k/input/post/final) so an ignored or misplaced norm fails."""
    from oracle.qwen3_ref import OracleDecoder
    from qwen_megakernel_amd.weights import make_prompt, make_weights, to_device

    w = make_weights(shape, seed=5, norm_std=0.1, num_layers=3, max_seq_len=256)
    ids = make_prompt(36, shape.vocab, seed=8)
    ref = _oracle_feed(OracleDecoder(w, shape, num_layers=3, max_seq_len=256), ids)
    dec = _decoder(to_device(w, "cuda"), num_layers=3, max_seq_len=256)
    toks, logits = _forward_rows(dec._forward, ids, 0, dec._k_cache, dec._v_cache)
    _check_rows(toks, logits, ref)


def test_qwen3_1p7b_prefill_and_batch():
    """Qwen3-1.7B (hidden 2048, MLP 6144), 4 layers: prefill rows and two batched steps."""
    from oracle.qwen3_ref import OracleDecoder
    from qwen_megakernel_amd.model import BatchDecoder
    from qwen_megakernel_amd.shapes import QWEN3_1_7B
    from qwen_megakernel_amd.weights import make_prompt, make_weights, to_device

    w = make_weights(QWEN3_1_7B, seed=0, num_layers=4, max_seq_len=256)
    wg = to_device(w, "cuda")
    prompts = [make_prompt(n, V, seed=20 + n) for n in (36, 6)]
    bd = BatchDecoder(weights=wg, batch_size=2, max_seq_len=256, num_layers=4, verbose=False)
    refs = []
    for b, p in enumerate(prompts):
        orc = OracleDecoder(w, QWEN3_1_7B, num_layers=4, max_seq_len=256)
        ref = _oracle_feed(orc, p)
        toks, logits = _forward_rows(bd._forward, p, 0, bd._k_cache, bd._v_cache, seq=b)
        bd._positions[b] = len(p)
        _check_rows(toks, logits, ref)
        refs.append((orc, ref))
    for s in range(2):
        inputs = [refs[b][1]["tokens"][-1] for b in range(2)]
        toks, logits = bd.step_logits(inputs)
        for b in range(2):
            orc, ref = refs[b]
            step = _oracle_feed(orc, inputs[b:b + 1])
            _check_step(s, logits[b].cpu(), step["logits"][0], toks[b], step["tokens"][0], step["gaps"][0])
            for key in ("logits", "tokens", "gaps"):
                ref[key] += step[key]


def test_invalid_entries_emit_minus_one(weights_gpu):
    """A token id outside the vocabulary, a position outside max_context and an emit row outside the
    batch give -1 and write no cache row; valid rows are unaffected."""
    dec = _decoder(weights_gpu, num_layers=2, max_seq_len=64)
    fwd = dec._forward
    out = torch.empty(5, dtype=torch.int32, device="cuda")
    tokens = _i32([5, V, 7, 9])
    positions = _i32([0, 1, 2, 40])  # max_context 8: position 40 is out of range
    fwd(tokens, _i32([0, 0, 0, 0]), positions, _i32([0, 1, 2, 3, 4]), out, None, dec._k_cache, dec._v_cache, 8)
    res = out.cpu().tolist()
    assert res[0] >= 0 and res[2] >= 0
    assert res[1] == -1 and res[3] == -1 and res[4] == -1
    kc = dec._k_cache.float().cpu()
    assert kc[:, :, 0].abs().sum() > 0 and kc[:, :, 2].abs().sum() > 0
    assert kc[:, :, 1].abs().sum() == 0 and kc[:, :, 40].abs().sum() == 0
    with pytest.raises(RuntimeError):
        fwd(tokens, _i32([0, 0, 0, 0]), positions, _i32([0]), out[:1], None, dec._k_cache, dec._v_cache, 65)


def test_batched_forward_deterministic(weights_gpu):
    """Fixed-order reductions: two identical forwards give bit-identical logits."""
    from qwen_megakernel_amd.weights import make_prompt

    ids = make_prompt(20, V, seed=9)
    outs = []
    for _ in range(2):
        dec = _decoder(weights_gpu, num_layers=4, max_seq_len=128)
        outs.append(_forward_rows(dec._forward, ids, 0, dec._k_cache, dec._v_cache)[1])
    assert torch.equal(outs[0], outs[1])


def test_decode_batch_16_sequences(shape, weights_cpu, weights_gpu):
    """A full 16-row MFMA tile of the fused decode step: 16 sequences, 2 layers, each row against its
    own oracle for three teacher-forced steps."""
    from oracle.qwen3_ref import OracleDecoder
    from qwen_megakernel_amd.model import BatchDecoder
    from qwen_megakernel_amd.weights import make_prompt

    B, layers = 16, 2
    prompts = [make_prompt(3 + b, shape.vocab, seed=40 + b) for b in range(B)]
    bd = BatchDecoder(weights=weights_gpu, batch_size=B, max_seq_len=128, num_layers=layers, verbose=False)
    orcs = [OracleDecoder(weights_cpu, shape, num_layers=layers, max_seq_len=128) for _ in range(B)]
    nxt = []
    for b, p in enumerate(prompts):
        ref = _oracle_feed(orcs[b], p)
        tok, lg = bd.prefill(b, p, return_logits=True)
        _check_step(len(p) - 1, lg.cpu(), ref["logits"][-1], tok, ref["tokens"][-1], ref["gaps"][-1])
        nxt.append(ref["tokens"][-1])
    for s in range(3):
        toks, logits = bd.step_logits(nxt)
        refs = [_oracle_feed(orcs[b], [nxt[b]]) for b in range(B)]
        for b in range(B):
            _check_step(s, logits[b].cpu(), refs[b]["logits"][0], toks[b], refs[b]["tokens"][0], refs[b]["gaps"][0])
        nxt = [r["tokens"][0] for r in refs]


def test_decode_batch_long_context_general_path(shape, weights_cpu, weights_gpu):
    """Contexts beyond the fused step's 4096 positions take the general path (split attention); two
    sequences after injected N(0,1) caches of 5000 and 4200 positions, 2 layers."""
    from oracle.qwen3_ref import OracleDecoder
    from qwen_megakernel_amd.model import BatchDecoder
    from qwen_megakernel_amd.weights import make_kv_prefill

    layers, max_seq = 2, 5100
    wc = _with_rope(weights_cpu, max_seq, "cpu")
    wg = _with_rope(weights_gpu, max_seq, "cuda")
    bd = BatchDecoder(weights=wg, batch_size=2, max_seq_len=max_seq, num_layers=layers, verbose=False)
    orcs = []
    for b, c0 in enumerate((5000, 4200)):
        k, v = make_kv_prefill(shape, c0, seed=2 + b)
        orc = OracleDecoder(wc, shape, num_layers=layers, max_seq_len=max_seq)
        orc.load_kv(k, v, c0)
        orcs.append(orc)
        bd.load_kv(b, k.cuda(), v.cuda(), c0)
    nxt = [11, 22]
    for s in range(2):
        toks, logits = bd.step_logits(nxt)
        refs = [_oracle_feed(orcs[b], [nxt[b]]) for b in range(2)]
        for b in range(2):
            _check_step(s, logits[b].cpu(), refs[b]["logits"][0], toks[b], refs[b]["tokens"][0], refs[b]["gaps"][0])
        nxt = [r["tokens"][0] for r in refs]


def test_decode_batch_equals_general_forward(weights_gpu):
    """The fused decode step and forward_tokens (general path) on the same inputs: same tokens
    wherever the logits' top two are not within rounding, logits within the same bar."""
    from qwen_megakernel_amd.model import BatchDecoder
    from qwen_megakernel_amd.weights import make_prompt

    bd = BatchDecoder(weights=weights_gpu, batch_size=4, max_seq_len=256, verbose=False)
    for b in range(4):
        bd.prefill(b, make_prompt(5 + 3 * b, V, seed=60 + b))
    k0, v0 = bd._k_cache.clone(), bd._v_cache.clone()
    toks = _i32([1, 2, 3, 4])
    pos = _i32(bd.positions)
    out_a = torch.empty(4, dtype=torch.int32, device="cuda")
    lg_a = torch.empty(4, V, dtype=torch.float32, device="cuda")
    bd._forward.decode(toks, pos, out_a, lg_a, bd._k_cache, bd._v_cache, 64)
    ka = bd._k_cache.clone()
    bd._k_cache.copy_(k0)
    bd._v_cache.copy_(v0)
    out_b = torch.empty(4, dtype=torch.int32, device="cuda")
    lg_b = torch.empty(4, V, dtype=torch.float32, device="cuda")
    ar = torch.arange(4, dtype=torch.int32, device="cuda")
    bd._forward(toks, ar, pos, ar, out_b, lg_b, bd._k_cache, bd._v_cache, 64)
    for b in range(4):
        cos = torch.nn.functional.cosine_similarity(lg_a[b].double(), lg_b[b].double(), dim=0).item()
        assert cos >= COS_MIN and (lg_a[b] - lg_b[b]).abs().max().item() <= ABS_MAX
    # the appended K rows agree up to rounding: layer 0 within 0.05 (one or two bf16 ulps of its
    # values), every layer's rows with cosine >= 0.999 (deeper layers carry the summation-order noise)
    d = (ka[:, 0].float() - bd._k_cache[:, 0].float()).abs().max().item()
    assert d <= 0.05, d
    cos = torch.nn.functional.cosine_similarity(ka.float().flatten().double(),
                                                bd._k_cache.float().flatten().double(), dim=0).item()
    assert cos >= 0.999, cos


@pytest.mark.parametrize("n", [128, 200, 300], ids=["128tok-64col-tiles", "200tok-128col-tiles", "300tok-mixed-tiles"])
def test_long_prefill_tiled_gemm(shape, weights_cpu, weights_gpu, n):
    """Prefills of 96+ tokens take the LDS-tiled MFMA GEMM: every 25th row and the last against
    the oracle, 2 layers, and a second identical forward bit-exact.  128 tokens: 64-column tiles
    for all four projections, o and down split 16 ways over K; 200 tokens: 128-column tiles with
    a partial last row tile; 300 tokens: 128-column tiles and 64-column tiles for down."""
    from oracle.qwen3_ref import OracleDecoder
    from qwen_megakernel_amd.weights import make_prompt

    layers = 2
    ids = make_prompt(n, shape.vocab, seed=13)
    ref = _oracle_feed(OracleDecoder(weights_cpu, shape, num_layers=layers, max_seq_len=512), ids)
    dec = _decoder(weights_gpu, num_layers=layers, max_seq_len=512)
    emit = list(range(0, n, 25)) + [n - 1]
    runs = []
    for _ in range(2):
        out = torch.empty(len(emit), dtype=torch.int32, device="cuda")
        logits = torch.empty(len(emit), V, dtype=torch.float32, device="cuda")
        dec._forward(_i32(ids), torch.zeros(n, dtype=torch.int32, device="cuda"),
                     torch.arange(n, dtype=torch.int32, device="cuda"), _i32(emit), out, logits, dec._k_cache,
                     dec._v_cache, n)
        runs.append((out.cpu().tolist(), logits.cpu()))
    toks, lg = runs[0]
    assert runs[1][0] == toks and torch.equal(runs[1][1], lg), "second forward differs"
    for r, e in enumerate(emit):
        _check_step(e, lg[r], ref["logits"][e], toks[r], ref["tokens"][e], ref["gaps"][e])
