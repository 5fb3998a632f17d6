"""GPU parity tests of the batched forward (prompt prefill and batched decode).

The batched path (qwen_megakernel/csrc/qmk_batch.hip, MFMA GEMMs) is checked
against the exact CPU oracle, which runs the same tokens in one pass over the
batched path's own cache: each of its rows is exactly a decode step at that
position on the inputs that row had (causal, exact reductions), so every
prefilled row and every batched step has its expected logits.  Same bar as the
decode kernel (tests/parity.py): cosine >= 0.999 and max abs <= 0.1 per row,
greedy tokens equal to the oracle's argmax except at near-ties, K/V rows equal
up to rounding.
"""

import pytest
import torch

from parity import (LAYERS28, LITERAL, Tally, check_kv_rows, check_row, check_rows, decoder, exact_oracle, fp32_oracle,
                    history_envelopes, lazy_envelopes, oracle_steps, stream_envelopes, stream_rows, with_rope)

pytestmark = pytest.mark.gpu

V = 151936


def _i32(values):
    return torch.tensor([int(v) for v in values], dtype=torch.int32, device="cuda")


def _forward_rows(fwd, ids, start, k_cache, v_cache, seq=0):
    """All rows of a one-sequence forward at positions start..; returns (tokens, logits [T, V])."""
    n = len(ids)
    out = torch.empty(n, dtype=torch.int32, device="cuda")
    logits = torch.empty(n, V, dtype=torch.float32, device="cuda")
    fwd(_i32(ids), torch.full((n,), seq, dtype=torch.int32, device="cuda"),
        torch.arange(start, start + n, dtype=torch.int32, device="cuda"),
        torch.arange(n, dtype=torch.int32, device="cuda"), out, logits, k_cache, v_cache, start + n)
    return out.cpu().tolist(), logits.cpu()


def test_mfma_operand_layout():
    """One v_mfma_f32_16x16x32_bf16 with the GEMM's lane layout equals A @ B^T."""
    from qwen_megakernel.build import get_extension

    ops = get_extension()
    g = torch.Generator().manual_seed(0)
    a = torch.randn(16, 32, generator=g).to(torch.bfloat16)
    b = torch.randn(16, 32, generator=g).to(torch.bfloat16)
    c = torch.empty(16, 16, dtype=torch.float32, device="cuda")
    ops.selftest_mfma(a.cuda(), b.cuda(), c)
    ref = a.double() @ b.double().t()
    err = (c.cpu().double() - ref).abs().max().item()
    assert err <= 1e-4, f"MFMA layout/result mismatch: max abs {err}"


@pytest.mark.parametrize("n,start", [(12, 0), (40, 0), (12, 200)],
                         ids=["12tok-rowwise-attention", "40tok-rowwise-attention", "12tok-after-200-split-attention"])
def test_prefill_all_rows_match_oracle(shape, exact06, weights_cpu, weights_gpu, n, start):
    """Every row of a 28-layer prefill at positions start.. against the oracle's row at that
    position (a token departure beyond one ulp only within the row's fp32 envelope); K/V written
    alike.  Fewer than 32 tokens take the row attention over at most 128 positions of context and
    the context-split attention beyond; the first `start` positions come from an earlier prefill."""
    from qwen_megakernel.weights import make_prompt

    ids = make_prompt(n, shape.vocab, seed=3)
    dec = decoder(weights_gpu)
    if start:
        dec.prefill(make_prompt(start, shape.vocab, seed=4))
    toks, logits = _forward_rows(dec._forward, ids, start, dec._k_cache, dec._v_cache)
    orc = exact_oracle(exact06, shape, 2048)
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, start, ids)
    envs = lazy_envelopes(weights_cpu, shape, 2048, dec._k_cache, dec._v_cache, start, ids, ref)
    print(check_rows(Tally(f"prefill {n} rows at {start}"), ref, toks, logits, bar=LAYERS28, envs=envs))
    check_kv_rows(f"prefill {n} rows at {start}", orc, dec._k_cache, dec._v_cache, start, n)


def test_prefill_then_decode_kernel(shape, exact06, weights_cpu, weights_gpu):
    """Decoder.prefill writes a cache the decode megakernel continues from: the prefill's last row
    and 12 decode steps on the decoder's own tokens against the oracle (a token departure beyond
    one ulp only within the step's fp32 envelope)."""
    from qwen_megakernel.weights import make_prompt

    prompt = make_prompt(24, shape.vocab, seed=5)
    dec = decoder(weights_gpu)
    tok, lg = dec.prefill(prompt, return_logits=True)
    assert dec.position == len(prompt)
    toks, lgs = [tok], [lg.cpu()]
    for _ in range(11):
        tok, lg = dec.step_logits(toks[-1])
        toks.append(tok)
        lgs.append(lg.cpu())
    orc = exact_oracle(exact06, shape, 2048)
    ref = stream_rows(orc, dec._k_cache, dec._v_cache, prompt, toks)
    envs = history_envelopes(weights_cpu, shape, 2048, dec._k_cache, dec._v_cache, prompt, toks, ref)
    print(check_rows(Tally("prefill + decode"), ref, toks, torch.stack(lgs), bar=LAYERS28, envs=envs))
    check_kv_rows("prefill + decode", orc, dec._k_cache, dec._v_cache, 0, len(prompt) + 11)


def test_generate_with_prefill_matches_oracle_stream(shape, exact06, weights_cpu, weights_gpu):
    """generate() feeds the prompt through prefill by default (use_prefill=False: one decode step per
    prompt token, as the reference); both streams are the oracle's up to near-ties."""
    from qwen_megakernel.weights import make_prompt

    prompt = make_prompt(20, V, seed=6)
    for use_prefill in (True, False):
        dec = decoder(weights_gpu, use_prefill=use_prefill)
        out = dec.generate(prompt, 24)
        ref = stream_rows(exact_oracle(exact06, shape, 2048), dec._k_cache, dec._v_cache, prompt, out)
        envs = history_envelopes(weights_cpu, shape, 2048, dec._k_cache, dec._v_cache, prompt, out, ref)
        print(check_rows(Tally(f"generate use_prefill={use_prefill}"), ref, out, bar=LAYERS28, envs=envs))


@pytest.fixture(scope="module")
def batch_prompts(shape):
    from qwen_megakernel.weights import make_prompt

    return [make_prompt(n, shape.vocab, seed=10 + b) for b, n in enumerate([5, 17, 33, 9])]


def test_batch_decode_matches_oracle(shape, exact06, weights_cpu, weights_gpu, batch_prompts):
    """BatchDecoder: per-sequence prefill, then 10 batched steps, each sequence on its own tokens at
    its own position; every sequence's rows against its own oracle (a token departure beyond one
    ulp only within the step's fp32 envelope)."""
    from qwen_megakernel.model import BatchDecoder

    prompts = batch_prompts
    bd = BatchDecoder(weights=weights_gpu, batch_size=4, max_seq_len=2048, verbose=False)
    toks, lgs = [], []
    for b, p in enumerate(prompts):
        tok, lg = bd.prefill(b, p, return_logits=True)
        toks.append([tok])
        lgs.append([lg.cpu()])
    assert bd.positions == [len(p) for p in prompts]
    for _ in range(10):
        nxt, logits = bd.step_logits([t[-1] for t in toks])
        for b in range(4):
            toks[b].append(nxt[b])
            lgs[b].append(logits[b].cpu())
    for b in range(4):
        orc = exact_oracle(exact06, shape, 2048)
        ref = stream_rows(orc, bd._k_cache[b], bd._v_cache[b], prompts[b], toks[b])
        envs = history_envelopes(weights_cpu, shape, 2048, bd._k_cache[b], bd._v_cache[b], prompts[b], toks[b], ref)
        print(check_rows(Tally(f"batched decode sequence {b}"), ref, toks[b], torch.stack(lgs[b]), bar=LAYERS28,
                         envs=envs))
        check_kv_rows(f"batched decode sequence {b}", orc, bd._k_cache[b], bd._v_cache[b], 0, len(prompts[b]) + 10)


def test_decode_batch_multi_launch_28_layers_long_prompts(shape, exact06, weights_cpu, weights_gpu):
    """Three sequences after prompts of 1300, 2100 and 3000 tokens, 28 layers, 4 batched steps:
    contexts above 2,048 positions take the multi-launch step (HF's two softmax passes split over
    every CU, the probabilities rounded to bf16).  Each sequence's prefill row and steps against
    its own oracle on the step's inputs, to the 28-layer bar (a token may leave the oracle's argmax
    beyond one ulp only within the step's fp32 envelope)."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_prompt

    lens, max_seq = (1300, 2100, 3000), 4096
    prompts = [make_prompt(n, V, seed=80 + i) for i, n in enumerate(lens)]
    bd = BatchDecoder(weights=with_rope(weights_gpu, max_seq, "cuda"), batch_size=3, max_seq_len=max_seq,
                      verbose=False)
    toks, lgs = [], []
    for b, p in enumerate(prompts):
        tok, lg = bd.prefill(b, p, return_logits=True)
        toks.append([tok])
        lgs.append([lg.cpu()])
    for _ in range(4):
        nxt, logits = bd.step_logits([t[-1] for t in toks])
        for b in range(3):
            toks[b].append(nxt[b])
            lgs[b].append(logits[b].cpu())
    forc = fp32_oracle(weights_cpu, shape, max_seq)
    for b in range(3):
        n0 = len(prompts[b]) - 1
        feed = [prompts[b][-1]] + toks[b][:-1]  # the rows at positions n0.. that produced toks[b]
        orc = exact_oracle(exact06, shape, max_seq)
        ref = oracle_steps(orc, bd._k_cache[b], bd._v_cache[b], n0, feed)
        envs = stream_envelopes(forc, bd._k_cache[b], bd._v_cache[b], n0, feed, ref)
        print(check_rows(Tally(f"multi-launch batched decode, 28 layers, sequence {b} after {lens[b]}"), ref,
                         toks[b], torch.stack(lgs[b]), bar=LAYERS28, envs=envs))


def test_batch_generate_matches_oracle_streams(shape, exact06, weights_cpu, weights_gpu, batch_prompts):
    """Device-fed batched generation: every sequence's stream is its oracle's up to near-ties (a
    token departure beyond one ulp only within the step's fp32 envelope)."""
    from qwen_megakernel.model import BatchDecoder

    prompts = batch_prompts
    bd = BatchDecoder(weights=weights_gpu, batch_size=4, max_seq_len=2048, verbose=False)
    out = bd.generate_ids(prompts, 11)
    for b in range(4):
        ref = stream_rows(exact_oracle(exact06, shape, 2048), bd._k_cache[b], bd._v_cache[b], prompts[b], out[b])
        envs = history_envelopes(weights_cpu, shape, 2048, bd._k_cache[b], bd._v_cache[b], prompts[b], out[b], ref)
        check_rows(Tally(f"batched generate sequence {b}"), ref, out[b], bar=LAYERS28, envs=envs)
    assert bd.positions == [len(p) + 10 for p in prompts]


def test_long_two_sequence_prefill_mfma_attention(shape, exact06, weights_gpu):
    """1100 tokens of two sequences (600 + 500) in one forward, 2 layers: the MFMA attention
    (1024+ tokens) over 64-token tiles, a partial last tile and the tile holding the end of
    sequence 0 and the start of sequence 1 (row-by-row fallback); every 50th row of each
    sequence and each sequence's last row against its own oracle, and a repeat bit-exact."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_prompt

    layers, lens = 2, (600, 500)
    prompts = [make_prompt(n, shape.vocab, seed=70 + i) for i, n in enumerate(lens)]
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
    refs = []
    for sq in range(2):
        orc = exact_oracle(exact06, shape, 1024, num_layers=layers)
        refs.append(oracle_steps(orc, bd._k_cache[sq], bd._v_cache[sq], 0, prompts[sq]))
        check_kv_rows(f"two-sequence prefill, sequence {sq}", orc, bd._k_cache[sq], bd._v_cache[sq], 0, lens[sq])
    t = Tally("two-sequence 1100-token prefill")
    for r, (sq, i) in enumerate(rows):
        check_row(t, (sq, i), refs[sq][i], got[r], lg[r], bar=LITERAL)
    print(t)


def test_long_single_sequence_prefill_mfma_attention(shape, exact06, weights_gpu):
    """A 2048-token prompt of one sequence, 2 layers: the MFMA attention's 32 tiles in 16 pairs
    (tiles i and 31 - i in one workgroup per query head), rows 0..2047 in every tile; every 97th
    row and the last against the oracle, and a repeat bit-exact."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_prompt

    layers, n = 2, 2048
    prompt = make_prompt(n, shape.vocab, seed=91)
    bd = BatchDecoder(weights=weights_gpu, batch_size=1, max_seq_len=n, num_layers=layers, verbose=False)
    rows = list(range(0, n, 97)) + [n - 1]
    runs = []
    for _ in range(2):
        out = torch.empty(len(rows), dtype=torch.int32, device="cuda")
        logits = torch.empty(len(rows), V, dtype=torch.float32, device="cuda")
        bd._forward(_i32(prompt), _i32([0] * n), _i32(list(range(n))), _i32(rows), out, logits, bd._k_cache,
                    bd._v_cache, n)
        runs.append((out.cpu().tolist(), logits.cpu()))
    got, lg = runs[0]
    assert runs[1][0] == got and torch.equal(runs[1][1], lg), "second forward differs"
    orc = exact_oracle(exact06, shape, n, num_layers=layers)
    ref = oracle_steps(orc, bd._k_cache[0], bd._v_cache[0], 0, prompt, emit=rows)
    check_kv_rows("2048-token prefill", orc, bd._k_cache[0], bd._v_cache[0], 0, n)
    t = Tally("2048-token prefill")
    for r, i in enumerate(rows):
        check_row(t, i, ref[r], got[r], lg[r], bar=LITERAL)
    print(t)


def test_prefill_all_matches_per_sequence_prefill(shape, weights_gpu):
    """Three prompts of different lengths in one forward (tokens of three sequences interleaved in
    one batch, each attending only to its own cache) against one prefill per sequence: the same
    logits to the decode bar, the same positions, and the next batched step continues alike."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_prompt

    prompts = [make_prompt(m, shape.vocab, seed=50 + m) for m in (5, 17, 33)]
    one = BatchDecoder(weights=weights_gpu, batch_size=3, max_seq_len=128, verbose=False)
    each = BatchDecoder(weights=weights_gpu, batch_size=3, max_seq_len=128, verbose=False)
    toks, lg = one.prefill_all(prompts, return_logits=True)
    ref = [each.prefill(b, p, return_logits=True) for b, p in enumerate(prompts)]
    assert one.positions == each.positions == [5, 17, 33]
    t = Tally("prefill_all vs per-sequence prefill")
    for b in range(3):
        check_row(t, b, ref[b][1].cpu(), toks[b], lg[b], bar=LAYERS28)
    feed = [ref[b][0] for b in range(3)]  # the same inputs to both
    s1, l1 = one.step_logits(feed)
    s2, l2 = each.step_logits(feed)
    for b in range(3):
        check_row(t, ("step", b), l2[b].cpu(), s1[b], l1[b], bar=LAYERS28)


@pytest.mark.parametrize("n", [2, 8, 40, 150],
                         ids=["2tok-split", "8tok-mfma-chunks", "40tok-mfma-chunks", "150tok-mfma-chunks"])
def test_long_context_prefill(shape, exact06, weights_gpu, n):
    """Prefill after an injected N(0,1) cache of 2100 positions: 2 tokens take the split attention
    (34 workgroups per head and token); 8, 40 and 150 tokens (one, one and three 64-token tiles,
    the last partial) the MFMA attention with its keys in chunks over the context (too few tiles
    to fill the chip)."""
    from qwen_megakernel.weights import make_kv_prefill, make_prompt

    c0, layers = 2100, 2
    max_seq = c0 + 192
    k, v = make_kv_prefill(shape, c0, seed=2)
    ids = make_prompt(n, shape.vocab, seed=7)
    dec = decoder(with_rope(weights_gpu, max_seq, "cuda"), num_layers=layers, max_seq_len=max_seq)
    dec.load_kv(k.cuda(), v.cuda(), c0)
    toks, logits = _forward_rows(dec._forward, ids, c0, dec._k_cache, dec._v_cache)
    orc = exact_oracle(exact06, shape, max_seq, num_layers=layers)
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, c0, ids)
    print(check_rows(Tally(f"long-context prefill {n} rows after {c0}"), ref, toks, logits, bar=LITERAL))
    check_kv_rows(f"long-context prefill {n}", orc, dec._k_cache, dec._v_cache, c0, n)


def test_prompt_after_long_context_28_layers(shape, exact06, weights_cpu, weights_gpu):
    """A new turn: 100 tokens after a 1200-token prefill, 28 layers (the MFMA attention over key
    chunks: two tiles, seven chunks of three 64-key blocks); every row against the exact oracle on
    the kernel's cache (a token departure beyond one ulp only within the row's fp32 envelope), and
    the K/V rows written."""
    from qwen_megakernel.weights import make_prompt

    c0, n = 1200, 100
    dec = decoder(weights_gpu)
    dec.prefill(make_prompt(c0, shape.vocab, seed=21))
    ids = make_prompt(n, shape.vocab, seed=22)
    toks, logits = _forward_rows(dec._forward, ids, c0, dec._k_cache, dec._v_cache)
    orc = exact_oracle(exact06, shape, 2048)
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, c0, ids)
    envs = lazy_envelopes(weights_cpu, shape, 2048, dec._k_cache, dec._v_cache, c0, ids, ref)
    print(check_rows(Tally(f"{n} rows after {c0}"), ref, toks, logits, bar=LAYERS28, envs=envs))
    check_kv_rows(f"{n} rows after {c0}", orc, dec._k_cache, dec._v_cache, c0, n)


def test_long_prompt_after_long_context(shape, exact06, weights_gpu):
    """600 tokens (ten 64-token tiles, the last partial) after a 1300-token prefill, 4 layers: the
    MFMA attention over six key chunks per tile (more than 8 tiles take up to 64 tile chunks);
    every 50th row and the last against the exact oracle at the literal bar, and the K/V rows."""
    from qwen_megakernel.weights import make_prompt

    layers, c0, n = 4, 1300, 600
    dec = decoder(weights_gpu, num_layers=layers)
    dec.prefill(make_prompt(c0, shape.vocab, seed=23))
    ids = make_prompt(n, shape.vocab, seed=24)
    rows = list(range(0, n, 50)) + [n - 1]
    out = torch.empty(len(rows), dtype=torch.int32, device="cuda")
    logits = torch.empty(len(rows), V, dtype=torch.float32, device="cuda")
    dec._forward(_i32(ids), torch.zeros(n, dtype=torch.int32, device="cuda"),
                 torch.arange(c0, c0 + n, dtype=torch.int32, device="cuda"), _i32(rows), out, logits, dec._k_cache,
                 dec._v_cache, c0 + n)
    orc = exact_oracle(exact06, shape, 2048, num_layers=layers)
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, c0, ids, emit=rows)
    print(check_rows(Tally(f"{n} rows after {c0}"), ref, out.cpu().tolist(), logits.cpu(), bar=LITERAL))
    check_kv_rows(f"{n} rows after {c0}", orc, dec._k_cache, dec._v_cache, c0, n)


@pytest.mark.parametrize(
    "n,start",
    [(31, 190), (32, 100), (33, 300), (320, 0), (700, 0), (64, 2000), (1, 3000), (3, 3000)],
    ids=["split-31@190", "rows-32@100", "mfma-chunks-33@300", "mfma-chunks-320@0", "mfma-pairs-700@0",
         "mfma-chunks-64@2000", "split-1@3000", "mfma-chunks-3@3000"])
def test_attention_form_matrix(shape, exact06, weights_gpu, n, start):
    """One prompt of n tokens after `start` prefilled positions, 2 layers, for each attention form
    the forward picks (the row kernel, the per-token context split, the MFMA attention in tile pairs
    or over key chunks) around the thresholds between them: the first, middle and last rows and
    every 100th against the exact oracle at the literal bar, and the K/V rows."""
    from qwen_megakernel.weights import make_prompt

    layers = 2
    max_seq = max(2048, start + n)
    w = with_rope(weights_gpu, max_seq, "cuda") if max_seq > 2048 else weights_gpu
    dec = decoder(w, num_layers=layers, max_seq_len=max_seq)
    if start:
        dec.prefill(make_prompt(start, shape.vocab, seed=25))
    ids = make_prompt(n, shape.vocab, seed=26)
    rows = sorted(set([0, n // 2, n - 1] + list(range(0, n, 100))))
    out = torch.empty(len(rows), dtype=torch.int32, device="cuda")
    logits = torch.empty(len(rows), V, dtype=torch.float32, device="cuda")
    dec._forward(_i32(ids), torch.zeros(n, dtype=torch.int32, device="cuda"),
                 torch.arange(start, start + n, dtype=torch.int32, device="cuda"), _i32(rows), out, logits,
                 dec._k_cache, dec._v_cache, start + n)
    orc = exact_oracle(exact06, shape, max_seq, num_layers=layers)
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, start, ids, emit=rows)
    print(check_rows(Tally(f"{n} tokens at {start}"), ref, out.cpu().tolist(), logits.cpu(), bar=LITERAL))
    check_kv_rows(f"{n} tokens at {start}", orc, dec._k_cache, dec._v_cache, start, n)


def test_long_context_prefill_rows_two_sequences(shape, exact06, weights_gpu):
    """Two sequences of 20 tokens each after injected N(0,1) caches of 2100 and 2060 positions, in
    one forward with their tokens interleaved: no 64-token tile is one sequence, so every row takes
    the row attention, which covers the contexts in two 2048-position chunks (scores recomputed per
    pass).  Every row against its sequence's oracle."""
    from dataclasses import replace

    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_kv_prefill, make_prompt

    c0s, layers, n = (2100, 2060), 2, 20
    max_seq = max(c0s) + 64
    bd = BatchDecoder(weights=with_rope(weights_gpu, max_seq, "cuda"), batch_size=2, max_seq_len=max_seq,
                      num_layers=layers, verbose=False)
    kvs = [make_kv_prefill(replace(shape, num_layers=layers), c, seed=20 + b) for b, c in enumerate(c0s)]
    for b, (k, v) in enumerate(kvs):
        bd.load_kv(b, k.cuda(), v.cuda(), c0s[b])
    ids = [make_prompt(n, shape.vocab, seed=30 + b) for b in range(2)]
    toks = [ids[i % 2][i // 2] for i in range(2 * n)]
    seqs = [i % 2 for i in range(2 * n)]
    pos = [c0s[i % 2] + i // 2 for i in range(2 * n)]
    out = torch.empty(2 * n, dtype=torch.int32, device="cuda")
    logits = torch.empty(2 * n, V, dtype=torch.float32, device="cuda")
    bd._forward(_i32(toks), _i32(seqs), _i32(pos), _i32(range(2 * n)), out, logits, bd._k_cache, bd._v_cache,
                max(c0s) + n)
    got, lg = out.cpu().tolist(), logits.cpu()
    t = Tally(f"two sequences x {n} rows after {c0s}")
    for b in range(2):
        orc = exact_oracle(exact06, shape, max_seq, num_layers=layers)
        ref = oracle_steps(orc, bd._k_cache[b], bd._v_cache[b], c0s[b], ids[b])
        rows = list(range(b, 2 * n, 2))
        check_rows(t, ref, [got[r] for r in rows], lg[rows], bar=LITERAL)
        check_kv_rows(f"two sequences, sequence {b}", orc, bd._k_cache[b], bd._v_cache[b], c0s[b], n)
    print(t)


@pytest.mark.parametrize("n,start", [(1, 0), (2, 0), (3, 0), (1, 150), (3, 150)],
                         ids=["1tok", "2tok", "3tok", "1tok-after-150", "3tok-after-150"])
def test_prefill_few_tokens(shape, exact06, weights_gpu, n, start):
    """Prompts of 1-3 tokens, 4 layers: the tiled GEMM's 128-row tile almost all repeats of the last
    row (rows past T), the row attention from position 0 and the split attention after a
    150-token prefix; every row against the oracle at the literal bar, and the K/V rows."""
    from qwen_megakernel.weights import make_prompt

    layers = 4
    dec = decoder(weights_gpu, num_layers=layers)
    if start:
        dec.prefill(make_prompt(start, shape.vocab, seed=12))
    ids = make_prompt(n, shape.vocab, seed=13 + n)
    toks, logits = _forward_rows(dec._forward, ids, start, dec._k_cache, dec._v_cache)
    orc = exact_oracle(exact06, shape, 2048, num_layers=layers)
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, start, ids)
    print(check_rows(Tally(f"{n}-token prefill at {start}"), ref, toks, logits, bar=LITERAL))
    check_kv_rows(f"{n}-token prefill at {start}", orc, dec._k_cache, dec._v_cache, start, n)


def test_random_norm_weights_prefill(shape):
    """Non-unit norm weights (q/k/input/post/final) so an ignored or misplaced norm fails."""
    from oracle.qwen3_exact import ExactOracle
    from qwen_megakernel.weights import make_prompt, make_weights, to_device

    w = make_weights(shape, seed=5, norm_std=0.1, num_layers=3, max_seq_len=256)
    ids = make_prompt(36, shape.vocab, seed=8)
    dec = decoder(to_device(w, "cuda"), num_layers=3, max_seq_len=256)
    toks, logits = _forward_rows(dec._forward, ids, 0, dec._k_cache, dec._v_cache)
    orc = ExactOracle(w, shape, num_layers=3, max_seq_len=256)
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, 0, ids)
    print(check_rows(Tally("random norm weights prefill"), ref, toks, logits, bar=LITERAL))
    check_kv_rows("random norm weights prefill", orc, dec._k_cache, dec._v_cache, 0, 36)


def test_qwen3_1p7b_prefill_and_batch():
    """Qwen3-1.7B (hidden 2048, MLP 6144), 4 layers: every prefill row of two prompts and two
    batched steps on the decoder's own tokens."""
    from oracle.qwen3_exact import ExactWeights
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.shapes import QWEN3_1_7B
    from qwen_megakernel.weights import make_prompt, make_weights, to_device

    w = make_weights(QWEN3_1_7B, seed=0, num_layers=4, max_seq_len=256)
    ew = ExactWeights(w, QWEN3_1_7B, num_layers=4)
    wg = to_device(w, "cuda")
    prompts = [make_prompt(n, V, seed=20 + n) for n in (36, 6)]
    bd = BatchDecoder(weights=wg, batch_size=2, max_seq_len=256, num_layers=4, verbose=False)
    t = Tally("qwen3-1.7b 4 layers batched")
    gen = []
    for b, p in enumerate(prompts):
        toks, logits = _forward_rows(bd._forward, p, 0, bd._k_cache, bd._v_cache, seq=b)
        bd._positions[b] = len(p)
        check_rows(t, oracle_steps(exact_oracle(ew, QWEN3_1_7B, 256), bd._k_cache[b], bd._v_cache[b], 0, p),
                   toks, logits, bar=LITERAL)
        gen.append([toks[-1]])
    lgs = [[], []]
    for _ in range(2):
        nxt, logits = bd.step_logits([g[-1] for g in gen])
        for b in range(2):
            gen[b].append(nxt[b])
            lgs[b].append(logits[b].cpu())
    for b in range(2):
        orc = exact_oracle(ew, QWEN3_1_7B, 256)
        ref = stream_rows(orc, bd._k_cache[b], bd._v_cache[b], prompts[b], gen[b])
        check_rows(t, ref[1:], gen[b][1:], torch.stack(lgs[b]), bar=LITERAL)
        check_kv_rows(f"qwen3-1.7b 4 layers sequence {b}", orc, bd._k_cache[b], bd._v_cache[b], 0, len(prompts[b]) + 2)
    print(t)


def test_invalid_entries_emit_minus_one(weights_gpu):
    """A token id outside the vocabulary, a position outside max_context and an emit row outside the
    batch give -1 and write no cache row; valid rows are unaffected."""
    dec = decoder(weights_gpu, num_layers=2, max_seq_len=64)
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


def test_invalid_entries_in_a_long_prompt(weights_gpu):
    """A 1024-token prompt (the fused q/k/v and gate/up epilogues, the MFMA attention) with a token
    id outside the vocabulary at row 300 and a position outside max_context at row 700: those rows
    emit -1 and write no cache row, the tiles holding them are redone row by row, the other rows
    emit tokens, and a second identical forward gives the same tokens and logits."""
    from qwen_megakernel.weights import make_prompt

    n = 1024
    dec = decoder(weights_gpu, num_layers=2, max_seq_len=n)
    fwd = dec._forward
    ids = make_prompt(n, V, seed=33)
    ids[300] = V
    pos = list(range(n))
    pos[700] = 5000
    emit = [0, 299, 300, 301, 700, 1023]
    runs = []
    for _ in range(2):
        dec._k_cache.zero_()
        dec._v_cache.zero_()
        out = torch.empty(len(emit), dtype=torch.int32, device="cuda")
        logits = torch.empty(len(emit), V, dtype=torch.float32, device="cuda")
        fwd(_i32(ids), _i32([0] * n), _i32(pos), _i32(emit), out, logits, dec._k_cache, dec._v_cache, n)
        runs.append((out.cpu().tolist(), logits.cpu()))
    res, lg = runs[0]
    assert runs[1][0] == res and torch.equal(runs[1][1], lg), "second forward differs"
    assert res[2] == -1 and res[4] == -1, res
    assert all(res[i] >= 0 for i in (0, 1, 3, 5)), res
    kc, vc = dec._k_cache.float().cpu(), dec._v_cache.float().cpu()
    for p in (300, 700):
        assert kc[:, :, p].abs().sum() == 0 and vc[:, :, p].abs().sum() == 0, p
    for p in (0, 299, 301, 1023):
        assert kc[:, :, p].abs().sum() > 0 and vc[:, :, p].abs().sum() > 0, p


def test_batched_forward_deterministic(weights_gpu):
    """Fixed-order reductions: two identical forwards give bit-identical logits."""
    from qwen_megakernel.weights import make_prompt

    ids = make_prompt(20, V, seed=9)
    outs = []
    for _ in range(2):
        dec = decoder(weights_gpu, num_layers=4, max_seq_len=128)
        outs.append(_forward_rows(dec._forward, ids, 0, dec._k_cache, dec._v_cache)[1])
    assert torch.equal(outs[0], outs[1])


def test_decode_batch_16_sequences(shape, exact06, weights_gpu):
    """A full 16-row MFMA tile of the fused decode step: 16 sequences, 2 layers, each sequence's
    prefill row and three batched steps on its own tokens against its own oracle."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_prompt

    B, layers = 16, 2
    prompts = [make_prompt(3 + b, shape.vocab, seed=40 + b) for b in range(B)]
    bd = BatchDecoder(weights=weights_gpu, batch_size=B, max_seq_len=128, num_layers=layers, verbose=False)
    gen, lgs = [], []
    for b, p in enumerate(prompts):
        tok, lg = bd.prefill(b, p, return_logits=True)
        gen.append([tok])
        lgs.append([lg.cpu()])
    for _ in range(3):
        nxt, logits = bd.step_logits([g[-1] for g in gen])
        for b in range(B):
            gen[b].append(nxt[b])
            lgs[b].append(logits[b].cpu())
    t = Tally("16-sequence batched decode")
    for b in range(B):
        orc = exact_oracle(exact06, shape, 128, num_layers=layers)
        ref = stream_rows(orc, bd._k_cache[b], bd._v_cache[b], prompts[b], gen[b])
        check_rows(t, ref, gen[b], torch.stack(lgs[b]), bar=LITERAL)
        check_kv_rows(f"16-sequence batched decode, sequence {b}", orc, bd._k_cache[b], bd._v_cache[b], 0,
                      len(prompts[b]) + 3)
    print(t)


def test_decode_batch_long_context_general_path(shape, exact06, weights_gpu):
    """Contexts beyond the fused step's 4096 positions take the general path (split attention); two
    sequences after injected N(0,1) caches of 5000 and 4200 positions, 2 layers, three steps."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_kv_prefill

    layers, max_seq = 2, 5100
    bd = BatchDecoder(weights=with_rope(weights_gpu, max_seq, "cuda"), batch_size=2, max_seq_len=max_seq,
                      num_layers=layers, verbose=False)
    c0s = (5000, 4200)
    for b, c0 in enumerate(c0s):
        k, v = make_kv_prefill(shape, c0, seed=2 + b)
        bd.load_kv(b, k.cuda(), v.cuda(), c0)
    feed, lgs = [[11], [22]], [[], []]
    for _ in range(3):
        nxt, logits = bd.step_logits([f[-1] for f in feed])
        for b in range(2):
            feed[b].append(nxt[b])
            lgs[b].append(logits[b].cpu())
    t = Tally("batched decode, general path, 5000/4200 context")
    for b in range(2):
        orc = exact_oracle(exact06, shape, max_seq, num_layers=layers)
        ref = oracle_steps(orc, bd._k_cache[b], bd._v_cache[b], c0s[b], feed[b][:-1])
        check_rows(t, ref, feed[b][1:], torch.stack(lgs[b]), bar=LITERAL)
        check_kv_rows(f"general path sequence {b}", orc, bd._k_cache[b], bd._v_cache[b], c0s[b], 3)
    print(t)


@pytest.mark.parametrize("c0s", [(3900,), (3000, 17), (2900, 1, 2500, 40)],
                         ids=["batch1-32splits", "batch2-16splits", "batch4-8splits"])
def test_decode_batch_fused_split_attention_contexts(shape, exact06, weights_gpu, c0s):
    """The fused step's attention splits each (sequence, KV head) over S = 256 / (8 B) workgroups.
    Injected N(0,1) caches: 2900-3900 positions give a split two or three 128-position batches
    (its running-maximum rescale), and 1, 17 or 40 positions leave some of the S splits empty.
    2 layers, three steps, every sequence against the exact oracle on its own cache."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_kv_prefill

    B, layers, max_seq = len(c0s), 2, 4096
    bd = BatchDecoder(weights=with_rope(weights_gpu, max_seq, "cuda"), batch_size=B, max_seq_len=max_seq,
                      num_layers=layers, verbose=False)
    for b, c0 in enumerate(c0s):
        k, v = make_kv_prefill(shape, c0, seed=5 + b)
        bd.load_kv(b, k.cuda(), v.cuda(), c0)
    feed, lgs = [[11 + 7 * b] for b in range(B)], [[] for _ in range(B)]
    for _ in range(3):
        nxt, logits = bd.step_logits([f[-1] for f in feed])
        for b in range(B):
            feed[b].append(nxt[b])
            lgs[b].append(logits[b].cpu())
    t = Tally(f"fused split attention, contexts {c0s}")
    for b in range(B):
        orc = exact_oracle(exact06, shape, max_seq, num_layers=layers)
        ref = oracle_steps(orc, bd._k_cache[b], bd._v_cache[b], c0s[b], feed[b][:-1])
        check_rows(t, ref, feed[b][1:], torch.stack(lgs[b]), bar=LITERAL)
        check_kv_rows(f"fused split attention sequence {b}", orc, bd._k_cache[b], bd._v_cache[b], c0s[b], 3)
    print(t)


def test_decode_batch_equals_general_forward(weights_gpu):
    """The fused decode step and forward_tokens (general path) on the same inputs: logits within
    the bar of each other and the same tokens up to near-ties."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_prompt

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
    t = Tally("fused decode step vs general forward")
    check_rows(t, lg_b.cpu(), out_a.cpu().tolist(), lg_a.cpu(), bar=LAYERS28)
    # the appended K rows agree up to rounding: layer 0 within one ulp at |k| < 8, every layer's
    # rows with cosine >= 0.999
    d = (ka[:, 0].float() - bd._k_cache[:, 0].float()).abs().max().item()
    assert d <= 0.0625, d
    cos = torch.nn.functional.cosine_similarity(ka.float().flatten().double(),
                                                bd._k_cache.float().flatten().double(), dim=0).item()
    assert cos >= 0.999, cos


@pytest.mark.parametrize("n", [128, 200, 300, 450],
                         ids=["128tok-64col-tiles", "200tok-128col-tiles", "300tok-mixed-tiles", "450tok-mfma-attention"])
def test_long_prefill_tiled_gemm(shape, exact06, weights_gpu, n):
    """Prefills of 96+ tokens take the LDS-tiled MFMA GEMM: every 25th row and the last against
    the oracle, 2 layers, and a second identical forward bit-exact.  128 tokens: 64-column tiles
    for all four projections, o and down split 16 ways over K; 200 tokens: 128-column tiles with
    a partial last row tile; 300 tokens: 128-column tiles and 64-column tiles for down; 450 tokens:
    the MFMA attention (8 tiles in 4 pairs, a partial last tile)."""
    from qwen_megakernel.weights import make_prompt

    layers = 2
    ids = make_prompt(n, shape.vocab, seed=13)
    emit = list(range(0, n, 25)) + [n - 1]
    dec = decoder(weights_gpu, num_layers=layers, max_seq_len=512)
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
    orc = exact_oracle(exact06, shape, 512, num_layers=layers)
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, 0, ids, emit=emit)
    print(check_rows(Tally(f"tiled-GEMM prefill {n}"), ref, toks, lg, labels=emit, bar=LITERAL))
    check_kv_rows(f"tiled-GEMM prefill {n}", orc, dec._k_cache, dec._v_cache, 0, n)


def test_prefill_emits_the_maximum_rows(shape, exact06, weights_gpu):
    """A 256-token prefill that emits every row: num_emit = 256, the most one forward takes (the
    LM-head GEMM over 16 row tiles), 2 layers; every row's token and logits against the exact
    oracle at the literal bar, and the rows in any order (emit reversed) give the same rows."""
    from qwen_megakernel.weights import make_prompt

    layers, n = 2, 256
    ids = make_prompt(n, shape.vocab, seed=29)
    dec = decoder(weights_gpu, num_layers=layers, max_seq_len=512)
    outs = []
    for emit in (list(range(n)), list(range(n - 1, -1, -1))):
        out = torch.empty(n, dtype=torch.int32, device="cuda")
        logits = torch.empty(n, V, dtype=torch.float32, device="cuda")
        dec._forward(_i32(ids), torch.zeros(n, dtype=torch.int32, device="cuda"),
                     torch.arange(n, dtype=torch.int32, device="cuda"), _i32(emit), out, logits, dec._k_cache,
                     dec._v_cache, n)
        outs.append((emit, out.cpu().tolist(), logits.cpu()))
    (e0, t0, l0), (e1, t1, l1) = outs
    assert t1[::-1] == t0 and torch.equal(l1.flip(0), l0), "the reversed emit list gave other rows"
    orc = exact_oracle(exact06, shape, 512, num_layers=layers)
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, 0, ids)
    print(check_rows(Tally("256 emitted rows"), ref, t0, l0, bar=LITERAL))
