"""GPU tests of the batched persistent decode kernel (qmk_decode_batch_persistent).

decode_batch runs it for 2 to 4 sequences at contexts up to 2048; it is the
decode kernel's tagged-exchange design with every weight slice applied to all
rows of the batch.  Each test compares every sequence's rows with the exact
CPU oracle on that sequence's own cache (tests/parity.py), and where useful
with the multi-launch batched step on identical inputs.
"""

import contextlib

import pytest
import torch

from parity import (LAYERS28, LITERAL, Tally, check_kv_rows, check_rows, exact_oracle, history_envelopes, oracle_steps,
                    stream_rows, with_rope)

pytestmark = pytest.mark.gpu

V = 151936


def _ops():
    return torch.ops.qwen_megakernel_C


@contextlib.contextmanager
def persistent(on: bool):
    was = _ops().set_batch_persistent(on)
    try:
        yield
    finally:
        _ops().set_batch_persistent(was)


def _i32(values):
    return torch.tensor([int(v) for v in values], dtype=torch.int32, device="cuda")


def _step(bd, tokens, positions, max_context):
    out = torch.empty(len(tokens), dtype=torch.int32, device="cuda")
    lg = torch.empty(len(tokens), V, dtype=torch.float32, device="cuda")
    bd._forward.decode(_i32(tokens), _i32(positions), out, lg, bd._k_cache, bd._v_cache, max_context)
    return out.cpu().tolist(), lg.cpu()


@pytest.mark.parametrize("B", [2, 3, 4])
def test_persistent_batch_matches_oracle_and_launch_path(shape, exact06, weights_gpu, B):
    """B sequences with prompts of different lengths, 4 layers: every persistent step against the
    oracle on the sequence's own cache (literal bar) and the K/V rows it appended; then the same
    steps replayed through the multi-launch path from the same cache and tokens, checked against
    the oracle on its own cache the same way, and its logits within cosine 0.999 / max abs 0.1 of
    the persistent kernel's (the two round the softmax probabilities differently, so their greedy
    tokens are each held to the oracle, not to each other)."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_prompt

    layers, steps, max_seq = 4, 6, 256
    prompts = [make_prompt(n, shape.vocab, seed=70 + b) for b, n in enumerate([7, 30, 2, 19][:B])]
    bd = BatchDecoder(weights=weights_gpu, batch_size=B, max_seq_len=max_seq, num_layers=layers, verbose=False)
    first = bd.prefill_all(prompts)
    start = bd.positions
    k0, v0 = bd._k_cache.clone(), bd._v_cache.clone()
    feed, lgs = [[t] for t in first], [[] for _ in range(B)]
    with persistent(True):
        for i in range(steps):
            pos = [start[b] + i for b in range(B)]
            nxt, lg = _step(bd, [f[-1] for f in feed], pos, max(pos) + 1)
            for b in range(B):
                feed[b].append(nxt[b])
                lgs[b].append(lg[b])
    assert int(_ops().device_error()) == 0
    t = Tally(f"persistent batch {B}, 4 layers")
    for b in range(B):
        orc = exact_oracle(exact06, shape, max_seq, num_layers=layers)
        ref = oracle_steps(orc, bd._k_cache[b], bd._v_cache[b], start[b], feed[b][:-1])
        check_rows(t, ref, feed[b][1:], torch.stack(lgs[b]), bar=LITERAL)
        check_kv_rows(f"persistent batch {B} sequence {b}", orc, bd._k_cache[b], bd._v_cache[b], start[b], steps)
    print(t)
    kp = bd._k_cache.clone()
    bd._k_cache.copy_(k0)
    bd._v_cache.copy_(v0)
    out_l, lg_l = [[] for _ in range(B)], [[] for _ in range(B)]
    with persistent(False):
        for i in range(steps):
            pos = [start[b] + i for b in range(B)]
            nxt, lg = _step(bd, [feed[b][i] for b in range(B)], pos, max(pos) + 1)
            for b in range(B):
                out_l[b].append(nxt[b])
                lg_l[b].append(lg[b])
    t2 = Tally(f"multi-launch replay, batch {B}")
    for b in range(B):
        orc = exact_oracle(exact06, shape, max_seq, num_layers=layers)
        ref = oracle_steps(orc, bd._k_cache[b], bd._v_cache[b], start[b], feed[b][:-1])
        check_rows(t2, ref, out_l[b], torch.stack(lg_l[b]), bar=LITERAL)
        for i in range(steps):
            x, y = lgs[b][i].double(), lg_l[b][i].double()
            assert torch.nn.functional.cosine_similarity(x, y, dim=0).item() >= 0.999
            assert (x - y).abs().max().item() <= 0.1
    d = (kp[:, 0].float() - bd._k_cache[:, 0].float()).abs().max().item()
    assert d <= 0.0625, d
    print(t2)


@pytest.mark.parametrize("c0s", [(2045, 1, 700, 64), (1, 2045), (33, 1000, 0)],
                         ids=["batch4-2048", "batch2-edges", "batch3-empty"])
def test_persistent_batch_context_edges(shape, exact06, weights_gpu, c0s):
    """Injected N(0,1) caches up to the kernel's limit (contexts 2046..2048: 64 positions per
    workgroup, a full K/V batch per wave) beside contexts of 1-3 positions (most workgroups hold
    none) and an empty cache; 2 layers, three steps, every sequence against the oracle."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_kv_prefill

    B, layers, max_seq = len(c0s), 2, 2048
    bd = BatchDecoder(weights=with_rope(weights_gpu, max_seq, "cuda"), batch_size=B, max_seq_len=max_seq,
                      num_layers=layers, verbose=False)
    for b, c0 in enumerate(c0s):
        if c0:
            k, v = make_kv_prefill(shape, c0, seed=80 + b)
            bd.load_kv(b, k.cuda(), v.cuda(), c0)
    feed, lgs = [[13 + 5 * b] for b in range(B)], [[] for _ in range(B)]
    with persistent(True):
        for i in range(3):
            pos = [c0s[b] + i for b in range(B)]
            nxt, lg = _step(bd, [f[-1] for f in feed], pos, max(pos) + 1)
            for b in range(B):
                feed[b].append(nxt[b])
                lgs[b].append(lg[b])
    assert int(_ops().device_error()) == 0
    t = Tally(f"persistent batch, contexts {c0s}")
    for b in range(B):
        orc = exact_oracle(exact06, shape, max_seq, num_layers=layers)
        ref = oracle_steps(orc, bd._k_cache[b], bd._v_cache[b], c0s[b], feed[b][:-1])
        check_rows(t, ref, feed[b][1:], torch.stack(lgs[b]), bar=LITERAL)
        check_kv_rows(f"persistent batch sequence {b}", orc, bd._k_cache[b], bd._v_cache[b], c0s[b], 3)
    print(t)


def test_persistent_batch_qwen3_1p7b_three_sequences():
    """Qwen3-1.7B (hidden 2048, MLP 6144) at batch 3, 2 layers, prompts prefilled together, four
    persistent steps against the Qwen3-1.7B oracle."""
    from oracle.qwen3_exact import ExactWeights
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.shapes import QWEN3_1_7B
    from qwen_megakernel.weights import make_prompt, make_weights, to_device

    layers, max_seq = 2, 128
    w = make_weights(QWEN3_1_7B, seed=0, max_seq_len=max_seq, num_layers=layers)
    ex = ExactWeights(w, QWEN3_1_7B, num_layers=layers)
    prompts = [make_prompt(n, QWEN3_1_7B.vocab, seed=90 + b) for b, n in enumerate([9, 3, 21])]
    bd = BatchDecoder(weights=to_device(w, "cuda"), batch_size=3, max_seq_len=max_seq, num_layers=layers,
                      verbose=False)
    first = bd.prefill_all(prompts)
    start = bd.positions
    feed, lgs = [[t] for t in first], [[], [], []]
    with persistent(True):
        for i in range(4):
            pos = [start[b] + i for b in range(3)]
            nxt, lg = _step(bd, [f[-1] for f in feed], pos, max(pos) + 1)
            for b in range(3):
                feed[b].append(nxt[b])
                lgs[b].append(lg[b])
    assert int(_ops().device_error()) == 0
    t = Tally("persistent batch 3, Qwen3-1.7B, 2 layers")
    for b in range(3):
        orc = exact_oracle(ex, QWEN3_1_7B, max_seq, num_layers=layers)
        ref = oracle_steps(orc, bd._k_cache[b], bd._v_cache[b], start[b], feed[b][:-1])
        check_rows(t, ref, feed[b][1:], torch.stack(lgs[b]), bar=LITERAL)
        check_kv_rows(f"Qwen3-1.7B persistent sequence {b}", orc, bd._k_cache[b], bd._v_cache[b], start[b], 4)
    print(t)


def test_persistent_batch_invalid_rows_emit_minus_one(weights_gpu):
    """A token outside the vocabulary and a position outside max_context emit -1 and write no
    cache row; the valid rows of the same step are unaffected (equal to a step without them)."""
    from qwen_megakernel.model import BatchDecoder

    bd = BatchDecoder(weights=weights_gpu, batch_size=4, max_seq_len=64, num_layers=2, verbose=False)
    with persistent(True):
        out, lg = _step(bd, [5, V, 7, 9], [0, 1, 2, 40], 8)
    assert out[0] >= 0 and out[2] >= 0 and out[1] == -1 and out[3] == -1
    kc = bd._k_cache.float().cpu()
    assert kc[0, :, :, 0].abs().sum() > 0 and kc[2, :, :, 2].abs().sum() > 0
    assert kc[1].abs().sum() == 0 and kc[3].abs().sum() == 0
    bd.reset()
    with persistent(True):
        out2, lg2 = _step(bd, [5, 3, 7, 4], [0, 1, 2, 3], 8)
    assert out2[0] == out[0] and out2[2] == out[2]
    assert torch.equal(lg2[0], lg[0]) and torch.equal(lg2[2], lg[2])
    assert int(_ops().device_error()) == 0


def test_persistent_batch_deterministic(weights_gpu):
    """Fixed-order reductions: the same step twice gives bit-identical logits."""
    from qwen_megakernel.model import BatchDecoder

    res = []
    for _ in range(2):
        bd = BatchDecoder(weights=weights_gpu, batch_size=4, max_seq_len=64, num_layers=4, verbose=False)
        bd.prefill_all([[1, 2, 3], [4], [5, 6], [7, 8, 9, 10]])
        with persistent(True):
            res.append(_step(bd, [11, 12, 13, 14], bd.positions, max(bd.positions) + 1)[1])
    assert torch.equal(res[0], res[1])


def test_persistent_batch_bounded_failure_and_reset(weights_gpu):
    """A forced one-tick wait bound makes the persistent step fail fast: -1 for every row, the
    error bit latched, later steps refused until reset(); after it the step is exact again."""
    from qwen_megakernel.model import BatchDecoder

    ops = _ops()
    bd = BatchDecoder(weights=weights_gpu, batch_size=2, max_seq_len=64, num_layers=2, verbose=False)
    with persistent(True):
        good, good_lg = _step(bd, [3, 4], [0, 0], 1)
        bd.reset()
        ops.set_wait_limit(1)
        try:
            out, _ = _step(bd, [3, 4], [0, 0], 1)
            assert out == [-1, -1]
            assert int(ops.device_error()) & 1
            with pytest.raises(RuntimeError):  # the stream is poisoned until reset
                _step(bd, [3, 4], [0, 0], 1)
        finally:
            ops.set_wait_limit(0)
            ops.reset()
        assert int(ops.device_error()) == 0
        bd.reset()
        again, again_lg = _step(bd, [3, 4], [0, 0], 1)
    assert again == good and torch.equal(again_lg, good_lg)


def test_persistent_batch_generate_28_layers(shape, exact06, weights_cpu, weights_gpu):
    """Device-fed batched generation on the 28-layer model (BatchDecoder.generate_ids: prompts
    prefilled together, then 12 persistent steps without host synchronisation): every sequence's
    stream is the oracle's greedy stream of its own history (a token departure beyond one ulp only
    within the step's fp32 envelope)."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_prompt

    prompts = [make_prompt(n, shape.vocab, seed=100 + b) for b, n in enumerate([12, 40, 5, 26])]
    bd = BatchDecoder(weights=weights_gpu, batch_size=4, max_seq_len=2048, verbose=False)
    with persistent(True):
        out = bd.generate_ids(prompts, 13)
    assert int(_ops().device_error()) == 0
    t = Tally("persistent batched generate, 28 layers")
    for b in range(4):
        ref = stream_rows(exact_oracle(exact06, shape, 2048), bd._k_cache[b], bd._v_cache[b], prompts[b], out[b])
        envs = history_envelopes(weights_cpu, shape, 2048, bd._k_cache[b], bd._v_cache[b], prompts[b], out[b], ref)
        check_rows(t, ref, out[b], bar=LAYERS28, envs=envs)
    print(t)


def test_persistent_batch_long_stream_across_tag_wraps(weights_gpu):
    """600 device-fed batched steps on the 28-layer model at batch 2 (the 16-bit exchange tags
    advance by 253 per step and wrap about twice), on two streams: a fresh one and one whose
    batched state was first advanced by 37 steps, so the two meet every wrap at different steps.
    No device error, and the two token streams are identical."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_prompt

    prompts = [make_prompt(9, V, seed=120), make_prompt(4, V, seed=121)]
    ops = _ops()
    logs = []
    for i, st in enumerate((torch.cuda.Stream(), torch.cuda.Stream())):
        with torch.cuda.stream(st), persistent(True):
            ops.reset()
            if i == 1:
                warm = BatchDecoder(weights=weights_gpu, batch_size=2, max_seq_len=64, verbose=False)
                warm.decode_steps(_i32([1, 2]), 37)
            bd = BatchDecoder(weights=weights_gpu, batch_size=2, max_seq_len=1024, verbose=False)
            first = bd.prefill_all(prompts)
            log = bd.decode_steps(_i32(first), 600).cpu()
            assert int(ops.device_error()) == 0
        assert int(log.min()) >= 0 and int(log.max()) < V
        logs.append(log)
    assert torch.equal(logs[0], logs[1])


def test_in_place_batched_step_takes_the_multi_launch_path(shape, weights_gpu):
    """decode_batch with out_tokens sharing memory with tokens (an in-place step, batch 4 at a
    context the persistent kernel serves) succeeds and gives, bit for bit, the tokens of the same
    step with separate buffers on the multi-launch path, which reads its inputs before writing."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_prompt

    B, layers, max_seq = 4, 4, 256
    prompts = [make_prompt(n, shape.vocab, seed=90 + b) for b, n in enumerate([5, 9, 3, 12])]
    bd = BatchDecoder(weights=weights_gpu, batch_size=B, max_seq_len=max_seq, num_layers=layers, verbose=False)
    first = bd.prefill_all(prompts)
    pos = bd.positions
    k0, v0 = bd._k_cache.clone(), bd._v_cache.clone()
    results = {}
    for name, persistent_on, in_place in (("launches", False, False), ("persistent", True, False),
                                          ("in place", True, True)):
        bd._k_cache.copy_(k0)
        bd._v_cache.copy_(v0)
        toks = _i32(first)
        out = toks if in_place else torch.empty(B, dtype=torch.int32, device="cuda")
        with persistent(persistent_on):
            bd._forward.decode(toks, _i32(pos), out, None, bd._k_cache, bd._v_cache, max(pos) + 1)
        results[name] = out.cpu().tolist()
    assert int(_ops().device_error()) == 0
    assert min(results["launches"]) >= 0
    assert results["in place"] == results["launches"], results
    assert min(results["persistent"]) >= 0
