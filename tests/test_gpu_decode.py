"""GPU parity tests: the HIP decode kernel against the exact CPU oracle.

The bar and the near-tie rule are in tests/parity.py: per step, on the inputs
the kernel's step had (its token and its cache), logits cosine >= 0.999 and
max abs <= 0.1 against oracle/qwen3_exact.py (HF Qwen3's bf16 rounding points,
exact arithmetic between them), the greedy token equal to the oracle's argmax
except at a near-tie (gap below max(1e-2, one bf16 ulp)), and the K/V rows
the step wrote equal to the oracle's up to rounding.  No bound depends on the
CPU the test runs on.
"""

import ctypes
import math

import pytest
import torch

from parity import (ENVELOPE, LAYERS28, LITERAL, Tally, check_kv_rows, check_row, check_rows, decoder, envelope, exact_oracle,
                    fp32_oracle, kernel_stream, oracle_steps, stream_envelopes, stream_rows, with_rope)

pytestmark = pytest.mark.gpu


def test_decode_parity_qwen3_0p6b(shape, exact06, weights_cpu, weights_gpu, prompt):
    """Config-0 shapes: 16-token prompt fed one step at a time, then 64 greedy steps; every row
    (a token departure beyond one ulp only within the step's fp32 envelope)."""
    dec = decoder(weights_gpu)
    feed, toks, lgs = kernel_stream(dec, prompt, 64)
    orc = exact_oracle(exact06, shape, 2048)
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, 0, feed)
    envs = stream_envelopes(fp32_oracle(weights_cpu, shape, 2048), dec._k_cache, dec._v_cache, 0, feed, ref)
    print(check_rows(Tally("qwen3-0.6b 16+64"), ref, toks, lgs, bar=LAYERS28, envs=envs))
    check_kv_rows("qwen3-0.6b 16+64", orc, dec._k_cache, dec._v_cache, 0, len(feed))


def test_decode_parity_random_norm_weights(shape, prompt):
    """Non-unit norm weights (q/k/input/post/final) so an ignored norm weight fails."""
    from oracle.qwen3_exact import ExactOracle
    from qwen_megakernel.weights import make_weights, to_device

    w = make_weights(shape, seed=5, norm_std=0.1, num_layers=3, max_seq_len=256)
    dec = decoder(to_device(w, "cuda"), num_layers=3, max_seq_len=256)
    feed, toks, lgs = kernel_stream(dec, prompt, 16)
    orc = ExactOracle(w, shape, num_layers=3, max_seq_len=256)
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, 0, feed)
    print(check_rows(Tally("random norm weights, 3 layers"), ref, toks, lgs, bar=LITERAL))
    check_kv_rows("random norm weights", orc, dec._k_cache, dec._v_cache, 0, len(feed))


def test_generate_nosync_matches_oracle_stream(shape, exact06, weights_cpu, weights_gpu, prompt):
    """The device-fed greedy stream (generate_nosync) is the oracle's, up to near-ties."""
    dec = decoder(weights_gpu)
    out = dec.generate(prompt, 64)
    assert len(out) == 64 and dec.position == len(prompt) - 1 + 64
    ref = stream_rows(exact_oracle(exact06, shape, 2048), dec._k_cache, dec._v_cache, prompt, out)
    n0 = len(prompt) - 1
    envs = stream_envelopes(fp32_oracle(weights_cpu, shape, 2048), dec._k_cache, dec._v_cache, n0,
                            [prompt[-1]] + out[:-1], ref)
    print(check_rows(Tally("generate 64"), ref, out, bar=LAYERS28, envs=envs))


@pytest.fixture(scope="module")
def bench_workload(shape, exact06, weights_cpu, weights_gpu):
    """The decode benchmark's workload: the seeded 128-token prompt (seed 1) through the batched
    prefill, then 1024 device-fed greedy steps (contexts 129..1152), the exact oracle's logits for
    every row that produced a generated token, and (lazily) the fp32 envelopes of those rows."""
    from qwen_megakernel.weights import make_prompt

    prompt = make_prompt(128, shape.vocab, seed=1)
    dec = decoder(weights_gpu)
    out = dec.generate(prompt, 1024)
    assert len(out) == 1024 and dec.position == len(prompt) - 1 + 1024
    assert int(torch.ops.qwen_megakernel_C.device_error()) == 0
    orc = exact_oracle(exact06, shape, 2048)
    seq = list(prompt) + out[:-1]
    n0 = len(prompt) - 1
    # over the kernel's cache; row n0-1 is the prefill's last row
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, 0, seq, emit=list(range(n0 - 1, len(seq))))
    check_kv_rows("1024-step stream", orc, dec._k_cache, dec._v_cache, 0, len(seq))
    kc, vc = dec._k_cache.cpu(), dec._v_cache.cpu()
    envs = stream_envelopes(fp32_oracle(weights_cpu, shape, 2048), kc, vc, n0, seq[n0:], ref[1:])
    return prompt, out, ref, envs


def test_bench_workload_1024_step_stream(bench_workload):
    """Every one of the 1024 generated tokens is the oracle's argmax given the same prefix (tokens
    and cache), up to near-ties: the stream is the greedy stream of its own history."""
    prompt, out, ref, envs = bench_workload
    print(check_rows(Tally("1024-step stream"), ref[1:], out, bar=LAYERS28, envs=envs))


def test_bench_workload_256_steps_with_logits(shape, exact06, weights_cpu, weights_gpu, bench_workload):
    """The same prompt prefilled, then 256 decode steps (one launch each, logits out) on the
    decoder's own tokens: every row's logits within the bar, the prefill's last row too."""
    prompt, out, ref, _ = bench_workload
    n0 = len(prompt) - 1
    dec = decoder(weights_gpu)
    tok, lg = dec.prefill(prompt[:-1], return_logits=True)
    t = Tally("prefill + 256 steps")
    check_rows(t, ref[:1], [tok], lg[None].cpu(), labels=["prefill"], bar=LAYERS28)
    feed, toks, lgs = [prompt[-1]], [], []
    for i in range(256):
        tk, l = dec.step_logits(feed[-1])
        toks.append(tk)
        lgs.append(l.cpu())
        feed.append(tk)
    assert toks == out[:256], "step-by-step launches and the device-fed loop gave different streams"
    orc = exact_oracle(exact06, shape, 2048)
    rows = stream_rows(orc, dec._k_cache, dec._v_cache, prompt, toks)
    envs = stream_envelopes(fp32_oracle(weights_cpu, shape, 2048), dec._k_cache, dec._v_cache, n0,
                            [prompt[-1]] + toks[:-1], rows)
    print(check_rows(t, rows, toks, torch.stack(lgs), bar=LAYERS28, envs=envs))


@pytest.mark.parametrize(
    "c0,layers,steps",
    [(1500, 4, 6), (1500, 28, 8), (2100, 4, 6), (2100, 28, 8), (8192, 4, 4), (8192, 28, 16), (12300, 4, 4),
     (32768, 28, 8)],
    ids=["1500-4layers", "1500-28layers", "2100-4layers", "2100-28layers", "8192-4layers", "8192-28layers",
         "12300-4layers", "32768-28layers"])
def test_long_context_parity(shape, exact06, weights_cpu, weights_gpu, c0, layers, steps):
    """Attention over an injected N(0,1) cache of c0 positions (split over the 32 workgroups of
    an XCD, two passes; above 2048 positions the long-context kernel runs, each wave streaming several K/V
    batches through the LDS ring; at 2100 wave 0 has a second, partial batch; above 12288 the
    deep form, which starts both passes with the ring full; at 12300 the waves have 7 and 6
    batches).  Every step against the exact oracle on the step's own inputs, and the K/V rows the
    kernel appended.  Four layers: the literal bar.  28 layers, where no fp32 implementation holds
    the literal 0.1 (tests/test_oracle_fp32.py): every step within the fp32 envelope of the same
    step (tests/parity.py)."""
    from qwen_megakernel.weights import make_kv_prefill

    max_seq = c0 + 64
    k, v = make_kv_prefill(shape, c0, seed=2)
    dec = decoder(with_rope(weights_gpu, max_seq, "cuda"), num_layers=layers, max_seq_len=max_seq)
    dec.load_kv(k.cuda(), v.cuda(), c0)
    feed, toks, lgs = kernel_stream(dec, [11, 22], steps)
    assert torch.equal(dec._k_cache[:, :, :c0].cpu(), k[:layers, :, :c0])  # the injected rows are untouched
    orc = exact_oracle(exact06, shape, max_seq, num_layers=layers)
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, c0, feed)
    envs = None
    if layers == 28:
        envs = envelope(fp32_oracle(weights_cpu, shape, max_seq), dec._k_cache, dec._v_cache, c0, feed, ref)
    print(check_rows(Tally(f"context {c0} x {layers} layers"), ref, toks, lgs, bar=ENVELOPE if envs else LITERAL, envs=envs))
    check_kv_rows(f"context {c0} x {layers} layers", orc, dec._k_cache, dec._v_cache, c0, len(feed))


def test_decode_at_the_maximum_sequence_length(shape, exact06, weights_gpu):
    """max_seq_len = 65536, the largest the entry points accept (the deep form, 2048 positions per
    workgroup): an injected N(0,1) cache of 65532 positions, 4 layers, and 4 steps up to position
    65535, the last one.  Every step against the exact oracle on the step's own inputs at the literal
    bar, and the K/V rows the kernel appended; a further step is refused."""
    from dataclasses import replace

    from qwen_megakernel.weights import make_kv_prefill

    layers, max_seq = 4, 65536
    c0 = max_seq - 4
    k, v = make_kv_prefill(replace(shape, num_layers=layers), c0, seed=5)
    dec = decoder(with_rope(weights_gpu, max_seq, "cuda"), num_layers=layers, max_seq_len=max_seq)
    dec.load_kv(k.cuda(), v.cuda(), c0)
    del k, v
    feed, toks, lgs = kernel_stream(dec, [11, 22], 3)
    assert dec.position == max_seq
    assert int(torch.ops.qwen_megakernel_C.device_error()) == 0
    with pytest.raises(ValueError):
        dec.step(5)
    orc = exact_oracle(exact06, shape, max_seq, num_layers=layers)
    ref = oracle_steps(orc, dec._k_cache, dec._v_cache, c0, feed)
    print(check_rows(Tally(f"context {c0}..{max_seq - 1} x {layers} layers"), ref, toks, lgs, bar=LITERAL))
    check_kv_rows(f"context {c0} x {layers} layers", orc, dec._k_cache, dec._v_cache, c0, len(feed))


@pytest.mark.parametrize("c0", [8192, 32768], ids=["8192", "32768"])
def test_long_context_256_step_stream(shape, exact06, weights_cpu, weights_gpu, c0):
    """The long-context workload's full length: 256 device-fed greedy steps (generate_nosync, the
    long-form kernel) after an injected N(0,1) cache of c0 positions, 28 layers.  No device error;
    every one of the 256 tokens is the exact oracle's argmax given the same prefix (one causal pass
    of the oracle over the kernel's own cache and tokens), up to the fp32 envelope of that step;
    rows 0, 63, 127, 191 and 255 are decoded again for their logits (each step rewrites only its own
    K/V row, with the same values) and checked within the fp32 envelope of the same step."""
    from qwen_megakernel.weights import make_kv_prefill

    steps, max_seq = 256, c0 + 272
    ops = torch.ops.qwen_megakernel_C
    k, v = make_kv_prefill(shape, c0, seed=2)
    dec = decoder(with_rope(weights_gpu, max_seq, "cuda"), max_seq_len=max_seq)
    dec.load_kv(k.cuda(), v.cuda(), c0)
    out = ops.generate_nosync(11, steps, *dec._scratch(), shape.num_layers, c0, max_seq, dec._attn_scale).cpu().tolist()
    assert int(ops.device_error()) == 0
    assert all(0 <= t < shape.vocab for t in out)
    feed = [11] + out[:-1]  # the input of step i; out[i] follows it
    rows = [0, 63, 127, 191, 255]
    lgs = []
    for i in rows:
        dec._position = c0 + i
        tok, lg = dec.step_logits(feed[i])
        assert tok == out[i], f"step {i}: the repeated step gave {tok}, the stream {out[i]}"
        lgs.append(lg.cpu())
    del k, v
    kc, vc = dec._k_cache.cpu(), dec._v_cache.cpu()
    del dec
    orc = exact_oracle(exact06, shape, max_seq)
    ref = oracle_steps(orc, kc, vc, c0, feed)  # every row of the stream
    forc = fp32_oracle(weights_cpu, shape, max_seq)
    t = Tally(f"context {c0}, 256-step stream")
    check_rows(t, ref, out, bar=ENVELOPE, envs=stream_envelopes(forc, kc, vc, c0, feed, ref))
    for j, i in enumerate(rows):
        env = envelope(forc, kc, vc, c0 + i, [feed[i]], ref[i:i + 1])[0]
        check_row(t, ("logits", i), ref[i], out[i], lgs[j], bar=ENVELOPE, env=env)
    print(t)


@pytest.mark.parametrize("c0", [1990, 12248], ids=["short-long", "long-deep"])
def test_generate_across_long_context_boundary(shape, weights_gpu, c0):
    """generate_nosync from position 1990 for 100 steps runs contexts 1991..2090: the loop switches
    from the short-context kernel to the long-context one after context 2048, each form with its
    own recorded graph (from 12248, contexts 12249..12348: from the long form to the deep one after
    context 12288).  Its tokens equal those of 100 per-step launches, which pick the kernel by the
    same rule, with graph replay and with direct launches."""
    from qwen_megakernel.build import get_extension
    from qwen_megakernel.weights import make_kv_prefill

    n = 100
    max_seq = c0 + 210
    wg = with_rope(weights_gpu, max_seq, "cuda")
    k, v = make_kv_prefill(shape, c0, seed=3)

    def fresh():
        d = decoder(wg, max_seq_len=max_seq)
        d.load_kv(k.cuda(), v.cuda(), c0)
        return d

    ref = fresh()
    toks, t = [], 11
    for _ in range(n):
        t = ref.step(t)
        toks.append(t)
    ops = get_extension()
    for graphs in (True, False, True):
        ops.set_graph_launch(graphs)
        try:
            dec = fresh()
            out = ops.generate_nosync(11, n, *dec._scratch(), shape.num_layers, c0, max_seq,
                                      dec._attn_scale).cpu().tolist()
        finally:
            ops.set_graph_launch(True)
        assert out == toks, f"graphs={graphs}: first difference at step {next(i for i in range(n) if out[i] != toks[i])}"
    assert int(ops.device_error()) == 0


def test_last_position_and_bounds(shape, weights_gpu):
    dec = decoder(weights_gpu, max_seq_len=64)
    dec._position = 63
    tok = dec.step(5)
    assert 0 <= tok < shape.vocab and dec.position == 64
    with pytest.raises(ValueError):
        dec.step(5)
    with pytest.raises(RuntimeError):
        # the op checks the position itself, independent of the Python wrapper
        torch.ops.qwen_megakernel_C.decode(dec._out_token, 5, *dec._scratch(), 28, 64, 64, dec._attn_scale)


def test_deterministic(weights_gpu, prompt):
    a = decoder(weights_gpu)
    b = decoder(weights_gpu)
    for t in prompt[:6]:
        ta, la = a.step_logits(t)
        tb, lb = b.step_logits(t)
        assert ta == tb and torch.equal(la, lb)


def test_two_streams_do_not_interfere(weights_gpu, prompt):
    """Per-stream device state: two decoders on two streams, interleaved step by step."""
    ref = decoder(weights_gpu)
    expect = [ref.step(t) for t in prompt[:8]]
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    d1, d2 = decoder(weights_gpu), decoder(weights_gpu)
    got1, got2 = [], []
    for t in prompt[:8]:
        with torch.cuda.stream(s1):
            got1.append(d1.step(t))
        with torch.cuda.stream(s2):
            got2.append(d2.step(t))
    assert got1 == expect and got2 == expect


def _c_generate(lib, dec, first, steps, start, out, stream):
    vp = ctypes.c_void_p
    st = lib.qmk_generate_model(
        ctypes.c_int(0), ctypes.c_int(first), ctypes.c_int(steps), vp(dec._embed_weight.data_ptr()),
        vp(dec._layer_weights_packed.data_ptr()), vp(dec._final_norm_weight.data_ptr()),
        vp(dec._lm_head_weight.data_ptr()), vp(dec._cos_table.data_ptr()), vp(dec._sin_table.data_ptr()),
        vp(dec._k_cache.data_ptr()), vp(dec._v_cache.data_ptr()), vp(dec._hidden.data_ptr()),
        vp(dec._norm_out.data_ptr()), vp(out.data_ptr()), ctypes.c_int(28), ctypes.c_int(start),
        ctypes.c_int(dec._max_seq_len), ctypes.c_float(dec._attn_scale), vp(stream.cuda_stream))
    assert st == 0, lib.qmk_status_string(st)


def test_concurrent_generate_on_two_streams(shape, weights_gpu, prompt):
    """Two device-fed generate loops enqueued on two streams with no host synchronisation in
    between (through the C ABI, which does not synchronise).  Every launch needs all 256 CUs, so
    the library orders the second loop's launches after the first's; without that the two
    kernels would share the chip, wait for absent workgroups and latch a time-out.  Both streams
    give the single-stream tokens and no device error."""
    from qwen_megakernel.build import load_c_library

    lib = load_c_library()
    lib.qmk_status_string.restype = ctypes.c_char_p
    steps = 200
    ref = decoder(weights_gpu)
    expect = ref.generate(prompt, steps)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    d1, d2 = decoder(weights_gpu), decoder(weights_gpu)
    for d in (d1, d2):
        d.prefill(prompt[:-1])
    torch.cuda.synchronize()
    o1 = torch.empty(steps, dtype=torch.int32, device="cuda")
    o2 = torch.empty(steps, dtype=torch.int32, device="cuda")
    start = len(prompt) - 1
    _c_generate(lib, d1, prompt[-1], steps, start, o1, s1)
    _c_generate(lib, d2, prompt[-1], steps, start, o2, s2)
    s1.synchronize()
    s2.synchronize()
    ops = torch.ops.qwen_megakernel_C
    for s in (s1, s2):
        with torch.cuda.stream(s):
            assert int(ops.device_error()) == 0
    assert o1.cpu().tolist() == expect and o2.cpu().tolist() == expect


def test_c_abi_matches_torch_op(weights_gpu, prompt):
    """launch_ldg_decode_direct / _persistent through ctypes give the op's token and cache."""
    from qwen_megakernel.build import load_c_library

    lib = load_c_library()
    a = decoder(weights_gpu)
    b = decoder(weights_gpu)
    vp = ctypes.c_void_p
    stream = vp(torch.cuda.current_stream().cuda_stream)

    def args(d):
        return [vp(t.data_ptr()) for t in d._scratch()]

    for i, t in enumerate(prompt[:4]):
        ta = a.step(t)
        sc = args(b)
        fn = lib.launch_ldg_decode_direct if i % 2 == 0 else lib.launch_ldg_decode_persistent
        extra = [ctypes.c_int(28), ctypes.c_int(b.position)]
        if i % 2 == 1:
            extra.append(ctypes.c_int(b.position + 1))
        fn(ctypes.c_int(t), vp(b._out_token.data_ptr()), *sc, *extra, ctypes.c_int(2048),
           ctypes.c_float(1.0 / math.sqrt(128)), stream)
        assert lib.qmk_last_status() == 0
        torch.cuda.synchronize()
        b._position += 1
        assert int(b._out_token.item()) == ta
    assert torch.equal(a._k_cache, b._k_cache) and torch.equal(a._v_cache, b._v_cache)


def test_failure_path_is_bounded_and_resettable(weights_gpu, prompt):
    """A forced one-tick wait bound makes the step fail fast; reset() recovers."""
    ops = torch.ops.qwen_megakernel_C
    dec = decoder(weights_gpu)
    good = dec.step(prompt[0])
    dec.reset()
    ops.set_wait_limit(1)
    try:
        with pytest.raises(RuntimeError):
            dec.step(prompt[0])
        assert int(ops.device_error()) & 1
        with pytest.raises(RuntimeError):  # poisoned until reset
            dec.step(prompt[1])
    finally:
        ops.set_wait_limit(0)
        dec.reset()
    assert int(ops.device_error()) == 0
    assert dec.step(prompt[0]) == good


def test_ten_thousand_step_stream(shape, weights_gpu, prompt):
    """10,000 consecutive device-fed steps (contexts 16..10,015; about 39 wraps of the 16-bit
    exchange tags, the long-context kernel from context 2049 on) without a device error, twice:
    on a fresh stream state, and on a second stream whose tags were first advanced by 37 launches,
    so the two runs meet every tag wrap at different steps.  The two streams are identical."""
    steps, max_seq = 10000, 10048
    wg = with_rope(weights_gpu, max_seq, "cuda")
    ops = torch.ops.qwen_megakernel_C
    outs = []
    for i, s in enumerate((torch.cuda.Stream(), torch.cuda.Stream())):
        with torch.cuda.stream(s):
            ops.reset()
            if i == 1:
                warm = decoder(wg, max_seq_len=max_seq)
                ops.generate_nosync(7, 37, *warm._scratch(), shape.num_layers, 0, max_seq, warm._attn_scale)
            dec = decoder(wg, max_seq_len=max_seq)
            dec.prefill(prompt[:-1])
            out = ops.generate_nosync(prompt[-1], steps, *dec._scratch(), shape.num_layers, len(prompt) - 1,
                                      max_seq, dec._attn_scale).cpu().tolist()
            assert int(ops.device_error()) == 0
        assert all(0 <= t < shape.vocab for t in out)
        outs.append(out)
    assert outs[0] == outs[1], f"first difference at step {next(i for i in range(steps) if outs[0][i] != outs[1][i])}"
