"""GPU tests of sampling (qwen_megakernel/csrc/qmk_sample.hip) against the
sampling oracle (oracle/sampling_ref.py, itself pinned against HF's warpers in
tests/test_sampling.py).

Tokens must equal the oracle's for the same (seed, counter, logits).  A
difference is accepted only where the oracle itself is on a knife edge: its
two best perturbed scores within 1e-4, or a top-p boundary token whose keep
decision flips when top_p moves by 1e-5 (the kernel's exp and log differ from
numpy's by an ulp, and masses are compared against p * Z exactly).
"""

import numpy as np
import pytest
import torch

from oracle import sampling_ref as S
from parity import decoder as _decoder

pytestmark = pytest.mark.gpu


def _ops():
    from qwen_megakernel.build import get_extension

    return get_extension()


def _gpu_sample(logits, T, k, p, seed, counters):
    lg = torch.as_tensor(logits, dtype=torch.float32).cuda().contiguous()
    out = torch.empty(lg.shape[0], dtype=torch.int32, device="cuda")
    _ops().sample(lg, T, k, p, seed, torch.as_tensor(counters, dtype=torch.int64).cuda(), out)
    return out.cpu().tolist()


def _explained(row, T, k, p, seed, counter, got):
    """Is a differing token a knife-edge case of the oracle?"""
    _, gap = S.sample_row(row, T, k, p, seed, counter)
    if gap < 1e-4:
        return True
    for dp in (-1e-5, 1e-5):
        if 0 < p + dp < 1 and S.sample_row(row, T, k, p + dp, seed, counter)[0] == got:
            return True
    return False


def _compare(logits, T, k, p, seed, counters):
    got = _gpu_sample(logits, T, k, p, seed, counters)
    bad = 0
    for r, c in enumerate(counters):
        want = S.sample_row(logits[r], T, k, p, seed, c)[0]
        if got[r] != want:
            assert _explained(logits[r], T, k, p, seed, c, got[r]), f"row {r}: {got[r]} != {want}"
            bad += 1
    assert bad <= max(1, len(counters) // 100)
    return got


@pytest.mark.parametrize("T,k,p", [(0.0, 0, 1.0), (1.0, 0, 1.0), (0.7, 0, 0.9), (1.0, 50, 1.0), (1.3, 40, 0.8),
                                   (0.6, 1, 1.0), (1.0, 0, 0.05)])
def test_sample_rows_match_oracle_small_vocab(T, k, p):
    rng = np.random.default_rng(1)
    logits = (rng.standard_normal((64, 1000)) * 3).astype(np.float32)
    _compare(logits, T, k, p, 1234, list(range(100, 164)))


@pytest.mark.parametrize("T,k,p", [(0.8, 0, 0.95), (1.0, 20, 0.9), (0.0, 0, 1.0)])
def test_sample_rows_match_oracle_full_vocab(T, k, p):
    """Rows of the real vocabulary size (151936), bf16-valued like the model's logits."""
    rng = np.random.default_rng(2)
    logits = torch.from_numpy(rng.standard_normal((4, 151936)).astype(np.float32) * 2).bfloat16().float().numpy()
    _compare(logits, T, k, p, 7, [5, 6, 7, 1 << 33])


def test_sample_rows_beyond_one_launch_sequence_and_repeatable():
    """300 rows: more than one launch sequence (256 rows each, the per-row work is reused and must
    be left zeroed); every row matches the oracle, and a second call gives the same tokens."""
    rng = np.random.default_rng(4)
    logits = (rng.standard_normal((300, 1000)) * 3).astype(np.float32)
    first = _compare(logits, 0.9, 20, 0.9, 99, list(range(300)))
    assert _gpu_sample(logits, 0.9, 20, 0.9, 99, list(range(300))) == first


def test_sample_rows_on_two_streams_at_once():
    """Each stream has its own sampler work: two calls in flight on two streams draw what the same
    calls draw one after the other."""
    rng = np.random.default_rng(6)
    lg = torch.from_numpy((rng.standard_normal((8, 20000)) * 2).astype(np.float32)).cuda()
    ctr = torch.arange(8, dtype=torch.int64).cuda()
    cfgs = [(0.9, 30, 0.95, 1), (1.2, 0, 0.8, 2)]

    def call(cfg):
        out = torch.empty(8, dtype=torch.int32, device="cuda")
        T, k, p, seed = cfg
        _ops().sample(lg, T, k, p, seed, ctr, out)
        return out

    seq = []
    for cfg in cfgs:
        seq.append(call(cfg).cpu().tolist())
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    outs = []
    for st, cfg in zip(streams, cfgs):
        with torch.cuda.stream(st):
            outs.append(call(cfg))
    torch.cuda.synchronize()
    assert [o.cpu().tolist() for o in outs] == seq


def test_gpu_draws_follow_softmax():
    """4096 draws from one row (distinct counters): frequencies within 5 sd of softmax(logits / T)."""
    row = np.array([1.0, 0.2, -0.5, 2.0, 0.0, -3.0, 1.5, 0.7], dtype=np.float32)
    n, T = 4096, 0.8
    got = _gpu_sample(np.tile(row, (n, 1)), T, 0, 1.0, 99, list(range(n)))
    counts = np.bincount(got, minlength=row.size)
    s = row.astype(np.float64) / T
    pr = np.exp(s - s.max())
    pr /= pr.sum()
    sd = np.sqrt(n * pr * (1 - pr))
    assert np.all(np.abs(counts - n * pr) <= 5 * sd + 1), (counts, n * pr)


def test_generate_sample_matches_host_loop(weights_gpu, prompt):
    """The sampled device loop: each step's token is the oracle's draw from that step's logits with
    counter = the step's position (logits from a per-step decode of the same kernel)."""
    T, k, p, seed, n = 0.9, 40, 0.92, 5, 24
    dec = _decoder(weights_gpu)
    out = dec.generate(prompt, n, temperature=T, top_k=k, top_p=p, seed=seed)
    host = _decoder(weights_gpu)
    host.prefill(prompt[:-1])
    tok = prompt[-1]
    for i in range(n):
        pos = host.position
        _, lg = host.step_logits(tok)
        want = S.sample_row(lg.cpu().numpy(), T, k, p, seed, pos)[0]
        if out[i] != want:
            assert _explained(lg.cpu().numpy(), T, k, p, seed, pos, out[i]), f"step {i}: {out[i]} != {want}"
        tok = out[i]  # continue on the device's stream


def test_generate_sample_greedy_at_zero_temperature(weights_gpu, prompt):
    a = _decoder(weights_gpu).generate(prompt, 40)
    dec = _decoder(weights_gpu)
    b = dec.generate_ids(list(prompt), 40, temperature=0.0)
    assert a == b
    # the sampled loop with T = 0 through the sampler (greedy path of the sampling kernel)
    dec.reset()
    dec.prefill(prompt[:-1])
    c = _ops().generate_sample(prompt[-1], 40, -1, 0.0, 0, 1.0, 0, dec._embed_weight, dec._layer_weights_packed,
                               dec._final_norm_weight, dec._lm_head_weight, dec._cos_table, dec._sin_table,
                               dec._k_cache, dec._v_cache, dec._hidden, dec._norm_out, 28, dec.position, 2048,
                               dec._attn_scale).cpu().tolist()
    assert c == a


def test_generate_sample_graph_equals_direct_and_seeds_differ(weights_gpu, prompt):
    outs = []
    for graphs in (True, False, True):
        _ops().set_graph_launch(graphs)
        try:
            outs.append(_decoder(weights_gpu).generate(prompt, 70, temperature=1.0, top_p=0.95, seed=11))
        finally:
            _ops().set_graph_launch(True)
    assert outs[0] == outs[1] == outs[2]
    other = _decoder(weights_gpu).generate(prompt, 70, temperature=1.0, top_p=0.95, seed=12)
    assert other != outs[0]


def test_generate_sample_stops_at_eos(weights_gpu, prompt):
    free = _decoder(weights_gpu).generate(prompt, 40, temperature=1.0, seed=3)
    eos = free[10]
    k = free.index(eos)
    dec = _decoder(weights_gpu)
    out = dec.generate_ids(list(prompt), 40, eos_token_id=eos, temperature=1.0, seed=3)
    assert out[: k + 1] == free[: k + 1] and out[k + 1:] == [eos] * (40 - k - 1)
    assert dec.position == len(prompt) - 1 + k + 1


def test_batch_sampled_generate_matches_host_loop(shape, weights_gpu):
    """BatchDecoder with sampling: per-sequence counters (position + sequence << 32), each row the
    oracle's draw from that row's logits."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_prompt

    T, k, p, seed, n = 1.1, 0, 0.9, 21, 8
    prompts = [make_prompt(m, shape.vocab, seed=30 + m) for m in (6, 11)]
    bd = BatchDecoder(weights=weights_gpu, batch_size=2, max_seq_len=256, verbose=False)
    out = bd.generate_ids(prompts, n, temperature=T, top_k=k, top_p=p, seed=seed)
    ref = BatchDecoder(weights=weights_gpu, batch_size=2, max_seq_len=256, verbose=False)
    _, lg_all = ref.prefill_all(prompts, return_logits=True)  # the prompts in one forward, as generate_ids
    for b, pr in enumerate(prompts):
        lg = lg_all[b]
        c = (len(pr) - 1) + (b << 32)
        want = S.sample_row(lg.cpu().numpy(), T, k, p, seed, c)[0]
        assert out[b][0] == want or _explained(lg.cpu().numpy(), T, k, p, seed, c, out[b][0])
    for i in range(1, n):
        pos = ref.positions
        toks, lg = ref.step_logits([out[0][i - 1], out[1][i - 1]])
        for b in range(2):
            c = pos[b] + (b << 32)
            row = lg[b].cpu().numpy()
            want = S.sample_row(row, T, k, p, seed, c)[0]
            assert out[b][i] == want or _explained(row, T, k, p, seed, c, out[b][i]), f"seq {b} step {i}"


def test_fused_temperature_draw_equals_sampler(weights_gpu, prompt):
    """Temperature-only sampling runs inside the decode kernel's LM-head argmax (perturbed keys);
    with top_k = vocab (a filter that keeps everything) the loop takes the separate sampling
    kernel instead. Same draws, so the same tokens, with and without graph replay."""
    T, seed = 0.85, 77
    fused = _decoder(weights_gpu).generate(prompt, 48, temperature=T, seed=seed)
    separate = _decoder(weights_gpu).generate(prompt, 48, temperature=T, top_k=151936, seed=seed)
    assert fused == separate
    _ops().set_graph_launch(False)
    try:
        direct = _decoder(weights_gpu).generate(prompt, 48, temperature=T, seed=seed)
    finally:
        _ops().set_graph_launch(True)
    assert direct == fused
