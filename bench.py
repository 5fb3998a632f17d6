#!/usr/bin/env python3
"""Decode throughput of the gfx950 Qwen3-0.6B megakernel (one JSON line on stdout).

Workload: Qwen3-0.6B architecture, seeded synthetic bf16 weights, a 128-token
random prompt prefilled into the KV cache (batched forward, untimed), then K
greedy batch-1 decode steps with device-side token feedback (the reference's
``generate_nosync`` path).  A "step" is one decode token = one kernel launch.
W warm-up steps run first on a separate pass (then the cache is reset and the
prompt re-prefilled), so the K timed steps always cover contexts 129..128+K.

``value`` is decode tok/s over the timed region (inputs resident in HBM).
``roofline`` relates the decode kernel's algorithmic bytes per launch
(weights + KV read + KV written, averaged over the timed contexts) to its
average launch duration measured with HIP events on the launch stream.
``roofline.traffic`` is the kernel's HBM traffic per launch from the committed
counter profile (see TRAFFIC_PROFILE).  ``cpu_baseline`` times the repo's
PyTorch bf16 decode path (the CPU oracle, HF Qwen3 bf16 eager semantics) on
every core of the host's affinity set: the CPU reference configuration (16-token
prompt, 2 warm-up and 64 timed greedy steps), and a bounded sample of the GPU
workload (the 128-token prompt, then 384 greedy steps).

``long_context`` (skip with ``--no-long-context``): the same model with the KV
cache prefilled to 8192 and to 32768 positions with seeded N(0, 1) bf16 K/V
(28 layers x 8 KV heads x 128 dims), then 256 device-fed greedy steps each,
in tok/s and algorithmic GB/s (weights + KV read + KV written per token).

``qwen3_1p7b`` (skip with ``--no-1p7b``): the Qwen3-1.7B shape (hidden 2048,
MLP 6144, seeded N(0, 0.02) weights): a 512-token prompt prefilled, then 256
device-fed greedy steps at batch 1 on the decode megakernel (context
513..768); and ``batch4``: four sequences with their own 512-token prompts,
256 device-fed steps of the batched forward (MFMA GEMMs), in tok/s over all
four and algorithmic GB/s per step (weights once + each sequence's KV).

``prefill``: the 128-token prompt through the batched forward, ms and tok/s;
``prefill_long``: a 2048-token prompt the same way (its attention on MFMA);
``prefill_after_context``: the 128-token prompt appended after 4000 positions (a new turn of a
conversation: the MFMA attention over key chunks);
``prefill_lens`` (only with ``--prefill-lens 4,32,...``): prompts of those lengths, from position 0 or
``--prefill-start`` (a new turn appended to a conversation).
``context_1024``: the decode rate at exactly 1024 positions of context (a
1023-token prompt prefilled, then 512 decode launches at position 1023).

``sampling`` (skip with ``--no-sampling``): the same prompt and model, 512
device-fed steps of the sampled generate loop (counter-based Gumbel-max draws,
seed 0) with temperature only (drawn inside the decode kernel), top-k 50,
top-p 0.9, and both (temperature 0.8), in tok/s; greedy is ``value``.

``phases`` (skip with ``--no-phases``) is the per-phase weight-streaming
microbenchmark: each GEMV phase of the step (RMSNorm + QKV, O, gate/up +
SiLU*mul, down, LM head + argmax) run alone over >= 1 GiB of rotating seeded
N(0, 0.02) weight copies with N(0, 1) activations, in GB/s.

Options for profiling runs: ``--phase-trace`` adds the in-kernel phase trace
of one more step (at the context after the timed ones) to the JSON line, for
the Qwen3-0.6B run, each long-context run and Qwen3-1.7B at batch 1;
``--copy-calibration`` first runs a plain 1 GiB device-to-device copy five
times, so that a counter run (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE) sees a
kernel of known traffic beside the decode kernel.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

PEAK_HBM_GBS = 8000.0
PROMPT_LEN = 128
# HBM traffic of the decode kernel per launch (FETCH_SIZE + WRITE_SIZE), from two rocprofv3 --pmc
# runs of this script with --copy-calibration, each counter scaled by its own reading for the
# 1 GiB calibration copy and averaged over the timed dispatches by ``python -m
# qwen_megakernel.counters``; remeasured whenever the kernel changes.  The traffic beyond the
# algorithmic bytes (exchange words and their write-backs, the last layer's QKV rows read twice)
# does not depend on the context, so a run at other contexts reports its own algorithmic bytes
# plus that excess.
TRAFFIC_PROFILE = {
    "file": "profiles/decode_kernel_qwen3_0p6b_ctx129-1152_xcd_parallel.md",
    "contexts": "129..1152",
    "measured_bytes": 1_344_236_094,
    "algorithmic_bytes": 1_265_674_240,
}
METRIC = "decode tok/s, batch 1, Qwen3-0.6B bf16; achieved HBM GB/s vs ~8 TB/s peak"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(sample_steps: int = 384):
    """The repo's PyTorch bf16 decode path (the CPU oracle: HF Qwen3's bf16 eager semantics with
    torch CPU ops) on the host, on every core of the process's affinity set.

    ``value``: the CPU reference configuration -- Qwen3-0.6B seeded weights, the seeded 16-token
    prompt fed one step at a time, 2 warm-up greedy steps, then 64 timed greedy steps.  Also
    reported: a bounded sample of the GPU workload itself (the 128-token prompt, then
    ``sample_steps`` timed greedy steps at contexts 129..)."""
    import torch

    from oracle.qwen3_ref import OracleDecoder
    from qwen_megakernel.shapes import QWEN3_0_6B
    from qwen_megakernel.weights import make_prompt, make_weights

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    max_seq = PROMPT_LEN + sample_steps + 8
    w = make_weights(QWEN3_0_6B, seed=0, max_seq_len=max_seq)

    def timed(prompt_len, warm, steps):
        dec = OracleDecoder(w, QWEN3_0_6B, max_seq_len=max_seq)
        tok = None
        for t in make_prompt(prompt_len, QWEN3_0_6B.vocab, seed=1):
            tok = dec.step(t)
        for _ in range(warm):
            tok = dec.step(tok)
        t0 = time.perf_counter()
        for _ in range(steps):
            tok = dec.step(tok)
        return time.perf_counter() - t0

    dt0 = timed(16, 2, 64)
    dt1 = timed(PROMPT_LEN, 0, sample_steps)
    cpu = _cpu_model()
    return {"value": round(64 / dt0, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "ms_per_token": round(dt0 * 1e3 / 64, 2),
            "sample": f"CPU reference configuration: the repo's PyTorch bf16 decode (HF Qwen3 bf16 eager "
                      f"semantics, torch CPU ops), Qwen3-0.6B seeded weights, seeded 16-token prompt fed one "
                      f"step at a time, 2 warm-up steps, 64 greedy steps timed ({dt0:.1f} s); {cpu}, "
                      f"{threads} threads",
            "bench_workload_sample": {
                "tok_per_s": round(sample_steps / dt1, 3),
                "sample": f"the GPU workload's 128-token prompt fed untimed, then {sample_steps} greedy steps "
                          f"timed at context {PROMPT_LEN + 1}..{PROMPT_LEN + sample_steps} ({dt1:.1f} s)"}}


def long_context(w, steps: int, contexts=(8192, 32768), phase_trace: bool = False):
    """Decode `steps` device-fed greedy tokens after a KV cache prefilled with N(0, 1) K/V.

    ``phase_trace``: one more step after the timed ones, with the in-kernel trace on."""
    import torch

    from qwen_megakernel.model import Decoder
    from qwen_megakernel.shapes import QWEN3_0_6B as S
    from qwen_megakernel.weights import rope_tables

    out = {}
    max_seq = max(contexts) + steps + 64
    ww = dict(w)
    cos, sin = rope_tables(max_seq, S.head_dim, 1e6)
    ww["cos_table"], ww["sin_table"] = cos.cuda(), sin.cuda()
    dec = Decoder(weights=ww, verbose=False, max_seq_len=max_seq)
    ops = torch.ops.qwen_megakernel_C
    shp = (S.num_layers, S.num_kv_heads, max(contexts), S.head_dim)
    g = torch.Generator(device="cuda").manual_seed(2)
    k = torch.randn(shp, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(shp, generator=g, device="cuda").to(torch.bfloat16)
    for c0 in contexts:
        dec.reset()
        dec.load_kv(k, v, c0)
        ops.generate_nosync(11, 4, *dec._scratch(), S.num_layers, c0, max_seq, dec._attn_scale)  # warm-up
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        stream = torch.cuda.current_stream()
        torch.cuda.synchronize()
        e0.record(stream)
        ops.generate_nosync(11, steps, *dec._scratch(), S.num_layers, c0 + 4, max_seq, dec._attn_scale)
        e1.record(stream)
        torch.cuda.synchronize()
        assert int(ops.device_error()) == 0
        t = e0.elapsed_time(e1) / 1e3 / steps
        mean_c = c0 + 5 + (steps - 1) / 2.0
        byts = S.weight_bytes_per_token() + S.kv_bytes_per_position() * (mean_c + 1)
        out[str(c0)] = {"tok_per_s": round(1.0 / t, 2), "ms_per_token": round(t * 1e3, 4), "steps": steps,
                        "context": f"{c0 + 5}..{c0 + 4 + steps}", "achieved_GBps": round(byts / t / 1e9, 1),
                        "roofline_frac": round(byts / t / 1e9 / PEAK_HBM_GBS, 4)}
        log(f"long context {c0}: {1.0 / t:.1f} tok/s, {byts / t / 1e9:.0f} GB/s algorithmic")
        if phase_trace:
            from qwen_megakernel import trace

            dec._position = c0 + 4 + steps  # the cache holds every position before it
            stamps = trace.capture(lambda: dec.step(11), S.num_layers)
            summ = trace.summarize(stamps, S.num_layers)
            summ["context"] = c0 + 5 + steps
            out[str(c0)]["phase_trace"] = summ
            log(f"long-context phase trace at context {c0 + 5 + steps}:\n" + trace.format_table(summ))
    del dec, k, v
    torch.cuda.empty_cache()
    return out


def qwen3_1p7b(steps: int = 256, prompt_len: int = 512, batch: int = 4, phase_trace: bool = False):
    """Qwen3-1.7B at batch 1 and at batch `batch`.

    Batch 1: a `prompt_len`-token prompt prefilled, then `steps` device-fed steps of the decode
    megakernel.  Batch `batch`: `batch` sequences, each with its own `prompt_len`-token prompt
    (seeds 1..batch), all prefilled together in one batched forward, then `steps` device-fed batched
    steps (context 513..768 per sequence): one launch of the batched persistent kernel per step,
    and for comparison the same steps on the multi-launch batched step (``multi_launch``).
    """
    import torch

    from qwen_megakernel.model import BatchDecoder, Decoder
    from qwen_megakernel.shapes import QWEN3_1_7B as S
    from qwen_megakernel.weights import make_prompt, make_weights

    max_seq = prompt_len + steps + 64
    w = make_weights(S, seed=0, max_seq_len=max_seq, device="cuda")
    dec = Decoder(weights=w, verbose=False, max_seq_len=max_seq)
    ops = torch.ops.qwen_megakernel_C
    prompt = make_prompt(prompt_len, S.vocab, seed=1)
    dec.prefill(prompt[:-1])
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    ops.generate_nosync(prompt[-1], steps, *dec._scratch(), S.num_layers, dec.position, max_seq, dec._attn_scale)
    e1.record(stream)
    torch.cuda.synchronize()
    assert int(ops.device_error()) == 0
    t = e0.elapsed_time(e1) / 1e3 / steps
    trace_summary = None
    if phase_trace:
        from qwen_megakernel import trace

        # one more step, at the context after the timed ones, with the in-kernel trace on
        dec._position = prompt_len - 1 + steps
        stamps = trace.capture(lambda: dec.step(11), S.num_layers)
        trace_summary = trace.summarize(stamps, S.num_layers)
        trace_summary["context"] = prompt_len + steps
        log(f"qwen3-1.7b phase trace at context {prompt_len + steps}:\n" + trace.format_table(trace_summary))
    mean_c = prompt_len + (steps - 1) / 2.0
    byts = S.weight_bytes_per_token() + S.kv_bytes_per_position() * (mean_c + 1)
    del dec
    torch.cuda.empty_cache()
    log(f"qwen3-1.7b batch 1: {1.0 / t:.1f} tok/s, {byts / t / 1e9:.0f} GB/s algorithmic")
    out = {"tok_per_s": round(1.0 / t, 2), "ms_per_token": round(t * 1e3, 4), "batch": 1, "steps": steps,
           "context": f"{prompt_len}..{prompt_len + steps - 1}", "bytes_per_token": int(byts),
           "achieved_GBps": round(byts / t / 1e9, 1), "roofline_frac": round(byts / t / 1e9 / PEAK_HBM_GBS, 4)}
    if trace_summary is not None:
        out["phase_trace"] = trace_summary

    bd = BatchDecoder(weights=w, batch_size=batch, max_seq_len=max_seq, verbose=False)
    prompts = [make_prompt(prompt_len, S.vocab, seed=1 + b) for b in range(batch)]
    bd.prefill_all(prompts)  # untimed: the workspace allocation and first launches
    bd.reset()
    torch.cuda.synchronize()
    tp = time.perf_counter()
    first = bd.prefill_all(prompts)  # every prompt in one forward
    prefill_s = time.perf_counter() - tp
    first_t = torch.tensor(first, dtype=torch.int32, device="cuda")
    start_pos = bd.positions

    def timed_steps():
        bd.decode_steps(first_t, 4)  # warm-up (contexts 513..516), then rewind to the prefilled state
        bd._positions = list(start_pos)
        torch.cuda.synchronize()
        e0.record(stream)
        log_t = bd.decode_steps(first_t, steps)
        e1.record(stream)
        torch.cuda.synchronize()
        assert int(log_t.min()) >= 0 and int(ops.device_error()) == 0
        bd._positions = list(start_pos)
        return e0.elapsed_time(e1) / 1e3 / steps, log_t  # seconds per batched step

    was = ops.set_batch_persistent(False)
    try:
        tm, _ = timed_steps()
    finally:
        ops.set_batch_persistent(was)
    tb, log_p = timed_steps()
    batch_trace = None
    if phase_trace:
        from qwen_megakernel import trace

        bd._positions = [p + steps for p in start_pos]
        nxt = [int(t) for t in log_p[-1].tolist()]
        stamps = trace.capture(lambda: bd.step(nxt), S.num_layers)
        batch_trace = trace.summarize(stamps, S.num_layers)
        batch_trace["context"] = prompt_len + steps + 1
        log(f"qwen3-1.7b batch {batch} phase trace (control wave of sequence 0) at context {prompt_len + steps + 1}:\n"
            + trace.format_table(batch_trace))
    # per step: the weights once, each sequence's KV read over its context plus its new K/V row
    byts_b = S.weight_bytes_per_token() + batch * S.kv_bytes_per_position() * (mean_c + 1)
    del bd, w
    torch.cuda.empty_cache()
    log(f"qwen3-1.7b batch {batch}: {batch / tb:.1f} tok/s ({tb * 1e3:.3f} ms/step; multi-launch path "
        f"{tm * 1e3:.3f} ms/step), {byts_b / tb / 1e9:.0f} GB/s algorithmic; prefill {batch} x {prompt_len} tokens "
        f"in one forward {prefill_s * 1e3:.1f} ms")
    out["batch4"] = {"tok_per_s": round(batch / tb, 2), "ms_per_step": round(tb * 1e3, 4), "batch": batch,
                     "steps": steps, "context": f"{prompt_len + 1}..{prompt_len + steps} per sequence",
                     "bytes_per_step": int(byts_b), "achieved_GBps": round(byts_b / tb / 1e9, 1),
                     "roofline_frac": round(byts_b / tb / 1e9 / PEAK_HBM_GBS, 4),
                     "prefill_ms": round(prefill_s * 1e3, 2),
                     "path": "decode_batch: one launch of the batched persistent kernel per step (256 workgroups of "
                             "one control wave per sequence and 8 compute waves, tagged-word exchanges, HF's "
                             "two-pass attention per sequence, LM head and argmax in the same launch)",
                     "multi_launch": {"tok_per_s": round(batch / tm, 2), "ms_per_step": round(tm * 1e3, 4),
                                      "path": "7 launches per layer (K-split MFMA GEMMs; HF's two-pass attention "
                                              "split over all CUs: scores, probabilities times V, sum), streamed "
                                              "LM head"}}
    if batch_trace is not None:
        out["batch4"]["phase_trace"] = batch_trace
    return out


def context_1024_rate(w, launches: int = 512):
    """Decode rate at exactly 1024 positions of context: a 1023-token prompt prefilled, then
    `launches` back-to-back `decode` launches at position 1023 (each rewrites that position's K/V
    and attends over 1024 positions), timed with HIP events on the launch stream."""
    import torch

    from qwen_megakernel.model import Decoder
    from qwen_megakernel.shapes import QWEN3_0_6B as S
    from qwen_megakernel.weights import make_prompt

    dec = Decoder(weights=w, verbose=False, max_seq_len=2048)
    dec.prefill(make_prompt(1023, S.vocab, seed=1))
    args = (*dec._scratch(), dec._num_layers, 1023, dec._max_seq_len, dec._attn_scale)

    def run(n):
        for _ in range(n):
            dec._ops.decode(dec._out_token, 11, *args)

    run(32)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    run(launches)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / launches
    if int(dec._out_token.item()) < 0:
        raise RuntimeError("decode at context 1024 failed on the device")
    del dec
    torch.cuda.empty_cache()
    log(f"context 1024: {1e6 / us:.1f} tok/s, {us:.1f} us per step")
    return {"context": 1024, "launches": launches, "us_per_step": round(us, 2), "tok_per_s": round(1e6 / us, 1)}


def prefill_rate(w, prompt_len: int = PROMPT_LEN, iters: int = 10, start: int = 0):
    """Qwen3-0.6B prompt prefill through the batched forward: ms and tokens/s for `prompt_len` tokens
    at positions start.. (the cache rows before `start` are zero: the work does not depend on their
    values)."""
    import torch

    from qwen_megakernel.model import Decoder
    from qwen_megakernel.shapes import QWEN3_0_6B as S
    from qwen_megakernel.weights import make_prompt, rope_tables

    max_seq = max(2048, start + prompt_len)
    if w["cos_table"].shape[0] < max_seq:
        w = dict(w)
        cos, sin = rope_tables(max_seq, S.head_dim, 1e6)
        w["cos_table"], w["sin_table"] = cos.cuda(), sin.cuda()
    dec = Decoder(weights=w, verbose=False, max_seq_len=max_seq)
    prompt = make_prompt(prompt_len, S.vocab, seed=1)
    dec._position = start
    dec.prefill(prompt)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(iters):
        dec._position = start
        dec.prefill(prompt)
    e1.record(stream)
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) / 1e3 / iters
    del dec
    torch.cuda.empty_cache()
    at = f" after {start} positions" if start else ""
    log(f"prefill {prompt_len} tokens{at}: {t * 1e3:.3f} ms ({prompt_len / t:.0f} tok/s); one decode step per "
        f"token would take {prompt_len} launches")
    out = {"prompt_len": prompt_len, "ms": round(t * 1e3, 3), "tok_per_s": round(prompt_len / t, 1)}
    if start:
        out["start"] = start
    return out


def sampling(dec, prompt, max_seq: int, steps: int):
    """Sampled generate loop (generate_sample) from the prefilled prompt, per sampling setting."""
    import torch

    from qwen_megakernel.shapes import QWEN3_0_6B as S

    ops = torch.ops.qwen_megakernel_C
    steps = min(steps, max_seq - len(prompt))
    out = {"steps": steps, "context": f"{len(prompt)}..{len(prompt) + steps - 1}"}

    def run(n, T, k, p):
        return ops.generate_sample(prompt[-1], n, -1, T, k, p, 0, dec._embed_weight, dec._layer_weights_packed,
                                   dec._final_norm_weight, dec._lm_head_weight, dec._cos_table, dec._sin_table,
                                   dec._k_cache, dec._v_cache, dec._hidden, dec._norm_out, S.num_layers,
                                   dec.position, max_seq, dec._attn_scale)

    for name, (T, k, p) in (("temperature_1.0", (1.0, 0, 1.0)), ("top_k_50", (1.0, 50, 1.0)),
                            ("top_p_0.9", (1.0, 0, 0.9)), ("top_k_50_top_p_0.9_T0.8", (0.8, 50, 0.9))):
        dec.reset()
        dec.prefill(prompt[:-1])
        run(min(64, steps), T, k, p)  # records the loop's graph for these arguments
        dec.reset()
        dec.prefill(prompt[:-1])
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        toks = run(steps, T, k, p)
        e1.record(stream)
        torch.cuda.synchronize()
        assert toks.numel() == steps and int(ops.device_error()) == 0
        t = e0.elapsed_time(e1) / 1e3 / steps
        out[name] = {"tok_per_s": round(1.0 / t, 1), "ms_per_token": round(t * 1e3, 4)}
        log(f"sampling {name}: {1.0 / t:.1f} tok/s")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-steps", type=int, default=384)
    ap.add_argument("--phase-trace", action="store_true")
    ap.add_argument("--no-phases", action="store_true")
    ap.add_argument("--no-long-context", action="store_true")
    ap.add_argument("--long-steps", type=int, default=256)
    ap.add_argument("--no-1p7b", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--no-sampling", action="store_true")
    ap.add_argument("--sample-steps", type=int, default=512)
    ap.add_argument("--prefill-lens", default="", help="comma-separated prompt lengths to time prefill at as well")
    ap.add_argument("--prefill-start", type=int, default=0, help="position the --prefill-lens prompts start at")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this path does not shard "
              f"across GPUs)", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        sys.exit("steps must be >= 1 and warmup >= 0")

    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from qwen_megakernel.model import Decoder, HEAD_DIM
    from qwen_megakernel.shapes import QWEN3_0_6B
    from qwen_megakernel.weights import make_prompt, make_weights

    max_seq = 2048
    while PROMPT_LEN + max(args.steps, args.warmup) > max_seq:
        max_seq *= 2
    t0 = time.time()
    w = make_weights(QWEN3_0_6B, seed=0, max_seq_len=max_seq, device="cuda")
    dec = Decoder(weights=w, verbose=False, max_seq_len=max_seq)
    prompt = make_prompt(PROMPT_LEN, QWEN3_0_6B.vocab, seed=1)
    ops = torch.ops.qwen_megakernel_C
    log(f"setup {time.time() - t0:.1f}s")

    def prefill():
        dec.reset()
        dec.prefill(prompt[:-1])

    def run(n):
        return ops.generate_nosync(prompt[-1], n, *dec._scratch(), QWEN3_0_6B.num_layers, dec.position,
                                   max_seq, dec._attn_scale)

    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        src.fill_(1)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log("copy calibration: 5 x 1 GiB device copies")

    if args.warmup:
        prefill()
        run(args.warmup)
    prefill()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    toks = run(args.steps)  # synchronises the stream at the end
    e1.record(stream)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    gpu_ms = e0.elapsed_time(e1)
    assert toks.numel() == args.steps and int(ops.device_error()) == 0

    first_c = PROMPT_LEN + 1  # cache_len of the first timed step (position 128)
    mean_c = first_c + (args.steps - 1) / 2.0
    bytes_per_launch = QWEN3_0_6B.weight_bytes_per_token() + QWEN3_0_6B.kv_bytes_per_position() * (mean_c + 1)
    avg_launch_s = gpu_ms / 1e3 / args.steps
    achieved = bytes_per_launch / avg_launch_s / 1e9
    value = args.steps / dt
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "qwen3-0.6b greedy decode, batch 1, 128-token prompt prefilled, "
                               f"{args.steps} device-fed decode steps (context {first_c}..{PROMPT_LEN + args.steps})",
                   "batch": 1, "prompt_len": PROMPT_LEN, "decode_steps": args.steps, "max_seq_len": max_seq,
                   "weights": "seeded N(0,0.02) bf16, norms 1, tied embeddings"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": int(bytes_per_launch + TRAFFIC_PROFILE["measured_bytes"]
                                    - TRAFFIC_PROFILE["algorithmic_bytes"]),
                     "traffic_source": f"{TRAFFIC_PROFILE['file']}: FETCH_SIZE + WRITE_SIZE per launch at contexts "
                                       f"{TRAFFIC_PROFILE['contexts']}, {TRAFFIC_PROFILE['measured_bytes']} B against "
                                       f"{TRAFFIC_PROFILE['algorithmic_bytes']} algorithmic; the same excess "
                                       f"added to this run's algorithmic bytes",
                     "bytes_per_launch": int(bytes_per_launch), "avg_launch_us": round(avg_launch_s * 1e6, 2),
                     "kernel": "qmk::decode_kernel<Qwen3_0_6B, false, false>"},
        "cpu_baseline": None,
    }
    if args.phase_trace:
        from qwen_megakernel import trace

        last = PROMPT_LEN - 1 + args.steps  # position after the timed steps
        dec._position = last

        stamps = trace.capture(lambda: dec.step(int(toks[-1])), QWEN3_0_6B.num_layers)
        summ = trace.summarize(stamps, QWEN3_0_6B.num_layers)
        summ["context"] = last + 1
        result["phase_trace"] = summ
        log(f"phase trace at context {last + 1}:\n" + trace.format_table(summ))
    if not args.no_sampling:
        result["sampling"] = sampling(dec, prompt, max_seq, args.sample_steps)
    del dec  # frees the 128-token run's caches; the weights stay for the long-context runs
    torch.cuda.empty_cache()
    result["context_1024"] = context_1024_rate(w)
    result["prefill"] = prefill_rate(w)
    result["prefill_long"] = prefill_rate(w, 2048, iters=5)
    result["prefill_after_context"] = prefill_rate(w, PROMPT_LEN, start=4000)
    if args.prefill_lens:
        result["prefill_lens"] = [prefill_rate(w, int(n), start=args.prefill_start) for n in args.prefill_lens.split(",")]
    if not args.no_long_context:
        result["long_context"] = long_context(w, args.long_steps, phase_trace=args.phase_trace)
    del w
    torch.cuda.empty_cache()
    if not args.no_1p7b:
        result["qwen3_1p7b"] = qwen3_1p7b(phase_trace=args.phase_trace)
    if not args.no_phases:
        from qwen_megakernel import phases as P

        result["phases"] = {}
        for ph in P.phases():
            r = P.bench(ph)
            r["frac_of_peak"] = round(r["GBps"] / PEAK_HBM_GBS, 4)
            result["phases"][ph.name] = r
            log(f"phase {ph.name:18s} {r['GBps']:8.1f} GB/s ({r['us_per_copy']:.2f} us per "
                f"{ph.bytes / 1e6:.1f} MB copy, {r['copies']} copies)")
            torch.cuda.empty_cache()
    log(f"decode: {value:.1f} tok/s, {dt * 1e3 / args.steps:.3f} ms/token, kernel avg {avg_launch_s * 1e6:.1f} us, "
        f"{achieved:.0f} GB/s algorithmic")
    if not args.no_cpu_baseline:
        t0 = time.time()
        result["cpu_baseline"] = cpu_baseline(args.cpu_steps)
        log(f"cpu baseline {result['cpu_baseline']['value']} tok/s ({time.time() - t0:.1f}s)")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
