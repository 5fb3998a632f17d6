"""Per-phase weight-streaming microbenchmark of the decode step's GEMVs.

Each phase of the decode kernel (RMSNorm + QKV 1024->4096, O 2048->1024,
gate/up 1024->2x3072 + SiLU*mul, down 3072->1024, LM head 1024->151936 +
argmax) is run on its own by ``torch.ops.qwen_megakernel_C.phase_bench`` over
a rotating set of distinct weight copies totalling at least ``min_bytes``
(1 GiB by default), so that neither L2 nor the 256 MB MALL serves repeats, as
the 1.19 GB weight stream of a real token does not fit them either.  Weights
are seeded N(0, 0.02) bf16, activations N(0, 1) bf16.  GB/s = copies x the
phase's weight bytes / kernel time (HIP events on the launch stream).

The reference has no such benchmark; it measures only whole-step throughput
(qwen_megakernel/bench.py).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .shapes import QWEN3_0_6B


@dataclass(frozen=True)
class Phase:
    name: str
    pid: int
    in_len: int
    weight_elems: int      # bf16 elements per copy
    extra_bytes: int = 0   # other bytes read per copy (norm weight)

    @property
    def bytes(self) -> int:
        return 2 * self.weight_elems + self.extra_bytes


def phases(shape=QWEN3_0_6B):
    h, i, q, kv, v = shape.hidden, shape.intermediate, shape.q_size, shape.kv_size, shape.vocab
    return [
        Phase("rmsnorm+qkv", 0, h, (q + 2 * kv) * h, 2 * h),
        Phase("o_proj", 1, q, h * q),
        Phase("gate_up+silu_mul", 2, h, 2 * i * h),
        Phase("down_proj", 3, i, h * i),
        Phase("lm_head+argmax", 4, h, v * h),
    ]


def out_buffer(ph: Phase, device) -> torch.Tensor:
    if ph.pid == 0:
        return torch.empty(4096, dtype=torch.bfloat16, device=device)
    if ph.pid in (1, 3):
        return torch.empty(8, 1024, dtype=torch.float32, device=device)
    if ph.pid == 2:
        return torch.empty(3072, dtype=torch.bfloat16, device=device)
    return torch.empty(256 * 8, dtype=torch.int64, device=device)


def make_inputs(ph: Phase, n_copies: int, seed: int = 0, device="cuda"):
    """``(weights [n_copies * elems] bf16, act bf16, norm_weight bf16 or None)``."""
    g = torch.Generator(device=device).manual_seed(seed)
    w = torch.empty(n_copies * ph.weight_elems, dtype=torch.bfloat16, device=device)
    for k in range(n_copies):
        seg = w[k * ph.weight_elems:(k + 1) * ph.weight_elems]
        seg.copy_(torch.randn(ph.weight_elems, generator=g, device=device) * 0.02)
    act = torch.randn(ph.in_len, generator=g, device=device).to(torch.bfloat16)
    norm = None
    if ph.pid == 0:
        norm = (1.0 + 0.1 * torch.randn(ph.in_len, generator=g, device=device)).to(torch.bfloat16)
    return w, act, norm


def run(ph: Phase, w, act, norm, n_copies: int, out=None):
    ops = torch.ops.qwen_megakernel_C
    if out is None:
        out = out_buffer(ph, w.device)
    ops.phase_bench(ph.pid, w, n_copies, norm, act, out)
    return out


def argmax_from_keys(keys: torch.Tensor) -> int:
    """Row index encoded by the largest (orderable logit << 32 | ~row) key."""
    k = keys.view(torch.int64).cpu()
    # keys are unsigned; compare as unsigned by flipping the sign bit
    best = int((k ^ (-(2 ** 63))).max().item() ^ (-(2 ** 63)))
    return 0xFFFFFFFF - (best & 0xFFFFFFFF)


def bench(ph: Phase, min_bytes: int = 1 << 30, iters: int = 5, seed: int = 0, device="cuda") -> dict:
    n = max(2, math.ceil(min_bytes / ph.bytes))
    w, act, norm = make_inputs(ph, n, seed, device)
    out = out_buffer(ph, device)
    run(ph, w, act, norm, n, out)  # warm-up (also pages the weights in)
    torch.cuda.synchronize()
    times = []
    stream = torch.cuda.current_stream()
    for _ in range(iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        run(ph, w, act, norm, n, out)
        e1.record(stream)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / 1e3)
    times.sort()
    t = times[len(times) // 2]
    del w
    return {"copies": n, "bytes_per_copy": ph.bytes, "rotation_bytes": n * ph.bytes,
            "us_per_copy": round(t / n * 1e6, 3), "GBps": round(n * ph.bytes / t / 1e9, 1)}
