"""In-kernel phase trace of one decode step.

A decode step is a single kernel launch, so kernel-level profilers see one
dispatch per token and cannot split it into phases.  The kernel therefore
stamps the 100 MHz device wall clock itself when a trace buffer is set
(``torch.ops.qwen_megakernel_C.set_trace``): the control wave of every
workgroup at 13 points per layer plus 3 after the last layer, and compute
wave 0 of every workgroup at the start and end of its 6 phases per layer.
The reference has no tracing (its phases were inspected with Nsight out of
band); this module turns the stamps into per-phase times, exchange latencies
and barrier wake-up delays.
"""

from __future__ import annotations

import numpy as np
import torch

CTL_POINTS = 13        # control-wave stamps per layer
COMPUTE_POINTS = 12    # compute-wave stamps per layer (start/end of 6 phases)
FINAL_POINTS = 3
NUM_WG = 256
TICK_US = 0.01         # 100 MHz

# control-wave segments: stamp k -> k+1 inside a layer, then the hand-off to the next layer
CTL_SEGMENTS = [
    "gather h + RMSNorm",
    "barrier a (wake-up)",
    "QKV rows + qkv exchange + q/k norm + RoPE + KV append",
    "scores (compute waves)",
    "softmax (max, sum) exchange",
    "probabilities + P@V (compute waves)",
    "P@V partial exchange + combine + attention-output exchange",
    "barrier g (wake-up)",
    "o_proj rows + o reduce-scatter across XCDs + h' exchange + RMSNorm",
    "gate/up rows (compute waves)",
    "SiLU*up + m exchange",
    "barrier k (wake-up)",
    "down_proj rows + d reduce-scatter across XCDs + publish h''",
]
COMPUTE_PHASES = ["QKV", "scores", "P@V", "O", "gate/up", "down"]
CTL_READY = [1, 3, 5, 7, 9, 11]  # control stamp after which each compute phase may start


def entries(num_layers: int) -> int:
    return (num_layers * (CTL_POINTS + COMPUTE_POINTS) + FINAL_POINTS) * NUM_WG


def capture(step_fn, num_layers: int, device="cuda") -> np.ndarray:
    """Runs ``step_fn()`` (one decode launch on the current stream) with tracing on.

    Returns the stamps as int64 ``[points, 256]`` (ticks)."""
    ops = torch.ops.qwen_megakernel_C
    buf = torch.zeros(entries(num_layers), dtype=torch.int64, device=device)
    ops.set_trace(buf)
    try:
        step_fn()
        torch.cuda.synchronize()
    finally:
        ops.set_trace(None)
    return buf.cpu().numpy().reshape(-1, NUM_WG)


def summarize(stamps: np.ndarray, num_layers: int) -> dict:
    """Per-segment times (us; mean/min/max over layers 1.. and workgroups)."""
    names = CTL_SEGMENTS
    nl = num_layers
    t = (stamps - stamps[0].min()).astype(np.float64) * TICK_US
    ctl = t[: nl * CTL_POINTS].reshape(nl, CTL_POINTS, NUM_WG)
    fin = t[nl * CTL_POINTS: nl * CTL_POINTS + FINAL_POINTS]
    comp = t[nl * CTL_POINTS + FINAL_POINTS:].reshape(nl, COMPUTE_POINTS, NUM_WG)
    first = 1 if nl > 1 else 0
    segs = {}
    for k in range(CTL_POINTS - 1):
        v = (ctl[first:, k + 1] - ctl[first:, k]).ravel()
        segs[names[k]] = v
    if nl > 1:
        segs[names[-1]] = (ctl[1:, 0] - ctl[:-1, CTL_POINTS - 1]).ravel()
    out = {"segments_us": {k: {"mean": round(float(v.mean()), 3), "min": round(float(v.min()), 3),
                               "max": round(float(v.max()), 3)} for k, v in segs.items()}}
    layer = ctl[:, CTL_POINTS - 1].mean(axis=1) - ctl[:, 0].mean(axis=1)
    if nl > 1:
        per_layer = float(np.mean(ctl[1:, 0].mean(axis=1) - ctl[:-1, 0].mean(axis=1)))
    else:
        per_layer = float(layer[0])
    out["per_layer_us"] = round(per_layer, 3)
    out["final_norm_done_us"] = round(float(fin[0].mean()), 3)
    out["lm_head_us"] = round(float((fin[1] - fin[0]).mean()), 3)
    out["launch_us"] = round(float(fin[2, 0]), 3)
    busy, wake = {}, {}
    for k, name in enumerate(COMPUTE_PHASES):
        b = (comp[first:, 2 * k + 1] - comp[first:, 2 * k]).ravel()
        w = (comp[first:, 2 * k] - ctl[first:, CTL_READY[k]]).ravel()
        busy[name] = round(float(b.mean()), 3)
        wake[name] = round(float(w.mean()), 3)
    out["compute_busy_us"] = busy
    # time from the control wave's last stamp before a barrier to compute wave 0 starting after it
    out["barrier_wake_us"] = wake
    return out


def format_table(summary: dict) -> str:
    lines = [f"{'segment':62s} {'mean':>7s} {'min':>7s} {'max':>7s}  (us)"]
    for k, v in summary["segments_us"].items():
        lines.append(f"{k:62s} {v['mean']:7.2f} {v['min']:7.2f} {v['max']:7.2f}")
    lines.append(f"per layer {summary['per_layer_us']:.2f} us; LM head {summary['lm_head_us']:.2f} us; "
                 f"launch {summary['launch_us']:.2f} us")
    lines.append("compute wave busy (us): " + ", ".join(f"{k} {v:.2f}" for k, v in summary["compute_busy_us"].items()))
    lines.append("barrier wake (us):      " + ", ".join(f"{k} {v:.2f}" for k, v in summary["barrier_wake_us"].items()))
    return "\n".join(lines)
