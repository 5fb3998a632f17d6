"""Phase-trace decoding on synthetic stamps (CPU)."""

import numpy as np

from qwen_megakernel import trace


def test_summarize_synthetic_stamps():
    nl = 3
    n_pts = nl * (trace.CTL_POINTS + trace.COMPUTE_POINTS) + trace.FINAL_POINTS
    st = np.zeros((n_pts, trace.NUM_WG), dtype=np.int64)
    layer_ticks, seg_ticks = 1000, 60  # 13 stamps 60 ticks apart: last at 720, next layer at 1000
    for L in range(nl):
        for k in range(trace.CTL_POINTS):
            st[L * trace.CTL_POINTS + k] = 5000 + L * layer_ticks + k * seg_ticks
        for k in range(6):
            base = nl * trace.CTL_POINTS + trace.FINAL_POINTS + L * trace.COMPUTE_POINTS
            ready = 5000 + L * layer_ticks + trace.CTL_READY[k] * seg_ticks
            st[base + 2 * k] = ready + 7      # wakes 7 ticks after the control wave's stamp
            st[base + 2 * k + 1] = ready + 37  # busy 30 ticks
    f0 = nl * trace.CTL_POINTS
    st[f0] = 5000 + nl * layer_ticks + 100
    st[f0 + 1] = st[f0] + 4600
    st[f0 + 2, 0] = st[f0 + 1, 0] + 50
    s = trace.summarize(st, nl)
    assert abs(s["per_layer_us"] - 10.0) < 1e-9
    segs = list(s["segments_us"].values())
    assert all(abs(v["mean"] - 0.6) < 1e-9 for v in segs[:-1])
    assert abs(segs[-1]["mean"] - (layer_ticks - 12 * seg_ticks) * 0.01) < 1e-9
    assert abs(s["lm_head_us"] - 46.0) < 1e-9
    assert abs(s["launch_us"] - (nl * layer_ticks + 100 + 4600 + 50) * 0.01) < 1e-9
    assert all(abs(v - 0.3) < 1e-9 for v in s["compute_busy_us"].values())
    assert all(abs(v - 0.07) < 1e-9 for v in s["barrier_wake_us"].values())
    assert "per layer" in trace.format_table(s)
    assert trace.entries(28) == (28 * 25 + 3) * 256
