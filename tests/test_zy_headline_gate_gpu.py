"""The headline's bandwidth gate as a test, as the reference gates achieved
bandwidth in its suite (tests/test_scan_scaling.py:41-80).

Config 1 exactly as bench.py measures it: gdn_decode_raw at B = 128 on a
160-slot fp16 pool with permuted slots and bf16 raw gates, step i on pool
i % 8 (8 pools of 160 MiB, so no state slab is cache-resident when it is
revisited). 256 steps are captured in one graph between two GPU clock stamps;
the graph is replayed for at least 50 ms first (the first replays after other
work run measurably slower), then 11 times timed. The median replay must move
the step's algorithmic bytes (274,744,064) at no less than 70% of the 8 TB/s
datasheet peak, the north star's target (<= 49.06 us a step).
"""
from __future__ import annotations

import time

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_config1_decode_sustains_70_percent_of_peak_hbm(kern):
    import bench

    pools, slot_maps, inputs, A, dtb = bench.make_workload(torch, 8)
    steps = 256

    def launch(i):
        p = i % len(pools)
        x = inputs[p]
        kern.gdn_decode_raw(pools[p], slot_maps[p], x["q"], x["k"], x["v"], x["a"], x["b"], A,
                            dtb, x["y"])

    for i in range(16):
        launch(i)
    torch.cuda.synchronize()
    clock = bench.GpuClock(torch)
    graph = bench.capture_clocked(torch, clock, lambda: [launch(i) for i in range(steps)])
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.05:
        graph.replay()
        torch.cuda.synchronize()
    times = sorted(bench.replay_times(torch, graph, 11, clock))
    secs = times[len(times) // 2] / steps
    gbs = bench.STEP_BYTES / secs / 1e9
    frac = gbs / bench.HBM_PEAK_GBS
    print(f"\nconfig 1 decode: {secs * 1e6:.2f} us/step, {gbs:.0f} GB/s, {frac * 100:.1f}% of "
          f"8 TB/s (replays {times[0] / steps * 1e6:.2f}-{times[-1] / steps * 1e6:.2f} us)")
    assert frac >= 0.70, (frac, [t / steps for t in times])
