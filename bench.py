"""Headline benchmark: batched GDN decode at B=128 on one MI355X.

Workload: one step = gdn_decode_raw over B=128 rows of a
Qwen3.5-9B-shaped GDN layer (32 value heads, 16 key heads, 128x128 fp16 state
per head, fp32 recurrence math, in-kernel gates from bf16 raw projections) on
a 160-slot fp16 state pool addressed through a random permutation of 128
distinct slots. Synthetic inputs, seeded.

Timing: K steps are captured in one hipGraph between two GPU wall-clock
stamps (a one-thread kernel writing s_memrealtime, libbraid_probe.so); the
graph is replayed 31 times, each replay between two synchronisations, and
timed between its stamps, so the graph's own launch latency (~10 us a replay)
is not charged to the K steps. `value` and `ms_per_step` are the median
replay (the reference's measure_graphed, noise_floor.py:52-105, which times
with events around the replay: that figure is reported beside it). The
default is COLD: step i runs on pool i % P, with P pools totalling > 1 GiB, so
neither the L2s nor the 256 MB Infinity Cache hold a state slab when it is
revisited (a single 160 MiB pool would fit and report above-HBM figures). The
HOT figure (one pool reused) is reported beside it, labelled.

Roofline: the decode is HBM-bound. Algorithmic bytes per step are
274,744,064 (state read + write 268,435,456; q/k/v/y 6,291,456; bf16 gates
16,384; A/dt_bias/slot map 768). achieved = bytes / mean step time; peak 8 TB/s.

stream_ceiling: the same 4096 state tiles streamed in place, read only and
written only by libbraid_probe.so at the decode's lane layout, with no
arithmetic and no q/k/v/y traffic: the ceiling the access pattern allows on
this box, beside the 8 TB/s datasheet peak.

cpu_baseline: the reference's CPU path, its batched torch decode restated in
oracle/torch_ref.py, timed on whole B=128 steps of the same workload with
torch's CPU threads (about 12 s of work). cpu_oracle_scalar: the scalar C
oracle on a sample of rows, one thread, scaled to steps/s at B=128.

"paths" (skip with --no-paths) times the other rows of the hot path on their
BASELINE shapes, each captured in a hipGraph and timed with events:
  decode_b128_*_pool  the config-1 step on a bf16 and on an fp32 pool
  prefill_config2   gdn_prefill_raw, 8 ragged rows of U[64, 1024] tokens, fp16
                    pool (tokens/s; FP32 flops vs the 157.3 TFLOP/s peak)
  prefill_tick      gdn_prefill_raw, 4 rows x 256 tokens (config 4's chunks)
  conv1d_prefill_config2  the chunked causal conv before config 2's scan
                    (bytes: bf16 x in, fp32 out over the padded [8, T, 8192])
  conv1d_decode     B=64, C=8192, K=4, bf16 in (HBM bytes per the layout)
  quantize_act      [64, 4096] bf16 (both launches)
  readout_quant_*   gated RMSNorm readout + out_proj input FP8 quant (both
                    launches), 64 decode tokens and config 2's 4073 tokens
  fp8_gemm_*        config 3's FP8 projection GEMMs at B=64, streaming kernel
                    (bytes: fp8 weight + x + bf16 out), weights cycled through
                    HBM; hipBLASLt and torch._scaled_mm beside it
  mixer_step        config 3: 24 GDN layers of quant -> conv -> gated decode at
                    B=64, one fp16 pool and conv pool per layer
  mixer_step_fused  the same step with conv + decode fused in one launch
  prefill_one_row_512, prefill_skewed_1x1024_15x128
                    small prefill batches: one long row; one long row among
                    short ones
  mixed_tick        config 4: 4 x 256-token prefill + 96 decode rows on one
                    192-slot fp16 pool; eager and graph-replayed per bucket, the
                    decode beside the prefill (MixedTick) and in sequence

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                       [--no-paths]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

H, G, D = 32, 16, 128
B, SLOTS = 128, 160
STATE_BYTES = B * H * D * D * 2 * 2                 # fp16 read + write
ACT_BYTES = B * (2 * G * D + 2 * H * D) * 4         # q, k, v in; y out (fp32)
GATE_BYTES = B * H * 2 * 2                          # a_raw, b_raw bf16
CONST_BYTES = 2 * H * 4 + B * 4                     # A, dt_bias, slot map
STEP_BYTES = STATE_BYTES + ACT_BYTES + GATE_BYTES + CONST_BYTES
HBM_PEAK_GBS = 8000.0
COLD_BYTES = 1.1 * 2 ** 30
TRAFFIC_FILE = ROOT / "profiles" / "gdn_decode_b128_traffic.json"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-paths", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="budget for the CPU-oracle baseline sample")
    return ap.parse_args()


def make_workload(torch, n_pools, seed=0):
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(seed)
    pools, slot_maps, inputs = [], [], []
    for p in range(n_pools):
        pools.append((torch.randn(SLOTS, H, D, D, generator=g, device=dev) * 0.02).half())
        perm = torch.randperm(SLOTS, generator=torch.Generator().manual_seed(seed + p))
        slot_maps.append(perm[:B].to(torch.int32).to(dev))
        inputs.append(dict(
            q=torch.randn(B, G, D, generator=g, device=dev),
            k=torch.randn(B, G, D, generator=g, device=dev),
            v=torch.randn(B, H, D, generator=g, device=dev),
            a=torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16),
            b=torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16),
            y=torch.empty(B, H, D, device=dev),
        ))
    A = -torch.exp(torch.rand(H, generator=g, device=dev) * 2)
    dt_bias = torch.rand(H, generator=g, device=dev) * 2 - 1
    return pools, slot_maps, inputs, A, dt_bias


def _busy(torch):
    """Keep the GPU busy for ~0.2 ms so that the host has queued the graph
    replay behind the start event before the GPU reaches it."""
    torch.cuda._sleep(200_000)


class GpuClock:
    """GPU wall-clock stamps inside a captured graph (libbraid_probe.so's
    braid_probe_clock: a one-thread kernel that writes the constant-rate
    s_memrealtime counter). A stamp before the first timed launch and one
    after the last bracket exactly the timed launches on the GPU's own clock,
    so the graph's launch latency (about 10 us per replay on MI355X, which
    events around graph.replay() include) stays outside the timed region; the
    second stamp's kernel runs only after the last timed launch completes."""

    def __init__(self, torch):
        import ctypes

        from braid_amd.build import PROBE_LIB

        lib = ctypes.CDLL(str(PROBE_LIB))
        self._stamp = lib.braid_probe_clock
        self._stamp.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self._stamp.restype = ctypes.c_int
        rate = lib.braid_probe_clock_hz
        rate.restype = ctypes.c_double
        self.hz = rate()
        if self.hz <= 0:
            raise RuntimeError("the GPU wall-clock rate is unknown")
        self.buf = torch.zeros(2, dtype=torch.int64, device="cuda")
        self.torch = torch

    def stamp(self, i):
        rc = self._stamp(self.buf[i:].data_ptr(), self.torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(f"braid_probe_clock failed ({rc})")

    def seconds(self):
        t0, t1 = self.buf.tolist()
        return (t1 - t0) / self.hz


def capture_clocked(torch, clock, body):
    """A graph of: stamp 0, body(), stamp 1."""
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        clock.stamp(0)
        body()
        clock.stamp(1)
    return graph


def replay_times(torch, graph, reps, clock=None):
    """Seconds of each of `reps` replays of `graph`, each bracketed by
    synchronisations: between the graph's two clock stamps when `clock` is
    given, else with events on the launch stream around the replay."""
    out = []
    for _ in range(reps):
        torch.cuda.synchronize()
        if clock is not None:
            graph.replay()
            torch.cuda.synchronize()
            out.append(clock.seconds())
            continue
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        _busy(torch)
        a.record()
        graph.replay()
        b.record()
        torch.cuda.synchronize()
        out.append(a.elapsed_time(b) / 1e3)
    return out


def time_steps(torch, kern, work, steps, warmup, reps=31):
    """Capture `steps` decode launches (step i on pool i % P) in one graph,
    bracketed by GPU clock stamps, and replay it `reps` times, each replay
    timed alone (the reference's measure_graphed, braid/bench/noise_floor.py
    :52-105, on the GPU's clock), after 50 ms of untimed replays. Returns the
    median seconds for the `steps` launches and the per-step spread, with the
    event-timed figure of the same replays (graph launch latency included)
    beside it."""
    pools, slot_maps, inputs, A, dtb = work
    P = len(pools)
    clock = GpuClock(torch)

    def launch(i):
        p = i % P
        x = inputs[p]
        kern.gdn_decode_raw(pools[p], slot_maps[p], x["q"], x["k"], x["v"], x["a"], x["b"], A,
                            dtb, x["y"])

    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    graph = capture_clocked(torch, clock, lambda: [launch(i) for i in range(steps)])
    # Untimed replays for at least 50 ms first (the first uploads the graph):
    # the first replays after other work run measurably slower, and with a
    # short graph (K = 20 is about 1 ms) they would set the upper percentiles.
    warm = time.perf_counter()
    n_warm = 0
    while n_warm < 2 or time.perf_counter() - warm < 0.05:
        graph.replay()
        torch.cuda.synchronize()
        n_warm += 1
    times = replay_times(torch, graph, reps, clock)
    ev = sorted(replay_times(torch, graph, 11))
    first = times[0]
    times.sort()
    q = lambda f: round(times[min(len(times) - 1, int(f * len(times)))] * 1e6 / steps, 3)
    median = times[len(times) // 2]
    return median, {"reps": reps, "steps_per_rep": steps, "p10_us": q(0.1),
                    "p50_us": q(0.5), "p90_us": q(0.9),
                    "first_rep_us": round(first * 1e6 / steps, 3),
                    "event_timed_p50_us": round(ev[len(ev) // 2] * 1e6 / steps, 3)}


def copy_bandwidth(torch, nbytes=2 ** 30):
    src = torch.empty(nbytes // 2, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 10
    start.record()
    for _ in range(reps):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    secs = start.elapsed_time(end) / 1e3 / reps
    del src, dst
    return 2 * nbytes / secs / 1e9


def stream_ceiling(torch, n_pools, launches=256, order="row_major"):
    """What an in-place stream of the step's state tiles reaches on this box:
    libbraid_probe.so's read-modify-write, read-only and write-only passes
    over the same 4096 tiles of 32 KiB (slot-permuted, cold pools, the
    decode's lane layout, nontemporal 128-bit accesses), without the
    arithmetic or the q/k/v/y traffic. Captured in one graph, timed on the
    GPU clock. GB/s count the state bytes each pass moves.

    `order` is the order the launch visits the same tiles in: "row_major" is
    the decode's (row b's 32 heads are consecutive tiles); "head_major" puts
    head h of every row together; "shuffled" is a seeded random order."""
    import ctypes

    from braid_amd.build import PROBE_LIB

    lib = ctypes.CDLL(str(PROBE_LIB))
    fn = lib.braid_probe_stream
    fn.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                   ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    dev = "cuda"
    pools = [torch.empty(SLOTS * H * D * D, dtype=torch.float16, device=dev)
             for _ in range(n_pools)]
    for p in pools:
        p.normal_()
    maps = []
    for p in range(n_pools):
        perm = torch.randperm(SLOTS, generator=torch.Generator().manual_seed(p))[:B]
        tiles = perm[:, None] * H + torch.arange(H)[None, :]
        if order == "head_major":
            tiles = tiles.t()
        tiles = tiles.reshape(-1)
        if order == "shuffled":
            tiles = tiles[torch.randperm(tiles.numel(),
                                         generator=torch.Generator().manual_seed(100 + p))]
        maps.append(tiles.to(torch.int32).to(dev))
    sink = torch.empty(1024, dtype=torch.int32, device=dev)
    n_tiles = B * H
    tile_bytes = D * D * 2
    out = {}
    for kind, label, nbytes in ((0, "rmw", 2 * n_tiles * tile_bytes),
                                (1, "read", n_tiles * tile_bytes),
                                (2, "write", n_tiles * tile_bytes)):
        def launch(i):
            st = torch.cuda.current_stream().cuda_stream
            rc = fn(kind, pools[i % n_pools].data_ptr(), n_tiles, maps[i % n_pools].data_ptr(),
                    sink.data_ptr(), st)
            if rc != 0:
                raise RuntimeError(f"braid_probe_stream failed ({rc})")

        for i in range(2 * n_pools):
            launch(i)
        torch.cuda.synchronize()
        clock = GpuClock(torch)
        graph = capture_clocked(torch, clock, lambda: [launch(i) for i in range(launches)])
        graph.replay()
        torch.cuda.synchronize()
        t = sorted(replay_times(torch, graph, 5, clock))
        secs = t[len(t) // 2] / launches
        out[f"{label}_us"] = round(secs * 1e6, 2)
        out[f"{label}_gbs"] = round(nbytes / secs / 1e9, 1)
    del pools
    return out


def cpu_baseline(budget_s):
    """The reference's CPU path: oracle/torch_ref.py restates its batched torch
    decode step (braid/reference/gdn_ref.py:69-99, gates gdn.py:299-300) over
    a slot-indexed fp16 pool. Timed on the host at the full config-1 step
    (B = 128, 160-slot fp16 pool, bf16 raw gates) with torch's CPU threads,
    as many whole steps as fit in `budget_s`."""
    import torch

    from oracle import torch_ref

    g = torch.Generator().manual_seed(0)
    pool = (torch.randn(SLOTS, H, D, D, generator=g) * 0.02).half()
    slots = torch.randperm(SLOTS, generator=g)[:B].to(torch.int32)
    A = -torch.exp(torch.rand(H, generator=g) * 2)
    dtb = torch.rand(H, generator=g) * 2 - 1

    def inputs():
        return (torch.randn(B, G, D, generator=g), torch.randn(B, G, D, generator=g),
                torch.randn(B, H, D, generator=g),
                torch.randn(B, H, generator=g).to(torch.bfloat16),
                torch.randn(B, H, generator=g).to(torch.bfloat16))

    torch_ref.decode_step(pool, slots, *inputs(), A, dtb)     # warm-up
    steps, spent = 0, 0.0
    while spent < budget_s and steps < 1000:
        x = inputs()
        t = time.perf_counter()
        torch_ref.decode_step(pool, slots, *x, A, dtb)
        spent += time.perf_counter() - t
        steps += 1
    threads = torch.get_num_threads()
    return {"value": round(steps / spent, 3), "unit": "steps/s", "cores": threads,
            "kind": "port",
            "sample": f"{steps} full B=128 steps of the reference's batched torch decode "
                      f"restated on the CPU (oracle/torch_ref.py: fp16 pool gathered by slot, "
                      f"fp32 math, bf16 raw gates), {spent:.1f} s on {threads} torch threads",
            "host_cpus": os.cpu_count()}


def cpu_oracle_scalar(budget_s):
    """The scalar C oracle (one thread) on whole rows of the same step, scaled
    to steps/s at B = 128: the per-element cost without vectorisation."""
    import numpy as np

    import oracle

    rng = np.random.default_rng(0)
    A = -np.exp(rng.uniform(0, 2, H)).astype(np.float32)
    dtb = rng.uniform(-1, 1, H).astype(np.float32)

    def one_row():
        pool = (rng.standard_normal((1, H, D, D)) * 0.02).astype(np.float16)
        q = rng.standard_normal((1, G, D)).astype(np.float32)
        k = rng.standard_normal((1, G, D)).astype(np.float32)
        v = rng.standard_normal((1, H, D)).astype(np.float32)
        a = oracle.bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
        b = oracle.bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
        t = time.perf_counter()
        al, be = oracle.gdn_gates(a, b, A, dtb, "bf16")
        oracle.gdn_decode(pool, [0], q, k, v, al, be, "f16")
        return time.perf_counter() - t

    one_row()
    rows, spent = 0, 0.0
    while spent < budget_s and rows < 64 * B:
        spent += one_row()
        rows += 1
    return {"value": round(1.0 / (spent / rows * B), 3), "unit": "steps/s", "cores": 1,
            "sample": f"{rows} rows on the scalar C oracle, {spent:.1f} s, scaled x{B}/rows"}


FP32_PEAK_TFLOPS = 157.3
FLOP_PER_TOKEN_HEAD = 7 * 128 * 128   # kv fma, alpha*S, update fma, readout fma (114,688)
CONV_BYTES_B64 = (64 * 8192 * 3 * 4 + 64 * 8192 * 4 * 4 + 64 * 8192 * 2 + 64 * 8192 * 4
                  + 8192 * 4 * 4 + 8192 * 4)
QUANT_BYTES_64x4096 = 64 * 4096 * 2 + 64 * 4096 + 4
ROW_BYTES = 2 * H * D * D * 2 + (2 * G * D + 2 * H * D) * 4 + H * 2 * 2 + 4
# readout per element: y fp32 + z bf16 read, core bf16 written and read back
# by the quantize pass, fp8 code written
READOUT_BYTES_PER_ELEM = 4 + 2 + 2 + 2 + 1


def graph_time(torch, fn, reps=11, inner=1, before_replay=None):
    """Median seconds per call of `fn`, replayed from a captured graph.
    `before_replay` runs once after capture (e.g. to point padded rows at a
    scratch slot, which eager validation would refuse as a duplicate)."""
    fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    clock = GpuClock(torch)
    graph = capture_clocked(torch, clock, lambda: [fn() for _ in range(inner)])
    if before_replay is not None:
        before_replay()
    # Replay for at least 20 ms first: the first replays of a kernel after other
    # work run measurably slower (config 2's prefill: 0.617 ms for about 20
    # launches, then 0.572 ms), so timing starts at the steady state.
    warm = time.perf_counter()
    n_warm = 0
    while n_warm < 3 or time.perf_counter() - warm < 0.02:
        graph.replay()
        torch.cuda.synchronize()
        n_warm += 1
    times = sorted(t / inner for t in replay_times(torch, graph, reps, clock))
    return times[len(times) // 2]


def measure_paths(torch, kern):
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(11)
    A = -torch.exp(torch.rand(H, generator=g, device=dev) * 2)
    dtb = torch.rand(H, generator=g, device=dev) * 2 - 1
    out = {}

    import ctypes
    import numpy as np

    def prefill_case(lens):
        """Kernel time of the plan an eager call runs (chosen on the host from
        seq_lens, braid_prefill_plan), captured with that plan forced; beside
        it the host's planning time, the time of a captured call, which plans
        in the kernel, and of a captured call given the host lengths to plan
        from (plan_lens)."""
        Bp, T = len(lens), max(lens)
        pool = (torch.randn(Bp + 4, H, D, D, generator=g, device=dev) * 0.02).half()
        slots = torch.arange(2, Bp + 2, dtype=torch.int32, device=dev)
        q = torch.randn(Bp, T, G, D, generator=g, device=dev)
        k = torch.randn(Bp, T, G, D, generator=g, device=dev)
        v = torch.randn(Bp, T, H, D, generator=g, device=dev)
        a = torch.randn(Bp, T, H, generator=g, device=dev)
        b = torch.randn(Bp, T, H, generator=g, device=dev)
        y = torch.empty(Bp, T, H, D, device=dev)
        sl = torch.tensor(lens, dtype=torch.int32, device=dev)
        call = lambda: kern.gdn_prefill_raw(pool, slots, q, k, v, a, b, A, dtb, y, sl)
        host = np.array(lens, dtype=np.int32)
        cus = torch.cuda.get_device_properties(0).multi_processor_count
        plan_times = []
        for _ in range(5):
            t_plan = time.perf_counter()
            plan = kern._lib.braid_prefill_plan(host.ctypes.data, Bp, T, H, cus)
            plan_times.append(time.perf_counter() - t_plan)
        n8, n4, n2 = plan >> 20, (plan >> 10) & 1023, plan & 1023
        # the launch an eager call makes: a launch small enough for the eighth
        # layout runs it without planning; one tier for every row runs that
        # layout's own kernel; otherwise the planned kernel with this plan
        if 8 * Bp * H <= cus:
            knobs, n8, n4, n2 = {}, Bp, 0, 0
        else:
            knobs = ({"prefill_layout": 8} if n8 == Bp else {"prefill_layout": 4} if n4 == Bp
                     else {"prefill_layout": 1} if n2 == Bp
                     else {"prefill_layout": 0, "prefill_plan": plan})
        with kern.launch_override(**knobs):
            t = graph_time(torch, call, reps=11)
        t_dev = graph_time(torch, call, reps=11)
        # a captured call handed the host lengths to plan from (plan_lens)
        t_hint = graph_time(torch, lambda: kern.gdn_prefill_raw(pool, slots, q, k, v, a, b, A,
                                                                dtb, y, sl, plan_lens=lens),
                            reps=11)
        tok = sum(lens)
        tf = tok * H * FLOP_PER_TOKEN_HEAD / t / 1e12
        return {"rows": Bp, "max_T": T, "tokens": tok, "ms": round(t * 1e3, 3),
                "tokens_per_s": round(tok / t, 1), "tflops": round(tf, 2),
                "fp32_frac": round(tf / FP32_PEAK_TFLOPS, 4),
                "plan": {"eighth_rows": n8, "quarter_rows": n4, "split_rows": n2},
                # the first call simulates; the library keeps the plan, so the
                # repeats are lookups
                "host_plan_us": round(plan_times[0] * 1e6, 1),
                "host_plan_cached_us": round(min(plan_times[1:]) * 1e6, 1),
                "captured_kernel_plan_ms": round(t_dev * 1e3, 3),
                "captured_plan_lens_ms": round(t_hint * 1e3, 3)}

    # the config-1 step on bf16 and fp32 pools (one 160-slot pool each; an fp32
    # pool is 320 MiB, past the 256 MB MALL; the bf16 pool's figure is hot)
    for label, dt, elem in (("decode_b128_bf16_pool", torch.bfloat16, 2),
                            ("decode_b128_fp32_pool", torch.float32, 4)):
        dpool = (torch.randn(SLOTS, H, D, D, generator=g, device=dev) * 0.02).to(dt)
        dslots = torch.randperm(SLOTS, generator=torch.Generator().manual_seed(7))[:B]
        dslots = dslots.to(torch.int32).to(dev)
        dq = torch.randn(B, G, D, generator=g, device=dev)
        dk = torch.randn(B, G, D, generator=g, device=dev)
        dv = torch.randn(B, H, D, generator=g, device=dev)
        da = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
        db = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
        dy = torch.empty(B, H, D, device=dev)
        t = graph_time(torch, lambda: kern.gdn_decode_raw(dpool, dslots, dq, dk, dv, da, db, A,
                                                          dtb, dy), reps=11, inner=20)
        nbytes = STEP_BYTES + B * H * D * D * 2 * (elem - 2)
        out[label] = {"us": round(t * 1e6, 2), "steps_per_s": round(1 / t, 1),
                      "gbs": round(nbytes / t / 1e9, 1),
                      "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}
        del dpool

    # gdn_decode (gates precomputed in fp32) on the config-1 fp16 pool shape:
    # alpha and beta are 8 bytes per head instead of the raw gates' 4
    dpool = (torch.randn(SLOTS, H, D, D, generator=g, device=dev) * 0.02).half()
    dalpha = torch.rand(B, H, generator=g, device=dev) * 0.5 + 0.5
    dbeta = torch.rand(B, H, generator=g, device=dev)
    t = graph_time(torch, lambda: kern.gdn_decode(dpool, dslots, dq, dk, dv, dalpha, dbeta, dy),
                   reps=11, inner=20)
    nbytes = STEP_BYTES + B * H * 4
    out["decode_b128_fp16_precomputed_gates"] = {
        "us": round(t * 1e6, 2), "steps_per_s": round(1 / t, 1),
        "gbs": round(nbytes / t / 1e9, 1), "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}
    del dpool

    lens = torch.randint(64, 1025, (8,), generator=torch.Generator().manual_seed(2)).tolist()
    out["prefill_config2"] = prefill_case(lens)
    # the small-batch regime: one 512-token row (eighth layout, eight workgroups
    # per tile) and one 1024-token row among 15 of 128 (planned)
    out["prefill_one_row_512"] = prefill_case([512])
    out["prefill_skewed_1x1024_15x128"] = prefill_case([1024] + [128] * 15)

    # config 2's causal conv prefill: 8 ragged rows, C=8192, K=4, bf16 in, fp32 out
    Cc, Tm = 2 * G * D + H * D, max(lens)
    cpool = torch.zeros(12, Cc, 4, device=dev)
    cslots = torch.arange(8, dtype=torch.int32, device=dev)
    cx = torch.randn(8, Tm, Cc, generator=g, device=dev).to(torch.bfloat16)
    cw = torch.randn(Cc, 4, generator=g, device=dev) * 0.1
    cout = torch.empty(8, Tm, Cc, device=dev)
    clens = torch.tensor(lens, dtype=torch.int32, device=dev)
    t = graph_time(torch, lambda: kern.conv1d_prefill(cpool, cslots, cx, cw, None, cout, clens),
                   reps=11)
    cbytes = 8 * Tm * Cc * (2 + 4) + 2 * 8 * Cc * 4 * 4 + Cc * 4 * 4
    out["conv1d_prefill_config2"] = {"tokens": sum(lens), "padded_T": Tm,
                                     "us": round(t * 1e6, 1),
                                     "gbs": round(cbytes / t / 1e9, 1),
                                     "hbm_frac": round(cbytes / t / 1e9 / HBM_PEAK_GBS, 4)}
    del cpool, cx, cout
    out["prefill_tick"] = prefill_case([256] * 4)

    # conv1d decode, config 3 shape
    C = 2 * G * D + H * D
    conv_pool = torch.randn(72, C, 4, generator=g, device=dev)
    slots64 = torch.randperm(72, generator=torch.Generator().manual_seed(3))[:64]
    slots64 = slots64.to(torch.int32).to(dev)
    w = torch.randn(C, 4, generator=g, device=dev) * 0.1
    bias = torch.randn(C, generator=g, device=dev) * 0.1
    xc = torch.randn(64, C, generator=g, device=dev).to(torch.bfloat16)
    co = torch.empty(64, C, device=dev)
    t = graph_time(torch, lambda: kern.conv1d_decode(conv_pool, slots64, xc, w, bias, co),
                   reps=11, inner=20)
    out["conv1d_decode"] = {"shape": "B=64 C=8192 K=4 bf16", "us": round(t * 1e6, 2),
                            "gbs": round(CONV_BYTES_B64 / t / 1e9, 1),
                            "hbm_frac": round(CONV_BYTES_B64 / t / 1e9 / HBM_PEAK_GBS, 4)}

    xq = torch.randn(64, 4096, generator=g, device=dev).to(torch.bfloat16)
    t = graph_time(torch, lambda: kern.quantize_act(xq), reps=11, inner=20)
    out["quantize_act"] = {"shape": "64x4096 bf16", "us": round(t * 1e6, 2),
                           "gbs": round(QUANT_BYTES_64x4096 / t / 1e9, 1)}

    # gated RMSNorm readout + out_proj input quant: decode (64 tokens) and
    # config 2's prefill (4073 tokens); y fp32, z/core bf16, q fp8
    gamma = 1.0 + 0.3 * torch.randn(D, generator=g, device=dev)
    for label, ntok in (("readout_quant_b64", 64), ("readout_quant_prefill", sum(lens))):
        ry = torch.randn(ntok, H, D, generator=g, device=dev)
        rz = torch.randn(ntok, H * D, generator=g, device=dev).to(torch.bfloat16)
        t = graph_time(torch, lambda: kern.gated_rmsnorm(ry, rz, gamma, 1e-6), reps=11,
                       inner=20 if ntok == 64 else 4)
        rbytes = ntok * H * D * READOUT_BYTES_PER_ELEM
        out[label] = {"tokens": ntok, "us": round(t * 1e6, 2),
                      "gbs": round(rbytes / t / 1e9, 1),
                      "hbm_frac": round(rbytes / t / 1e9 / HBM_PEAK_GBS, 4)}
        del ry, rz

    # FP8 projection GEMMs of config 3's layer at B=64 (the streaming kernel):
    # in_proj qkv + z (N = 8192 + 4096) and out_proj (N = 4096), K = 4096;
    # HBM-bound on the fp8 weight bytes. `us` cycles through distinct weights
    # totalling >= 512 MB, so each call reads its weight from HBM as a model's
    # layers do (one weight timed over and over stays in the 256 MB MALL:
    # `us_mall_resident`). hipBLASLt (the library path, BRAID_FP8_GEMM=0) and
    # torch._scaled_mm, the reference's call, are timed the same two ways.
    xg = torch.randn(64, 4096, generator=g, device=dev).to(torch.bfloat16)
    xgq, sxg = kern.quantize_act(xg)
    for label, N in (("fp8_gemm_in_proj_b64", 12288), ("fp8_gemm_out_proj_b64", 4096)):
        n_w = -(-(512 << 20) // (N * 4096))
        ws = [kern.quantize_act(torch.randn(N, 4096, generator=g, device=dev) * 0.02)
              for _ in range(n_w)]

        def cycle(fn):
            def run():
                for wq, sw in ws:
                    fn(wq, sw)
            return run

        ours = lambda wq, sw: kern.fp8_matmul(xgq, sxg, wq, sw)  # noqa: E731
        ref = lambda wq, sw: torch._scaled_mm(xgq, wq.t(), scale_a=sxg, scale_b=sw,  # noqa: E731
                                              out_dtype=torch.bfloat16)
        t = graph_time(torch, cycle(ours), reps=11, inner=2) / n_w
        t_res = graph_time(torch, lambda: ours(*ws[0]), reps=11, inner=20)
        with kern.launch_override(fp8_gemm=0):
            t_lib = graph_time(torch, cycle(ours), reps=11, inner=2) / n_w
            t_lib_res = graph_time(torch, lambda: ours(*ws[0]), reps=11, inner=20)
        t_ref = graph_time(torch, cycle(ref), reps=11, inner=2) / n_w
        t_ref_res = graph_time(torch, lambda: ref(*ws[0]), reps=11, inner=20)
        gbytes = N * 4096 + 64 * 4096 + 64 * N * 2
        out[label] = {"shape": f"M=64 N={N} K=4096", "weights_cycled": n_w,
                      "us": round(t * 1e6, 2), "gbs": round(gbytes / t / 1e9, 1),
                      "hbm_frac": round(gbytes / t / 1e9 / HBM_PEAK_GBS, 4),
                      "us_mall_resident": round(t_res * 1e6, 2),
                      "hipblaslt_us": round(t_lib * 1e6, 2),
                      "hipblaslt_us_mall_resident": round(t_lib_res * 1e6, 2),
                      "torch_scaled_mm_us": round(t_ref * 1e6, 2),
                      "torch_scaled_mm_us_mall_resident": round(t_ref_res * 1e6, 2)}
        del ws

    # config 3: 24-layer mixer decode step at B=64
    L, Bm, S = 24, 64, 72
    layers = []
    for _ in range(L):
        layers.append(dict(
            pool=(torch.randn(S, H, D, D, generator=g, device=dev) * 0.02).half(),
            conv=torch.randn(S, C, 4, generator=g, device=dev) * 0.5,
            w=torch.randn(C, 4, generator=g, device=dev) * 0.1,
            bias=torch.randn(C, generator=g, device=dev) * 0.1,
            x=torch.randn(Bm, 4096, generator=g, device=dev).to(torch.bfloat16),
            xin=torch.randn(Bm, C, generator=g, device=dev).to(torch.bfloat16),
            a=torch.randn(Bm, H, generator=g, device=dev).to(torch.bfloat16),
            b=torch.randn(Bm, H, generator=g, device=dev).to(torch.bfloat16),
            cout=torch.empty(Bm, C, device=dev), y=torch.empty(Bm, H, D, device=dev)))

    def mixer_step():
        for ly in layers:
            kern.quantize_act(ly["x"])
            kern.conv1d_decode(ly["conv"], slots64, ly["xin"], ly["w"], ly["bias"], ly["cout"])
            q, k, v = torch.split(ly["cout"], [G * D, G * D, H * D], dim=-1)
            kern.gdn_decode_raw(ly["pool"], slots64, q.unflatten(-1, (G, D)),
                                k.unflatten(-1, (G, D)), v.unflatten(-1, (H, D)), ly["a"],
                                ly["b"], A, dtb, ly["y"])

    t = graph_time(torch, mixer_step, reps=11)
    step_bytes = L * (QUANT_BYTES_64x4096 + CONV_BYTES_B64 + Bm * ROW_BYTES)

    def mixer_step_fused():
        for ly in layers:
            kern.quantize_act(ly["x"])
            kern.gdn_conv_decode_raw(ly["pool"], ly["conv"], slots64, ly["xin"], ly["w"],
                                     ly["bias"], ly["a"], ly["b"], A, dtb, ly["y"], G)

    t_fused = graph_time(torch, mixer_step_fused, reps=11)

    # The step's parts, each as its own 24-launch sequence, and the dispatch
    # floor: 24 one-thread kernels (braid_probe_clock) in the same kind of
    # graph. A dependent launch costs about that much even when it does nothing.
    def quant_only():
        for ly in layers:
            kern.quantize_act(ly["x"])

    def fused_only():
        for ly in layers:
            kern.gdn_conv_decode_raw(ly["pool"], ly["conv"], slots64, ly["xin"], ly["w"],
                                     ly["bias"], ly["a"], ly["b"], A, dtb, ly["y"], G)

    floor_clock = GpuClock(torch)
    floor_buf = torch.zeros(L, dtype=torch.int64, device=dev)

    def empty_launches():
        st = torch.cuda.current_stream().cuda_stream
        for i in range(L):
            floor_clock._stamp(floor_buf[i:].data_ptr(), st)

    parts = {"quantize_act_us": round(graph_time(torch, quant_only, reps=11) * 1e6, 1),
             "conv_decode_us": round(graph_time(torch, fused_only, reps=11) * 1e6, 1),
             "dispatch_floor_us_per_launch":
                 round(graph_time(torch, empty_launches, reps=11) / L * 1e6, 2)}
    out["mixer_step_fused"] = {"layers": L, "batch": Bm, "us": round(t_fused * 1e6, 1),
                               "gbs": round(step_bytes / t_fused / 1e9, 1),
                               "hbm_frac": round(step_bytes / t_fused / 1e9 / HBM_PEAK_GBS, 4),
                               "note": "conv + decode in one launch per layer; same bytes "
                                       "credited as mixer_step",
                               "parts_24_layers": parts}
    out["mixer_step"] = {"layers": L, "batch": Bm, "us": round(t * 1e6, 1),
                         "gbs": round(step_bytes / t / 1e9, 1),
                         "hbm_frac": round(step_bytes / t / 1e9 / HBM_PEAK_GBS, 4),
                         "bytes": step_bytes}
    del layers

    # config 4: mixed tick on one 192-slot fp16 pool
    pool = (torch.randn(192, H, D, D, generator=g, device=dev) * 0.02).half()
    pre_slots = torch.arange(96, 100, dtype=torch.int32, device=dev)
    pq = torch.randn(4, 256, G, D, generator=g, device=dev)
    pk = torch.randn(4, 256, G, D, generator=g, device=dev)
    pv = torch.randn(4, 256, H, D, generator=g, device=dev)
    pa = torch.randn(4, 256, H, generator=g, device=dev).to(torch.bfloat16)
    pb = torch.randn(4, 256, H, generator=g, device=dev).to(torch.bfloat16)
    py = torch.empty(4, 256, H, D, device=dev)
    plen = torch.full((4,), 256, dtype=torch.int32, device=dev)
    tick = {}
    from braid_amd.tick import MixedTick
    mixed = MixedTick(kern)
    for bucket in (16, 32, 64, 96, 128):
        live = min(bucket, 96)
        # Captured (and run eagerly) with distinct slots apart from the prefill
        # rows' 96..99: the live rows 0..live-1, then free slots 100..; the
        # graphs are then replayed with the pad rows on one scratch slot, 191.
        eager_sl = torch.cat([torch.arange(live, dtype=torch.int32, device=dev),
                              torch.arange(100, 100 + bucket - live, dtype=torch.int32,
                                           device=dev)])
        sl = eager_sl.clone()
        padded = torch.cat([torch.arange(live, dtype=torch.int32, device=dev),
                            torch.full((bucket - live,), 191, dtype=torch.int32, device=dev)])
        dq = torch.randn(bucket, G, D, generator=g, device=dev)
        dk = torch.randn(bucket, G, D, generator=g, device=dev)
        dv = torch.randn(bucket, H, D, generator=g, device=dev)
        da = torch.randn(bucket, H, generator=g, device=dev).to(torch.bfloat16)
        db = torch.randn(bucket, H, generator=g, device=dev).to(torch.bfloat16)
        dy = torch.empty(bucket, H, D, device=dev)

        def tick_seq():
            kern.gdn_prefill_raw(pool, pre_slots, pq, pk, pv, pa, pb, A, dtb, py, plen)
            kern.gdn_decode_raw(pool, sl, dq, dk, dv, da, db, A, dtb, dy)

        # The tick as the library runs it: the decode on a side stream beside
        # the prefill (braid_amd/tick.py); the sequential tick beside it.
        pre_args = dict(slots=pre_slots, q=pq, k=pk, v=pv, a_raw=pa, b_raw=pb, A=A,
                        dt_bias=dtb, y=py, seq_lens=plen)
        dec_args = dict(slots=sl, q=dq, k=dk, v=dv, a_raw=da, b_raw=db, A=A, dt_bias=dtb,
                        y=dy)

        def tick_fn():
            mixed(pool, pre_args, dec_args)

        entry = {"graph_us": round(graph_time(torch, tick_fn, reps=11,
                                              before_replay=lambda: sl.copy_(padded)) * 1e6, 1)}
        sl.copy_(eager_sl)
        entry["graph_sequential_us"] = round(graph_time(
            torch, tick_seq, reps=11, before_replay=lambda: sl.copy_(padded)) * 1e6, 1)
        # eager: the kernels' eager validation wants distinct slots, so the
        # pad rows of bucket 128 take distinct free slots (100..131) instead
        # of one scratch slot
        sl.copy_(eager_sl)
        for label, fn in (("eager_us", tick_fn), ("eager_sequential_us", tick_seq)):
            fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(5):
                fn()
            torch.cuda.synchronize()
            entry[label] = round((time.perf_counter() - t0) / 5 * 1e6, 1)
        if bucket > live:
            entry["eager_pad"] = f"{bucket - live} pad rows on distinct free slots"
        tick[str(bucket)] = entry
    tick_bytes = 96 * ROW_BYTES + 4 * 2 * H * D * D * 2 + 4 * 256 * (
        (2 * G * D + 2 * H * D) * 4 + H * 2 * 2)
    tick["bytes_b96"] = tick_bytes
    tick["gbs_b96_graph"] = round(tick_bytes / (tick["96"]["graph_us"] * 1e-6) / 1e9, 1)
    out["mixed_tick"] = tick
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path and the box has "
              f"one GPU (asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)
    import torch

    from braid_amd.kernels.loader import load_gdn

    kern = load_gdn()
    n_cold = max(2, math.ceil(COLD_BYTES / (SLOTS * H * D * D * 2)))
    work = make_workload(torch, n_cold)
    t_cold, spread = time_steps(torch, kern, work, args.steps, args.warmup)
    hot_work = tuple([x[:1] for x in work[:3]] + list(work[3:]))
    t_hot, _ = time_steps(torch, kern, hot_work, args.steps, args.warmup, reps=11)
    del work, hot_work
    torch.cuda.empty_cache()
    copy_gbs = copy_bandwidth(torch)
    ceiling = stream_ceiling(torch, n_cold)
    orders = {o: stream_ceiling(torch, n_cold, launches=64, order=o)
              for o in ("head_major", "shuffled")}
    torch.cuda.empty_cache()

    step_s = t_cold / args.steps
    achieved = STEP_BYTES / step_s / 1e9
    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
    out = {
        "metric": "GDN decode steps/s and achieved HBM GB/s (% of peak) at B=128, 1 MI355X",
        "value": round(args.steps / t_cold, 2),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "config1: batched GDN decode (gdn_decode_raw), B=128, "
                               "160-slot fp16 pool, permuted slots, cold pools",
                   "batch": B, "value_heads": H, "key_heads": G, "state": "128x128 fp16",
                   "gates": "in-kernel from bf16 raw", "cold_pools": n_cold},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic},
        # roofline.traffic: HBM bytes per launch of this kernel from two rocprofv3
        # counter passes (FETCH_SIZE, WRITE_SIZE) over this command, calibrated on
        # the stream probes' exact bytes in the same passes
        "traffic_source": "profiles/gdn_decode_b128_hbm_traffic.md",
        "achieved_gbs": round(achieved, 1),
        "hbm_frac": round(achieved / HBM_PEAK_GBS, 4),
        # value and ms_per_step are the median of these replays (each of all
        # K steps, timed alone); first_rep_us is the first timed replay alone
        "spread_us_per_step": spread,
        "hot_steps_per_s": round(args.steps / t_hot, 2),
        "hot_achieved_gbs": round(STEP_BYTES / (t_hot / args.steps) / 1e9, 1),
        "copy_gbs": round(copy_gbs, 1),
        "bytes_per_step": STEP_BYTES,
        # the same tiles streamed in place with no arithmetic and no q/k/v/y
        # (libbraid_probe.so); decode_vs_rmw = probe time / decode time
        "stream_ceiling": dict(ceiling, decode_vs_rmw=round(ceiling["rmw_us"] / (step_s * 1e6),
                                                            4)),
        # the same probe passes over the same tiles visited in other orders
        "stream_ceiling_other_orders": orders,
    }
    if not args.no_paths:
        out["paths"] = measure_paths(torch, kern)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        out["cpu_oracle_scalar"] = cpu_oracle_scalar(args.cpu_seconds / 4)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
