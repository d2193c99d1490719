"""Benchmark: µs per Qwen3-4B decode-step linear stack (3-bit packed TCQ, batch 1).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S]

Workload: the 7 projections (q, k, v, o, gate, up,
down) of each of Qwen3-4B's 36 decoder layers, as 252 distinct packed linears
(k = 3 bits/weight, S = 64 trellis states, seeded synthetic streams and
activations), all captured in one HIP graph and replayed once per step.  The
weights (1.37 GB) exceed the 256 MB Infinity Cache, so each replay streams
them from HBM.

Prints ONE JSON line: ``value`` is µs per decode step (lower is better), with
the step's algorithmic GB/s and % of MI355X's 8 TB/s HBM peak; ``roofline``
covers the dominant kernel (the gate/up-shaped decode-GEMV, timed per launch
with HIP events over 36 distinct weight sets on the stream it runs on), and
``cpu_baseline`` times the reference's CPU tiled path (the oracle's op-for-op
restatement) on a bounded sample on this host.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

HBM_PEAK_GBPS = 8000.0
N_LAYERS = 36
BITS = 3
N_STATES = 64
BATCH = 1


def _bytes(n: int, d: int, bits: int, batch: int) -> int:
    # k-bit codes + fp16 scales, codebook, rot_scale, x in, y out
    return n * d * bits // 8 + 2 * n + 2 * (1 << (bits + 1)) + 2 * d + 2 * batch * d + 2 * batch * n


def build_stack(device, n_layers=N_LAYERS, bits=BITS):
    from turbopress_amd.runtime import PackedTCQLinear
    from turbopress_amd.synthetic import QWEN3_4B_LAYER, make_activation, make_payload
    layers = []
    for li in range(n_layers):
        mods = {}
        for j, (name, (d, n)) in enumerate(QWEN3_4B_LAYER.items()):
            seed = 1000 * li + j
            mods[name] = (PackedTCQLinear(make_payload(n, d, bits, N_STATES, seed=seed), mode="hip"),
                          make_activation(BATCH, d, seed=seed).to(device))
        layers.append(mods)
    return layers


def step_bytes(layers) -> int:
    return sum(_bytes(m.out_features, m.in_features, m.bits, BATCH)
               for mods in layers for (m, _) in mods.values())


def run_step(layers, outs):
    i = 0
    for mods in layers:
        for name in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
            m, x = mods[name]
            outs[i] = m(x)
            i += 1


def time_graph(layers, steps, warmup):
    outs = [None] * (7 * len(layers))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(max(warmup, 1)):
            run_step(layers, outs)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run_step(layers, outs)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) / steps, wall / steps * 1e3, g, outs


def time_dominant_kernel(layers, reps=3):
    """Per-launch HIP-event timing of the gate-shaped GEMV (9728 x 2560) over the
    36 layers' distinct weights, on the stream the kernel is launched on."""
    from turbopress_amd import hip_kernel as hk
    stream = torch.cuda.current_stream()
    zs = []
    for mods in layers:
        m, x = mods["gate_proj"]
        zs.append((m, hk.fwht_scale(x, m.rot_scale, m.block)))
    for m, z in zs:  # warm
        hk.packed_gemv(z, m)
    torch.cuda.synchronize()
    evs = []
    for _ in range(reps):
        for m, z in zs:
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            hk.packed_gemv(z, m)
            b.record(stream)
            evs.append((a, b))
    torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in evs]
    m0 = zs[0][0]
    return sum(ms) / len(ms), _bytes(m0.out_features, m0.in_features, m0.bits, BATCH)


def cpu_baseline(budget_s: float):
    """The reference's CPU tiled path (oracle restatement), one Qwen3-4B layer
    at k=3, B=1, repeated until ~budget_s of CPU work, scaled to 36 layers."""
    from oracle.tiled_baseline import TiledLinearCPU
    from turbopress_amd.synthetic import QWEN3_4B_LAYER, make_activation, make_payload
    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    mods = []
    for j, (name, (d, n)) in enumerate(QWEN3_4B_LAYER.items()):
        mods.append((TiledLinearCPU(make_payload(n, d, BITS, N_STATES, seed=j)),
                     make_activation(BATCH, d, seed=j)))
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        for lin, x in mods:
            lin(x)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s or len(times) >= 20:
            break
    times.sort()
    per_layer = times[len(times) // 2]
    return {
        "value": round(per_layer * N_LAYERS * 1e6, 1), "unit": "us/step", "cores": threads,
        "kind": "port",
        "sample": (f"1 of 36 Qwen3-4B layers (q,k,v,o,gate,up,down; k=3, S=64, B=1) through "
                   f"oracle/tiled_baseline.py (torch CPU, {threads} threads), median of "
                   f"{len(times)} runs, scaled x36"),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: the packed-TCQ decode path is built and measured "
              "on a single GPU only (multi-GPU sharding is design-only); run with --gpus 1.",
              file=sys.stderr)
        return 2
    torch.manual_seed(0)
    dev = torch.device("cuda", 0)
    print(f"[bench] building {N_LAYERS}x7 packed linears (k={BITS}, S={N_STATES})", file=sys.stderr, flush=True)
    layers = build_stack(dev)
    nbytes = step_bytes(layers)
    print(f"[bench] capturing graph; {nbytes / 1e9:.4f} GB per step", file=sys.stderr, flush=True)
    ms_ev, ms_wall, _, _ = time_graph(layers, args.steps, args.warmup)
    ms = ms_ev
    print(f"[bench] graph step {ms * 1e3:.1f} us (wall {ms_wall * 1e3:.1f} us)", file=sys.stderr, flush=True)
    dom_ms, dom_bytes = time_dominant_kernel(layers)
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    print(f"[bench] dominant kernel {dom_ms * 1e3:.2f} us/launch, {achieved:.0f} GB/s", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(args.cpu_seconds)
    gbps = nbytes / (ms * 1e-3) / 1e9
    line = {
        "metric": "µs per decode-step linear stack + HBM GB/s (% peak), 3-bit TCQ, Qwen3-4B b=1",
        "value": round(ms * 1e3, 2), "unit": "us/step", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "qwen3-4b decode-step linear stack: 36 layers x (q,k,v,o,gate,up,down), "
                               "one HIP graph", "layers": N_LAYERS, "bits": BITS, "n_states": N_STATES,
                   "batch": BATCH, "bytes_per_step": nbytes},
        "gbps": round(gbps, 1), "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
        "wall_ms_per_step": round(ms_wall, 5),
        "roofline": {"kernel": "tcq decode-GEMV, gate/up shape 9728x2560 k=3 B=1",
                     "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "us_per_launch": round(dom_ms * 1e3, 3), "bytes_per_launch": dom_bytes},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
