"""Benchmark: µs per Qwen3-4B decode-step linear stack (3-bit packed TCQ, batch 1).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S]

Workload: the 7 projections (q, k, v, o, gate, up,
down) of each of Qwen3-4B's 36 decoder layers -- 252 distinct packed linears
at k = 3 bits/weight, S = 64 trellis states, seeded synthetic streams -- with
seeded fp16 activations (N(0,1), 1 % of channels x20), one input per
shared-input group (q/k/v, o, gate/up, down) of every layer.  The weights
(1.37 GB) exceed the 256 MB Infinity Cache, so every step streams them from
HBM.  A step is captured once in a HIP graph and replayed; K replays are
timed with HIP events between two device synchronisations.

Clock settling: under this load the GPU's power management lowers the clock
after ~1.5 ms and settles within ~100 steps.  Every timed leg first replays
its graph for a fixed wall time (``settle_ms``, default 500 ms) and only then
runs the W warm-up and K timed replays, so the figures are the sustained
rate whatever W is.

``value`` (µs per step, lower is better) is the primary executor, the
decode-step stack (tp_stack_run): one small launch rotates all 252 inputs
(z = blockFWHT(x * rot_scale) / sqrt(block), fp16) into the plan's z buffer,
then ONE persistent launch streams every linear's packed weights.  After the
timed region one replay's 252 outputs are compared with the per-linear
``PackedTCQLinear.forward`` (itself oracle-checked in the tests) at max-rel
2e-3; a mismatch fails the run.  The line also reports the same stack with
the decoder's phase order enforced on the device (q/k/v | o | gate/up | down
of each layer, 144 phases, a phase starts after all of the previous one),
one launch per shared-input group (144 launches) and one launch per linear
(252 launches, the drop-in PackedTCQLinear.forward path), and
``chained_step``: a decode step that respects the data dependencies (each
layer's q/k/v group, o, gate/up group and down each read the output of the
launch before; down feeds the next layer; decode_step.ChainedDecodeStep),
checked against the per-linear forward on the inputs each launch read.

``roofline`` covers the dominant kernel, the stack's GEMV launch
(tcq_stack_slot_kernel): its algorithmic bytes (the step's bytes minus the
rot_scale vectors, which only the rotation launch reads) over its own
duration, timed with HIP events around back-to-back launches on the stream
they run on.  ``traffic`` is the HBM bytes per launch of the committed
rocprofv3 counter summary named in ``traffic_source`` (FETCH_SIZE and
WRITE_SIZE passes, each calibrated on a known-size copy), not measured in
this run.  ``read_reference`` is a plain streaming read of the step's byte
count (``tp_read_probe``): the read bandwidth the box reaches with no
compute, i.e. the practical ceiling the kernel is compared against.

``per_linear`` is the one-linear-at-a-time table of BASELINE.json configs[0]
(SmolLM2-135M up-proj, k=2), configs[1] (the Qwen3-0.6B layer, k=3),
configs[3] (Qwen3-4B gate/up/down, k in {2,3,4}, B in {1,4,8}) and the
batch-32 shapes of configs[4]: PackedTCQLinear.forward, one launch per call,
each case cycling over >= 320 MB of distinct copies of the linear inside one
graph so no call reads cached weights; per case µs, GB/s over the algorithmic
bytes and over the reference's (k+1)-bit level-stream bytes, the time one
streaming-read launch of the same byte count takes (``floor_us``) and the
fraction of HBM peak.  ``c1_layer_stack`` is the Qwen3-0.6B layer's 7 linears
as one stack (96 distinct layer copies, 575 MB: over twice the 256 MB
Infinity Cache).
``batch32`` is the batch >= 16 path, the MFMA skinny GEMM of configs[4]: the
same 36-layer stack at batch 32, as time, TFLOP/s and fraction of the
2.5 PFLOP/s dense fp16 MFMA peak.
``encoder`` times the compress-time TCQ Viterbi search on a gate_proj-sized
matrix; its CPU comparison sits in the CPU-baseline leg.
``cpu_baseline`` times the reference's CPU tiled path (the oracle's
op-for-op restatement) on a bounded sample on this host, on every CPU this
process may run on.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import torch

HBM_PEAK_GBPS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
N_LAYERS = 36
BITS = 3
N_STATES = 64
BATCH = 1
PARITY_TOL = 2e-3
ORDER = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
GROUP_INPUT = {"q_proj": "attn", "k_proj": "attn", "v_proj": "attn", "o_proj": "o",
               "gate_proj": "mlp", "up_proj": "mlp", "down_proj": "down"}
GROUP_DIM = {"attn": 2560, "o": 4096, "mlp": 2560, "down": 9728}


def _bytes(n: int, d: int, bits: int, batch: int) -> int:
    # k-bit codes + fp16 scales, codebook, rot_scale, x in, y out
    return n * d * bits // 8 + 2 * n + 2 * (1 << (bits + 1)) + 2 * d + 2 * batch * d + 2 * batch * n


def _ref_bytes(n: int, d: int, bits: int, batch: int) -> int:
    """Bytes the reference's Triton path moves for the same linear: the
    (k+1)-bit level stream with rows padded to 4 bytes (runtime.py:253-277)
    instead of the k-bit codes, the same side tensors."""
    row = -(-d * (bits + 1) // 32) * 4
    return n * row + _bytes(n, d, bits, batch) - n * d * bits // 8


def build_layers(device, n_layers=N_LAYERS, bits=BITS, batch=BATCH, shapes=None):
    from turbopress_amd.runtime import PackedTCQLinear
    from turbopress_amd.synthetic import QWEN3_4B_LAYER, make_activation, make_payload
    shapes = shapes or QWEN3_4B_LAYER
    layers, inputs = [], []
    for li in range(n_layers):
        mods = {}
        for j, name in enumerate(ORDER):
            d, n = shapes[name]
            mods[name] = PackedTCQLinear(make_payload(n, d, bits, N_STATES, seed=1000 * li + j), mode="hip")
        xs = {}
        for k, g in enumerate(("attn", "o", "mlp", "down")):
            d = mods[{"attn": "q_proj", "o": "o_proj", "mlp": "gate_proj", "down": "down_proj"}[g]].in_features
            xs[g] = make_activation(batch, d, seed=1000 * li + 100 + k).to(device)
        layers.append(mods)
        inputs.append(xs)
    return layers, inputs


def step_bytes(layers, batch=BATCH) -> int:
    return sum(_bytes(m.out_features, m.in_features, m.bits, batch) for mods in layers for m in mods.values())


def make_stack(layers, inputs, ordered):
    from turbopress_amd.decode_step import QWEN_PHASES, LinearStack
    entries = []
    for li, (mods, xs) in enumerate(zip(layers, inputs)):
        for name in ORDER:
            entries.append((mods[name], xs[GROUP_INPUT[name]], 4 * li + QWEN_PHASES[name]))
    return LinearStack(entries, ordered=ordered)


def settle(run, settle_ms: float) -> int:
    """Run `run` (one replay / launch sequence) back to back for `settle_ms`
    of wall time so the GPU reaches its sustained clock; returns the count."""
    if settle_ms <= 0:
        return 0
    torch.cuda.synchronize()
    t_end = time.perf_counter() + settle_ms * 1e-3
    count = 0
    while time.perf_counter() < t_end:
        for _ in range(16):
            run()
        count += 16
        torch.cuda.synchronize()
    return count


def capture(step_fn):
    """Warm `step_fn` once on a side stream, then capture it in a graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step_fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step_fn()
    return g


def time_graph(step_fn, steps, warmup, settle_ms=0.0):
    """Capture step_fn once, replay it for `settle_ms`, then `warmup` times,
    then time `steps` replays between device synchronisations.  Returns ms
    per step (events, wall) and the graph."""
    g = capture(step_fn)
    settle(g.replay, settle_ms)
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
    return start.elapsed_time(end) / steps, wall / steps * 1e3, g


def time_gemv_kernel(stack, steps, warmup, settle_ms=0.0):
    """Average duration (µs) of the stack's GEMV launch alone: the z buffer is
    filled once, then `steps` GEMV launches run back to back between two
    events on the stream they are launched on (torch's current stream)."""
    stack.rotate()
    settle(stack.gemv, settle_ms)
    for _ in range(warmup):
        stack.gemv()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        stack.gemv()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps * 1e3


def chained_step(device, steps: int, warmup: int, settle_ms: float, n_layers: int = N_LAYERS) -> dict:
    """A data-dependent decode step over 36 Qwen3-4B layers
    (decode_step.ChainedDecodeStep): in every layer the q/k/v group reads
    the layer input, o reads q's output, the gate/up group reads o's output,
    down reads gate's output and feeds the next layer -- 4 launches per
    layer, each on the previous one's output, one HIP graph per step.  The
    layers are seeded like the headline's, with each linear's row scales
    divided by its expected gain (synthetic.unit_gain) so that activations
    keep their magnitude along the 144 chained projections (a real decoder
    has RMS norms between them; here fp16 would overflow by layer ~12).  Every
    output of the captured step is checked against the per-linear forward
    on the same inputs (the tests check the chain against the oracle)."""
    from turbopress_amd.decode_step import ChainedDecodeStep
    from turbopress_amd.runtime import PackedTCQLinear
    from turbopress_amd.synthetic import QWEN3_4B_LAYER, make_activation, make_payload, unit_gain
    layers = []
    for li in range(n_layers):
        mods = {}
        for j, name in enumerate(ORDER):
            d, n = QWEN3_4B_LAYER[name]
            mods[name] = PackedTCQLinear(unit_gain(make_payload(n, d, BITS, N_STATES, seed=1000 * li + j)),
                                         mode="hip")
        layers.append(mods)
    x = make_activation(BATCH, QWEN3_4B_LAYER["q_proj"][0], seed=7).to(device)
    chain = ChainedDecodeStep(layers, x)
    ms, _, _ = time_graph(chain.run, steps, warmup, settle_ms)
    torch.cuda.synchronize()
    worst, where = 0.0, None
    for li in range(n_layers):
        ins = chain.layer_inputs(li)
        for name in ORDER:
            ref = layers[li][name](ins[name]).float()
            got = chain.outputs[li][name].float()
            err = float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))
            if not err <= worst:  # (a NaN counts as the worst)
                worst, where = err, f"layer {li} {name}"
    final = chain.outputs[-1]["down_proj"].float()
    nbytes = step_bytes(layers)
    out = {"us_per_step": round(ms * 1e3, 2), "launches_per_step": 4 * n_layers, "bytes_per_step": nbytes,
           "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
           "parity_vs_per_linear": {"max_rel": worst, "worst": where, "tol": PARITY_TOL, "ok": worst <= PARITY_TOL},
           "final_rms": round(float(final.pow(2).mean().sqrt()), 4)}
    del chain, layers
    torch.cuda.empty_cache()
    return out


def check_stack_outputs(stack, layers, inputs) -> dict:
    """One replay's outputs of the timed plan against the per-linear HIP
    forward of the same linears on the same inputs (max-rel, normalised by
    the largest reference magnitude, as the tests use)."""
    stack.run()
    torch.cuda.synchronize()
    worst, where, i = 0.0, None, 0
    for li, (mods, xs) in enumerate(zip(layers, inputs)):
        for name in ORDER:
            ref = mods[name](xs[GROUP_INPUT[name]]).float()
            got = stack.outputs[i].float()
            err = float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))
            if err > worst:
                worst, where = err, f"layer {li} {name}"
            i += 1
    return {"linears_checked": i, "max_rel": worst, "worst": where, "tol": PARITY_TOL, "ok": worst <= PARITY_TOL}


TRAFFIC_PROFILE = Path(__file__).resolve().parent / "profiles" / "tcq_stack_slot_kernel_qwen3-4b_b1_hbm_traffic.md"


def measured_traffic():
    """HBM bytes per GEMV launch from the committed counter summary (FETCH_SIZE
    and WRITE_SIZE passes calibrated against a known-size copy) and where it
    came from, or (None, None)."""
    try:
        value, build = None, None
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                value = int(line.split(":")[1])
            if line.startswith("build:"):
                build = line.split(":", 1)[1].strip()
        if value is not None:
            src = f"profiles/{TRAFFIC_PROFILE.name}" + (f" ({build})" if build else "")
            return value, src
    except (OSError, ValueError):
        pass
    return None, None


def copy_reference(mib: int, reps: int = 10):
    """A plain device-to-device copy of `mib` MiB (read + write), timed like
    the GEMV: the practical streaming bandwidth of this box, and the known-size
    kernel that HBM byte counters are calibrated against."""
    a = torch.ones(mib << 18, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        b.copy_(a)
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) / reps * 1e3
    moved = 2 * a.numel() * 4
    del a, b
    return {"bytes_read": moved // 2, "bytes_written": moved // 2, "us": round(us, 2),
            "gbps": round(moved / (us * 1e-6) / 1e9, 1)}


def read_reference(nbytes: int, reps: int = 20, settle_ms: float = 0.0):
    """A plain streaming read (tp_read_probe: every wave streams its own
    contiguous slice with 16-byte loads, no compute) of as many bytes as one
    step moves: the read bandwidth this box reaches at all, i.e. the
    practical ceiling of an HBM-bound read stream."""
    from turbopress_amd import _lib
    lib = _lib.lib()
    nbytes = (nbytes + 15) & ~15
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def run():
        _lib.check(lib.tp_read_probe(buf.data_ptr(), nbytes, sink.data_ptr(), stream), "read_probe")

    settle(run, settle_ms)
    for _ in range(reps):
        run()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        run()
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) / reps * 1e3
    del buf, sink
    return {"bytes_read": nbytes, "us": round(us, 2), "gbps": round(nbytes / (us * 1e-6) / 1e9, 1)}


def encoder_reference(rows: int = 9728, dim: int = 2560, cpu_rows: int = 256):
    """Compress-time leg (not the headline): the TCQ Viterbi search
    (tp_tcq_viterbi) over a Qwen3-4B gate_proj-sized matrix (k=3, S=64, the
    stored trellis codebook).  Returns the figures and the first `cpu_rows`
    rows with their GPU codes, which the CPU-baseline leg times and checks."""
    from turbopress_amd.codebooks import default_codebook
    from turbopress_amd.encoder import viterbi
    gen = torch.Generator().manual_seed(0)
    z = torch.randn(rows, dim, generator=gen)
    cb = default_codebook(BITS, N_STATES).to(torch.float32)
    zg = z.to("cuda")
    viterbi(zg, cb, N_STATES)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 3
    start.record()
    for _ in range(reps):
        out = viterbi(zg, cb, N_STATES)
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) / reps * 1e3
    figures = {"rows": rows, "dim": dim, "bits": BITS, "n_states": N_STATES, "gpu_us": round(us, 1),
               "gpu_weights_per_s": round(rows * dim / (us * 1e-6), 1)}
    return figures, (z[:cpu_rows], cb, out[0][:cpu_rows].cpu(), rows)


def host_cpus() -> tuple[int, str]:
    """CPUs this process may run on: its affinity set, further limited by a
    cgroup CPU quota when one is set; and how that was found."""
    total = os.cpu_count() or 1
    try:
        n = len(os.sched_getaffinity(0))
        how = f"sched_getaffinity ({n} of os.cpu_count() {total})"
    except (AttributeError, OSError):
        n, how = total, "os.cpu_count()"
    try:
        quota, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if quota != "max":
            q = max(1, int(int(quota) // int(period)))
            if q < n:
                n, how = q, f"cgroup cpu.max quota ({q} CPUs; affinity {how})"
    except (OSError, ValueError):
        pass
    return n, how


def cpu_encoder_baseline(sample) -> dict:
    """The reference's fp32 Viterbi search restated on the CPU
    (oracle.codebook_oracle.viterbi_full, torch) over the encoder leg's
    sample rows, scaled to the whole matrix; also checks the GPU codes."""
    from oracle.codebook_oracle import viterbi_full
    z, cb, gpu_codes, rows = sample
    threads, how = host_cpus()
    torch.set_num_threads(threads)
    t0 = time.perf_counter()
    ref = viterbi_full(z, cb, N_STATES)
    secs = time.perf_counter() - t0
    return {"value": round(secs * rows / z.shape[0], 3), "unit": "s/matrix", "cores": threads,
            "cores_source": how, "kind": "port",
            "sample": f"{z.shape[0]} of {rows} rows through the fp32 reference search (torch CPU), scaled",
            "codes_match_gpu": bool(torch.equal(gpu_codes, ref[0]))}


def batch32_reference(layers, steps: int, warmup: int, settle_ms: float) -> dict:
    """The batch >= 16 path (MFMA skinny GEMM): the same 36-layer stack at
    batch 32 (one rotation launch + one wide-kernel launch).  Achieved
    TFLOP/s = 2*B*n*d / time of the GEMV launch."""
    dev = layers[0]["q_proj"].scales.device
    batch = 32
    from turbopress_amd.synthetic import make_activation
    inputs = []
    for li in range(len(layers)):
        inputs.append({g: make_activation(batch, d, seed=5000 + 10 * li + k).to(dev)
                       for k, (g, d) in enumerate(GROUP_DIM.items())})
    weights = sum(m.out_features * m.in_features for mods in layers for m in mods.values())
    stack = make_stack(layers, inputs, ordered=False)
    ms, _, _ = time_graph(stack.run, steps, warmup, settle_ms)
    us_gemv = time_gemv_kernel(stack, steps, warmup, settle_ms / 2)
    tf = 2 * batch * weights / (us_gemv * 1e-6) / 1e12
    return {"batch": batch, "stack_us_per_step": round(ms * 1e3, 2), "stack_gemv_us": round(us_gemv, 2),
            "stack_gemv_tflops": round(tf, 1), "stack_gemv_mfma_frac": round(tf / MFMA_FP16_PEAK_TFLOPS, 4)}


def _graph_us_per_call(step_fn, calls: int, steps: int = 20, settle_ms: float = 0.0) -> float:
    """µs per call of a graph of `calls` back-to-back calls (step_fn makes
    them), replayed `steps` times after settling and 5 warm-up replays."""
    ms, _, _ = time_graph(step_fn, steps, 5, settle_ms)
    return ms * 1e3 / calls


def default_cases():
    """(config, name, in, out, bits, batch) of the per-linear table."""
    from turbopress_amd.synthetic import QWEN3_0_6B_LAYER, QWEN3_4B_LAYER
    cases = [("c0", "smollm2_up_proj", 576, 1536, 2, 1)]
    cases += [("c1", name, *QWEN3_0_6B_LAYER[name], 3, 1) for name in ORDER]
    cases += [("c3", name, *QWEN3_4B_LAYER[name], k, b)
              for k in (2, 3, 4) for b in (1, 4, 8) for name in ("gate_proj", "up_proj", "down_proj")]
    cases += [("c4", name, *QWEN3_4B_LAYER[name], 3, 32) for name in ("gate_proj", "down_proj")]
    return cases


def per_linear_sweep(cases=None, min_bytes: float = 320e6, settle_ms: float = 50.0, steps: int = 10,
                     log=None) -> list:
    """PackedTCQLinear.forward one linear at a time.  Each case builds R >=
    min_bytes / bytes distinct device copies of one seeded linear and times
    one graph of R forwards (so no call reads cached weights).  `floor_us`
    is the same byte count read by one plain streaming-read launch
    (tp_read_probe) per call, R distinct buffers in one graph: what a single
    launch of that size reaches at all."""
    from turbopress_amd import _lib
    from turbopress_amd.runtime import PackedTCQLinear
    from turbopress_amd.synthetic import make_activation, make_payload, payload_to
    cases = cases or default_cases()
    lib = _lib.lib()
    floors = {}
    out = []
    for cfg, name, d, n, k, b in cases:
        nb = _bytes(n, d, k, b)
        reps = max(8, -(-int(min_bytes) // nb))
        p = payload_to(make_payload(n, d, k, N_STATES, seed=k), "cuda")
        mods = [PackedTCQLinear(p, mode="hip") for _ in range(reps)]
        x = make_activation(b, d, seed=1).cuda()

        def step(mods=mods, x=x):
            for m in mods:
                m(x)

        us = _graph_us_per_call(step, reps, steps, settle_ms)
        del mods
        key = (nb + 15) & ~15
        if key not in floors:
            bufs = [torch.ones(key // 4, dtype=torch.int32, device="cuda") for _ in range(reps)]
            sink = torch.zeros(1, dtype=torch.int32, device="cuda")

            def probe(bufs=bufs, sink=sink, key=key):
                st = torch.cuda.current_stream().cuda_stream
                for buf in bufs:
                    _lib.check(lib.tp_read_probe(buf.data_ptr(), key, sink.data_ptr(), st), "read_probe")

            floors[key] = _graph_us_per_call(probe, reps, steps)
            del bufs
        torch.cuda.empty_cache()
        gbps = nb / (us * 1e-6) / 1e9
        row = {"config": cfg, "linear": name, "shape": [d, n], "bits": k, "batch": b, "us": round(us, 2),
               "bytes": nb, "gbps": round(gbps, 1),
               "gbps_ref_bytes": round(_ref_bytes(n, d, k, b) / (us * 1e-6) / 1e9, 1),
               "floor_us": round(floors[key], 2), "frac_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4)}
        if b >= 16:
            tfl = 2 * b * n * d / (us * 1e-6) / 1e12
            row["tflops"] = round(tfl, 2)
            row["mfma_frac"] = round(tfl / MFMA_FP16_PEAK_TFLOPS, 4)
        if log:
            log(f"{cfg} {name} k={k} B={b}: {row['us']} us, {row['gbps']} GB/s "
                f"(one read launch of the same bytes: {row['floor_us']} us)")
        out.append(row)
    return out


def c1_layer_stack(steps: int, warmup: int, settle_ms: float, copies: int = 96) -> dict:
    """the Qwen3-0.6B layer's 7 linears (k=3, B=1) as one stack
    launch pair, over `copies` distinct seeded layers (> 256 MB)."""
    from turbopress_amd.synthetic import QWEN3_0_6B_LAYER
    dev = torch.device("cuda", 0)
    layers, inputs = build_layers(dev, n_layers=copies, shapes=QWEN3_0_6B_LAYER)
    stack = make_stack(layers, inputs, ordered=False)
    ms, _, _ = time_graph(stack.run, steps, warmup, settle_ms)
    nb = step_bytes(layers)
    us = ms * 1e3
    out = {"layers": copies, "bytes_per_layer": nb // copies, "us_per_layer": round(us / copies, 3),
           "gbps": round(nb / (us * 1e-6) / 1e9, 1), "frac_hbm_peak": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}
    del stack, layers, inputs
    torch.cuda.empty_cache()
    return out


def cpu_baseline(budget_s: float):
    """The reference's CPU tiled path (oracle restatement), one Qwen3-4B layer
    at k=3, B=1, repeated until ~budget_s of CPU work, scaled to 36 layers."""
    from oracle.tiled_baseline import TiledLinearCPU
    from turbopress_amd.synthetic import QWEN3_4B_LAYER, make_activation, make_payload
    threads, how = host_cpus()
    torch.set_num_threads(threads)
    mods = []
    for j, name in enumerate(ORDER):
        d, n = QWEN3_4B_LAYER[name]
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
        "cores_source": how, "host_cpu_count": os.cpu_count(), "kind": "port",
        "sample": (f"1 of 36 Qwen3-4B layers (q,k,v,o,gate,up,down; k=3, S=64, B=1) through "
                   f"oracle/tiled_baseline.py (torch CPU, {threads} threads), median of "
                   f"{len(times)} runs, scaled x36"),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--settle-ms", type=float, default=500.0,
                    help="wall time each timed leg replays its graph before warm-up (clock settling)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--copy-mib", type=int, default=1024,
                    help="size of the device copy reported as copy_reference (0: skip)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only-primary", action="store_true", help="skip every comparison leg")
    ap.add_argument("--only-batch32", action="store_true",
                    help="run only the batch-32 leg (profiling the MFMA path) and print its figures")
    ap.add_argument("--per-linear", action="store_true",
                    help="run only the one-linear-at-a-time table (configs c0, c1, c3, c4) and print it")
    ap.add_argument("--cases", default=None,
                    help="with --per-linear: comma-separated cfg:name:in:out:bits:batch cases")
    ap.add_argument("--only-chained", action="store_true",
                    help="run only the data-dependent (chained) decode step and print its figures")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: the packed-TCQ decode path is built and measured "
              "on a single GPU only (multi-GPU sharding is design-only); run with --gpus 1.",
              file=sys.stderr)
        return 2
    from turbopress_amd import decode_step

    torch.manual_seed(0)
    dev = torch.device("cuda", 0)
    log = lambda m: print(f"[bench] {m}", file=sys.stderr, flush=True)  # noqa: E731
    if args.per_linear:
        cases = None
        if args.cases:
            cases = [(c[0], c[1], int(c[2]), int(c[3]), int(c[4]), int(c[5]))
                     for c in (s.split(":") for s in args.cases.split(","))]
        print(json.dumps({"per_linear": per_linear_sweep(cases, log=log)}), flush=True)
        return 0
    if args.only_chained:
        print(json.dumps({"chained_step": chained_step(dev, max(5, args.steps // 5), 2, args.settle_ms / 2)}),
              flush=True)
        return 0
    log(f"building {N_LAYERS}x7 packed linears (k={BITS}, S={N_STATES}, batch {BATCH})")
    layers, inputs = build_layers(dev)
    nbytes = step_bytes(layers)
    log(f"{nbytes / 1e9:.4f} GB per step")
    if args.only_batch32:
        print(json.dumps({"batch32": batch32_reference(layers, args.steps, args.warmup, args.settle_ms)}),
              flush=True)
        return 0

    stack = make_stack(layers, inputs, ordered=False)
    ms, ms_wall, _ = time_graph(stack.run, args.steps, args.warmup, args.settle_ms)
    log(f"stack (rotation launch + 1 GEMV launch): {ms * 1e3:.1f} us/step")
    us_gemv = time_gemv_kernel(stack, args.steps, args.warmup, args.settle_ms / 2)
    log(f"stack GEMV kernel alone: {us_gemv:.1f} us/launch")
    parity = check_stack_outputs(stack, layers, inputs)
    log(f"timed plan vs per-linear forward: max-rel {parity['max_rel']:.2e} over "
        f"{parity['linears_checked']} linears ({parity['worst']})")
    if not parity["ok"]:
        print(json.dumps({"error": "stack outputs differ from the per-linear forward", "parity": parity}),
              flush=True)
        return 1
    extra = {}
    if not args.only_primary:
        stack_o = make_stack(layers, inputs, ordered=True)
        ms_o, _, _ = time_graph(stack_o.run, max(5, args.steps // 5), 2, args.settle_ms / 2)
        if stack_o.error():
            raise RuntimeError("stack phase wait timed out")
        log(f"stack, phase-ordered: {ms_o * 1e3:.1f} us/step")
        del stack_o
        steps_slow = max(5, args.steps // 5)

        def grouped():
            for mods, xs in zip(layers, inputs):
                decode_step.layer_forward(mods, xs)

        ms_g, _, _ = time_graph(grouped, steps_slow, 2, args.settle_ms / 2)
        log(f"grouped launches (144/step): {ms_g * 1e3:.1f} us/step")

        def per_linear():
            for mods, xs in zip(layers, inputs):
                for name in ORDER:
                    mods[name](xs[GROUP_INPUT[name]])

        ms_p, _, _ = time_graph(per_linear, steps_slow, 2, args.settle_ms / 2)
        log(f"per-linear launches (252/step): {ms_p * 1e3:.1f} us/step")
        chained = chained_step(dev, steps_slow, 2, args.settle_ms / 2)
        log(f"chained decode step (144 dependent launches): {chained['us_per_step']} us/step, "
            f"parity vs per-linear max-rel {chained['parity_vs_per_linear']['max_rel']:.2e}")
        if not chained["parity_vs_per_linear"]["ok"]:
            print(json.dumps({"error": "chained step outputs differ from the per-linear forward",
                              "chained": chained}), flush=True)
            return 1
        extra = {"phase_ordered_stack_us": round(ms_o * 1e3, 2), "grouped_launches_us": round(ms_g * 1e3, 2),
                 "per_linear_launches_us": round(ms_p * 1e3, 2), "chained_step_us": chained["us_per_step"],
                 "chained_step": chained}

    copy_ref = copy_reference(args.copy_mib) if args.copy_mib > 0 and not args.only_primary else None
    if copy_ref:
        log(f"device copy {args.copy_mib} MiB: {copy_ref['gbps']} GB/s (read + write)")
    read_ref = read_reference(nbytes, settle_ms=args.settle_ms / 2)
    log(f"streaming read of {nbytes / 1e9:.4f} GB: {read_ref['us']} us, {read_ref['gbps']} GB/s")
    enc, enc_sample, b32, table, c1 = None, None, None, None, None
    if not args.only_primary:
        b32 = batch32_reference(layers, args.steps, args.warmup, args.settle_ms)
        log(f"batch 32: stack {b32['stack_gemv_us']} us/GEMV launch, {b32['stack_gemv_tflops']} TFLOP/s")
        del stack
        torch.cuda.empty_cache()
        table = per_linear_sweep(log=log)
        c1 = c1_layer_stack(args.steps, args.warmup, args.settle_ms / 2)
        log(f"c1 Qwen3-0.6B layer as one stack: {c1['us_per_layer']} us/layer, {c1['gbps']} GB/s")
        enc, enc_sample = encoder_reference()
        log(f"TCQ Viterbi encoder, {enc['rows']}x{enc['dim']}: GPU {enc['gpu_us']} us")
    cpu = None
    if not args.no_cpu_baseline:
        log("CPU baseline")
        cpu = cpu_baseline(args.cpu_seconds)
        if enc_sample is not None:
            enc["cpu_baseline"] = cpu_encoder_baseline(enc_sample)
            log(f"encoder CPU baseline (scaled): {enc['cpu_baseline']['value']} s, "
                f"codes match GPU: {enc['cpu_baseline']['codes_match_gpu']}")
    gbps = nbytes / (ms * 1e-3) / 1e9
    gemv_bytes = nbytes - sum(2 * m.in_features for mods in layers for m in mods.values())
    gemv_gbps = gemv_bytes / (us_gemv * 1e-6) / 1e9
    traffic, traffic_src = measured_traffic()
    line = {
        "metric": "µs per decode-step linear stack + HBM GB/s (% peak), 3-bit TCQ, Qwen3-4B b=1",
        "value": round(ms * 1e3, 2), "unit": "us/step", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "settle_ms": args.settle_ms, "ms_per_step": round(ms, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic (seeded codes, codebook, scales, signs, activations)",
        "config": {"workload": "qwen3-4b decode-step linear stack: 36 layers x (q,k,v,o,gate,up,down), "
                               "one HIP graph: rotation launch + one persistent GEMV launch",
                   "layers": N_LAYERS, "bits": BITS, "n_states": N_STATES, "batch": BATCH,
                   "bytes_per_step": nbytes},
        "gbps": round(gbps, 1), "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
        "wall_ms_per_step": round(ms_wall, 5),
        "roofline": {"kernel": "tcq_stack_slot_kernel<3,64,4> (all 252 linears, one launch per step)",
                     "bound": "hbm", "achieved": round(gemv_gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gemv_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "us_per_launch": round(us_gemv, 2), "bytes_per_launch": gemv_bytes},
        "parity": parity,
        "executors": extra,
        "copy_reference": copy_ref,
        "read_reference": read_ref,
        "per_linear": table,
        "c1_layer_stack": c1,
        "batch32": b32,
        "encoder": enc,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
