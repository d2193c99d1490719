"""Decode-step stack (one persistent launch for many linears) vs the oracle (GPU)."""

import numpy as np
import pytest
import torch

from oracle import tcq_oracle as O
from turbopress_amd.synthetic import QWEN3_4B_LAYER, make_activation, make_payload, payload_numpy

pytestmark = pytest.mark.gpu

GEMV_TOL = 2e-3

MIXED = [  # (d, n, phase): hb 512, 512, 4096, 64, 512
    (2560, 4096, 0), (2560, 1024, 0), (4096, 2560, 1), (576, 1536, 2), (9728, 2560, 3),
]


def _build(cuda, shapes, batch, bits=3, ordered=False, bias=False):
    from turbopress_amd.decode_step import LinearStack
    from turbopress_amd.runtime import PackedTCQLinear
    payloads, entries = [], []
    for i, (d, n, ph) in enumerate(shapes):
        p = make_payload(n, d, bits, 64, seed=100 + i, bias=bias and i % 2 == 0)
        payloads.append(p)
        x = make_activation(batch, d, seed=200 + i).to(cuda)
        entries.append((PackedTCQLinear(p, mode="hip"), x, ph))
    return payloads, LinearStack(entries, ordered=ordered)


def _check(payloads, stack):
    for p, x, y in zip(payloads, stack.inputs, stack.outputs):
        ref = O.tiled_forward(payload_numpy(p), x.cpu().numpy())
        assert O.max_rel(y.float().cpu().numpy(), ref) <= GEMV_TOL


@pytest.mark.parametrize("ordered", [False, True])
@pytest.mark.parametrize("batch", [1, 2, 3, 5, 8, 12, 20])
def test_stack_matches_oracle(cuda, ordered, batch):
    """Batch 1-2 / 3-4 / 5-8: slot kernel with 8 / 4 / 2 slots per z load;
    9-16 / 17-32: wide kernel with one / two batch tiles."""
    payloads, stack = _build(cuda, MIXED, batch, ordered=ordered, bias=True)
    stack.run()
    torch.cuda.synchronize()
    _check(payloads, stack)
    assert stack.error() == 0


RAGGED = [  # (d, n, phase): odd n, n below one 16-row tile, n one past a tile
    (2560, 4095, 0), (1024, 1, 0), (576, 17, 1), (2560, 1537, 1), (4096, 33, 2), (1024, 15, 2),
]


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("ordered", [False, True])
@pytest.mark.parametrize("batch", [1, 3, 8, 12, 24])
def test_stack_ragged_rows(cuda, bits, ordered, batch):
    """Row counts that are odd or not a multiple of 16 (the last row shares
    its row-scale and bias dword with the row past the end), with bias:
    every row of every output within 2e-3 of the oracle, in the slot
    kernel (batch <= 4), the wide kernel (batch 5..32) and, phase-ordered at
    batch <= 4, the ordered kernel."""
    payloads, stack = _build(cuda, RAGGED, batch, bits=bits, ordered=ordered, bias=True)
    for o in stack.outputs:
        o.fill_(float("nan"))
    stack.run()
    torch.cuda.synchronize()
    _check(payloads, stack)
    assert stack.error() == 0


def test_stack_k2_and_repeat_runs_reset_counters(cuda):
    payloads, stack = _build(cuda, [(1024, 3072, 0), (3072, 1024, 1), (2048, 1024, 1)], 1, bits=2,
                             ordered=True)
    firsts = None
    for _ in range(3):
        stack.run()
        torch.cuda.synchronize()
        header = stack.plan[:8].cpu()
        assert int(header.count_nonzero()) == 0  # ticket and exit counters back to zero
        outs = [o.clone() for o in stack.outputs]
        if firsts is None:
            firsts = outs
        for a, b in zip(firsts, outs):
            assert torch.equal(a, b)  # full-K blocks: deterministic
    _check(payloads, stack)


@pytest.mark.parametrize("batch", [1, 4, 8, 12])
def test_stack_k4(cuda, batch):
    """4 bits/weight: slot kernel (batch <= 8) and wide kernel."""
    payloads, stack = _build(cuda, MIXED, batch, bits=4, bias=True)
    stack.run()
    torch.cuda.synchronize()
    _check(payloads, stack)
    assert stack.error() == 0


@pytest.mark.parametrize("ordered", [False, True])
def test_stack_graph_replay_with_new_inputs(cuda, ordered):
    """Every replay rotates the new inputs before any z is read."""
    payloads, stack = _build(cuda, [(d, n, ph) for (d, n), ph in
                                    zip(QWEN3_4B_LAYER.values(), (0, 0, 0, 1, 2, 2, 3))], 1, ordered=ordered)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        stack.run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        stack.run()
    for rep in range(3):
        for i, x in enumerate(stack.inputs):
            x.copy_(make_activation(1, x.shape[1], seed=300 + 10 * rep + i).to(x.device))
        g.replay()
        torch.cuda.synchronize()
        _check(payloads, stack)


@pytest.mark.parametrize("batch", [1, 4])
def test_stack_split_launches_match_run(cuda, batch):
    """The two launches called one by one (rotate(), gemv()) give run()'s
    outputs bit for bit (full-K blocks are deterministic)."""
    payloads, stack = _build(cuda, MIXED, batch, bias=True)
    stack.run()
    torch.cuda.synchronize()
    fused = [o.clone() for o in stack.outputs]
    for o in stack.outputs:
        o.zero_()
    stack.rotate()
    stack.gemv()
    torch.cuda.synchronize()
    for a, b in zip(fused, stack.outputs):
        assert torch.equal(a, b)
    _check(payloads, stack)
    assert stack.error() == 0


@pytest.mark.parametrize("shapes", ["mixed", "ragged"])
@pytest.mark.parametrize("ordered", [False, True])
@pytest.mark.parametrize("batch", [1, 3, 4])
def test_stack_unaligned_output_rows(cuda, shapes, ordered, batch):
    """Outputs through the C ABI at an odd element offset with an odd row
    stride: a lane's four rows are not 8-byte aligned there, so the slot
    kernel stores them one by one instead of in one 8-byte store.  Same bits
    as the plan with aligned outputs, and nothing written outside the rows."""
    import ctypes

    from turbopress_amd import _lib
    from turbopress_amd import hip_kernel as hk
    shape_list = MIXED if shapes == "mixed" else RAGGED
    payloads, stack = _build(cuda, shape_list, batch, ordered=ordered)
    stack.run()
    torch.cuda.synchronize()
    ref = [o.clone() for o in stack.outputs]
    arr = (_lib.StackLinear * len(stack.linears))()
    bufs, lds = [], []
    for i, (lin, x, ph) in enumerate(zip(stack.linears, stack.inputs, stack.phases)):
        ldy = lin.out_features + 3
        buf = torch.full((batch * ldy + 1,), float("nan"), dtype=torch.float16, device=cuda)
        bufs.append(buf)
        lds.append(ldy)
        pb = lin._tiled_geo["path_bytes"]
        arr[i] = _lib.StackLinear(
            lin.tiled_packed.data_ptr(), lin.tiled_packed.data_ptr() + pb, x.data_ptr(), lin.in_features,
            lin.rot_scale.data_ptr(), lin.block, lin.scales.data_ptr(), 0, buf.data_ptr() + 2, ldy,
            lin.out_features, lin.in_features, ph, 0)
    lib = _lib.lib()
    nbytes = int(lib.tp_stack_plan_bytes(arr, len(stack.linears), stack.bits, batch))
    plan = torch.zeros(nbytes, dtype=torch.uint8, device=cuda)
    torch.cuda.synchronize()
    _lib.check(lib.tp_stack_plan_init(arr, len(stack.linears), stack.bits, batch, plan.data_ptr(), nbytes),
               "stack_plan_init")
    _lib.check(lib.tp_stack_run(plan.data_ptr(), batch, stack.codebook.data_ptr(), stack.bits, stack.n_states,
                                int(ordered), stack.total_blocks, hk.current_stream_ptr(cuda)), "stack_run")
    torch.cuda.synchronize()
    for lin, buf, ldy, r in zip(stack.linears, bufs, lds, ref):
        rows = buf[1:].view(batch, ldy)
        assert torch.equal(rows[:, :lin.out_features].view(torch.int16), r.view(torch.int16))
        assert torch.isnan(rows[:, lin.out_features:]).all() and torch.isnan(buf[0])
    err = ctypes.c_int()
    _lib.check(lib.tp_stack_error(plan.data_ptr(), ctypes.byref(err)), "stack_error")
    assert err.value == 0


def test_stack_rejects_mixed_codebooks(cuda):
    from turbopress_amd.decode_step import LinearStack
    from turbopress_amd.runtime import PackedTCQLinear
    a = PackedTCQLinear(make_payload(64, 256, 3, 64, seed=1), mode="hip")
    b = PackedTCQLinear(make_payload(64, 256, 2, 64, seed=2), mode="hip")
    x = torch.zeros(1, 256, dtype=torch.float16, device=cuda)
    with pytest.raises(ValueError):
        LinearStack([(a, x, 0), (b, x, 0)])
    with pytest.raises(ValueError):
        LinearStack([(a, x, 1), (a, x, 0)])  # phases must not decrease
    with pytest.raises(ValueError):
        LinearStack([(a, x, 0), (a, x, 2)])  # nor skip a phase
    with pytest.raises(ValueError):
        LinearStack([(a, x, 1), (a, x, 1)])  # and start at 0


def test_headline_plan_matches_per_linear_and_oracle(cuda):
    """The exact plan bench.py times: Qwen3-4B, 36 layers x 7 linears (252
    linears, 144 phases, 1.37 GB), k=3, S=64, batch 1.  Every stack output,
    unordered and phase-ordered, within max-rel 2e-3 of the per-linear
    PackedTCQLinear.forward on the same input, and layers 0 and 35 within
    2e-3 of the oracle's tiled forward."""
    import bench
    layers, inputs = bench.build_layers(cuda)
    payload_of = {}
    from turbopress_amd.synthetic import QWEN3_4B_LAYER as SH
    for li in (0, 35):
        for j, name in enumerate(bench.ORDER):
            d, n = SH[name]
            payload_of[(li, name)] = make_payload(n, d, 3, 64, seed=1000 * li + j)
    refs = [mods[name](xs[bench.GROUP_INPUT[name]]).float()
            for mods, xs in zip(layers, inputs) for name in bench.ORDER]
    for ordered in (False, True):
        stack = bench.make_stack(layers, inputs, ordered=ordered)
        assert len(stack.linears) == 252 and stack.n_phases == 144
        for _ in range(2):  # the second run starts from the counters the first one reset
            for o in stack.outputs:
                o.fill_(float("nan"))
            stack.run()
            torch.cuda.synchronize()
            for i, (got, ref) in enumerate(zip(stack.outputs, refs)):
                err = float((got.float() - ref).abs().max() / ref.abs().max())
                assert err <= GEMV_TOL, (ordered, i // 7, bench.ORDER[i % 7], err)
        assert stack.error() == 0
        if not ordered:
            for (li, name), p in payload_of.items():
                i = 7 * li + bench.ORDER.index(name)
                x = inputs[li][bench.GROUP_INPUT[name]].cpu().numpy()
                ref = O.tiled_forward(payload_numpy(p), x)
                assert O.max_rel(stack.outputs[i].float().cpu().numpy(), ref) <= GEMV_TOL, (li, name)
        del stack


def test_batch32_stack_mixed_blocks(cuda):
    """192 linears at batch 32 (9216 rotation tiles, the wide kernel), with
    Hadamard blocks 64..8192 (8192: two 4096-column sub-tiles summed) and
    bias on every third.  Every output within 2e-3 of the per-linear forward
    on the same input, and one linear of each shape within 2e-3 of the
    oracle's tiled forward."""
    from turbopress_amd.decode_step import LinearStack
    from turbopress_amd.runtime import PackedTCQLinear
    shapes = [(2560, 48), (576, 32), (8192, 32), (4096, 48), (9728, 32), (1024, 32)]  # (d, n)
    payloads, entries = [], []
    for g in range(32):
        for j, (d, n) in enumerate(shapes):
            p = make_payload(n, d, 3, 64, seed=5000 + 6 * g + j, bias=(g + j) % 3 == 0)
            payloads.append(p)
            x = make_activation(32, d, seed=7000 + 6 * g + j).to(cuda)
            entries.append((PackedTCQLinear(p, mode="hip"), x, 0))
    stack = LinearStack(entries)
    for o in stack.outputs:
        o.fill_(float("nan"))
    stack.run()
    torch.cuda.synchronize()
    assert stack.error() == 0
    for i, ((lin, x, _), y) in enumerate(zip(entries, stack.outputs)):
        ref = lin(x).float()
        err = float((y.float() - ref).abs().max() / ref.abs().max())
        assert err <= GEMV_TOL, (i, shapes[i % 6], err)
    for i in range(6):
        ref = O.tiled_forward(payload_numpy(payloads[i]), entries[i][1].cpu().numpy())
        assert O.max_rel(stack.outputs[i].float().cpu().numpy(), ref) <= GEMV_TOL, shapes[i]


@pytest.mark.parametrize("batch", [1, 3, 9, 32])
def test_stack_rotation_bit_exact(cuda, batch):
    """The rotation launch's z rows (the plan's last region, one [batch,
    G4 * 256] fp16 block per linear in order) equal the oracle's
    fp16(blockFWHT(x * rot_scale)) bit for bit, zero past d, for Hadamard
    blocks 4..16384.  Blocks of at most 4096 columns are packed across batch
    rows into 4096-column tiles (d = 12, block 4: one tile holds every row;
    d = 2560 at batch 3: a tile of 8 blocks spans rows 0 and 1, the last
    tile is partial); larger blocks run per row."""
    _rotation_bit_exact(cuda, batch, ROT_DS)


ROT_DS = [12, 40, 96, 128, 576, 1024, 2048, 2560, 3072, 4096, 6144, 8192, 9728, 16384]


def test_stack_rotation_bit_exact_many_tiles(cuda):
    """The same at batch 32 with every width three times: more than four
    4096-column tiles per CU, where the launch takes its bpermute butterflies
    at lane distance 16 / 32 (the permlane swaps below that)."""
    ds = ROT_DS * 3
    tiles = sum(-(-32 * d // 4096) if d <= 4096 or d % 4096 else 32 * d // 4096 for d in ds)
    assert tiles > 4 * torch.cuda.get_device_properties(cuda).multi_processor_count
    _rotation_bit_exact(cuda, 32, ds)


def _rotation_bit_exact(cuda, batch, ds):
    from turbopress_amd.decode_step import LinearStack
    from turbopress_amd.runtime import PackedTCQLinear
    payloads, entries = [], []
    for i, d in enumerate(ds):
        p = make_payload(16, d, 3, 64, seed=400 + i)
        payloads.append(p)
        gen = torch.Generator().manual_seed(500 + i)
        x = (torch.randn(batch, d, generator=gen) * 3).to(torch.float16)
        entries.append((PackedTCQLinear(p, mode="hip"), x.to(cuda), 0))
    stack = LinearStack(entries)
    stack.rotate()
    torch.cuda.synchronize()
    widths = [-(-d // 256) * 256 for d in ds]
    zbytes = [batch * w * 2 for w in widths]
    plan = stack.plan.cpu().numpy()
    off = plan.size - sum(zbytes)
    for p, (_, x, _), w, nb in zip(payloads, entries, widths, zbytes):
        got = plan[off:off + nb].view(np.uint16).reshape(batch, w)
        off += nb
        d = int(p["d"])
        ref = O.rotate_activations(payload_numpy(p), x.cpu().numpy()).astype(np.float16).view(np.uint16)
        assert np.array_equal(got[:, :d], ref), (d, int(p["block"]))
        assert not got[:, d:].any(), d


@pytest.mark.parametrize("batch", [3, 5])
def test_stack_rotation_special_values(cuda, batch):
    """Zeros of both signs and infinities through the rotation launch (16 and
    64 columns per thread at batch 3 and 5; blocks 4, 512, 4096 and 8192):
    a row of +0, a row of -0 (products with the negative signs are -0, and
    every zero z carries the sign IEEE arithmetic gives it, which the
    division's fix-up keeps), a row of random values with -0 entries and
    one +inf per Hadamard block (an infinite z everywhere in that block).  z
    equals the oracle's bit for bit wherever the oracle's is not NaN, and is
    NaN where it is."""
    from turbopress_amd.decode_step import LinearStack
    from turbopress_amd.runtime import PackedTCQLinear
    ds = [12, 2560, 4096, 8192]
    payloads, entries = [], []
    for i, d in enumerate(ds):
        p = make_payload(16, d, 3, 64, seed=700 + i)
        payloads.append(p)
        gen = torch.Generator().manual_seed(800 + i)
        x = (torch.randn(batch, d, generator=gen) * 3).to(torch.float16)
        x[0] = 0.0
        x[1] = -0.0
        x[2, 5::13] = -0.0
        x[2, ::int(p["block"])] = float("inf")
        entries.append((PackedTCQLinear(p, mode="hip"), x.to(cuda), 0))
    stack = LinearStack(entries)
    stack.rotate()
    torch.cuda.synchronize()
    widths = [-(-d // 256) * 256 for d in ds]
    zbytes = [batch * w * 2 for w in widths]
    plan = stack.plan.cpu().numpy()
    off = plan.size - sum(zbytes)
    for p, (_, x, _), w, nb in zip(payloads, entries, widths, zbytes):
        got = plan[off:off + nb].view(np.uint16).reshape(batch, w)
        off += nb
        d = int(p["d"])
        with np.errstate(invalid="ignore"):
            ref = O.rotate_activations(payload_numpy(p), x.cpu().numpy()).astype(np.float16)
        g16 = got[:, :d].view(np.float16)
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(g16), nan), d
        assert np.array_equal(got[:, :d][~nan], ref.view(np.uint16)[~nan]), d
        # (the cases occur: zeros of both signs, infinities)
        assert np.signbit(ref[:2]).any() and (~np.signbit(ref[:2])).any() and np.isinf(ref[2]).all(), d


@pytest.mark.parametrize("shapes", ["qwen3-0.6b", "qwen3-4b"])
def test_chained_step_matches_oracle_layer_by_layer(cuda, shapes):
    """The data-dependent decode step (q/k/v group -> o -> gate/up group ->
    down -> next layer, 4 launches per layer) captured in a graph and
    replayed on a new input: every projection of every layer within the
    GEMV tolerance of the oracle on the input that launch read (the previous
    launch's GPU output), so the chain passes data, and o / gate / down
    really consume q / o / gate."""
    from turbopress_amd.decode_step import ChainedDecodeStep
    from turbopress_amd.runtime import PackedTCQLinear
    from turbopress_amd.synthetic import QWEN3_0_6B_LAYER, unit_gain
    table = QWEN3_0_6B_LAYER if shapes == "qwen3-0.6b" else QWEN3_4B_LAYER
    n_layers = 3 if shapes == "qwen3-0.6b" else 2
    names = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
    payloads, layers = [], []
    for li in range(n_layers):
        ps, mods = {}, {}
        for j, name in enumerate(names):
            d, n = table[name]
            p = unit_gain(make_payload(n, d, 3, 64, seed=500 * li + j, bias=(name == "o_proj")))
            ps[name], mods[name] = p, PackedTCQLinear(p, mode="hip")
        payloads.append(ps)
        layers.append(mods)
    x = make_activation(1, table["q_proj"][0], seed=3).to(cuda)
    chain = ChainedDecodeStep(layers, x)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        chain.run()
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g):
        chain.run()
    x.copy_(make_activation(1, table["q_proj"][0], seed=4).to(cuda))
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    for li in range(n_layers):
        ins = chain.layer_inputs(li)
        for name in names:
            got = chain.outputs[li][name].float().cpu().numpy()
            ref = O.tiled_forward(payload_numpy(payloads[li][name]), ins[name].float().cpu().numpy())
            assert O.max_rel(got, ref) <= GEMV_TOL, (li, name)
    assert torch.equal(chain.layer_inputs(1)["q_proj"], chain.outputs[0]["down_proj"])
    with pytest.raises(ValueError):
        ChainedDecodeStep([layers[0], {**layers[1], "q_proj": layers[1]["o_proj"]}], x)
