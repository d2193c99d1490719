"""Bandwidth path (device layout + MFMA decode-GEMV) vs the CPU oracle (GPU).

The decode check runs the GEMV kernel's own decode front-end (subset bits by
funnel-shift XORs, pair-table lookups) through tp_decode_tiled and requires
bit-exact fp16 weights; GEMV outputs must be within max-rel 2e-3 of the fp64
product on the same decoded weights.  Shapes cover ragged rows (n not a
multiple of 16), ragged columns (d not a multiple of 64/256), single-unit and
split-K tiles, every supported trellis, and batches across the 16-column
MFMA tiles (1, 3, 16, 17, 32, 40).
"""

import numpy as np
import pytest
import torch

from oracle import tcq_oracle as O
from turbopress_amd import hip_kernel as hk
from turbopress_amd.synthetic import (
    QWEN3_4B_LAYER, make_activation, make_payload, payload_numpy)

pytestmark = pytest.mark.gpu

GEMV_TOL = 2e-3

DECODE_CASES = [
    (16, 64, 3, 64), (17, 64, 2, 64), (33, 576, 2, 64), (40, 1000, 3, 64),
    (5, 200, 3, 16), (31, 328, 2, 8), (20, 130, 3, 4), (48, 2560, 3, 64), (64, 9728, 2, 64),
    (16, 64, 4, 64), (33, 576, 4, 64), (40, 1000, 4, 16), (20, 130, 4, 4), (31, 328, 4, 8), (48, 2560, 4, 64),
]


@pytest.mark.parametrize("n,d,bits,n_states", DECODE_CASES)
def test_tiled_decode_bit_exact(cuda, n, d, bits, n_states):
    from turbopress_amd.runtime import PackedTCQLinear
    p = make_payload(n, d, bits, n_states, seed=n + 7 * d)
    lin = PackedTCQLinear(p, mode="hip")
    assert lin.tiled_packed is not None and lin.path_packed is None
    got = lin.decode_rows(0, n).cpu().numpy()
    ref = O.decode_rows(payload_numpy(p))
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


def test_retiled_bytes_are_true_rate(cuda):
    from turbopress_amd.hip_kernel import tiled_layout
    for (d, n) in QWEN3_4B_LAYER.values():
        for bits in (2, 3, 4):
            g = tiled_layout(n, d, bits)
            assert g["path_bytes"] + g["member_bytes"] == g["tiles"] * 16 * g["segments"] * 64 * bits // 8
            assert g["tiles"] * 16 == -(-n // 16) * 16 and g["z_cols"] >= d


GEMV_CASES = [
    # n, d, bits, S, batch
    (1536, 576, 2, 64, 1),
    (192, 256, 3, 64, 2),
    (100, 700, 3, 16, 3),
    (4096, 2560, 3, 64, 1),
    (1024, 2560, 3, 64, 16),
    (2560, 9728, 3, 64, 17),
    (9728, 2560, 2, 64, 32),
    (300, 512, 3, 8, 40),
    (2560, 4096, 3, 64, 4),
    (9728, 2560, 4, 64, 1),      # k=4: one-pass kernel
    (2560, 9728, 4, 64, 3),
    (130, 200, 4, 16, 2),
    (1024, 2560, 4, 64, 8),      # k=4: split-K kernel
    (300, 512, 4, 8, 20),        # k=4: wide kernel (rotated input)
]


@pytest.mark.parametrize("n,d,bits,n_states,batch", GEMV_CASES)
def test_tiled_gemv_matches_fp64(cuda, n, d, bits, n_states, batch):
    from turbopress_amd.hip_kernel import packed_gemv
    from turbopress_amd.runtime import PackedTCQLinear
    p = make_payload(n, d, bits, n_states, seed=n * 3 + d)
    lin = PackedTCQLinear(p, mode="hip")
    z = torch.randn(batch, d, generator=torch.Generator().manual_seed(2)).to(torch.float16)
    y = packed_gemv(z.to(cuda), lin).float().cpu().numpy()
    ref = O.gemv_fp64(payload_numpy(p), z.numpy().astype(np.float64))
    assert O.max_rel(y, ref) <= GEMV_TOL


@pytest.mark.parametrize("name", sorted(QWEN3_4B_LAYER))
def test_qwen3_4b_forward_matches_tiled_oracle(cuda, name):
    """Config 2 shapes, one layer, batch 1: rotation + GEMV end to end."""
    from turbopress_amd.runtime import PackedTCQLinear
    d, n = QWEN3_4B_LAYER[name]
    p = make_payload(n, d, 3, 64, seed=len(name) * 31 + n)
    lin = PackedTCQLinear(p, mode="hip")
    x = make_activation(1, d, seed=3)
    y = lin(x.to(cuda)).float().cpu().numpy()
    assert O.max_rel(y, O.tiled_forward(payload_numpy(p), x.numpy())) <= GEMV_TOL


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("name", ["gate_proj", "down_proj"])
def test_c3_mlp_rates_and_batches(cuda, name, bits):
    """Config 3: Qwen3-4B MLP shapes at k = 2, 3, 4 and batch 1, 4, 8 (plus 2
    and 5: the one-pass kernel where the input fits -- down_proj up to batch
    2, gate_proj up to 8 --, the split-K kernel otherwise), each batch a
    separate forward checked against one oracle evaluation."""
    from turbopress_amd.runtime import PackedTCQLinear
    d, n = QWEN3_4B_LAYER[name]
    p = make_payload(n, d, bits, 64, seed=40 + bits)
    lin = PackedTCQLinear(p, mode="hip")
    xs = [make_activation(b, d, seed=10 * bits + b) for b in (1, 2, 4, 5, 8)]
    ref = O.tiled_forward(payload_numpy(p), np.concatenate([x.numpy() for x in xs]))
    r0 = 0
    for x in xs:
        y = lin(x.to(cuda)).float().cpu().numpy()
        assert O.max_rel(y, ref[r0:r0 + x.shape[0]]) <= GEMV_TOL, (name, bits, x.shape[0])
        r0 += x.shape[0]


@pytest.mark.parametrize("name", ["gate_proj", "down_proj"])
def test_c4_batch32(cuda, name):
    """Config 4: down / gate at batch 32, k=3 (rotation + wide kernel with
    split-K sums in the workspace), twice in a row (the workspace returns to
    zero)."""
    from turbopress_amd.runtime import PackedTCQLinear
    d, n = QWEN3_4B_LAYER[name]
    p = make_payload(n, d, 3, 64, seed=77)
    lin = PackedTCQLinear(p, mode="hip")
    x = make_activation(32, d, seed=5)
    ref = O.tiled_forward(payload_numpy(p), x.numpy())
    for _ in range(2):
        y = lin(x.to(cuda)).float().cpu().numpy()
        assert O.max_rel(y, ref) <= GEMV_TOL
    assert int(hk.shared_workspace(cuda, 0).count_nonzero()) == 0


def test_workspace_returns_to_zero_and_calls_repeat(cuda):
    from turbopress_amd.runtime import PackedTCQLinear
    p = make_payload(2560, 9728, 3, 64, seed=5, bias=True)
    lin = PackedTCQLinear(p, mode="hip")
    x = make_activation(2, 9728, seed=4).to(cuda)
    ys = [lin(x) for _ in range(3)]
    torch.cuda.synchronize()
    assert int(hk.shared_workspace(cuda, 0).count_nonzero()) == 0
    for y in ys[1:]:
        assert float((y.float() - ys[0].float()).abs().max()) <= 2e-3 * float(ys[0].float().abs().max())
    ref = O.tiled_forward(payload_numpy(p), x.cpu().numpy())
    assert O.max_rel(ys[0].float().cpu().numpy(), ref) <= GEMV_TOL


def test_graph_replays_match_eager(cuda):
    from turbopress_amd.runtime import PackedTCQLinear
    lins, xs = [], []
    for i, (d, n) in enumerate([(2560, 4096), (4096, 2560), (2560, 9728)]):
        lins.append(PackedTCQLinear(make_payload(n, d, 3, 64, seed=40 + i), mode="hip"))
        xs.append(make_activation(1, d, seed=i).to(cuda))
    eager = [lin(x).clone() for lin, x in zip(lins, xs)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for lin, x in zip(lins, xs):
            lin(x)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [lin(x) for lin, x in zip(lins, xs)]
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert float((o.float() - e.float()).abs().max()) <= 2e-3 * float(e.float().abs().max()), rep
        _ = [lin(x) for lin, x in zip(lins, xs)]  # eager work between replays
        torch.cuda.synchronize()


FUSED_CASES = [  # (n, d, bits): Hadamard block d & -d = 2, 4, 64, 512, 1024, 2048, 4096
    (40, 130, 3), (48, 100, 2), (1536, 576, 2), (256, 2560, 3), (200, 3072, 3),
    (300, 2048, 2), (2560, 4096, 3), (1536, 576, 4), (256, 2560, 4), (200, 3072, 4), (2560, 4096, 4),
]


@pytest.mark.parametrize("n,d,bits", FUSED_CASES)
@pytest.mark.parametrize("batch", [1, 4, 12, 20])
def test_fused_forward_matches_oracle(cuda, n, d, bits, batch):
    """tp_packed_linear_forward: rotation computed per workgroup in LDS (full
    blocks, partial blocks of a larger Hadamard, unaligned d fallback); at
    batch 12 / 20 with blocks <= 512 the wide kernel rotates each 512-column
    chunk itself (one and two 16-row batch tiles)."""
    from turbopress_amd.runtime import PackedTCQLinear
    p = make_payload(n, d, bits, 64, seed=d + batch, bias=True)
    lin = PackedTCQLinear(p, mode="hip")
    x = make_activation(batch, d, seed=batch)
    y = lin(x.to(cuda)).float().cpu().numpy()
    assert O.max_rel(y, O.tiled_forward(payload_numpy(p), x.numpy())) <= GEMV_TOL


def test_fused_equals_two_launch_path(cuda):
    from turbopress_amd import hip_kernel as hk
    from turbopress_amd.runtime import PackedTCQLinear
    p = make_payload(2560, 9728, 3, 64, seed=9)
    lin = PackedTCQLinear(p, mode="hip")
    x = make_activation(3, 9728, seed=9).to(cuda)
    fused = lin(x).float()
    two = hk.packed_gemv(hk.fwht_scale(x, lin.rot_scale, lin.block), lin).float()
    assert float((fused - two).abs().max()) <= 2e-3 * float(two.abs().max())


@pytest.mark.parametrize("batch", [12, 32])
def test_fused_wide_equals_two_launch_path(cuda, batch):
    """Batch 9..32 at Hadamard block 512: the wide kernel rotating in the
    launch matches the rotation launch + wide kernel on z."""
    from turbopress_amd import hip_kernel as hk
    from turbopress_amd.runtime import PackedTCQLinear
    p = make_payload(9728, 2560, 3, 64, seed=11)
    lin = PackedTCQLinear(p, mode="hip")
    x = make_activation(batch, 2560, seed=12).to(cuda)
    fused = lin(x).float()
    zpad = hk.rotate_padded(x, lin.rot_scale, lin.block, lin._tiled_geo["z_cols"])
    two = hk.gemv_tiled(zpad, lin, lin.bias, torch.empty(batch, 9728, dtype=torch.float16, device=cuda)).float()
    assert float((fused - two).abs().max()) <= 2e-3 * float(two.abs().max())


@pytest.mark.parametrize("shapes,batch,bits", [
    ([(1024, 2048), (1024, 1024), (1024, 1024)], 1, 3),   # Qwen3-0.6B q/k/v
    ([(2560, 9728), (2560, 9728)], 1, 3),                 # Qwen3-4B gate/up
    ([(2560, 4096), (2560, 1024), (2560, 1024)], 5, 3),
    # Hadamard blocks of 1024 / 2048 columns at the other rates
    ([(1024, 2048), (1024, 1024), (1024, 1024)], 3, 2),
    ([(2048, 1024), (2048, 512)], 2, 4),
])
def test_group_forward_matches_oracle(cuda, shapes, batch, bits):
    """tp_packed_linear_forward_group: several linears on one input, one launch."""
    from turbopress_amd import hip_kernel as hk
    from turbopress_amd.runtime import PackedTCQLinear
    d = shapes[0][0]
    payloads = [make_payload(n, dd, bits, 64, seed=60 + i, bias=(i == 1))
                for i, (dd, n) in enumerate(shapes)]
    lins = [PackedTCQLinear(p, mode="hip") for p in payloads]
    x = make_activation(batch, d, seed=8)
    outs = hk.forward_group(lins, x.to(cuda))
    for p, o, (dd, n) in zip(payloads, outs, shapes):
        assert o.shape == (batch, n)
        ref = O.tiled_forward(payload_numpy(p), x.numpy())
        assert O.max_rel(o.float().cpu().numpy(), ref) <= GEMV_TOL


def test_shared_workspace_two_linears_back_to_back(cuda):
    """Two linears of different shapes take turns on the one split-K
    workspace of the stream (batch 12 and 24: both split K), then a grouped
    launch gives each member a disjoint region of it; every output matches
    the oracle and the workspace is zero after each launch.  No linear holds
    a workspace of its own."""
    from turbopress_amd.runtime import PackedTCQLinear
    shapes = [(9728, 2560, 12), (2560, 9728, 24), (9728, 2560, 24)]
    lins, ps = [], []
    for i, (n, d, _) in enumerate(shapes):
        ps.append(make_payload(n, d, 3, 64, seed=300 + i, bias=(i == 1)))
        lins.append(PackedTCQLinear(ps[-1], mode="hip"))
        assert not any(t.numel() > 0 and name.endswith("ws") for name, t in lins[-1].named_buffers())
    for rnd in range(2):
        for lin, p, (n, d, batch) in zip(lins, ps, shapes):
            x = make_activation(batch, d, seed=10 * rnd + batch)
            y = lin(x.to(cuda))
            torch.cuda.synchronize()
            assert int(hk.shared_workspace(cuda, 0).count_nonzero()) == 0, (rnd, n, d)
            ref = O.tiled_forward(payload_numpy(p), x.numpy())
            assert O.max_rel(y.float().cpu().numpy(), ref) <= GEMV_TOL, (rnd, n, d, batch)
    # a group of two linears sharing the input (disjoint workspace regions)
    x = make_activation(12, 2560, seed=99)
    outs = hk.forward_group([lins[0], lins[2]], x.to(cuda))
    torch.cuda.synchronize()
    assert int(hk.shared_workspace(cuda, 0).count_nonzero()) == 0
    for y, p in zip(outs, (ps[0], ps[2])):
        assert O.max_rel(y.float().cpu().numpy(), O.tiled_forward(payload_numpy(p), x.numpy())) <= GEMV_TOL


KSPLIT_CASES = [  # (n, d, batch): K long against the rows (down_proj and kin), Hadamard blocks <= 512
    (2560, 9728, 1), (2560, 9728, 2), (2560, 9728, 4), (2560, 9728, 8),
    (1024, 3584, 4), (333, 4864, 3), (1537, 2624, 8), (96, 9728, 5)]


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("n,d,batch", KSPLIT_CASES)
def test_ksplit_shapes_match_oracle_deterministically(cuda, bits, n, d, batch):
    """Shapes whose K range is long against their rows, where the one-pass
    forward cuts K into parts of whole Hadamard blocks summed through the
    shared workspace (n odd or not a multiple of 16, d not a multiple of
    256, bias): outputs within the GEMV tolerance of the oracle, a second
    call bit-identical to the first (the parts are added in a fixed order),
    and the workspace zero after each call."""
    from turbopress_amd.runtime import PackedTCQLinear
    p = make_payload(n, d, bits, 64, seed=n + d + batch, bias=bool(n % 2))
    lin = PackedTCQLinear(p, mode="hip")
    x = make_activation(batch, d, seed=batch).to(cuda)
    y1 = lin(x)
    torch.cuda.synchronize()
    assert int(hk.shared_workspace(cuda, 0).count_nonzero()) == 0
    y2 = lin(x)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    assert int(hk.shared_workspace(cuda, 0).count_nonzero()) == 0
    ref = O.tiled_forward(payload_numpy(p), x.cpu().numpy())
    assert O.max_rel(y1.float().cpu().numpy(), ref) <= GEMV_TOL, (n, d, bits, batch)


@pytest.mark.parametrize("d,block", [(3072, 1024), (4096, 4096), (2560, 512)])
@pytest.mark.parametrize("batch", [12, 20])
@pytest.mark.parametrize("x_offset", [0, 8])
def test_packed_linear_forward_abi_batch_9_to_32(cuda, d, block, batch, x_offset):
    """tp_packed_linear_forward called through the C ABI at batch 9..32: with a
    Hadamard block over 512 or an x that is only 8-byte aligned it runs the
    split-K kernel with the rotation fused per workgroup (the path Python's
    forward_tiled routes around); with block 512 and 16-byte aligned x the
    wide kernel rotating each chunk itself."""
    from turbopress_amd import _lib
    from turbopress_amd.runtime import PackedTCQLinear
    n = 200
    p = make_payload(n, d, 3, 64, seed=d + batch, bias=True)
    assert p["block"] == block
    lin = PackedTCQLinear(p, mode="hip")
    x = make_activation(batch, d, seed=batch + x_offset)
    # x placed `x_offset` bytes past a 16-byte aligned base
    raw = torch.zeros(batch * d + 8, dtype=torch.float16, device=cuda)
    xs = raw[x_offset // 2: x_offset // 2 + batch * d].view(batch, d)
    xs.copy_(x.to(cuda))
    assert xs.data_ptr() % 16 == x_offset
    y = torch.full((batch, n), float("nan"), dtype=torch.float16, device=cuda)
    buf, pb = lin.tiled_packed, lin._tiled_geo["path_bytes"]
    ws = hk.gemv_workspace(n, 32, cuda)
    st = _lib.lib().tp_packed_linear_forward(
        xs.data_ptr(), d, batch, lin.rot_scale.data_ptr(), block, buf.data_ptr(), buf.data_ptr() + pb,
        lin.scales.data_ptr(), lin.codebook.data_ptr(), lin.bias.data_ptr(), n, d, 3, 64, y.data_ptr(), n,
        ws.data_ptr(), ws.numel(), torch.cuda.current_stream(cuda).cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    ref = O.tiled_forward(payload_numpy(p), x.numpy())
    assert O.max_rel(y.float().cpu().numpy(), ref) <= GEMV_TOL
    assert int(ws.count_nonzero()) == 0  # split-K workspace back to zero


@pytest.mark.parametrize("batch", [1, 4])
def test_packed_linear_forward_abi_misaligned_codebook(cuda, batch):
    """A codebook only 2-byte aligned: the one-pass kernel reads it as dwords
    through the scalar cache and declines it, and the call runs the older
    tiled kernels, with the same results (the aligned call beside it takes
    the one-pass kernel)."""
    from turbopress_amd import _lib
    from turbopress_amd.runtime import PackedTCQLinear
    n, d = 200, 2560
    p = make_payload(n, d, 3, 64, seed=31 + batch)
    lin = PackedTCQLinear(p, mode="hip")
    x = make_activation(batch, d, seed=batch).to(cuda)
    cb = lin.codebook
    raw = torch.zeros(cb.numel() + 1, dtype=torch.float16, device=cuda)
    cbs = raw[1: 1 + cb.numel()]
    cbs.copy_(cb)
    assert cbs.data_ptr() % 4 == 2
    buf, pb = lin.tiled_packed, lin._tiled_geo["path_bytes"]
    ws = hk.gemv_workspace(n, 32, cuda)
    ys = []
    for cbp in (cb.data_ptr(), cbs.data_ptr()):
        y = torch.full((batch, n), float("nan"), dtype=torch.float16, device=cuda)
        st = _lib.lib().tp_packed_linear_forward(
            x.data_ptr(), d, batch, lin.rot_scale.data_ptr(), p["block"], buf.data_ptr(), buf.data_ptr() + pb,
            lin.scales.data_ptr(), cbp, 0, n, d, 3, 64, y.data_ptr(), n,
            ws.data_ptr(), ws.numel(), torch.cuda.current_stream(cuda).cuda_stream)
        assert st == 0
        ys.append(y)
    torch.cuda.synchronize()
    ref = O.tiled_forward(payload_numpy(p), x.cpu().numpy())
    for y in ys:
        assert O.max_rel(y.float().cpu().numpy(), ref) <= GEMV_TOL
    assert int(ws.count_nonzero()) == 0


def _random_case(seed):
    """A seeded (n, d, bits, n_states, batch): d with Hadamard blocks from 32
    to 2048 columns, n not a multiple of the 16-row tile, batch 1..32."""
    rng = np.random.default_rng(1000 + seed)
    d = int(rng.choice([96, 160, 192, 320, 576, 640, 1024, 1152, 1536, 2048, 2560, 3072]))
    n = int(rng.integers(1, 70)) * 16 + int(rng.integers(0, 16))
    bits = int(rng.choice([2, 3, 4]))
    n_states = int(rng.choice([4, 8, 16, 64]))
    batch = int(rng.choice([1, 2, 3, 4, 5, 6, 8, 9, 12, 16, 17, 24, 32]))
    return n, d, bits, n_states, batch


@pytest.mark.parametrize("seed", range(40))
def test_random_shapes_match_oracle(cuda, seed):
    """PackedTCQLinear.forward at seeded random shapes, rates, trellis sizes
    and batches (every launch route: one-pass, split-K, wide, rotation
    launch + GEMV) against the CPU oracle's tiled forward, to the GEMV
    tolerance."""
    from turbopress_amd.runtime import PackedTCQLinear
    n, d, bits, n_states, batch = _random_case(seed)
    p = make_payload(n, d, bits, n_states, seed=seed, bias=bool(seed % 2))
    lin = PackedTCQLinear(p, mode="hip")
    x = make_activation(batch, d, seed=seed)
    y = lin(x.to(cuda)).float().cpu().numpy()
    assert y.shape == (batch, n)
    assert O.max_rel(y, O.tiled_forward(payload_numpy(p), x.numpy())) <= GEMV_TOL, (n, d, bits, n_states, batch)
