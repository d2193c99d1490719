"""HIP kernels vs the CPU oracle on the same seeded inputs (GPU).

Bars (from the north-star specification):
  * decoded levels and decoded fp16 weights: bit-exact with the reference
    decode (runtime.py:122-139, 291-301);
  * rotation: the fp32 transform matches the oracle's fp32 transform, so the
    fp16 result is compared bit-for-bit against fp16(oracle);
  * GEMV / forward: max-rel = max|y - y_ref| / max|y_ref| <= 2e-3 against
    the fp32/fp64-accumulated oracle (fp16 output).
"""

import zlib

import numpy as np
import pytest
import torch

from oracle import tcq_oracle as O
from turbopress_amd.synthetic import (
    QWEN3_0_6B_LAYER, make_activation, make_payload, payload_numpy, payload_to)

pytestmark = pytest.mark.gpu

GEMV_TOL = 2e-3


def _stream():
    return torch.cuda.current_stream().cuda_stream


# ------------------------------------------------------------------ rotation
ROT_CASES = [(576, 64), (1536, 512), (1024, 1024), (3072, 1024), (128, 128),
             (2560, 512), (4096, 4096), (9728, 512), (2048, 2048), (96, 32), (8, 8)]


@pytest.mark.parametrize("d,block", ROT_CASES)
@pytest.mark.parametrize("batch", [1, 5])
def test_fwht_scale_matches_oracle(cuda, d, block, batch):
    from turbopress_amd.hip_kernel import fwht_scale
    gen = torch.Generator().manual_seed(7 + d + batch)
    rs = ((torch.randn(d, generator=gen).sign()) * (torch.rand(d, generator=gen) + 0.5)).to(torch.float16)
    x = (torch.randn(batch, d, generator=gen) * 3).to(torch.float16)
    got = fwht_scale(x.to(cuda), rs.to(cuda), block).cpu().numpy()
    ref32 = O.block_fwht(x.numpy().astype(np.float32) * rs.numpy().astype(np.float32), block)
    ref16 = ref32.astype(np.float16)
    assert got.shape == (batch, d)
    assert np.array_equal(got.view(np.uint16), ref16.view(np.uint16))


def test_fwht_scale_rejects_bad_block(cuda):
    from turbopress_amd.hip_kernel import fwht_scale
    x = torch.zeros(1, 96, dtype=torch.float16, device=cuda)
    with pytest.raises(ValueError):
        fwht_scale(x, torch.ones(96, dtype=torch.float16, device=cuda), 64)


# -------------------------------------------------------------------- decode
DECODE_CASES = [(n, d, k, s) for s in (4, 8, 16, 64) for (n, d, k) in
                ((5, 77, 1), (9, 96, 2), (7, 102, 3), (3, 130, 4), (4, 64, 5), (2, 40, 7))]


@pytest.mark.parametrize("n,d,bits,n_states", DECODE_CASES)
def test_window_decode_levels_bit_exact(cuda, n, d, bits, n_states):
    from turbopress_amd.hip_kernel import window_decode_levels
    p = make_payload(n, d, bits, n_states, seed=n * d + bits)
    got = window_decode_levels(p["path_packed"].to(cuda),
                               None if p["member_packed"] is None else p["member_packed"].to(cuda),
                               d, bits, n_states).cpu().numpy()
    assert np.array_equal(got, O.levels_of(payload_numpy(p)))


@pytest.mark.parametrize("n,d,bits,n_states", [(33, 576, 2, 64), (17, 1024, 3, 64),
                                               (11, 2560, 4, 64), (9, 200, 3, 16)])
def test_decode_rows_bit_exact(cuda, n, d, bits, n_states):
    from turbopress_amd.runtime import PackedTCQLinear
    p = make_payload(n, d, bits, n_states, seed=3)
    lin = PackedTCQLinear(p, mode="hip")
    pn = payload_numpy(p)
    for r0, r1 in ((0, n), (3, 8), (n - 1, n)):
        got = lin.decode_rows(r0, r1).cpu().numpy()
        ref = O.decode_rows(pn, r0, r1)
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), (r0, r1)


# ---------------------------------------------------------------------- GEMV
GEMV_CASES = [
    # (n, d, bits, n_states, batch)
    (1536, 576, 2, 64, 1),      # config 0: SmolLM2-135M up-proj
    (192, 256, 3, 64, 2),       # tests/test_runtime.py:164-174 shape
    (200, 96, 2, 8, 4),
    (130, 200, 4, 16, 3),
    (64, 128, 1, 4, 1),
    (96, 320, 5, 64, 9),
]


@pytest.mark.parametrize("n,d,bits,n_states,batch", GEMV_CASES)
def test_packed_gemv_matches_fp64_oracle(cuda, n, d, bits, n_states, batch):
    from turbopress_amd.hip_kernel import packed_gemv
    from turbopress_amd.runtime import PackedTCQLinear
    p = make_payload(n, d, bits, n_states, seed=n + d)
    lin = PackedTCQLinear(p, mode="hip")
    z = (torch.randn(batch, d, generator=torch.Generator().manual_seed(1))).to(torch.float16)
    y = packed_gemv(z.to(cuda), lin).float().cpu().numpy()
    ref = O.gemv_fp64(payload_numpy(p), z.numpy().astype(np.float64))
    assert O.max_rel(y, ref) <= GEMV_TOL


@pytest.mark.parametrize("mode", ["hip", "triton", "tiled", "cached"])
@pytest.mark.parametrize("n,d,bits", [(1536, 576, 2), (256, 1024, 3), (72, 640, 4)])
def test_forward_modes_match_tiled_oracle(cuda, mode, n, d, bits):
    from turbopress_amd.runtime import PackedTCQLinear
    p = make_payload(n, d, bits, 64, seed=11, bias=True)
    lin = PackedTCQLinear(p, mode=mode, tile_rows=100)
    x = make_activation(2, d, seed=5)
    y = lin(x.to(cuda)).float().cpu().numpy()
    ref = O.tiled_forward(payload_numpy(p), x.numpy())
    assert y.shape == (2, n)
    assert O.max_rel(y, ref) <= GEMV_TOL, mode


@pytest.mark.parametrize("name", sorted(QWEN3_0_6B_LAYER))
def test_qwen3_0_6b_layer_linears(cuda, name):
    """Config 1: every Qwen3-0.6B projection at k=3, batch 1."""
    from turbopress_amd.runtime import PackedTCQLinear
    d, n = QWEN3_0_6B_LAYER[name]
    p = make_payload(n, d, 3, 64, seed=zlib.crc32(name.encode()) % 1000)
    lin = PackedTCQLinear(p, mode="hip")
    x = make_activation(1, d, seed=1)
    y = lin(x.to(cuda)).float().cpu().numpy()
    assert O.max_rel(y, O.tiled_forward(payload_numpy(p), x.numpy())) <= GEMV_TOL


def test_forward_errors_match_reference(cuda):
    from turbopress_amd.runtime import PackedTCQLinear
    p = make_payload(64, 128, 2, 8)
    lin = PackedTCQLinear(p, mode="hip")
    with pytest.raises(ValueError):
        lin(torch.randn(2, 64, device=cuda, dtype=torch.float16))
    with pytest.raises(RuntimeError):
        lin(torch.randn(2, 128, dtype=torch.float16))  # CPU input: no CPU path
    with pytest.raises(ValueError):
        PackedTCQLinear(p, mode="warp")
    with pytest.raises(ValueError):
        PackedTCQLinear({"format": 1})


@pytest.mark.parametrize("n,d,bits", [(9728, 2560, 3), (2560, 9728, 2), (100, 300, 4)])
def test_packed_bytes_exact(cuda, n, d, bits):
    """packed_bytes follows the reference's accounting (runtime.py:337-356)
    with the device layout in place of the (k+1)-bit level stream: exactly
    k bits per weight of the padded 16-row x 256-column tiles, plus the fp16
    side tensors; cached mode counts the fp16 weights."""
    from turbopress_amd.runtime import PackedTCQLinear
    p = make_payload(n, d, bits, 64, seed=5, bias=True)
    n_pad, d_pad = -(-n // 16) * 16, -(-d // 256) * 256
    side = 2 * (n + (1 << (bits + 1))) + 2 * n  # scales, codebook, bias
    signs = (d + 7) // 8
    hip = PackedTCQLinear(p, mode="hip")
    assert hip.tiled_packed.numel() == n_pad * d_pad * bits // 8
    assert hip.packed_bytes() == n_pad * d_pad * bits // 8 + signs + 2 * (2 * d) + side
    tiled = PackedTCQLinear(p, mode="tiled")
    natural = n * ((d + 7) // 8) + n * ((d * (bits - 1) + 7) // 8)
    assert tiled.packed_bytes() == natural + signs + 2 * (2 * d) + side
    if n * d <= 1 << 20:
        cached = PackedTCQLinear(p, mode="cached")
        assert cached.packed_bytes() == 2 * n * d + side


def test_packed_bytes_and_attributes(cuda):
    from turbopress_amd.runtime import PackedTCQLinear
    p = make_payload(256, 256, 2, 8)
    hip = PackedTCQLinear(p, mode="hip")
    cached = PackedTCQLinear(p, mode="cached")
    assert hip.levels_packed is not None and hip._w_cache is None
    assert cached.path_packed is None and cached._w_cache is not None
    assert hip.packed_bytes() < 2 * 256 * 256 / 6
    assert cached.packed_bytes() >= 2 * 256 * 256


@pytest.mark.gpu
def test_read_probe_runs_and_checks_arguments(cuda):
    """The streaming-read probe reads a buffer without writing it (its sink
    stays zero for an all-zero buffer) and rejects sizes that are not whole
    16-byte words."""
    from turbopress_amd import _lib
    lib = _lib.lib()
    buf = torch.zeros(1 << 20, dtype=torch.int32, device=cuda)
    sink = torch.zeros(1, dtype=torch.int32, device=cuda)
    stream = torch.cuda.current_stream(cuda).cuda_stream
    assert lib.tp_read_probe(buf.data_ptr(), buf.numel() * 4, sink.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
    assert lib.tp_read_probe(buf.data_ptr(), 20, sink.data_ptr(), stream) != 0
