"""Pin the CPU oracle before trusting it (CPU only).

Each check is chosen so that a plausible mistake in the oracle (a dropped
generator tap, a reversed window, a wrong byte order, a transposed operand,
a missing normalisation) fails it, independently of how the oracle states
the formula:
  * closed forms (hand-worked LUT, Lloyd-Max 1/2-bit values, dense Sylvester);
  * brute force (sequential shift-register walk over every window);
  * the reference's own invariants (tests/test_trellis.py:10-21,
    tests/test_runtime.py:18-49, tests/test_hadamard.py:18-58);
  * golden vectors imported from the reference (tests/golden/*.json).
"""

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import tcq_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- bit layout
@pytest.mark.parametrize("width", [1, 2, 3, 5, 8])
def test_pack_le_roundtrip(width):
    rng = np.random.default_rng(0)
    vals = rng.integers(0, 1 << width, (5, 77), dtype=np.uint8)
    packed = O.pack_le(vals, width)
    assert packed.shape == (5, -(-77 * width // 8))
    assert np.array_equal(O.unpack_le(packed, 77, width), vals)


def test_pack_le_known_answer():
    # width 3, values 5 (101b) then 6 (110b): stream bits LSB-first are
    # 1,0,1, 0,1,1 -> byte 0b00110101 = 0x35.
    assert O.pack_le(np.array([[5, 6]], dtype=np.uint8), 3).tolist() == [[0x35]]
    # width 1: column c at bit c, row padded to a byte.
    bits = np.array([[1, 0, 0, 0, 0, 0, 0, 1, 1]], dtype=np.uint8)
    assert O.pack_le(bits, 1).tolist() == [[0x81, 0x01]]


def test_unpack_bits_v1_is_msb_first_flat():
    # pipeline.py:106-117: numpy packbits (MSB-first), flat over the matrix.
    vals = np.array([1, 2, 3, 0, 1], dtype=np.uint8)  # width 2
    bits = ((vals[:, None] >> np.arange(2, dtype=np.uint8)) & 1).reshape(-1)
    buf = np.packbits(bits)
    assert np.array_equal(O.unpack_bits_v1(buf, 5, 2), vals)
    # value bits 1,0 | 0,1 | 1,1 | 0,0 -> 0b10011100 = 0x9C, then 0b10 << 6
    assert buf.tolist() == [0x9C, 0x80]


# ------------------------------------------------------------ trellis tables
def test_subset_table_s4_hand_worked():
    # S=4, (g0, g1) = (5, 7), m = 2, x = (b << 2) | s.
    # s=0,b=0: x=0 -> 0;  s=0,b=1: x=4 -> par(4&7)=1, par(4&5)=1 -> 3
    # s=1,b=0: x=1 -> par(1)=1, par(1)=1 -> 3;  s=1,b=1: x=5 -> par(5)=0, par(5)=0 -> 0
    # s=2,b=0: x=2 -> par(2&7)=1, par(2&5)=0 -> 2; s=2,b=1: x=6 -> par(6)=0, par(4)=1 -> 1
    # s=3,b=0: x=3 -> par(3)=0, par(1)=1 -> 1;  s=3,b=1: x=7 -> par(7)=1, par(5)=0 -> 2
    assert O.subset_table(4).tolist() == [[0, 3], [3, 0], [2, 1], [1, 2]]


@pytest.mark.parametrize("n_states", [4, 8, 16, 64])
def test_trellis_structure(n_states):
    t = O.subset_table(n_states)
    assert set(t.flatten().tolist()) == {0, 1, 2, 3}
    assert np.all(t[:, 0] != t[:, 1])


def test_subset_lut_size_and_range():
    lut = O.subset_lut(64)
    assert lut.shape == (128,)
    assert set(np.unique(lut).tolist()) == {0, 1, 2, 3}


@pytest.mark.parametrize("n_states", [4, 8, 16, 64])
def test_lut_matches_sequential_walk_on_every_window(n_states):
    """Brute force: for every (m+1)-bit window, run the shift register from
    state 0 over the window bits (oldest first) and read the last subset."""
    m = O.log2_states(n_states)
    lut = O.subset_lut(n_states)
    table = O.subset_table(n_states)
    for x in range(1 << (m + 1)):
        bits = [(x >> j) & 1 for j in range(m + 1)]  # b[t-m], ..., b[t]
        state = 0
        for b in bits[:-1]:
            state = ((state << 1) | b) & (n_states - 1)
        assert lut[x] == table[state, bits[-1]], (n_states, x)


@pytest.mark.parametrize("n_states", [4, 8, 16, 64])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_window_decode_equals_sequential_walk(n_states, bits):
    rng = np.random.default_rng(n_states * 10 + bits)
    path = rng.integers(0, 2, (7, 101), dtype=np.uint8)
    memb = rng.integers(0, 1 << (bits - 1), (7, 101), dtype=np.uint8)
    a = O.window_decode_levels(path, memb, n_states)
    b = O.decode_levels_sequential(path, memb, n_states)
    assert np.array_equal(a, b)
    assert a.max() < 1 << (bits + 1)


def test_window_decode_exhaustive_short_rows():
    # Every 9-bit path on S=16 (window spans the row start).
    paths = ((np.arange(512)[:, None] >> np.arange(9)) & 1).astype(np.uint8)
    memb = np.zeros_like(paths)
    assert np.array_equal(O.window_decode_levels(paths, memb, 16),
                          O.decode_levels_sequential(paths, memb, 16))


@pytest.mark.parametrize("n_states,bits", [(8, 2), (16, 3), (64, 3)])
def test_window_decode_on_viterbi_output(n_states, bits):
    """tests/test_runtime.py:28-42: decode of real encoder output reproduces
    the encoder's own level codes."""
    from oracle.codebook_oracle import lloyd_max_gaussian, viterbi
    gen = torch.Generator().manual_seed(0)
    w = torch.randn(6, 96, generator=gen)
    cb = lloyd_max_gaussian(bits + 1)[0].to(torch.float32)
    level, path, memb = viterbi(w, cb, n_states)
    assert np.array_equal(O.window_decode_levels(path.numpy(), memb.numpy(), n_states), level.numpy())


def test_viterbi_is_min_distortion_on_tiny_rows():
    """Brute force over all 2^d paths x best member per position (d=6, S=4)."""
    from oracle.codebook_oracle import lloyd_max_gaussian, viterbi
    n_states, d = 4, 6
    cb = lloyd_max_gaussian(3)[0].to(torch.float32)
    gen = torch.Generator().manual_seed(3)
    z = torch.randn(3, d, generator=gen)
    level, _, _ = viterbi(z, cb, n_states)
    got = ((cb[level.long()] - z) ** 2).sum(1)
    table = O.subset_table(n_states)
    for r in range(3):
        best = math.inf
        for p in range(1 << d):
            state, cost = 0, 0.0
            for t in range(d):
                b = (p >> t) & 1
                sub = table[state, b]
                cost += float(((cb[sub::4] - z[r, t]) ** 2).min())
                state = ((state << 1) | b) & (n_states - 1)
            best = min(best, cost)
        assert abs(float(got[r]) - best) < 1e-5


# ------------------------------------------------------------------ rotation
def test_fwht_matches_dense_sylvester():
    d = 16
    h = np.array([[1.0]])
    while h.shape[0] < d:
        h = np.block([[h, h], [h, -h]])
    h /= math.sqrt(d)
    x = np.random.default_rng(0).standard_normal((5, d))
    assert np.allclose(O.fwht(x), x @ h.T, atol=1e-12)
    # entry (i, j) = (-1)^popcount(i & j) / sqrt(d)
    i, j = 5, 11
    assert h[i, j] == (-1) ** bin(i & j).count("1") / math.sqrt(d)


def test_fwht_is_orthonormal_involution():
    x = np.random.default_rng(1).standard_normal((3, 4, 64))
    y = O.fwht(x)
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1))
    assert np.allclose(O.fwht(y), x)


def test_block_fwht_is_blockwise():
    x = np.random.default_rng(2).standard_normal((2, 96))
    y = O.block_fwht(x, 32)
    for b in range(3):
        assert np.allclose(y[:, 32 * b: 32 * (b + 1)], O.fwht(x[:, 32 * b: 32 * (b + 1)]))
    assert O.largest_pow2_divisor(576) == 64 and O.largest_pow2_divisor(9728) == 512


def test_rotation_preserves_matmul():
    # (W R^T)(R x) = W x with R = H diag(signs) (tests/test_hadamard.py:59-67).
    rng = np.random.default_rng(3)
    d = 96
    signs = rng.integers(0, 2, d) * 2 - 1
    w = rng.standard_normal((8, d))
    x = rng.standard_normal((4, d))
    rot = lambda v: O.block_fwht(v * signs, 32)  # noqa: E731
    assert np.allclose(rot(x) @ rot(w).T, x @ w.T)


# ------------------------------------------------------------------ codebooks
def test_lloyd_max_closed_forms():
    from oracle.codebook_oracle import lloyd_max_gaussian
    lv, mse = lloyd_max_gaussian(1)
    assert np.allclose(lv.numpy(), [-math.sqrt(2 / math.pi), math.sqrt(2 / math.pi)])
    assert abs(mse - (1 - 2 / math.pi)) < 1e-10
    lv2, mse2 = lloyd_max_gaussian(2)
    assert abs(float(lv2[2]) - 0.4528) < 2e-3 and abs(float(lv2[3]) - 1.510) < 2e-3
    assert abs(mse2 - 0.1175) < 1e-3
    lv4, _ = lloyd_max_gaussian(4)
    assert torch.allclose(lv4, -lv4.flip(0), atol=1e-8) and bool((lv4[1:] > lv4[:-1]).all())


def _golden_codebooks():
    return json.loads((GOLDEN / "codebooks.json").read_text())


def test_package_codebook_table_matches_reference_golden():
    from turbopress_amd.codebooks import default_codebook
    g = _golden_codebooks()["trellis"]
    for key, v in g.items():
        bits, s = (int(t) for t in key.split(","))
        cb = default_codebook(bits, s)
        assert cb.view(torch.int16).to(torch.int32).bitwise_and(0xFFFF).tolist() == v["f16"], key
        # subsets stay sorted (trellis.py:249-250)
        f = cb.float()
        for j in range(4):
            assert bool((f[j::4][1:] >= f[j::4][:-1]).all())


@pytest.mark.slow
@pytest.mark.parametrize("bits,n_states", [(2, 64), (3, 16)])
def test_codebook_restatement_matches_reference_golden(bits, n_states):
    from oracle.codebook_oracle import tcq_optimized_codebook
    g = _golden_codebooks()["trellis"][f"{bits},{n_states}"]
    cb = tcq_optimized_codebook(bits, n_states)
    assert [float(v).hex() for v in cb.tolist()] == g["f32"]


@pytest.mark.slow
def test_pipeline_codebook_restatement_matches_reference_golden():
    from oracle.codebook_oracle import pipeline_tcq_codebook
    g = _golden_codebooks()["pipeline"]["3,16"]
    cb = pipeline_tcq_codebook(3, 16)
    assert [float(v).hex() for v in cb.tolist()] == g["f32"]


def test_rademacher_signs_match_reference_golden():
    from oracle.codebook_oracle import rademacher_signs
    g = json.loads((GOLDEN / "signs.json").read_text())["cases"]
    for key, hexbytes in g.items():
        d, seed = (int(t) for t in key.split(","))
        s01 = rademacher_signs(d, seed).numpy().astype(np.uint8)
        assert np.packbits(s01, bitorder="little").tobytes().hex() == hexbytes, key


# ---------------------------------------------------------- decode & forward
def _payload(n=40, d=96, bits=3, n_states=16, seed=0, bias=True):
    from turbopress_amd.synthetic import make_payload, payload_numpy
    return payload_numpy(make_payload(n, d, bits, n_states, seed=seed, bias=bias))


def test_decode_rows_is_codebook_times_scale():
    p = _payload()
    w = O.decode_rows(p)
    lv = O.decode_levels_sequential(O.unpack_le(p["path_packed"], 96, 1),
                                    O.unpack_le(p["member_packed"], 96, 2), 16)
    ref = (p["codebook"].astype(np.float32)[lv] * p["scales"].astype(np.float32)[:, None]).astype(np.float16)
    assert np.array_equal(w.view(np.uint16), ref.view(np.uint16))


def test_tiled_forward_matches_fp64_dense():
    p = _payload(n=64, d=128, bits=2, n_states=8)
    x = np.random.default_rng(4).standard_normal((3, 128)).astype(np.float16)
    y = O.tiled_forward(p, x, tile_rows=24)
    # independent: dense weights in the original basis, W = W' R D^-1 per row
    w_rot = O.decode_rows(p).astype(np.float64)
    signs = O.unpack_le(p["signs_packed"], 128, 1)[0].astype(np.float64) * 2 - 1
    w = O.block_fwht(w_rot, int(p["block"])) * signs * p["inv_equil"].astype(np.float64)
    ref = x.astype(np.float64) @ w.T + p["bias"].astype(np.float64)
    assert O.max_rel(y, ref) < 1e-3


@pytest.mark.parametrize("bits,n_states,batch", [(2, 8, 1), (3, 64, 3), (4, 16, 2)])
def test_gemv_fp64_matches_independent_dense_product(bits, n_states, batch):
    """gemv_fp64 (window decode, row scale factored out of the sum) against
    an independent statement: levels from the sequential shift-register walk
    (trellis.py:182-199), dense weights cb[level] * scale in fp64, then a
    plain row-by-row dot product.  A transposed operand, a dropped scale or a
    reversed window fails it."""
    p = _payload(n=24, d=80, bits=bits, n_states=n_states, seed=7, bias=False)
    z = np.random.default_rng(bits).standard_normal((batch, 80))
    got = O.gemv_fp64(p, z)
    lv = O.decode_levels_sequential(O.unpack_le(p["path_packed"], 80, 1),
                                    O.unpack_le(p["member_packed"], 80, bits - 1), n_states)
    cb = p["codebook"].astype(np.float64)
    sc = p["scales"].astype(np.float64)
    ref = np.empty((batch, 24))
    for b in range(batch):
        for r in range(24):
            ref[b, r] = sum(cb[lv[r, c]] * sc[r] * z[b, c] for c in range(80))
    assert got.shape == (batch, 24)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_torch_tiled_baseline_agrees_with_numpy_oracle():
    from oracle.tiled_baseline import TiledLinearCPU
    from turbopress_amd.synthetic import make_payload, payload_numpy
    pt = make_payload(50, 192, 3, 64, seed=2, bias=True)
    pn = payload_numpy(pt)
    lin = TiledLinearCPU(pt, tile_rows=16)
    w_t = lin.decode_rows(0, 50).numpy()
    assert np.array_equal(w_t.view(np.uint16), O.decode_rows(pn).view(np.uint16))
    x = torch.randn(2, 192)
    assert O.max_rel(lin(x).numpy(), O.tiled_forward(pn, x.numpy())) < 1e-5


def test_algorithmic_bytes_qwen3_4b_mlp():
    # 9728 x 2560 at k=3, B=1: 9.388 MB
    assert abs(O.algorithmic_bytes(9728, 2560, 3, 1) / 1e6 - 9.388) < 1e-3
