"""numpy restatement of the reference packed-TCQ decode path (TEST ORACLE).

Test infrastructure only: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s CPU-baseline leg, never by the ``turbopress_amd`` package.

Every function cites the reference lines it restates (paths relative to the
reference checkout).  Integer work is exact; floating-point work follows the
reference's precision choices (fp32 compute, fp16 storage) so that decoded
weights can be compared bit-for-bit.

Pinning (what checks each function beyond retyping the formula):
  * ``subset_table`` / ``subset_lut``: brute force against the sequential
    shift-register walk (``decode_levels_sequential``) over every window,
    structural invariants of ``tests/test_trellis.py:10-21`` and
    ``tests/test_runtime.py:45-49``, and a hand-worked S=4 table.
  * ``pack_le`` / ``unpack_le``: round trip (``tests/test_runtime.py:18-25``)
    plus hand-packed known answers.
  * ``window_decode_levels``: equality with the sequential walk on random
    and exhaustive inputs (``tests/test_runtime.py:28-42``) and on the output
    of the Viterbi encoder in ``codebook_oracle``.
  * ``fwht`` / ``block_fwht``: dense Sylvester matrix, involution, isometry
    (``tests/test_hadamard.py:18-58``).
  * ``decode_rows`` / ``tiled_forward``: fp64 dense product on the decoded
    weights and the golden vectors written by ``tests/golden/make_golden.py``.
  * ``unpack_bits_v1``: round trip with ``numpy.packbits`` and a hand vector.
"""

from __future__ import annotations

import math

import numpy as np

# Best-known rate-1/2 convolutional generators (octal), trellis.py:47-52.
GENERATORS: dict[int, tuple[int, int]] = {
    4: (0o5, 0o7),
    8: (0o15, 0o17),
    16: (0o23, 0o35),
    64: (0o133, 0o171),
}
N_SUBSETS = 4  # trellis.py:43


def log2_states(n_states: int) -> int:
    if n_states not in GENERATORS:
        raise ValueError(f"n_states must be one of {sorted(GENERATORS)}, got {n_states}")
    return n_states.bit_length() - 1


# ---------------------------------------------------------------------------
# bit layout, format v2 (runtime.py:73-100)
# ---------------------------------------------------------------------------
def pack_le(vals: np.ndarray, width: int) -> np.ndarray:
    """runtime.py:73-90: bit j of element c -> stream bit c*width+j, LSB-first
    within each byte, each row padded to whole bytes."""
    vals = np.asarray(vals)
    if vals.ndim != 2 or vals.dtype != np.uint8:
        raise ValueError("expected a 2D uint8 array")
    if not 1 <= width <= 8:
        raise ValueError(f"width must be in [1, 8], got {width}")
    n, d = vals.shape
    bits = (vals[:, :, None] >> np.arange(width, dtype=np.uint8)) & 1
    stream = bits.reshape(n, d * width)
    pad = (-stream.shape[1]) % 8
    if pad:
        stream = np.pad(stream, ((0, 0), (0, pad)))
    return np.packbits(stream.reshape(n, -1, 8), axis=-1, bitorder="little").reshape(n, -1)


def unpack_le(packed: np.ndarray, d: int, width: int) -> np.ndarray:
    """runtime.py:93-100: inverse of ``pack_le`` -> uint8 [n, d]."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    n = packed.shape[0]
    bits = np.unpackbits(packed, axis=1, bitorder="little")[:, : d * width]
    bits = bits.reshape(n, d, width).astype(np.uint32)
    weights = (1 << np.arange(width, dtype=np.uint32))
    return (bits * weights).sum(-1).astype(np.uint8)


def unpack_bits_v1(buf: np.ndarray, count: int, width: int) -> np.ndarray:
    """pipeline.py:114-117 (format v1): numpy ``packbits`` order, i.e. MSB-first
    within each byte, one flat stream over the whole matrix; value bit j of
    element i sits at stream position i*width + j."""
    bits = np.unpackbits(np.asarray(buf, dtype=np.uint8))[: count * width].reshape(count, width)
    return (bits.astype(np.uint32) << np.arange(width, dtype=np.uint32)).sum(axis=1).astype(np.uint8)


# ---------------------------------------------------------------------------
# trellis tables (trellis.py:55-87) and the window LUT (runtime.py:106-119)
# ---------------------------------------------------------------------------
def _parity(x: int) -> int:
    return bin(x).count("1") & 1


def subset_table(n_states: int) -> np.ndarray:
    """trellis.py:64-80: subset[s, b] = (par(x & g1) << 1) | par(x & g0),
    x = (b << m) | s."""
    m = log2_states(n_states)
    g0, g1 = GENERATORS[n_states]
    out = np.empty((n_states, 2), dtype=np.int64)
    for s in range(n_states):
        for b in (0, 1):
            x = (b << m) | s
            out[s, b] = (_parity(x & g1) << 1) | _parity(x & g0)
    return out


def subset_lut(n_states: int) -> np.ndarray:
    """runtime.py:106-119: LUT over the natural (m+1)-bit stream window.

    Window bit j holds path bit b[t-m+j]; the state is the bit-reverse of the
    low m bits and the current bit is bit m.
    """
    m = log2_states(n_states)
    xs = np.arange(1 << (m + 1))
    b_cur = (xs >> m) & 1
    state = np.zeros_like(xs)
    for k in range(m):
        state |= ((xs >> (m - 1 - k)) & 1) << k
    return subset_table(n_states)[state, b_cur].astype(np.uint8)


def window_decode_levels(path_bits: np.ndarray, member_codes: np.ndarray,
                         n_states: int) -> np.ndarray:
    """runtime.py:122-139: level[t] = member[t]*4 + LUT[window(t)], the window
    zero-padded before each row start (the encoder starts in state 0)."""
    path_bits = np.asarray(path_bits, dtype=np.uint8)
    n, d = path_bits.shape
    m = log2_states(n_states)
    lut = subset_lut(n_states)
    padded = np.pad(path_bits.astype(np.int64), ((0, 0), (m, 0)))
    x = padded[:, m:] << m
    for j in range(m):
        x = x | (padded[:, j: j + d] << j)
    subsets = lut[x]
    return (np.asarray(member_codes, dtype=np.int64) * N_SUBSETS + subsets).astype(np.uint8)


def decode_levels_sequential(path_bits: np.ndarray, member_codes: np.ndarray,
                             n_states: int) -> np.ndarray:
    """trellis.py:182-199: the sequential shift-register walk from state 0."""
    path_bits = np.asarray(path_bits, dtype=np.int64)
    member_codes = np.asarray(member_codes, dtype=np.int64)
    n, d = path_bits.shape
    table = subset_table(n_states)
    mask = n_states - 1
    out = np.empty((n, d), dtype=np.uint8)
    state = np.zeros(n, dtype=np.int64)
    for t in range(d):
        b = path_bits[:, t]
        sub = table[state, b]
        out[:, t] = (member_codes[:, t] * N_SUBSETS + sub).astype(np.uint8)
        state = ((state << 1) | b) & mask
    return out


# ---------------------------------------------------------------------------
# rotation: orthonormal Sylvester FWHT per block (hadamard.py:30-56,
# runtime.py:192-208) and the fused activation scale (runtime.py:243-249)
# ---------------------------------------------------------------------------
def largest_pow2_divisor(n: int) -> int:
    """hadamard.py:30-34."""
    if n < 1:
        raise ValueError(f"n must be >= 1, got {n}")
    return n & (-n)


def fwht(x: np.ndarray) -> np.ndarray:
    """hadamard.py:37-56 / runtime.py:192-201: natural-order butterflies
    (pairs at distance h = 1, 2, 4, ...), then one division by sqrt(d).
    Computes in the input's float dtype."""
    x = np.asarray(x)
    d = x.shape[-1]
    if d & (d - 1):
        raise ValueError(f"fwht requires a power-of-2 last dimension, got {d}")
    y = x.reshape(-1, d)
    h = 1
    while h < d:
        y = y.reshape(-1, d // (2 * h), 2, h)
        even, odd = y[:, :, 0, :], y[:, :, 1, :]
        y = np.stack((even + odd, even - odd), axis=2).reshape(-1, d)
        h *= 2
    return (y / y.dtype.type(math.sqrt(d))).reshape(x.shape)


def block_fwht(x: np.ndarray, block: int) -> np.ndarray:
    """runtime.py:204-208: independent FWHT of every contiguous ``block``."""
    x = np.asarray(x)
    if block == x.shape[-1]:
        return fwht(x)
    m = x.shape[-1] // block
    return fwht(x.reshape(*x.shape[:-1], m, block)).reshape(x.shape)


def rot_scale(signs_packed: np.ndarray, inv_equil_f16: np.ndarray, d: int) -> np.ndarray:
    """runtime.py:245-249: fp16((2*sign-1) * f32(inv_equil))."""
    signs = unpack_le(np.asarray(signs_packed).reshape(1, -1), d, 1)[0]
    return ((signs.astype(np.float32) * 2 - 1)
            * np.asarray(inv_equil_f16, dtype=np.float16).astype(np.float32)).astype(np.float16)


# ---------------------------------------------------------------------------
# decode and forward (runtime.py:291-334)
# ---------------------------------------------------------------------------
def levels_of(payload: dict, r0: int = 0, r1: int | None = None) -> np.ndarray:
    """Unpack + window-decode rows [r0, r1) of a format-v2 payload
    (runtime.py:293-299)."""
    d = int(payload["d"])
    bits = int(payload["bits"])
    r1 = int(payload["n"]) if r1 is None else r1
    pathb = unpack_le(payload["path_packed"][r0:r1], d, 1)
    if payload.get("member_packed") is not None:
        memb = unpack_le(payload["member_packed"][r0:r1], d, bits - 1)
    else:
        memb = np.zeros_like(pathb)
    return window_decode_levels(pathb, memb, int(payload["n_states"]))


def decode_rows(payload: dict, r0: int = 0, r1: int | None = None) -> np.ndarray:
    """runtime.py:291-301: fp16(codebook.f32[level] * scale.f32) for rows
    [r0, r1).  Both operands are fp16 values, so the fp32 product is exact
    and the single fp16 rounding is the only rounding."""
    r1 = int(payload["n"]) if r1 is None else r1
    levels = levels_of(payload, r0, r1)
    cb = np.asarray(payload["codebook"], dtype=np.float16).astype(np.float32)
    sc = np.asarray(payload["scales"], dtype=np.float16)[r0:r1].astype(np.float32)
    return (cb[levels.astype(np.int64)] * sc[:, None]).astype(np.float16)


def payload_rot_scale(payload: dict) -> np.ndarray:
    return rot_scale(payload["signs_packed"], payload["inv_equil"], int(payload["d"]))


def rotate_activations(payload: dict, x: np.ndarray) -> np.ndarray:
    """runtime.py:323-324 (CPU branch): z = blockFWHT(x.f32 * rot_scale.f32)."""
    rs = payload_rot_scale(payload).astype(np.float32)
    return block_fwht(np.asarray(x, dtype=np.float32) * rs, int(payload["block"]))


def tiled_forward(payload: dict, x: np.ndarray, tile_rows: int = 1024) -> np.ndarray:
    """runtime.py:322-334, the CPU ``mode="tiled"`` forward: fp32 rotation,
    per-tile fp16 decode, fp32 matmul, fp16 bias added in fp32, returned fp32."""
    x = np.asarray(x)
    d, n = int(payload["d"]), int(payload["n"])
    if x.shape[-1] != d:
        raise ValueError(f"expected last dim {d}, got {x.shape[-1]}")
    z = rotate_activations(payload, x)
    flat = z.reshape(-1, d)
    y = np.empty((flat.shape[0], n), dtype=np.float32)
    for r0 in range(0, n, tile_rows):
        r1 = min(r0 + tile_rows, n)
        y[:, r0:r1] = flat @ decode_rows(payload, r0, r1).astype(np.float32).T
    y = y.reshape(*z.shape[:-1], n)
    if payload.get("bias") is not None:
        y = y + np.asarray(payload["bias"], dtype=np.float16).astype(np.float32)
    return y


def gemv_fp64(payload: dict, z: np.ndarray) -> np.ndarray:
    """fp64 product of rotated activations with the decoded codebook values:
    y[b, r] = scale[r] * sum_c cb[level[r, c]] * z[b, c] (the quantity the
    reference's fused GEMV accumulates, triton_kernel.py:70-73, 123)."""
    levels = levels_of(payload)
    cb = np.asarray(payload["codebook"], dtype=np.float16).astype(np.float64)
    sc = np.asarray(payload["scales"], dtype=np.float16).astype(np.float64)
    w = cb[levels.astype(np.int64)]
    return (np.asarray(z, dtype=np.float64).reshape(-1, w.shape[1]) @ w.T) * sc[None, :]


def algorithmic_bytes(n: int, d: int, bits: int, batch: int) -> int:
    """Bytes one packed linear must move: k-bit codes + fp16 scales,
    codebook, rot_scale, x in and y out."""
    return n * d * bits // 8 + 2 * n + 2 * (1 << (bits + 1)) + 2 * d + 2 * batch * d + 2 * batch * n


def max_rel(got: np.ndarray, ref: np.ndarray) -> float:
    """Max-scaled relative error: max|got - ref| / max|ref|."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))
