"""Op-for-op torch-CPU restatement of the reference's ``mode="tiled"`` forward.

Test infrastructure only (see ``oracle/__init__.py``).  ``bench.py`` times it
as the CPU baseline (``cpu_baseline.kind == "port"``): the reference's own
Python cannot travel to the GPU box, so this file repeats its CPU path with
the same torch calls in the same order:

  * ``unpack_le``             runtime.py:93-100  (8 int lanes per packed byte)
  * ``window_decode_levels``  runtime.py:122-139 (m shift/OR passes + LUT gather)
  * ``decode_rows``           runtime.py:291-301 (fp16(cb.f32[level]*scale.f32))
  * ``block_fwht``            runtime.py:192-208
  * ``tiled_forward``         runtime.py:322-334 (1024-row tiles, fp32 matmul)

The numpy oracle (``tcq_oracle``) is the checker; the tests assert that this
restatement agrees with it bit-for-bit on decoded weights.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle.tcq_oracle import subset_lut as _np_subset_lut


def unpack_le(packed: torch.Tensor, d: int, width: int) -> torch.Tensor:
    n = packed.shape[0]
    shifts = torch.arange(8, dtype=torch.uint8)
    bits = (packed[:, :, None] >> shifts) & 1
    stream = bits.reshape(n, -1)[:, : d * width]
    weights = (1 << torch.arange(width, dtype=torch.int32))
    return (stream.reshape(n, d, width).to(torch.int32) * weights).sum(-1).to(torch.uint8)


def window_decode_levels(path_bits: torch.Tensor, member_codes: torch.Tensor,
                         n_states: int, lut: torch.Tensor) -> torch.Tensor:
    n, d = path_bits.shape
    m = n_states.bit_length() - 1
    padded = F.pad(path_bits.to(torch.int32), (m, 0))
    x = padded[:, m:] << m
    for j in range(m):
        x = x | (padded[:, j: j + d] << j)
    subsets = lut[x.long()]
    return (member_codes.to(torch.int32) * 4 + subsets).to(torch.uint8)


def _fwht(x: torch.Tensor) -> torch.Tensor:
    d = x.shape[-1]
    y = x.reshape(-1, d)
    h = 1
    while h < d:
        y = y.reshape(-1, d // (2 * h), 2, h)
        even, odd = y[:, :, 0, :], y[:, :, 1, :]
        y = torch.stack((even + odd, even - odd), dim=2).reshape(-1, d)
        h *= 2
    return (y / math.sqrt(d)).reshape(x.shape)


def block_fwht(x: torch.Tensor, block: int) -> torch.Tensor:
    if block == x.shape[-1]:
        return _fwht(x)
    m = x.shape[-1] // block
    return _fwht(x.reshape(*x.shape[:-1], m, block)).reshape(x.shape)


class TiledLinearCPU:
    """The CPU state ``PackedTCQLinear(payload, mode="tiled")`` holds
    (runtime.py:226-250) and its forward (runtime.py:304-334)."""

    def __init__(self, payload: dict, tile_rows: int = 1024) -> None:
        def t(v):
            return v if isinstance(v, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(v))

        self.n, self.d = int(payload["n"]), int(payload["d"])
        self.bits, self.n_states = int(payload["bits"]), int(payload["n_states"])
        self.block = int(payload["block"])
        self.tile_rows = tile_rows
        self.path_packed = t(payload["path_packed"])
        mp = payload.get("member_packed")
        self.member_packed = None if mp is None else t(mp)
        self.scales = t(payload["scales"]).to(torch.float16)
        self.codebook = t(payload["codebook"]).to(torch.float16)
        b = payload.get("bias")
        self.bias = None if b is None else t(b).to(torch.float16)
        self.lut = torch.from_numpy(_np_subset_lut(self.n_states))
        signs = unpack_le(t(payload["signs_packed"]).reshape(1, -1), self.d, 1)[0]
        self.rot_scale = ((signs.float() * 2 - 1)
                          * t(payload["inv_equil"]).to(torch.float16).float()).to(torch.float16)

    def decode_rows(self, r0: int, r1: int) -> torch.Tensor:
        pathb = unpack_le(self.path_packed[r0:r1], self.d, 1)
        if self.member_packed is not None:
            memb = unpack_le(self.member_packed[r0:r1], self.d, self.bits - 1)
        else:
            memb = torch.zeros_like(pathb)
        levels = window_decode_levels(pathb, memb, self.n_states, self.lut)
        w = self.codebook.float()[levels.long()] * self.scales[r0:r1].float()[:, None]
        return w.to(torch.float16)

    @torch.no_grad()
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.d:
            raise ValueError(f"expected last dim {self.d}, got {x.shape[-1]}")
        compute_dtype = torch.float32
        z = block_fwht(x.to(compute_dtype) * self.rot_scale.to(compute_dtype), self.block)
        flat = z.reshape(-1, self.d)
        y = torch.empty(flat.shape[0], self.n, dtype=compute_dtype)
        for r0 in range(0, self.n, self.tile_rows):
            r1 = min(r0 + self.tile_rows, self.n)
            y[:, r0:r1] = flat @ self.decode_rows(r0, r1).to(compute_dtype).T
        y = y.reshape(*z.shape[:-1], self.n)
        if self.bias is not None:
            y = y + self.bias.to(y.dtype)
        return y.to(x.dtype)

    __call__ = forward
