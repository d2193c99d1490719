"""Compress time: an ``nn.Linear`` into the format-v2 payload that
``PackedTCQLinear`` reads, and the whole-model swap.

``pack_linear`` follows ``turbopress/runtime.py:143-186``: quarter-power
equilibration of the input channels against activation RMS (the factors
rounded to their stored fp16 precision before use), a seeded randomized
Hadamard rotation (``hadamard.py:59-108``: Rademacher signs from
``torch.Generator().manual_seed(seed)``, then the orthonormal block
Walsh-Hadamard transform over the largest power-of-2 block), TCQ of every
row (``encoder.tcq_quantize_rows``: the row statistics with the reference's
torch CPU ops, the Viterbi searches on the GPU, ``tp_tcq_viterbi``), and
LSB-first packing of the path bits and member codes (``runtime.py:73-86``).
Given the same inputs the payload equals the reference's bit for bit.

``pack_model`` follows ``runtime.py:368-411``: every ``nn.Linear`` of every
decoder block becomes a ``PackedTCQLinear``, with the reference's per-linear
seed ``seed + 7919 * block + crc32(name) % 1000``.
"""

from __future__ import annotations

import math
import zlib
from typing import Any

import numpy as np
import torch
from torch import Tensor, nn

__all__ = ["pack_rows_le", "equilibration", "rademacher_signs", "block_hadamard_rows", "pack_linear",
           "pack_model"]


def pack_rows_le(vals: Tensor, width: int) -> Tensor:
    """uint8 values < 2^width [n, d] -> uint8 [n, ceil(d * width / 8)]: bit
    j of element c at stream position c * width + j, stream bit i in byte
    i >> 3, bit i & 7, every row starting on a byte (runtime.py:73-86)."""
    if vals.ndim != 2 or vals.dtype != torch.uint8:
        raise ValueError("expected a 2D uint8 tensor")
    if not 1 <= width <= 8:
        raise ValueError(f"width must be in [1, 8], got {width}")
    a = vals.detach().cpu().numpy()
    n, d = a.shape
    bits = ((a[:, :, None] >> np.arange(width, dtype=np.uint8)) & 1).reshape(n, d * width)
    return torch.from_numpy(np.packbits(bits, axis=1, bitorder="little"))


def equilibration(w: Tensor, act_rms: Tensor) -> Tensor:
    """Per-input-channel factor s (fp32 holding fp16 values) of the
    quarter-power equilibration w * s, from the weight's column norms and
    the activation RMS, both clamped at 5 % of their RMS (runtime.py:157-162)."""
    act = act_rms.to(torch.float32).cpu().clamp_min(1e-8)
    act = act.clamp_min(0.05 * float(act.pow(2).mean().sqrt()))
    cn = w.norm(dim=0)
    cn = cn.clamp_min(max(0.05 * float(cn.pow(2).mean().sqrt()), 1e-12))
    return (act / cn).sqrt().to(torch.float16).float()


def rademacher_signs(dim: int, seed: int) -> Tensor:
    """0/1 int64 [dim]: the seeded sign draw of the rotation (hadamard.py:76-78)."""
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(0, 2, (dim,), generator=gen, dtype=torch.int64)


def block_hadamard_rows(x: Tensor, block: int) -> Tensor:
    """Orthonormal Walsh-Hadamard transform of every `block`-column block of
    the rows of x (fp32): butterflies at distance 1, 2, 4, ..., block / 2,
    then one division by sqrt(block) -- the reference's stage order and
    rounding (hadamard.py:37-56, 100-106)."""
    n, d = x.shape
    if block < 1 or block & (block - 1) or d % block:
        raise ValueError(f"block must be a power of 2 dividing {d}, got {block}")
    y = x.reshape(-1, block)
    h = 1
    while h < block:
        pairs = y.reshape(-1, block // (2 * h), 2, h)
        lo, hi = pairs[:, :, 0, :], pairs[:, :, 1, :]
        y = torch.stack((lo + hi, lo - hi), dim=2).reshape(-1, block)
        h *= 2
    return (y / math.sqrt(block)).reshape(n, d)


@torch.no_grad()
def pack_linear(linear: nn.Linear, act_rms: Tensor, bits: int, n_states: int = 64,
                seed: int = 0) -> dict[str, Any]:
    """TurboPress-quantize ``linear`` and return its format-v2 payload
    (runtime.py:143-186); tensors on the CPU, as the reference returns them.

    ``in_features`` must have a power-of-2 factor: the packed format's
    rotation is a block Walsh-Hadamard transform (the reference falls back to
    a dense orthogonal matrix for odd sizes, which its packed forward does not
    apply)."""
    from turbopress_amd.encoder import tcq_quantize_rows
    w = linear.weight.detach().to(torch.float32).cpu()
    n, d = w.shape
    block = d & -d
    if block == 1 and d > 1:
        raise ValueError(f"in_features={d} has no power-of-2 factor: the packed rotation needs one")
    if not 1 <= bits <= 4:
        raise ValueError(f"bits must be in [1, 4] for the GPU encoder, got {bits}")
    s = equilibration(w, act_rms)
    signs01 = rademacher_signs(d, seed)
    signs = (signs01 * 2 - 1).to(torch.float32)
    w_rot = block_hadamard_rows((w * s[None, :]) * signs, block)
    q = tcq_quantize_rows(w_rot, bits=bits, n_states=n_states)
    return {
        "format": 2,
        "n": n,
        "d": d,
        "bits": bits,
        "n_states": n_states,
        "block": block,
        "path_packed": pack_rows_le(q.path_bits, 1),
        "member_packed": pack_rows_le(q.member_codes, bits - 1) if bits > 1 else None,
        "scales": q.scales.to(torch.float16),
        "signs_packed": pack_rows_le(signs01.to(torch.uint8)[None, :], 1),
        "inv_equil": (1.0 / s).to(torch.float16),
        "codebook": q.codebook.to(torch.float16),
        "bias": None if linear.bias is None else linear.bias.detach().to(torch.float16).cpu(),
        "seed": seed,
    }


@torch.no_grad()
def pack_model(model: nn.Module, stats: dict[str, Tensor], bits: int, n_states: int = 64,
               mode: str = "cached", seed: int = 0, log=None) -> dict[str, Any]:
    """Replace every ``nn.Linear`` of every decoder block of ``model`` with a
    ``PackedTCQLinear`` in place (runtime.py:368-411).  ``stats`` maps
    ``"{block}.{name}"`` to the per-channel activation RMS of that linear's
    input.  Returns the byte accounting."""
    from turbopress_amd.artifact import decoder_layers
    from turbopress_amd.runtime import PackedTCQLinear
    layers = decoder_layers(model)
    packed_total = fp16_total = 0
    for i, block in enumerate(layers):
        replacements = []
        for name, mod in block.named_modules():
            if isinstance(mod, nn.Linear):
                payload = pack_linear(mod, stats[f"{i}.{name}"], bits=bits, n_states=n_states,
                                      seed=seed + 7919 * i + zlib.crc32(name.encode()) % 1000)
                replacements.append((name, payload, mod.weight.device))
        for name, payload, device in replacements:
            parent = block
            *parents, leaf = name.split(".")
            for p in parents:
                parent = getattr(parent, p)
            if device.type == "cuda":
                from turbopress_amd.synthetic import payload_to
                payload = payload_to(payload, device)
            qlin = PackedTCQLinear(payload, mode=mode)
            setattr(parent, leaf, qlin.to(device))
            packed_total += qlin.packed_bytes()
            fp16_total += 2 * qlin.in_features * qlin.out_features
        if log is not None:
            log.info(f"packed block {i + 1}/{len(layers)}")
    return {"packed_bytes": packed_total, "fp16_bytes": fp16_total,
            "compression": fp16_total / max(packed_total, 1)}
