"""TCQ encoder on MI355X (compress time): the Viterbi search of
``turbopress/trellis.py:111-179`` (and ``pipeline.py:209-276``'s copy) and
the per-row quantizer around it (``trellis.py:256-320``).

``viterbi`` returns exactly what the reference's ``_viterbi`` returns --
``(level_codes, path_bits, member_codes, end_state)`` -- computed by
``tp_tcq_viterbi`` (one wave per row, one lane per trellis state; see
``csrc/tp_viterbi.hip``) with the reference's fp32 arithmetic and
tie-breaking, so the codes are identical.  Rows are processed in chunks so
the branch-decision workspace (8 bytes per weight) stays bounded.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from turbopress_amd import _lib
from turbopress_amd import hip_kernel as hk

__all__ = ["viterbi", "TCQQuantized", "tcq_quantize_rows"]

_WORKSPACE_BUDGET = 1 << 30  # bytes of branch decisions per launch


def viterbi(z: Tensor, codebook: Tensor, n_states: int, start_state: Tensor | None = None):
    """Minimum-distortion trellis path of every row of ``z`` (fp32 [n, d] on
    the GPU) against the doubled ``codebook``; rows start in ``start_state``
    (default state 0).  Returns uint8 level codes, path bits and member codes
    [n, d] and int64 end states [n]."""
    if z.ndim != 2:
        raise ValueError(f"expected z of shape [n, d], got {tuple(z.shape)}")
    if not z.is_cuda:
        raise RuntimeError("viterbi runs on a ROCm GPU; move z to CUDA")
    n, d = z.shape
    levels = codebook.numel()
    bits = levels.bit_length() - 2
    if levels != 1 << (bits + 1) or not 1 <= bits <= 4:
        raise ValueError(f"codebook must have 2^(bits+1) entries for bits in 1..4, got {levels}")
    dev = z.device
    z32 = z.to(torch.float32).contiguous()
    cb = codebook.to(device=dev, dtype=torch.float32).contiguous()
    level = torch.empty(n, d, dtype=torch.uint8, device=dev)
    path = torch.empty_like(level)
    member = torch.empty_like(level)
    end = torch.empty(n, dtype=torch.int32, device=dev)
    start = None if start_state is None else start_state.to(device=dev, dtype=torch.int32).contiguous()
    lib = _lib.lib()
    chunk = max(1, min(n, _WORKSPACE_BUDGET // max(1, d * 8)))
    ws = torch.empty(int(lib.tp_viterbi_workspace_bytes(chunk, d)), dtype=torch.uint8, device=dev)
    stream = hk.current_stream_ptr(dev)
    for r0 in range(0, n, chunk):
        r1 = min(n, r0 + chunk)
        st = lib.tp_tcq_viterbi(
            z32[r0].data_ptr(), z32.stride(0), r1 - r0, d, cb.data_ptr(), bits, n_states,
            None if start is None else start[r0].data_ptr(),
            level[r0].data_ptr(), path[r0].data_ptr(), member[r0].data_ptr(), end[r0].data_ptr(),
            ws.data_ptr(), ws.numel(), stream)
        _lib.check(st, "tcq_viterbi")
    return level, path, member, end.to(torch.int64)


@dataclass
class TCQQuantized:
    """TCQ-coded rows (trellis.py:93-108): ``w ~= scales[:, None] *
    codebook[level_codes]``; ``path_bits`` + ``member_codes`` are the
    ``bits``-bit stored stream."""

    level_codes: Tensor
    path_bits: Tensor
    member_codes: Tensor
    scales: Tensor
    codebook: Tensor
    bits: int
    n_states: int

    def dequantize(self) -> Tensor:
        return self.scales[:, None] * self.codebook[self.level_codes.long()]


def tcq_quantize_rows(w: Tensor, bits: int, n_states: int = 8, scale_iters: int = 1,
                      codebook: Tensor | None = None) -> TCQQuantized:
    """TCQ-quantize each row of ``w`` [n_rows, dim] at ``bits`` bits/weight
    (trellis.py:256-320): per-row RMS scale, Viterbi on w/scale, then
    ``scale_iters`` least-squares scale refits each followed by a new search.
    Zero rows get scale 0.  ``codebook`` (fp32 [2^(bits+1)]) defaults to the
    trellis-optimised codebook for (bits, n_states), the reference's default
    (``codebook_mode="optimized"``).

    The row statistics and refits run on ``w``'s device with the reference's
    torch ops (so a CPU ``w``, as ``pack_linear`` passes, gives the
    reference's scales bit for bit); only the Viterbi searches run on the
    GPU (``tp_tcq_viterbi``).  The results are on ``w``'s device."""
    if w.ndim != 2:
        raise ValueError(f"expected a 2D tensor [n_rows, dim], got shape {tuple(w.shape)}")
    if not torch.is_floating_point(w):
        raise TypeError(f"expected a floating-point tensor, got {w.dtype}")
    if not 1 <= bits <= 4:
        raise ValueError(f"tcq bits must be in [1, 4] on the GPU encoder, got {bits}")
    if scale_iters < 0:
        raise ValueError(f"scale_iters must be >= 0, got {scale_iters}")
    if codebook is None:
        from turbopress_amd.codebooks import available_codebooks, optimized_codebook_f32
        if (bits, n_states) not in available_codebooks():
            raise ValueError(f"no stored codebook for bits={bits}, n_states={n_states}: pass one")
        codebook = optimized_codebook_f32(bits, n_states)
    gpu = w.device if w.is_cuda else torch.device("cuda", torch.cuda.current_device())
    w32 = w.to(torch.float32)
    cb = codebook.to(device=w32.device, dtype=torch.float32)
    cb_gpu = cb.to(gpu)

    def search(z: Tensor):
        level, path, member, _ = viterbi(z.to(gpu), cb_gpu, n_states)
        return level.to(w32.device), path.to(w32.device), member.to(w32.device)

    scales = w32.pow(2).mean(dim=1).sqrt()
    nonzero = scales > 0
    safe = torch.where(nonzero, scales, torch.ones_like(scales))
    level, path, member = search(w32 / safe[:, None])
    for _ in range(scale_iters):
        q = cb[level.long()]
        num = (w32 * q).sum(dim=1)
        den = (q * q).sum(dim=1)
        new_scale = torch.where(den > 0, num / den.clamp_min(1e-30), safe)
        safe = torch.where(new_scale > 0, new_scale, safe)
        level, path, member = search(w32 / safe[:, None])
    scales = torch.where(nonzero, safe, torch.zeros_like(safe))
    return TCQQuantized(level, path, member, scales, cb, bits, n_states)
