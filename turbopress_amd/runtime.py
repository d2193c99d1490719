"""Packed-TCQ linear layer on MI355X: the drop-in for turbopress/runtime.py.

``PackedTCQLinear(payload, mode, tile_rows)`` accepts the reference's
format-v2 payload (runtime.py:171-186) and keeps its public surface
(runtime.py:211-362): ``in_features``, ``out_features``, ``bits``,
``n_states``, ``block``, ``mode``, ``levels_packed``, ``_w_cache``,
``decode_rows``, ``forward`` and ``packed_bytes``.

Modes (runtime.py:67):
  * ``"hip"``    -- weights stay packed at the true k bits/weight; every
                    forward runs the HIP rotation + decode-GEMV kernels.
                    ``"triton"`` is accepted as an alias so scripts written for
                    the reference keep working; no Triton code exists here.
  * ``"cached"`` -- load-time decompression: decode + fold the rotation back
                    into fp16 weights with HIP kernels, then a library GEMM.
  * ``"tiled"``  -- packed streams resident; each forward decodes 1024-row
                    tiles with the HIP decode kernel and multiplies them.

Every mode computes on the GPU.  A payload on the CPU is moved to the current
ROCm device at construction; a CPU activation raises RuntimeError -- there is
no CPU fallback.
"""

from __future__ import annotations

from typing import Any

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from turbopress_amd import hip_kernel as hk

__all__ = ["PackedTCQLinear", "MODES", "Trellis", "trellis_generators", "pack_linear", "pack_model"]

MODES = ("hip", "triton", "cached", "tiled")

_GENERATORS = {4: (0o5, 0o7), 8: (0o15, 0o17), 16: (0o23, 0o35), 64: (0o133, 0o171)}


def trellis_generators(n_states: int) -> tuple[int, int]:
    """(g0, g1) of the S-state bitshift trellis (trellis.py:47-52); artifacts
    record them so a loader can refuse an incompatible trellis."""
    if n_states not in _GENERATORS:
        raise ValueError(f"n_states must be one of {sorted(_GENERATORS)}, got {n_states}")
    return _GENERATORS[n_states]


class Trellis:
    """Shift-register trellis tables (trellis.py:55-87), derived from the C
    library's window LUT: subset_table[s, b] = LUT[rev_m(s) | b << m]."""

    def __init__(self, n_states: int) -> None:
        if n_states not in _GENERATORS:
            raise ValueError(f"n_states must be one of {sorted(_GENERATORS)}, got {n_states}")
        self.n_states = n_states
        m = n_states.bit_length() - 1
        lut = hk.subset_lut(n_states).long()
        sub = torch.empty(n_states, 2, dtype=torch.int64)
        for s in range(n_states):
            rev = sum(((s >> k) & 1) << (m - 1 - k) for k in range(m))
            for b in (0, 1):
                sub[s, b] = lut[rev | (b << m)]
        self.subset_table = sub
        ns = torch.arange(n_states)
        self.prev0 = ns >> 1
        self.prev1 = (ns >> 1) | (n_states >> 1)
        bit = ns & 1
        self.sub0 = sub[self.prev0, bit]
        self.sub1 = sub[self.prev1, bit]


def _target_device(payload: dict) -> torch.device:
    p = payload["path_packed"]
    if isinstance(p, Tensor) and p.is_cuda:
        return p.device
    if not torch.cuda.is_available():
        raise RuntimeError("turbopress_amd.PackedTCQLinear needs a ROCm GPU (no CPU path)")
    return torch.device("cuda", torch.cuda.current_device())


class PackedTCQLinear(nn.Module):
    """Linear layer that runs from packed trellis-coded weights on MI355X."""

    def __init__(self, payload: dict[str, Any], mode: str = "cached", tile_rows: int = 1024) -> None:
        super().__init__()
        if payload.get("format") != 2:
            raise ValueError("expected a format-v2 payload from pack_linear()")
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
        if not hk.HAS_HIP:
            raise RuntimeError("turbopress_amd needs libturbopress_amd.so and a ROCm GPU")
        self.out_features: int = int(payload["n"])
        self.in_features: int = int(payload["d"])
        self.bits: int = int(payload["bits"])
        self.n_states: int = int(payload["n_states"])
        self.block: int = int(payload["block"])
        # The mode string is kept as given (runtime.py:231): the reference's
        # scripts check ``module.mode == "triton"`` (bench_packed.py:286-293).
        # "triton" and "hip" select the same packed HIP path.
        self.mode = mode
        self._packed_path = mode in ("hip", "triton")
        self.tile_rows = tile_rows
        self._trellis = Trellis(self.n_states)
        dev = _target_device(payload)

        def buf(name, dtype=None):
            v = payload.get(name)
            if v is None:
                return None
            v = v if isinstance(v, Tensor) else torch.as_tensor(v)
            v = v.to(device=dev, dtype=dtype) if dtype is not None else v.to(dev)
            return v.contiguous()

        self.register_buffer("path_packed", buf("path_packed", torch.uint8))
        self.register_buffer("member_packed", buf("member_packed", torch.uint8))
        self.register_buffer("scales", buf("scales", torch.float16))
        self.register_buffer("signs_packed", buf("signs_packed", torch.uint8))
        self.register_buffer("inv_equil", buf("inv_equil", torch.float16))
        self.register_buffer("codebook", buf("codebook", torch.float16))
        self.register_buffer("bias", buf("bias", torch.float16))
        self.register_buffer("lut", hk.subset_lut(self.n_states).to(dev))
        self._check_shapes()
        # Host-side codebook fingerprint: grouped launches compare it without
        # touching the device (legal while a graph is being captured).
        self.codebook_key = tuple(self.codebook.cpu().view(torch.int16).tolist())
        # Fused activation-side scale (runtime.py:243-249): fp16((2s-1)*inv_equil),
        # formed on the GPU from the packed sign bits.
        d = self.in_features
        sp = self.signs_packed.reshape(-1)
        bits01 = ((sp[:, None] >> torch.arange(8, device=dev, dtype=torch.uint8)) & 1).reshape(-1)[:d]
        self.register_buffer(
            "rot_scale", ((bits01.float() * 2 - 1) * self.inv_equil.float()).to(torch.float16))
        self.register_buffer("_w_cache", None)
        self.register_buffer("levels_packed", None)

        self.register_buffer("tiled_packed", None)
        self._tiled_geo = None
        self._ws_bytes = (0, 0)  # split-K workspace need at batch <= 16 / <= 32
        self._group = None       # SharedInputGroup this layer belongs to (decode_step)
        self._group_index = 0
        if self._packed_path:
            if self.bits in hk.TILED_BITS:
                # Load-time re-tile into the MFMA kernel's layout, still at the
                # true k bits/weight (the reference re-packs (k+1)-bit levels
                # here, runtime.py:253-277); the natural streams are freed.
                self._tiled_geo = hk.tiled_layout(self.out_features, d, self.bits)
                self.tiled_packed = hk.retile(self.path_packed, self.member_packed,
                                              self.out_features, d, self.bits)
                # The split-K workspace (batch 5..32 and some larger shapes)
                # is not the layer's own: one zeroed buffer per device and
                # stream is shared by every packed linear (hip_kernel.
                # shared_workspace), where the reference allocates its fp32
                # output per call (triton_kernel.py:141).
                self._ws_bytes = hk.workspace_bytes(self.out_features)
                for name in ("path_packed", "member_packed"):
                    setattr(self, name, None)
                self.levels_packed = self.tiled_packed
            else:
                # Other rates run the general kernels on the natural streams.
                self.levels_packed = self.path_packed
        elif self.mode == "cached":
            w_rot = self.decode_rows(0, self.out_features)
            w = torch.empty_like(w_rot)
            hk._lib.check(hk._lib.lib().tp_block_fwht_rows(
                w_rot.data_ptr(), 0, self.rot_scale.data_ptr(), w.data_ptr(),
                self.out_features, d, self.block, hk.current_stream_ptr(dev)), "cached fold")
            self._w_cache = w
            for name in ("path_packed", "member_packed", "signs_packed", "lut"):
                setattr(self, name, None)

    def _check_shapes(self) -> None:
        n, d, k = self.out_features, self.in_features, self.bits
        if not 1 <= k <= 7:
            raise ValueError(f"bits must be in [1, 7], got {k}")
        if self.block < 1 or d % self.block or self.block & (self.block - 1):
            raise ValueError(f"block {self.block} is not a power of 2 dividing d={d}")
        if tuple(self.path_packed.shape) != (n, (d + 7) // 8):
            raise ValueError(f"path_packed shape {tuple(self.path_packed.shape)} != {(n, (d + 7) // 8)}")
        if k > 1:
            want = (n, (d * (k - 1) + 7) // 8)
            if self.member_packed is None or tuple(self.member_packed.shape) != want:
                raise ValueError(f"member_packed must have shape {want}")
        if self.scales.numel() != n or self.inv_equil.numel() != d:
            raise ValueError("scales/inv_equil sizes do not match (n, d)")
        if self.codebook.numel() != 1 << (k + 1):
            raise ValueError(f"codebook must have {1 << (k + 1)} entries")

    # -- decode -----------------------------------------------------------
    def decode_rows(self, r0: int, r1: int) -> Tensor:
        """Decode rows [r0, r1) of the rotated weight matrix to fp16 (GPU)."""
        if self.tiled_packed is not None:
            return hk.decode_tiled(self)[max(0, r0):min(self.out_features, r1)].contiguous()
        return hk.decode_rows(self, r0, r1)

    # -- forward ----------------------------------------------------------
    def forward(self, x: Tensor) -> Tensor:
        if x.shape[-1] != self.in_features:
            raise ValueError(f"expected last dim {self.in_features}, got {x.shape[-1]}")
        if not x.is_cuda:
            raise RuntimeError("PackedTCQLinear runs on a ROCm GPU; move the input to CUDA")
        if self._group is not None:
            return self._group.run(self._group_index, x)
        if self.mode == "cached":
            y = F.linear(x.to(torch.float16), self._w_cache)
            if self.bias is not None:
                y = y + self.bias
            return y.to(x.dtype)
        if self.tiled_packed is not None:
            return hk.forward_tiled(self, x).to(x.dtype)
        z = hk.fwht_scale(x, self.rot_scale, self.block)
        if self._packed_path:
            y = hk.packed_gemv(z, self, bias=self.bias)
        else:  # tiled
            flat = z.reshape(-1, self.in_features)
            y = torch.empty(flat.shape[0], self.out_features, dtype=torch.float16, device=z.device)
            for r0 in range(0, self.out_features, self.tile_rows):
                r1 = min(r0 + self.tile_rows, self.out_features)
                y[:, r0:r1] = flat @ self.decode_rows(r0, r1).T
            y = y.reshape(*z.shape[:-1], self.out_features)
            if self.bias is not None:
                y = y + self.bias
        return y.to(x.dtype)

    def _apply(self, fn, recurse=True):
        """Device moves apply; dtype casts of the whole model (``.half()``,
        ``.to(dtype=...)``) leave the packed buffers in the fp16/uint8 storage
        the kernels read."""
        dtypes = {name: b.dtype for name, b in self._buffers.items() if b is not None}
        super()._apply(fn, recurse)
        for name, dt in dtypes.items():
            b = self._buffers.get(name)
            if b is not None and b.dtype != dt:
                self._buffers[name] = b.to(dt)
        return self

    # -- accounting ---------------------------------------------------------
    def packed_bytes(self) -> int:
        """Resident weight bytes under the current mode (runtime.py:337-356)."""
        if self._w_cache is not None:
            total = self._w_cache.numel() * self._w_cache.element_size()
        elif self.tiled_packed is not None:
            total = self.tiled_packed.numel() + self.signs_packed.numel()
            total += 2 * (self.inv_equil.numel() + self.rot_scale.numel())
        else:
            total = self.path_packed.numel() + self.signs_packed.numel()
            if self.member_packed is not None:
                total += self.member_packed.numel()
            total += 2 * (self.inv_equil.numel() + self.rot_scale.numel())
        total += 2 * (self.scales.numel() + self.codebook.numel())
        if self.bias is not None:
            total += 2 * self.bias.numel()
        return total

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bits={self.bits}, n_states={self.n_states}, mode={self.mode!r}, "
                f"resident={self.packed_bytes() / 2**20:.1f} MiB "
                f"(fp16 {2 * self.in_features * self.out_features / 2**20:.1f} MiB)")


# The reference's runtime module also holds the compress-time entry points
# (runtime.py:143-186, 368-411); they live in turbopress_amd.pack.
from turbopress_amd.pack import pack_linear, pack_model  # noqa: E402
