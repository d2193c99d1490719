"""Torch-facing wrappers of the HIP kernels (the reference's triton_kernel.py API).

``HAS_HIP``, ``fwht_scale(x, rot_scale, block)`` and ``packed_gemv(z, layer)``
keep the names, arguments and error behaviour of
turbopress/triton_kernel.py:19-27, 132-157, 235-260.  Each call launches
hand-written HIP kernels from libturbopress_amd.so on torch's current stream;
nothing here computes on the CPU, and nothing synchronises the host, so the
calls can be captured in a HIP graph.
"""

from __future__ import annotations

import torch
from torch import Tensor

from turbopress_amd import _lib

__all__ = ["HAS_HIP", "fwht_scale", "packed_gemv", "decode_rows", "window_decode_levels",
           "subset_lut", "current_stream_ptr", "tiled_layout", "retile", "TILED_BITS"]

# bits per weight served by the device-layout MFMA kernels
TILED_BITS = (2, 3, 4)


def _has_hip() -> bool:
    try:
        return _lib.available() and torch.cuda.is_available()
    except Exception:  # pragma: no cover - defensive: a broken ROCm install
        return False


HAS_HIP: bool = _has_hip()


def current_stream_ptr(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(t: Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA (ROCm) tensor; turbopress_amd has no CPU path")


def subset_lut(n_states: int) -> Tensor:
    """uint8 [2*S] window -> subset LUT (runtime.py:106-119), from the C library."""
    import ctypes
    size = 2 * n_states
    buf = (ctypes.c_uint8 * max(size, 1))()
    _lib.check(_lib.lib().tp_subset_lut(n_states, buf, size), "subset_lut")
    return torch.tensor(list(buf), dtype=torch.uint8)


def fwht_scale(x: Tensor, rot_scale: Tensor, block: int) -> Tensor:
    """``blockFWHT(x * rot_scale)`` in one HIP launch (triton_kernel.py:235-260).

    fp32 butterflies, fp16 result; x may be any float dtype (cast to fp16 as the
    reference does, triton_kernel.py:244)."""
    _require_cuda(x, "x")
    d = x.shape[-1]
    flat = x.reshape(-1, d).to(torch.float16).contiguous()
    rs = rot_scale.to(device=x.device, dtype=torch.float16).contiguous()
    if rs.numel() != d:
        raise ValueError(f"rot_scale has {rs.numel()} entries, expected {d}")
    out = torch.empty_like(flat)
    st = _lib.lib().tp_fwht_scale(flat.data_ptr(), rs.data_ptr(), out.data_ptr(),
                                  flat.shape[0], d, int(block), current_stream_ptr(x.device))
    _lib.check(st, "fwht_scale")
    return out.reshape(x.shape)


def window_decode_levels(path_packed: Tensor, member_packed: Tensor | None, d: int,
                         bits: int, n_states: int) -> Tensor:
    """uint8 level codes [n, d] straight from the packed v2 streams
    (runtime.py:122-139 after unpack_le, runtime.py:93-100)."""
    _require_cuda(path_packed, "path_packed")
    path = path_packed.contiguous()
    n = path.shape[0]
    mem = None if member_packed is None else member_packed.contiguous()
    out = torch.empty(n, d, dtype=torch.uint8, device=path.device)
    st = _lib.lib().tp_window_decode_levels(
        path.data_ptr(), path.shape[1], 0 if mem is None else mem.data_ptr(),
        0 if mem is None else mem.shape[1], n, d, bits, n_states, out.data_ptr(), d,
        current_stream_ptr(path.device))
    _lib.check(st, "window_decode_levels")
    return out


def decode_rows(layer, r0: int, r1: int) -> Tensor:
    """fp16 rotated weight rows [r0, r1) of a packed layer (runtime.py:291-301)."""
    path = layer.path_packed
    if path is None:
        raise RuntimeError("layer no longer holds its packed streams")
    _require_cuda(path, "path_packed")
    d = layer.in_features
    r0, r1 = max(0, r0), min(layer.out_features, r1)
    out = torch.empty(max(r1 - r0, 0), d, dtype=torch.float16, device=path.device)
    if r1 <= r0:
        return out
    mem = layer.member_packed
    ps = path.stride(0)
    ms = 0 if mem is None else mem.stride(0)
    st = _lib.lib().tp_decode_rows(
        path.data_ptr() + r0 * ps, ps,
        0 if mem is None else mem.data_ptr() + r0 * ms, ms,
        layer.scales.data_ptr() + 2 * r0, layer.codebook.data_ptr(),
        r1 - r0, d, layer.bits, layer.n_states, out.data_ptr(), d,
        current_stream_ptr(path.device))
    _lib.check(st, "decode_rows")
    return out


def packed_gemv(z: Tensor, layer, bias: Tensor | None = None) -> Tensor:
    """y = z @ W_packed^T (+ bias) for a packed layer (triton_kernel.py:132-157).

    ``layer`` is duck-typed: ``in_features``, ``out_features``, ``bits``,
    ``n_states``, ``scales``, ``codebook`` and the packed streams
    ``path_packed``/``member_packed``.  Returns fp16 [..., n]."""
    _require_cuda(z, "z")
    n, d = layer.out_features, layer.in_features
    flat = z.reshape(-1, d).to(torch.float16).contiguous()
    out = torch.empty(flat.shape[0], n, dtype=torch.float16, device=z.device)
    if getattr(layer, "tiled_packed", None) is not None:
        ldz = layer._tiled_geo["z_cols"]
        zpad = flat if ldz == d else torch.nn.functional.pad(flat, (0, ldz - d))
        gemv_tiled(zpad, layer, bias, out)
        return out.reshape(*z.shape[:-1], n)
    if getattr(layer, "path_packed", None) is None:
        raise RuntimeError("layer was not built with mode='hip'")
    path, mem = layer.path_packed, layer.member_packed
    st = _lib.lib().tp_tcq_gemv(
        flat.data_ptr(), flat.shape[0], path.data_ptr(), path.stride(0),
        0 if mem is None else mem.data_ptr(), 0 if mem is None else mem.stride(0),
        layer.scales.data_ptr(), layer.codebook.data_ptr(),
        0 if bias is None else bias.data_ptr(),
        n, d, layer.bits, layer.n_states, out.data_ptr(), current_stream_ptr(z.device))
    _lib.check(st, "packed_gemv")
    return out.reshape(*z.shape[:-1], n)


# ---------------------------------------------------------------------------
# bandwidth path: device layout + MFMA decode-GEMV
# ---------------------------------------------------------------------------
def tiled_layout(n: int, d: int, bits: int) -> dict:
    """Geometry of the device layout (tp_tiled_layout)."""
    import ctypes
    vals = [ctypes.c_int64() for _ in range(5)]
    _lib.check(_lib.lib().tp_tiled_layout(n, d, bits, *[ctypes.byref(v) for v in vals]), "tiled_layout")
    keys = ("tiles", "segments", "path_bytes", "member_bytes", "z_cols")
    return dict(zip(keys, (v.value for v in vals)))


def retile(path_packed: Tensor, member_packed: Tensor, n: int, d: int, bits: int) -> Tensor:
    """One uint8 device buffer [path words | member words] in the kernel's
    layout (replaces the load-time stream build of runtime.py:253-277)."""
    _require_cuda(path_packed, "path_packed")
    geo = tiled_layout(n, d, bits)
    pb, mb = geo["path_bytes"], geo["member_bytes"]
    buf = torch.empty(pb + mb, dtype=torch.uint8, device=path_packed.device)
    path, mem = path_packed.contiguous(), member_packed.contiguous()
    st = _lib.lib().tp_retile(path.data_ptr(), path.stride(0), mem.data_ptr(), mem.stride(0),
                              n, d, bits, buf.data_ptr(), buf.data_ptr() + pb,
                              current_stream_ptr(path.device))
    _lib.check(st, "retile")
    return buf


def gemv_workspace(n: int, batch: int, device) -> Tensor:
    """A zeroed split-K workspace of its own for an n-row linear at `batch`
    rows (tp_gemv_workspace_bytes)."""
    nbytes = int(_lib.lib().tp_gemv_workspace_bytes(n, batch))
    return torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=device)


def workspace_bytes(n: int) -> tuple:
    """Split-K workspace bytes of an n-row linear at batch <= 16 and <= 32."""
    lib = _lib.lib()
    return int(lib.tp_gemv_workspace_bytes(n, 16)), int(lib.tp_gemv_workspace_bytes(n, 32))


# One split-K workspace per (device, stream), shared by every packed linear
# launched on that stream.  The kernels leave it zero when they finish, so
# launches in stream order can share it; launches that overlap on one
# workspace (two streams would need two) are not allowed, hence one per
# stream.  A workspace that grows is replaced, and the old one stays alive:
# a captured graph may still name it.
_WORKSPACES: dict = {}
_RETIRED_WORKSPACES: list = []
_WS_ALIGN = 256


def _aligned(nbytes: int) -> int:
    return (nbytes + _WS_ALIGN - 1) // _WS_ALIGN * _WS_ALIGN


def shared_workspace(device, nbytes: int) -> Tensor:
    """The zeroed split-K workspace of `device` and its current stream, at
    least `nbytes` long (allocated or grown on first need)."""
    dev = torch.device(device)
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (index, torch.cuda.current_stream(index).cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _RETIRED_WORKSPACES.append(ws)
        ws = torch.zeros(max(_aligned(nbytes), _WS_ALIGN), dtype=torch.uint8,
                         device=torch.device("cuda", index))
        _WORKSPACES[key] = ws
    return ws


def layer_workspace(layer, batch: int) -> tuple:
    """(pointer, bytes) of the shared workspace for one launch of `layer` at
    `batch` rows (<= 32)."""
    need = layer._ws_bytes[0 if batch <= 16 else 1]
    ws = shared_workspace(layer.tiled_packed.device, need)
    return ws.data_ptr(), need


def group_workspaces(layers, batch: int) -> tuple:
    """Disjoint regions of the shared workspace for the linears of one group
    launch (they run concurrently): lists of pointers and sizes."""
    needs = [lyr._ws_bytes[0 if batch <= 16 else 1] for lyr in layers]
    offs, total = [], 0
    for need in needs:
        offs.append(total)
        total += _aligned(need)
    ws = shared_workspace(layers[0].tiled_packed.device, total)
    base = ws.data_ptr()
    return [base + o for o in offs], needs


def decode_tiled(layer) -> Tensor:
    """fp16 rotated weights [n, d] decoded through the tiled GEMV's decode path."""
    n, d = layer.out_features, layer.in_features
    buf = layer.tiled_packed
    out = torch.empty(n, d, dtype=torch.float16, device=buf.device)
    st = _lib.lib().tp_decode_tiled(buf.data_ptr(), buf.data_ptr() + layer._tiled_geo["path_bytes"],
                                    layer.scales.data_ptr(), layer.codebook.data_ptr(), n, d,
                                    layer.bits, layer.n_states, out.data_ptr(), d,
                                    current_stream_ptr(buf.device))
    _lib.check(st, "decode_tiled")
    return out


def rotate_padded(x: Tensor, rot_scale: Tensor, block: int, ldz: int) -> Tensor:
    """fp16 z [B, ldz] = blockFWHT(x * rot_scale) with zero columns [d, ldz)."""
    _require_cuda(x, "x")
    d = x.shape[-1]
    flat = x.reshape(-1, d).to(torch.float16).contiguous()
    z = torch.empty(flat.shape[0], ldz, dtype=torch.float16, device=x.device)
    st = _lib.lib().tp_fwht_scale_padded(flat.data_ptr(), rot_scale.data_ptr(), z.data_ptr(),
                                         flat.shape[0], d, int(block), ldz,
                                         current_stream_ptr(x.device))
    _lib.check(st, "fwht_scale_padded")
    return z


def gemv_tiled(zpad: Tensor, layer, bias: Tensor | None, out: Tensor) -> Tensor:
    """out[B, n] = packed GEMV over the device layout; zpad fp16 [B, ldz]."""
    n, d = layer.out_features, layer.in_features
    buf = layer.tiled_packed
    pb = layer._tiled_geo["path_bytes"]
    ldz = zpad.shape[1]
    stream = current_stream_ptr(zpad.device)
    lib = _lib.lib()
    for b0 in range(0, zpad.shape[0], 32):
        nb = min(32, zpad.shape[0] - b0)
        ws, ws_bytes = layer_workspace(layer, nb)
        st = lib.tp_tcq_gemv_tiled(
            zpad.data_ptr() + 2 * b0 * ldz, ldz, nb, buf.data_ptr(), buf.data_ptr() + pb,
            layer.scales.data_ptr(), layer.codebook.data_ptr(),
            0 if bias is None else bias.data_ptr(), n, d, layer.bits, layer.n_states,
            out.data_ptr() + 2 * b0 * n, n, ws, ws_bytes, stream)
        _lib.check(st, "tcq_gemv_tiled")
    return out


def forward_tiled(layer, x: Tensor) -> Tensor:
    """Rotation + decode-GEMV + bias: one fused launch per 32 rows
    (tp_packed_linear_forward) when the rotation fits the launch (up to 8
    rows, or Hadamard blocks <= 512); otherwise the rows rotate once into the
    padded layout and run the batched decode-GEMV (tp_tcq_gemv_tiled) per 32
    rows.  fp16 [..., n]."""
    _require_cuda(x, "x")
    n, d = layer.out_features, layer.in_features
    flat = x.reshape(-1, d).to(torch.float16).contiguous()
    y = torch.empty(flat.shape[0], n, dtype=torch.float16, device=x.device)
    if d % 4 or (flat.shape[0] > 8 and (layer.block > 512 or d % 8)):
        # Rows not 8-byte aligned, or a batch whose Hadamard blocks span more
        # than one 512-column chunk: rotate into the padded layout, then GEMV.
        zpad = rotate_padded(flat, layer.rot_scale, layer.block, layer._tiled_geo["z_cols"])
        gemv_tiled(zpad, layer, layer.bias, y)
        return y.reshape(*x.shape[:-1], n)
    buf = layer.tiled_packed
    pb = layer._tiled_geo["path_bytes"]
    bias = layer.bias
    stream = current_stream_ptr(x.device)
    lib = _lib.lib()
    for b0 in range(0, flat.shape[0], 32):
        nb = min(32, flat.shape[0] - b0)
        ws, ws_bytes = layer_workspace(layer, nb)
        st = lib.tp_packed_linear_forward(
            flat.data_ptr() + 2 * b0 * d, d, nb, layer.rot_scale.data_ptr(), layer.block,
            buf.data_ptr(), buf.data_ptr() + pb, layer.scales.data_ptr(), layer.codebook.data_ptr(),
            0 if bias is None else bias.data_ptr(), n, d, layer.bits, layer.n_states,
            y.data_ptr() + 2 * b0 * n, n, ws, ws_bytes, stream)
        _lib.check(st, "packed_linear_forward")
    return y.reshape(*x.shape[:-1], n)


def forward_group(layers, x: Tensor) -> list:
    """One launch for up to 4 tiled layers sharing the input x and codebook
    (tp_packed_linear_forward_group); returns their fp16 outputs."""
    import ctypes
    if not 1 <= len(layers) <= 4:
        raise ValueError("forward_group takes 1 to 4 layers")
    _require_cuda(x, "x")
    l0 = layers[0]
    d = l0.in_features
    for lyr in layers:
        if lyr.tiled_packed is None or lyr.in_features != d or lyr.bits != l0.bits \
                or lyr.n_states != l0.n_states:
            raise ValueError("grouped layers need the device layout and equal in_features/bits/S")
        if lyr.codebook_key != l0.codebook_key:
            raise ValueError("grouped layers must share one codebook")
    if d % 4 or x.numel() // d > 8:
        return [forward_tiled(lyr, x) for lyr in layers]
    flat = x.reshape(-1, d).to(torch.float16).contiguous()
    k = len(layers)
    outs = [torch.empty(flat.shape[0], lyr.out_features, dtype=torch.float16, device=x.device)
            for lyr in layers]
    P = ctypes.c_void_p * k
    I = ctypes.c_int64 * k
    stream = current_stream_ptr(x.device)
    lib = _lib.lib()
    for b0 in range(0, flat.shape[0], 32):
        nb = min(32, flat.shape[0] - b0)
        ws_ptrs, ws_sizes = group_workspaces(layers, nb)
        st = lib.tp_packed_linear_forward_group(
            k, flat.data_ptr() + 2 * b0 * d, d, nb,
            P(*[lyr.rot_scale.data_ptr() for lyr in layers]), I(*[lyr.block for lyr in layers]),
            P(*[lyr.tiled_packed.data_ptr() for lyr in layers]),
            P(*[lyr.tiled_packed.data_ptr() + lyr._tiled_geo["path_bytes"] for lyr in layers]),
            P(*[lyr.scales.data_ptr() for lyr in layers]), l0.codebook.data_ptr(),
            P(*[0 if lyr.bias is None else lyr.bias.data_ptr() for lyr in layers]),
            I(*[lyr.out_features for lyr in layers]), d, l0.bits, l0.n_states,
            P(*[o.data_ptr() + 2 * b0 * o.shape[1] for o in outs]), I(*[o.shape[1] for o in outs]),
            P(*ws_ptrs), I(*ws_sizes),
            stream)
        _lib.check(st, "packed_linear_forward_group")
    return [o.reshape(*x.shape[:-1], o.shape[1]) for o in outs]

