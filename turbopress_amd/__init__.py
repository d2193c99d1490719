"""turbopress_amd: TurboPress's packed-TCQ decode path, native to MI355X (gfx950).

Drop-in for the reference's packed runtime (turbopress/runtime.py,
turbopress/triton_kernel.py): ``PackedTCQLinear`` takes the same format-v2
payload and forward signature; ``fwht_scale``/``packed_gemv`` keep the
reference kernel wrappers' names.  All compute runs in hand-written HIP
kernels from ``libturbopress_amd.so`` (C ABI in ``include/turbopress_amd.h``).
"""

from __future__ import annotations

__version__ = "0.1.0"

_LAZY = {
    "PackedTCQLinear": ("turbopress_amd.runtime", "PackedTCQLinear"),
    "Trellis": ("turbopress_amd.runtime", "Trellis"),
    "HAS_HIP": ("turbopress_amd.hip_kernel", "HAS_HIP"),
    "fwht_scale": ("turbopress_amd.hip_kernel", "fwht_scale"),
    "packed_gemv": ("turbopress_amd.hip_kernel", "packed_gemv"),
    "subset_lut": ("turbopress_amd.hip_kernel", "subset_lut"),
    "window_decode_levels": ("turbopress_amd.hip_kernel", "window_decode_levels"),
    "default_codebook": ("turbopress_amd.codebooks", "default_codebook"),
    "pack_linear": ("turbopress_amd.pack", "pack_linear"),
    "pack_model": ("turbopress_amd.pack", "pack_model"),
    "load_packed_model": ("turbopress_amd.artifact", "load_packed_model"),
    "tcq_quantize_rows": ("turbopress_amd.encoder", "tcq_quantize_rows"),
}

__all__ = list(_LAZY)


def __getattr__(name):
    if name in _LAZY:
        import importlib
        mod, attr = _LAZY[name]
        return getattr(importlib.import_module(mod), attr)
    raise AttributeError(f"module 'turbopress_amd' has no attribute {name!r}")
