"""Default trellis-optimised codebooks (data).

``default_codebook(bits, n_states)`` returns the fp16 codebook that
``turbopress.trellis.tcq_optimized_codebook(bits, n_states)`` (seed 0,
trellis.py:206-253) produces and ``pack_linear`` stores (runtime.py:183);
``optimized_codebook_f32`` its fp32 values, which the encoder searches with
(trellis.py:296).  The values are read from ``data/tcq_codebooks.json``
(bit patterns); nothing is computed at run time.
"""

from __future__ import annotations

import json
from functools import lru_cache
from pathlib import Path

import torch

_DATA = Path(__file__).resolve().parent / "data" / "tcq_codebooks.json"


@lru_cache(maxsize=None)
def _data() -> dict:
    return json.loads(_DATA.read_text())


def _table() -> dict[str, list[int]]:
    return _data()["codebooks"]


def available_codebooks() -> list[tuple[int, int]]:
    return sorted(tuple(int(v) for v in k.split(",")) for k in _table())


def default_codebook(bits: int, n_states: int = 64) -> torch.Tensor:
    """fp16 [2**(bits+1)] codebook for (bits, n_states)."""
    key = f"{bits},{n_states}"
    tab = _table()
    if key not in tab:
        raise ValueError(f"no default codebook for bits={bits}, n_states={n_states}; "
                         f"have {available_codebooks()}")
    raw = torch.tensor(tab[key], dtype=torch.int32).to(torch.int16)
    return raw.view(torch.float16).clone()


def optimized_codebook_f32(bits: int, n_states: int = 64) -> torch.Tensor:
    """fp32 [2**(bits+1)] trellis-optimised codebook for (bits, n_states):
    the values the encoder searches with (default_codebook is their fp16
    rounding)."""
    key = f"{bits},{n_states}"
    tab = _data().get("codebooks_f32", {})
    if key not in tab:
        raise ValueError(f"no default codebook for bits={bits}, n_states={n_states}; "
                         f"have {available_codebooks()}")
    raw = torch.tensor(tab[key], dtype=torch.int64).to(torch.int32)
    return raw.view(torch.float32).clone()
