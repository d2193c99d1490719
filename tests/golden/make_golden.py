"""Write the golden vectors that no closed form or invariant pins.

Run in the build container only (the reference checkout does not exist on
the GPU box):

    python tests/golden/make_golden.py [--reference /root/reference]

It imports exactly the reference functions whose outputs depend on torch's
RNG stream and tie-breaking, and records their outputs as small JSON
fixtures next to this script:

  * ``codebooks.json``: ``turbopress.trellis.tcq_optimized_codebook(bits, S)``
    (the codebook ``pack_linear`` stores, trellis.py:206-253) and
    ``turbopress.pipeline.tcq_codebook(bits, S)`` (the codebook format-v1
    artifacts store, pipeline.py:282-301), as fp32 hex strings plus the fp16
    bit patterns the packed runtime keeps (runtime.py:183).
  * ``signs.json``: ``turbopress.hadamard.RandomizedOrthogonal(d, seed).signs``
    (hadamard.py:76-80) for a few (d, seed), stored as 0/1 bits.

Everything else on the decode path (LUT, bit layout, window decode, FWHT) is
pinned by closed forms and brute force in the tests, so it is not imported.
"""

from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

CODEBOOK_CASES = [(b, s) for s in (4, 8, 16, 64) for b in (1, 2, 3, 4)]
PIPELINE_CASES = [(b, s) for s in (16, 64) for b in (2, 3, 4)]
SIGN_CASES = [(576, 0), (1024, 0), (2560, 0), (96, 3), (9728, 11)]


def _f32_hex(t) -> list[str]:
    return [float(v).hex() for v in t.to(dtype=__import__("torch").float32).tolist()]


def _f16_bits(t) -> list[int]:
    import torch
    return t.to(torch.float16).view(torch.int16).to(torch.int32).bitwise_and(0xFFFF).tolist()


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    sys.path.insert(0, args.reference)
    import torch
    from turbopress import pipeline as ref_pipeline
    from turbopress.hadamard import RandomizedOrthogonal
    from turbopress.trellis import tcq_optimized_codebook

    out = {"source": "turbopress 0.5.2 (reference), imported by tests/golden/make_golden.py",
           "torch": torch.__version__, "trellis": {}, "pipeline": {}}
    for bits, s in CODEBOOK_CASES:
        t0 = time.time()
        cb = tcq_optimized_codebook(bits, s)
        out["trellis"][f"{bits},{s}"] = {"f32": _f32_hex(cb), "f16": _f16_bits(cb)}
        print(f"trellis codebook bits={bits} S={s}: {time.time() - t0:.1f}s", flush=True)
    for bits, s in PIPELINE_CASES:
        t0 = time.time()
        cb = ref_pipeline.tcq_codebook(bits, s)
        out["pipeline"][f"{bits},{s}"] = {"f32": _f32_hex(cb), "f16": _f16_bits(cb)}
        print(f"pipeline codebook bits={bits} S={s}: {time.time() - t0:.1f}s", flush=True)
    (HERE / "codebooks.json").write_text(json.dumps(out, indent=1) + "\n")

    signs = {"source": out["source"], "cases": {}}
    for d, seed in SIGN_CASES:
        s01 = (RandomizedOrthogonal(d, seed=seed).signs > 0).to(torch.uint8).numpy()
        signs["cases"][f"{d},{seed}"] = np.packbits(s01, bitorder="little").tobytes().hex()
    (HERE / "signs.json").write_text(json.dumps(signs, indent=1) + "\n")
    print("wrote", HERE / "codebooks.json", HERE / "signs.json")


if __name__ == "__main__":
    main()
