"""Write turbopress_amd/data/tcq_codebooks.json from the oracle's restatement.

    python tests/golden/make_codebook_table.py [--check-only]

The packed runtime stores the trellis-optimised codebook of each linear as
fp16 (turbopress/runtime.py:183), and ``pack_linear`` searches with its fp32
values (runtime.py:166, trellis.py:296).  The synthetic workloads, the tests
and the encoder need the default codebook for (bits, S) without running the
codebook training on the GPU box, so this script computes it once with
``oracle.codebook_oracle.tcq_optimized_codebook`` (a restatement of
turbopress/trellis.py:206-253, seed 0) and writes the fp16 and fp32 bit
patterns into the package's data file.  ``tests/test_oracle.py`` checks the
table against the golden vectors imported from the reference
(``codebooks.json``).
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle.codebook_oracle import tcq_optimized_codebook  # noqa: E402

OUT = ROOT / "turbopress_amd" / "data" / "tcq_codebooks.json"
CASES = [(b, s) for s in (4, 8, 16, 64) for b in (1, 2, 3, 4)]


def table() -> dict:
    import torch
    out = {"what": "fp16 (codebooks) and fp32 (codebooks_f32) bit patterns of "
                   "tcq_optimized_codebook(bits, n_states, seed=0)",
           "generated_by": "tests/golden/make_codebook_table.py", "codebooks": {}, "codebooks_f32": {}}
    for bits, s in CASES:
        cb32 = tcq_optimized_codebook(bits, s).to(torch.float32)
        cb = cb32.to(torch.float16)
        out["codebooks"][f"{bits},{s}"] = cb.view(torch.int16).to(torch.int32).bitwise_and(0xFFFF).tolist()
        out["codebooks_f32"][f"{bits},{s}"] = [int(v) & 0xFFFFFFFF for v in cb32.view(torch.int32).tolist()]
        print(f"bits={bits} S={s} done", flush=True)
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--check-only", action="store_true")
    args = ap.parse_args()
    t = table()
    golden = json.loads((Path(__file__).parent / "codebooks.json").read_text())["trellis"]
    bad = [k for k, v in t["codebooks"].items() if golden[k]["f16"] != v]
    import struct
    for k, v in t["codebooks_f32"].items():
        want = [struct.unpack("<I", struct.pack("<f", float.fromhex(h)))[0] for h in golden[k]["f32"]]
        if want != v:
            bad.append(k + " (f32)")
    print("mismatches vs reference golden:", bad)
    if not args.check_only:
        OUT.parent.mkdir(parents=True, exist_ok=True)
        OUT.write_text(json.dumps(t, indent=1) + "\n")
        print("wrote", OUT)
    if bad:
        raise SystemExit(1)


if __name__ == "__main__":
    main()
