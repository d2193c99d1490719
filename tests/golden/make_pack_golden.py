"""Write the golden vectors of ``pack_linear`` (nn.Linear -> format-v2 payload).

Run in the build container only (the reference checkout does not exist on
the GPU box):

    python tests/golden/make_pack_golden.py [--reference /root/reference]

For a few seeded small linears it calls ``turbopress.runtime.pack_linear``
(runtime.py:143-186: equilibration, seeded rotation, TCQ with the reference's
CPU Viterbi) and records inputs and outputs in ``pack_linear.json`` next to
this script: the weight, bias and activation RMS as fp32/fp16 bit patterns,
and every payload field (packed bytes, fp16 bit patterns, ints).
"""

from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent

# (n, d, bits, n_states, seed, bias)
CASES = [(24, 256, 3, 64, 5, True), (16, 96, 2, 16, 0, False), (12, 512, 4, 8, 7, False),
         (8, 128, 1, 4, 3, True)]


def case_inputs(n: int, d: int, seed: int, bias: bool):
    import torch
    gen = torch.Generator().manual_seed(1000 + seed)
    w = torch.randn(n, d, generator=gen) * 0.02
    w[:, :: max(1, d // 8)] *= 6.0  # a few outlier input channels
    b = (torch.randn(n, generator=gen) * 0.1) if bias else None
    act = torch.randn(d, generator=gen).abs() + 0.1
    return w, b, act


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    sys.path.insert(0, args.reference)
    import torch
    from torch import nn
    from turbopress.runtime import pack_linear  # the reference implementation

    def f32_bits(t):
        return t.to(torch.float32).contiguous().view(torch.int32).tolist()

    def f16_bits(t):
        return t.to(torch.float16).contiguous().view(torch.int16).to(torch.int32).bitwise_and(0xFFFF).tolist()

    out = {"source": "turbopress.runtime.pack_linear (runtime.py:143-186)", "torch": torch.__version__,
           "cases": []}
    for n, d, bits, s, seed, bias in CASES:
        t0 = time.time()
        w, b, act = case_inputs(n, d, seed, bias)
        lin = nn.Linear(d, n, bias=bias)
        with torch.no_grad():
            lin.weight.copy_(w)
            if bias:
                lin.bias.copy_(b)
        p = pack_linear(lin, act, bits=bits, n_states=s, seed=seed)
        out["cases"].append({
            "n": n, "d": d, "bits": bits, "n_states": s, "seed": seed,
            "weight_f32": f32_bits(w), "bias_f32": None if b is None else f32_bits(b), "act_rms_f32": f32_bits(act),
            "payload": {
                "block": int(p["block"]),
                "path_packed": p["path_packed"].flatten().tolist(),
                "member_packed": None if p["member_packed"] is None else p["member_packed"].flatten().tolist(),
                "scales_f16": f16_bits(p["scales"]),
                "signs_packed": p["signs_packed"].flatten().tolist(),
                "inv_equil_f16": f16_bits(p["inv_equil"]),
                "codebook_f16": f16_bits(p["codebook"]),
                "bias_f16": None if p["bias"] is None else f16_bits(p["bias"]),
            },
        })
        print(f"n={n} d={d} bits={bits} S={s}: {time.time() - t0:.1f} s", flush=True)
    (HERE / "pack_linear.json").write_text(json.dumps(out) + "\n")
    print("wrote", HERE / "pack_linear.json")


if __name__ == "__main__":
    main()
