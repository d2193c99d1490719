"""Build libturbopress_amd.so (hipcc, gfx950) in-tree.

    python -m turbopress_amd.build [--jobs N] [--verbose]

Every ``csrc/*.hip`` file is compiled for gfx950 to an object under
``csrc/_build/`` and linked into ``turbopress_amd/libturbopress_amd.so``,
next to this file, so the library travels with the source tree.  The build
always recompiles (it is also the CPU-side "does it build" check).
"""

from __future__ import annotations

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ_DIR = CSRC / "_build"
INCLUDE = PKG.parent / "include"
LIB_NAME = "libturbopress_amd.so"
LIB_PATH = PKG / LIB_NAME
ARCH = os.environ.get("TP_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
# atomic optimizer off: it turns a one-lane ticket atomicAdd into a wave
# reduction whose result is read back at once, i.e. a wait that would drain
# every weight prefetch in flight; the kernels consume ticket results later.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function",
    f"-I{INCLUDE}",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}")
    noise = [ln for ln in res.stderr.splitlines()
             if ln.strip() and "packed-fp32-ops" not in ln and "not a recognized feature" not in ln]
    if verbose and noise:
        sys.stderr.write("\n".join(noise) + "\n")


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    objs = [OBJ_DIR / (s.stem + ".o") for s in sources]
    cmds = [[HIPCC, *HIP_FLAGS, "-c", str(s), "-o", str(o)] for s, o in zip(sources, objs)]
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs)], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose))


if __name__ == "__main__":
    main()
