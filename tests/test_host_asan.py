"""Host-side sanitizer build of the C ABI (no GPU): every csrc/*.hip file is
compiled with AddressSanitizer and UndefinedBehaviorSanitizer on its host
side (-Xarch_host; the gfx950 device code is built as usual and never run
here), linked with tests/asan/host_driver.cpp, and run.  The driver
walks the plan builder (layout, schedules, ordered-kernel blocks), the
layout and workspace size functions, the trellis tables and the argument
checks of every GPU entry point; a sanitizer report or an unexpected status
fails the test."""

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "turbopress_amd" / "csrc"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = ROCM / "bin" / "hipcc"
CLANG = ROCM / "llvm" / "bin" / "clang++"
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=all"]


def test_host_code_under_address_and_ub_sanitizers(tmp_path):
    if not HIPCC.exists() or not CLANG.exists():
        pytest.skip("ROCm compilers not available")
    common = ["-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fPIC", f"-I{ROOT / 'include'}",
              f"-I{CSRC}"]
    srcs = sorted(CSRC.glob("*.hip"))

    def compile_one(src):
        obj = tmp_path / (src.stem + ".o")
        cmd = [str(HIPCC), "--offload-arch=gfx950", *common, *SAN, "-c", str(src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        assert res.returncode == 0, res.stderr[-3000:]
        return obj

    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(compile_one, srcs))
    drv = tmp_path / "host_driver.o"
    res = subprocess.run([str(HIPCC), "--offload-arch=gfx950", "-x", "hip", *common, *SAN, "-c",
                          str(ROOT / "tests" / "asan" / "host_driver.cpp"), "-o", str(drv)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    exe = tmp_path / "host_driver"
    res = subprocess.run([str(CLANG), "-fsanitize=address,undefined", "-o", str(exe), str(drv),
                          *map(str, objs), f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}"],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", HIP_VISIBLE_DEVICES="")
    res = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=600)
    assert res.returncode == 0, (res.stdout + res.stderr)[-4000:]
    assert "0 unexpected results" in res.stdout
