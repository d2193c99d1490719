"""The C-ABI library loads, exports every declared symbol, and validates
arguments on the host (CPU only: no call here reaches the GPU)."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(tp_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    names = _declared_symbols()
    for required in ("tp_abi_version", "tp_fwht_scale", "tp_decode_rows",
                     "tp_window_decode_levels", "tp_tcq_gemv", "tp_subset_lut"):
        assert required in names


def test_library_exports_every_declared_symbol(built_lib):
    for name in _declared_symbols():
        assert hasattr(built_lib, name), name


def test_ctypes_table_covers_header():
    from turbopress_amd import _lib
    assert set(_lib.SIGNATURES) == set(_declared_symbols())


def test_abi_version_and_status_strings(built_lib):
    from turbopress_amd import _lib
    assert built_lib.tp_abi_version() == _lib.ABI_VERSION
    for code in range(10):
        assert _lib.status_string(code) != "unknown status"
    assert _lib.status_string(99) == "unknown status"


@pytest.mark.parametrize("n_states", [4, 8, 16, 64])
def test_subset_lut_host_function_matches_oracle(built_lib, n_states):
    from oracle.tcq_oracle import subset_lut
    buf = (ctypes.c_uint8 * (2 * n_states))()
    assert built_lib.tp_subset_lut(n_states, buf, 2 * n_states) == 0
    assert np.array_equal(np.frombuffer(bytes(buf), dtype=np.uint8), subset_lut(n_states))


def test_host_side_argument_validation(built_lib):
    from turbopress_amd import _lib
    buf = (ctypes.c_uint8 * 256)()
    assert built_lib.tp_subset_lut(6, buf, 256) == _lib.TP_ERR_UNSUPPORTED_STATES
    assert built_lib.tp_subset_lut(64, buf, 64) == _lib.TP_ERR_BAD_DIMS
    # Null pointers, bad block and bad bits are rejected before any GPU call.
    assert built_lib.tp_fwht_scale(None, None, None, 1, 64, 64, None) == _lib.TP_ERR_NULL_POINTER
    fake = ctypes.c_void_p(16)
    assert built_lib.tp_fwht_scale(fake, fake, fake, 1, 96, 64, None) == _lib.TP_ERR_BAD_BLOCK
    assert built_lib.tp_fwht_scale(fake, fake, fake, 1, 96, 48, None) == _lib.TP_ERR_BAD_BLOCK
    assert built_lib.tp_decode_rows(fake, 12, fake, 24, fake, fake, 4, 96, 9, 64, fake, 96, None) \
        == _lib.TP_ERR_UNSUPPORTED_BITS
    assert built_lib.tp_decode_rows(fake, 12, fake, 24, fake, fake, 4, 96, 3, 32, fake, 96, None) \
        == _lib.TP_ERR_UNSUPPORTED_STATES
    assert built_lib.tp_decode_rows(fake, 11, fake, 24, fake, fake, 4, 96, 3, 64, fake, 96, None) \
        == _lib.TP_ERR_BAD_DIMS
    assert built_lib.tp_tcq_gemv(fake, 1, fake, 12, None, 24, fake, fake, None, 4, 96, 3, 64,
                                 fake, None) == _lib.TP_ERR_NULL_POINTER
    assert built_lib.tp_read_probe(None, 64, fake, None) == _lib.TP_ERR_NULL_POINTER
    assert built_lib.tp_read_probe(fake, 20, fake, None) == _lib.TP_ERR_BAD_DIMS
    assert built_lib.tp_read_probe(ctypes.c_void_p(24), 64, fake, None) == _lib.TP_ERR_MISALIGNED
    # the stack's codebook is read as dwords through the scalar cache
    assert built_lib.tp_stack_gemv(ctypes.c_void_p(256), 1, ctypes.c_void_p(258), 3, 64, 0, 1, None) \
        == _lib.TP_ERR_MISALIGNED


def _stack_array(count, n=256, d=256):
    from turbopress_amd import _lib
    arr = (_lib.StackLinear * count)()
    for i in range(count):
        arr[i].n, arr[i].d, arr[i].ldx, arr[i].ldy, arr[i].block, arr[i].phase = n, d, d, n, d & -d, 0
    return arr


def test_stack_plan_size_limits(built_lib):
    """Schedule entries hold (linear << 14) | block in a positive int32: the
    plan accepts up to 65536 linears of up to 2^14 blocks (128 rows each) and
    refuses anything larger on the host."""
    assert built_lib.tp_stack_plan_bytes(_stack_array(1), 1, 3, 1) > 0
    assert built_lib.tp_stack_plan_bytes(_stack_array(2048), 2048, 3, 1) > 0
    big = _stack_array(65536, n=16, d=64)
    assert built_lib.tp_stack_plan_bytes(big, 65536, 3, 1) > 0
    assert built_lib.tp_stack_plan_bytes(_stack_array(65537, n=16, d=64), 65537, 3, 1) == 0
    assert built_lib.tp_stack_plan_bytes(_stack_array(1, n=128 << 14, d=64), 1, 3, 1) == 0
    assert built_lib.tp_stack_plan_bytes(_stack_array(1, n=(128 << 14) - 128, d=64), 1, 3, 1) > 0
    assert built_lib.tp_stack_plan_bytes(_stack_array(1), 1, 5, 1) == 0
    assert built_lib.tp_stack_plan_bytes(_stack_array(1), 1, 3, 33) == 0


def test_stack_plan_phases_start_at_zero_without_gaps(built_lib):
    """A phase waits for the one before it only, so plans whose phases skip
    a number (or do not start at 0) are refused on the host."""
    arr = _stack_array(4)
    for i, ph in enumerate((0, 0, 1, 2)):
        arr[i].phase = ph
    assert built_lib.tp_stack_plan_bytes(arr, 4, 3, 1) > 0
    arr[3].phase = 3  # phase 2 empty
    assert built_lib.tp_stack_plan_bytes(arr, 4, 3, 1) == 0
    for i, ph in enumerate((1, 1, 2, 3)):
        arr[i].phase = ph
    assert built_lib.tp_stack_plan_bytes(arr, 4, 3, 1) == 0


def test_split_k_route_reports_a_short_workspace_before_any_launch(built_lib):
    """A call routed to the split-K kernel (batch 6 with 1024-column Hadamard
    blocks: not the one-pass kernel) whose workspace is one word short
    returns TP_ERR_WORKSPACE on the host, before any launch; the no-allocation
    forward uses the same routing with its fixed array, whose limit the GPU
    test checks.  Out-of-range batches are refused first."""
    from turbopress_amd import _lib
    fake = ctypes.c_void_p(256)
    n, d, batch = 33000, 1024, 6
    T = (n + 15) // 16
    need = T * 16 * 16 * 4 + T * 4  # split-K sums (batch <= 16) + counters
    assert built_lib.tp_gemv_workspace_bytes(n, batch) >= need
    args = [fake, d, batch, fake, 1024, fake, fake, fake, fake, None, n, d, 3, 64, fake, n, fake, need - 4, None]
    assert built_lib.tp_packed_linear_forward(*args) == _lib.TP_ERR_WORKSPACE
    args[16] = None
    assert built_lib.tp_packed_linear_forward(*args) == _lib.TP_ERR_WORKSPACE
    noalloc = [fake, 256, 33, fake, 256, fake, fake, fake, fake, None, 16400, 256, 3, 64, fake, 16400, None]
    assert built_lib.tp_packed_linear_forward_noalloc(*noalloc) == _lib.TP_ERR_BAD_DIMS


def test_check_maps_status_to_reference_exceptions():
    from turbopress_amd import _lib
    with pytest.raises(ValueError):
        _lib.check(_lib.TP_ERR_BAD_DIMS, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.TP_ERR_HIP, "x")
    _lib.check(_lib.TP_OK, "x")


def test_device_code_indexes_no_register_arrays(tmp_path):
    """Every loop over a register array unrolls to constant indices: the
    device code holds no VGPR-indexed moves (and no spills to scratch).  (A loop the compiler cannot
    unroll turns v[e + h] into indexed moves, and once if-converted those
    write past the array into unrelated live registers.)"""
    import shutil
    import subprocess
    from concurrent.futures import ThreadPoolExecutor
    from turbopress_amd import build as B
    if not Path(B.HIPCC).exists() and shutil.which(B.HIPCC) is None:
        pytest.skip("hipcc not available")

    def compile_asm(src):
        out = tmp_path / (src.stem + ".s")
        res = subprocess.run([B.HIPCC, *B.HIP_FLAGS, f"-I{B.CSRC}", "--cuda-device-only", "-S", str(src),
                              "-o", str(out)], capture_output=True, text=True)
        assert res.returncode == 0, res.stderr[-2000:]
        return src.name, out.read_text(), res.stderr

    with ThreadPoolExecutor(max_workers=4) as ex:
        results = list(ex.map(compile_asm, sorted(B.CSRC.glob("*.hip"))))
    for name, asm, log in results:
        assert "loop not unrolled" not in log, name
        for insn in ("s_set_gpr_idx_on", "v_movrels", "v_movreld", "v_movrelsd"):
            assert insn not in asm, (name, insn)
        # No register spills to scratch memory, and no kernel with a private
        # segment (whose scratch is set up at every wave launch).
        assert "scratch_load" not in asm and "scratch_store" not in asm, name
        for kern, body in re.findall(r"\.amdhsa_kernel (\S+)\n(.*?)\.end_amdhsa_kernel", asm, re.S):
            assert ".amdhsa_enable_private_segment 1" not in body, (name, kern)


def _plan(lib, ns, d, block, batch, bits=3, ws=1 << 21, cus=256, lds=160 * 1024):
    arr = (ctypes.c_int64 * len(ns))(*ns)
    out = (ctypes.c_int64 * 6)()
    assert lib.tp_linear_forward_plan(arr, len(ns), d, block, bits, batch, ws, cus, lds, out) == 0
    return dict(zip(("kparts", "units_per_part", "units_per_wave", "chunks", "tiles_per_group", "workgroups"),
                    list(out)))


def test_linear_planner_cuts_at_the_qwen3_4b_shapes(built_lib):
    """The one-pass kernel's plan on a 256-CU, 160 KiB-LDS device (host only):
    down_proj (2560 x 9728) cuts K into parts of whole 512-column Hadamard
    blocks at batch 1..8 (many parts at batch 4 / 8, where one part would
    stage the whole input in every workgroup); gate_proj keeps one part at
    batch 1 and 4 and takes 3 at batch 8; the gate/up pair fits one round of
    workgroups with 4 units per wave; o_proj's 4096-column block is never
    split; without a workspace nothing is split; batch 9 is not this
    kernel's."""
    lib = built_lib
    for batch in (1, 4, 8):
        p = _plan(lib, [2560], 9728, 512, batch)
        assert p["kparts"] >= 3 and p["units_per_part"] % 2 == 0, (batch, p)
        assert p["workgroups"] <= 256 and p["units_per_part"] * p["kparts"] >= 38
    assert _plan(lib, [2560], 9728, 512, 4)["kparts"] >= 5
    assert _plan(lib, [9728], 2560, 512, 1) == {"kparts": 1, "units_per_part": 10, "units_per_wave": 2,
                                                  "chunks": 5, "tiles_per_group": 3, "workgroups": 203}
    assert _plan(lib, [9728], 2560, 512, 4)["kparts"] == 1
    assert _plan(lib, [9728], 2560, 512, 8)["kparts"] == 3
    pair = _plan(lib, [9728, 9728], 2560, 512, 1)
    assert pair["kparts"] == 1 and pair["units_per_wave"] == 4 and pair["workgroups"] <= 256
    o = _plan(lib, [2560], 4096, 4096, 1)
    assert o["kparts"] == 1 and o["workgroups"] == 160
    assert _plan(lib, [2560], 9728, 512, 4, ws=0)["kparts"] == 0  # no workspace: the split-K kernel
    assert _plan(lib, [2560], 9728, 512, 9)["kparts"] == 0
