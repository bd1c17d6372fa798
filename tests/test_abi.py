"""C-ABI library checks that need no GPU: it loads, exports every symbol the
header declares, and rejects bad arguments before launching anything.
Also the engine's host-side mapping logic (letter grouping, stride merging).
"""

import ctypes
import os
import re

import pytest
import torch

from trntensor_amd.hip import _lib, engine

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "trntensor_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|size_t|const char\*)\s+(tt_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    handle = _lib.load()
    assert handle is not None, _lib.load_error()
    return handle


def test_header_declares_the_bound_symbols():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(raw, name), name


def test_version_and_status_strings(lib):
    assert lib.tt_abi_version() == _lib.ABI_VERSION
    assert lib.tt_status_string(0) == b"ok"
    assert lib.tt_status_string(1) == b"invalid argument"
    assert lib.tt_status_string(2).startswith(b"unsupported")
    assert lib.tt_status_string(3).startswith(b"HIP")


def test_gemm_argument_errors_need_no_device(lib):
    st = lib.tt_gemm(1, 0, 0, -1, 4, 4, 1.0, None, 4, 0, None, 4, 0, 0.0, None, 4, 0, None, 4, 0, 1, None)
    assert st == _lib.TT_INVALID and b"negative" in lib.tt_last_error()
    # empty problem: nothing to do
    assert lib.tt_gemm(1, 0, 0, 0, 4, 4, 1.0, None, 4, 0, None, 4, 0, 0.0, None, 4, 0, None, 4, 0, 1, None) == 0
    dummy = ctypes.c_void_p(16)
    st = lib.tt_gemm(1, 0, 0, 4, 4, 4, 1.0, dummy, 2, 0, dummy, 4, 0, 0.0, None, 4, 0, dummy, 4, 0, 1, None)
    assert st == _lib.TT_INVALID and b"leading dimension" in lib.tt_last_error()
    st = lib.tt_gemm(7, 0, 0, 4, 4, 4, 1.0, dummy, 4, 0, dummy, 4, 0, 0.0, None, 4, 0, dummy, 4, 0, 1, None)
    assert st == _lib.TT_UNSUPPORTED


def test_mp2_workspace_and_errors(lib):
    # 64 occupied -> 2080 pairs; 320 virtuals -> 5 blocks -> 15 block pairs
    need = lib.tt_mp2_energy_workspace_bytes(1, 64, 320, 1200)
    assert need >= (2080 * 15 + 1) * 8 and need % 256 == 0
    dummy = ctypes.c_void_p(256)
    st = lib.tt_mp2_energy(1, 64, 320, 1200, dummy, dummy, dummy, dummy, dummy, 8, 1, None)
    assert st == _lib.TT_INVALID and b"workspace" in lib.tt_last_error()
    st = lib.tt_mp2_energy(1, -1, 3, 3, dummy, dummy, dummy, dummy, dummy, 1 << 20, 1, None)
    assert st == _lib.TT_INVALID
    st = lib.tt_mp2_energy(5, 2, 3, 3, dummy, dummy, dummy, dummy, dummy, 1 << 20, 1, None)
    assert st == _lib.TT_UNSUPPORTED


def test_mp2_workspace_holds_a_row_padded_copy_for_unaligned_naux(lib):
    part = (((2080 * 15 + 1) * 8 + 255) // 256) * 256
    for code, elem in ((1, 8), (0, 4)):
        # naux a multiple of 16: the partials only
        assert lib.tt_mp2_energy_workspace_bytes(code, 64, 320, 1200) == part
        assert lib.tt_mp2_energy_workspace_bytes(code, 64, 320, 1216) == part
        # otherwise also B with rows padded to the next multiple of 16
        for naux, pitch in ((1199, 1200), (1190, 1200), (1201, 1216), (1, 16)):
            pad = (64 * 320 * pitch * elem + 255) // 256 * 256
            assert lib.tt_mp2_energy_workspace_bytes(code, 64, 320, naux) == part + pad
    assert lib.tt_mp2_energy_workspace_bytes(1, 0, 320, 1199) == 256
    # Both entry points accept the partials' size for any naux: below it they refuse.
    dummy = ctypes.c_void_p(256)
    st = lib.tt_mp2_energy(1, 64, 320, 1199, dummy, dummy, dummy, dummy, dummy, part - 8, 1, None)
    assert st == _lib.TT_INVALID and f"need {part}".encode() in lib.tt_last_error()
    st = lib.tt_mp2_energy_shard(1, 64, 320, 1199, dummy, dummy, dummy, 0, 1, dummy, dummy, part - 8, 1, None)
    assert st == _lib.TT_INVALID and f"need {part}".encode() in lib.tt_last_error()


def test_ao2mo_and_strided_errors(lib):
    dummy = ctypes.c_void_p(256)
    assert lib.tt_ao_to_mo_workspace_bytes(1, 512, 64, 320, 1536) >= 64 * 512 * 1536 * 8
    st = lib.tt_ao_to_mo_transform(1, 8, 2, 3, 4, dummy, dummy, dummy, dummy, dummy, 8, None)
    assert st == _lib.TT_INVALID
    shape = _lib.i64_array([2] * 9)
    st = lib.tt_strided_contract(1, 9, shape, shape, shape, 0, shape, shape, shape, dummy, None, 1.0, 0.0, None, dummy, None, 0, None)
    assert st == _lib.TT_INVALID
    big = _lib.i64_array([1 << 31])
    st = lib.tt_strided_contract(1, 1, big, shape, shape, 0, shape, shape, shape, dummy, None, 1.0, 0.0, None, dummy, None, 0, None)
    assert st == _lib.TT_UNSUPPORTED


def test_strided_workspace_only_for_split_reductions(lib):
    one = _lib.i64_array([1])
    red = _lib.i64_array([10_000_000])
    assert lib.tt_strided_contract_workspace_bytes(1, 1, one, 1, red) > 0
    # column tiles may split the reduction of up to 2^18 outputs
    some = _lib.i64_array([100_000])
    assert lib.tt_strided_contract_workspace_bytes(1, 1, some, 1, red) > 0
    many = _lib.i64_array([1 << 18])
    assert lib.tt_strided_contract_workspace_bytes(1, 1, many, 1, red) == 0
    short = _lib.i64_array([1])
    assert lib.tt_strided_contract_workspace_bytes(1, 1, many, 1, short) == 0


# ---------------------------------------------------------------------------
# engine host logic
# ---------------------------------------------------------------------------
def test_operand_diagonal_and_merge():
    x = torch.empty(4, 5, 6)
    op = engine.Operand("iji", torch.empty(4, 5, 4))
    assert op.letters == ["i", "j"] and op.strd["i"] == 20 + 1
    op = engine.Operand("abc", x)
    assert engine._merge(op, ["a", "b"]) == (20, 6)
    assert engine._merge(op, ["b", "c"]) == (30, 1)
    assert engine._merge(op, ["a", "c"]) is None
    assert engine._merge(op, []) == (1, 0)


def test_gemm_layout_choice():
    A = engine.Operand("ij", torch.empty(8, 6))  # rows i (stride 6), k=j contiguous
    assert engine._gemm_layout(A, ["i"], ["j"]) == (True, 6)
    assert engine._gemm_layout(A, ["j"], ["i"]) == (False, 6)
    Bt = engine.Operand("ab", torch.empty(8, 6).t())  # non-contiguous view
    assert engine._gemm_layout(Bt, ["a"], ["b"]) == (False, 6)
    bc = engine.Operand("ab", torch.empty(1, 6).expand(8, 6))  # stride-0 rows
    assert engine._gemm_layout(bc, ["a"], ["b"]) is None


def test_merge_dims():
    # (extent, a_stride, b_stride): contiguous in both -> one dim
    assert engine._merge_dims([(4, 30, 6), (6, 5, 1)]) == [(24, 5, 1)]
    assert engine._merge_dims([(4, 6, 6), (6, 1, 1)]) == [(24, 1, 1)]
    assert engine._merge_dims([(4, 6, 1), (6, 1, 4)]) == [(4, 6, 1), (6, 1, 4)]
    assert engine._merge_dims([(1, 9, 9), (3, 1, 0)]) == [(3, 1, 0)]


def test_fast_division_formula():
    """The multiplier scheme of tt_common.hpp (FastDiv) is exact for n < 2^31."""
    import random

    rng = random.Random(0)
    for d in list(range(1, 300)) + [rng.randint(1, (1 << 31) - 1) for _ in range(300)]:
        s = 0
        while (1 << s) < d:
            s += 1
        m = ((1 << 32) * ((1 << s) - d)) // d + 1
        assert m < (1 << 32)
        for n in [0, 1, d - 1, d, d + 1, (1 << 31) - 1] + [rng.randint(0, (1 << 31) - 1) for _ in range(50)]:
            if n < 0:
                continue
            q = (((n * m) >> 32) + n) >> s
            assert q == n // d, (n, d)


def test_strided_int64_needs_integral_scalars(lib):
    dummy = ctypes.c_void_p(256)
    shape = _lib.i64_array([4])
    st = lib.tt_strided_contract(_lib.TT_I64, 1, shape, shape, shape, 0, shape, shape, shape, dummy, None, 1.5, 0.0, None, dummy, None, 0, None)
    assert st == _lib.TT_INVALID and b"integral" in lib.tt_last_error()
    st = lib.tt_strided_contract(_lib.TT_I64, 1, shape, shape, shape, 0, shape, shape, shape, dummy, None, 1.0, 0.25, None, dummy, None, 0, None)
    assert st == _lib.TT_INVALID


def test_plain_c_client_compiles_links_and_runs(tmp_path):
    """tests/c_abi/abi_smoke.c: the header compiles as C (gcc -std=c99), the
    program links against the built library and its host-side checks pass."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    src = os.path.join(ROOT, "tests", "c_abi", "abi_smoke.c")
    exe = str(tmp_path / "abi_smoke")
    libdir = os.path.dirname(_lib.LIB_PATH)
    cmd = [gcc, "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), src, "-o", exe,
           "-L", libdir, "-ltrntensor_hip", f"-Wl,-rpath,{libdir}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    run = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "c abi ok" in run.stdout


def test_mp2_shard_range_checks_need_no_device(lib):
    assert lib.tt_mp2_energy_unit_count(64, 320) == 2080 * 15
    assert lib.tt_mp2_energy_unit_count(0, 320) == 0
    dummy = ctypes.c_void_p(256)
    ws = lib.tt_mp2_energy_workspace_bytes(1, 4, 70, 16)
    st = lib.tt_mp2_energy_shard(1, 4, 70, 16, dummy, dummy, dummy, 25, 6, dummy, dummy, ws, 1, None)
    assert st == _lib.TT_INVALID and b"outside" in lib.tt_last_error()  # 10 pairs x 3 block pairs = 30 units
    st = lib.tt_mp2_energy_shard(1, 4, 70, 16, dummy, dummy, dummy, -1, 2, dummy, dummy, ws, 1, None)
    assert st == _lib.TT_INVALID


def test_launch_table_loads_and_misses_without_a_device(lib):
    """The host launch table (tt_fastpath.so) loads against the library's
    entry points; a lookup of CPU operands is a miss (no launch), and only
    operands on one GPU in one dtype can be recorded."""
    from trntensor_amd.hip import _fastpath

    assert os.path.exists(_fastpath.PATH), "tt_fastpath.so is not built"
    tab = _fastpath.table(8)
    assert tab is not None, _fastpath.error()
    a, b = torch.randn(32, 96), torch.randn(32, 96)
    assert tab.run("ap,bp->ab", a, b, 1.0) is None
    with pytest.raises(RuntimeError, match="one device"):
        tab.add("ap,bp->ab", a, b, [0] * 15, [32, 32], False)
    with pytest.raises(TypeError):
        tab.run("ap,bp->ab", a.numpy(), b, 1.0)
    assert len(tab) == 0
