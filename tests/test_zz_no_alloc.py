"""tt_mp2_energy_noalloc: the MP2 entry point that allocates nothing.

Its partials live in a static device array of the library. These tests call
it through the C ABI and check it against tt_mp2_energy (caller workspace)
on the same inputs: bitwise in deterministic mode, on two calls in a row with
the second problem smaller than the first (the array keeps the first call's
partials), and in atomic mode within the fp64 bar. The size limit is checked
without a device: the call must refuse before any HIP call.
"""

import ctypes

import pytest
import torch

from oracle import cpu_ref
from trntensor_amd.hip import _lib, engine
from util import rel

SCRATCH_DOUBLES = 1 << 21


def _inputs(nocc, nvir, naux, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    B = torch.randn(nocc, nvir, naux, generator=g, dtype=torch.float64) * 0.05
    eo = torch.sort(-20 + 19.7 * torch.rand(nocc, generator=g, dtype=torch.float64))[0]
    ev = torch.sort(0.1 + 4.9 * torch.rand(nvir, generator=g, dtype=torch.float64))[0]
    return B.to(dtype), eo.to(dtype), ev.to(dtype)


def _run(lib, B, eo, ev, deterministic, noalloc):
    """One call on cuda:0; returns the energy as a Python float (after a sync)."""
    code = engine.dtype_code(B.dtype)
    nocc, nvir, naux = B.shape
    b, o, v = (t.to("cuda:0").contiguous() for t in (B, eo, ev))
    e = torch.full((), float("nan"), dtype=B.dtype, device="cuda:0")
    stream = engine._stream_ptr(b.device)
    if noalloc:
        st = lib.tt_mp2_energy_noalloc(code, nocc, nvir, naux, b.data_ptr(), o.data_ptr(), v.data_ptr(),
                                       e.data_ptr(), int(deterministic), stream)
        _lib.check(st, "tt_mp2_energy_noalloc")
    else:
        wsb = lib.tt_mp2_energy_workspace_bytes(code, nocc, nvir, naux)
        ws = torch.empty(int(wsb), dtype=torch.uint8, device="cuda:0")
        st = lib.tt_mp2_energy(code, nocc, nvir, naux, b.data_ptr(), o.data_ptr(), v.data_ptr(), e.data_ptr(),
                               ws.data_ptr(), wsb, int(deterministic), stream)
        _lib.check(st, "tt_mp2_energy")
    torch.cuda.synchronize()
    return float(e.cpu())


@pytest.fixture(scope="module")
def lib():
    handle = _lib.load()
    assert handle is not None, _lib.load_error()
    return handle


def test_noalloc_refuses_beyond_its_scratch_without_a_device(lib):
    # 2048 occupied, 1024 virtuals: 2,098,176 pairs x 136 block pairs > 2^21 partials
    dummy = ctypes.c_void_p(256)
    st = lib.tt_mp2_energy_noalloc(1, 2048, 1024, 64, dummy, dummy, dummy, dummy, 1, None)
    assert st == _lib.TT_INVALID
    msg = lib.tt_last_error()
    assert b"static scratch" in msg and str(SCRATCH_DOUBLES).encode() in msg
    st = lib.tt_mp2_energy_noalloc(1, -1, 3, 3, dummy, dummy, dummy, dummy, 1, None)
    assert st == _lib.TT_INVALID
    st = lib.tt_mp2_energy_noalloc(5, 2, 3, 3, dummy, dummy, dummy, dummy, 1, None)
    assert st == _lib.TT_UNSUPPORTED


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_noalloc_matches_workspace_entry_point_twice(hip, lib, dtype):
    # Second problem smaller: its partials overwrite only a prefix of the array.
    for shape, seed in (((12, 150, 200), 1), ((5, 70, 37), 2)):
        B, eo, ev = _inputs(*shape, dtype, seed)
        print(f"noalloc det {dtype} {shape}", flush=True)
        ref = _run(lib, B, eo, ev, True, noalloc=False)
        got = _run(lib, B, eo, ev, True, noalloc=True)
        assert got == ref, (shape, got, ref)
        oracle = float(cpu_ref.mp2_energy(B.double(), eo.double(), ev.double()))
        assert rel(got, oracle) <= (1e-10 if dtype == torch.float64 else 1e-5)


@pytest.mark.gpu
def test_noalloc_atomic_mode_twice(hip, lib):
    # The accumulator starts at zero on every call (zeroed by a kernel).
    for shape, seed in (((10, 130, 96), 3), ((4, 64, 40), 4)):
        B, eo, ev = _inputs(*shape, torch.float64, seed)
        print(f"noalloc atomic {shape}", flush=True)
        ref = _run(lib, B, eo, ev, True, noalloc=False)
        got = _run(lib, B, eo, ev, False, noalloc=True)
        assert rel(got, ref) <= 1e-12, (shape, got, ref)


@pytest.mark.gpu
def test_noalloc_config4_fp64(hip, lib):
    B, eo, ev = _inputs(64, 320, 1200, torch.float64, 0)
    print("noalloc config 4 fp64", flush=True)
    ref = _run(lib, B, eo, ev, True, noalloc=False)
    got = _run(lib, B, eo, ev, True, noalloc=True)
    assert got == ref
