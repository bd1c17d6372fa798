"""Backend control and residency on the host: the reference's tests/test_nki.py
(lines 10-44) restated for this build. Where the reference's behaviour hinges
on the Neuron compiler, the HIP counterpart is asserted instead (the message
names the HIP runtime); without a gfx950 device, as on a CPU-only host, the
"no runtime" branches are the ones exercised.
"""

import pytest
import torch

import trntensor_amd as trntensor
from trntensor_amd.hip import dispatch


@pytest.fixture(autouse=True)
def _restore_backend():
    prev = trntensor.get_backend()
    yield
    dispatch._backend = prev


def test_set_backend_auto():
    trntensor.set_backend("auto")
    assert trntensor.get_backend() == "auto"


def test_set_backend_pytorch():
    trntensor.set_backend("pytorch")
    assert trntensor.get_backend() == "pytorch"
    trntensor.set_backend("auto")


def test_set_backend_invalid():
    with pytest.raises(AssertionError):
        trntensor.set_backend("tpu")


@pytest.mark.skipif(dispatch.HAS_HIP, reason="asserts the no-runtime guard")
def test_set_backend_hip_raises_without_runtime():
    """Reference: set_backend('nki') without neuronxcc raises RuntimeError and
    leaves the backend unchanged (tests/test_nki.py:27-31); 'nki' is an alias
    of 'hip' here."""
    for name in ("hip", "nki"):
        with pytest.raises(RuntimeError, match="HIP backend"):
            trntensor.set_backend(name)
        assert trntensor.get_backend() not in ("hip", "nki")


def test_from_xla_cpu_tensor_is_noop():
    t = torch.randn(3, 4)
    assert trntensor.from_xla(t) is t
    assert trntensor.from_device(t) is t


@pytest.mark.skipif(dispatch.HAS_HIP, reason="to_xla without a HIP runtime raises; a GPU host has one")
def test_to_xla_without_runtime_raises():
    t = torch.randn(3, 4)
    with pytest.raises(RuntimeError, match="HIP runtime"):
        trntensor.to_xla(t)


@pytest.mark.skipif(dispatch.HAS_HIP, reason="asserts the no-runtime behaviour")
def test_contractions_raise_without_runtime():
    """No host fallback: without the HIP runtime every entry point raises."""
    A, B = torch.randn(4, 3), torch.randn(3, 5)
    with pytest.raises(RuntimeError, match="HIP runtime unavailable"):
        trntensor.einsum("ij,jk->ik", A, B)
    with pytest.raises(RuntimeError, match="HIP runtime unavailable"):
        trntensor.mp2_energy(torch.randn(2, 3, 4), torch.randn(2), torch.randn(3))
    # the planner itself is host logic and still answers
    assert trntensor.plan_contraction("ij,jk->ik", A, B).backend == "pytorch"


def test_force_backend_env(monkeypatch):
    monkeypatch.setenv("TRNTENSOR_FORCE_BACKEND", "pytorch")
    assert dispatch._use_hip() is False
    monkeypatch.setenv("TRNTENSOR_FORCE_BACKEND", "nki")
    assert dispatch._use_hip() is True
    monkeypatch.delenv("TRNTENSOR_FORCE_BACKEND")
    trntensor.set_backend("pytorch")
    assert dispatch._use_hip() is False


class _FakeMp2Lib:
    """tt_mp2_energy_workspace_bytes with the library's sizes: partials for
    the work units plus, for naux off a multiple of 16, the padded copy."""

    def tt_mp2_energy_workspace_bytes(self, code, nocc, nvir, naux):
        part = 8 * (nocc * (nocc + 1) // 2 * 3 + 1)
        pad = 0 if naux % 16 == 0 else nocc * nvir * ((naux + 15) // 16 * 16) * 8
        return part + pad


def test_mp2_workspace_falls_back_to_partials_on_oom():
    """An unaligned naux asks for the padded copy first; when the device cannot
    hold it (OutOfMemoryError), the call gets the partials-only workspace, with
    which the library runs on B as given."""
    lib = _FakeMp2Lib()
    asked = []

    def alloc_oom_above(limit):
        def alloc(n):
            asked.append(n)
            if n > limit:
                raise torch.OutOfMemoryError("no room for the padded copy")
            return torch.empty(n, dtype=torch.uint8)

        return alloc

    full = lib.tt_mp2_energy_workspace_bytes(1, 4, 100, 1199)
    part = lib.tt_mp2_energy_workspace_bytes(1, 4, 100, 1200)
    assert full > part
    ws, nb = dispatch._mp2_workspace(lib, 1, 4, 100, 1199, None, _alloc=alloc_oom_above(part))
    assert nb == part and ws.numel() == part and asked == [full, part]
    asked.clear()
    ws, nb = dispatch._mp2_workspace(lib, 1, 4, 100, 1199, None, _alloc=alloc_oom_above(full))
    assert nb == full and ws.numel() == full and asked == [full]
    asked.clear()
    # naux a multiple of 16: no copy is asked for.
    ws, nb = dispatch._mp2_workspace(lib, 1, 4, 100, 1200, None, _alloc=alloc_oom_above(full))
    assert nb == part and asked == [part]
