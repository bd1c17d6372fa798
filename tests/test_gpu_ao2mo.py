"""GPU parity of the full AO->MO transform (tt_ao_to_mo_transform via
trntensor_amd.ao_to_mo_transform).

Oracle: the reference's 3-operand einsum (trntensor/quantum.py:188-194) at
small sizes, and the two-step form its own test uses
(tests/test_quantum.py:72-74) at config-3 scale, where the 3-operand form
would materialise an (m, i, n, a) product. Shapes include those of the
reference's simulator and hardware tests (tests/test_nki_sim.py:93-152,
tests/test_nki_kernels.py:194-259), including nbasis not a multiple of 128.
"""

import pytest
import torch

import trntensor_amd as tt
from oracle import brute, cpu_ref
from tests.util import normwise, rel

pytestmark = pytest.mark.gpu


def inputs(nbasis, nocc, nvir, naux, dtype=torch.float64, seed=0):
    g = torch.Generator().manual_seed(seed)
    eri = torch.randn(nbasis, nbasis, naux, generator=g, dtype=torch.float64) * 0.1
    Co = torch.randn(nbasis, nocc, generator=g, dtype=torch.float64)
    Cv = torch.randn(nbasis, nvir, generator=g, dtype=torch.float64)
    return eri.to(dtype), Co.to(dtype), Cv.to(dtype)


SHAPES = [
    (8, 3, 5, 12),
    (32, 5, 10, 16),
    (256, 8, 16, 16),
    (200, 6, 12, 12),
    (256, 16, 32, 32),
    (200, 10, 20, 24),
    (97, 70, 130, 33),
    (1, 1, 1, 1),
]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
def test_matches_oracle(hip, shape, dt):
    eri, Co, Cv = inputs(*shape, dtype=dt, seed=sum(shape))
    ref = cpu_ref.ao_to_mo_transform(eri, Co, Cv)
    got = tt.ao_to_mo_transform(eri.cuda(), Co.cuda(), Cv.cuda())
    assert got.device.type == "cuda" and got.dtype == dt and tuple(got.shape) == (shape[1], shape[2], shape[3])
    assert normwise(got, ref) <= (1e-12 if dt == torch.float64 else 1e-5)


def test_golden_fixture(hip):
    import os

    import numpy as np

    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "ao2mo_small.npz"))
    for k in range(2):
        eri, Co, Cv = (torch.from_numpy(g[n + str(k)]).cuda() for n in ("eri", "Co", "Cv"))
        got = tt.ao_to_mo_transform(eri, Co, Cv)
        assert normwise(got, torch.from_numpy(g[f"B{k}"])) <= 1e-13


def test_cpu_operands_round_trip(hip):
    eri, Co, Cv = inputs(40, 4, 9, 10, seed=3)
    got = tt.ao_to_mo_transform(eri, Co, Cv)
    assert got.device.type == "cpu"
    assert normwise(got, torch.from_numpy(brute.ao_to_mo_loops(eri, Co, Cv))) <= 1e-12


def test_composes_with_mp2_energy(hip):
    """tests/test_nki_kernels.py:244-268: AO -> MO -> E with B resident on the device."""
    eri, Co, Cv = inputs(256, 10, 30, 32, seed=52)
    g = torch.Generator().manual_seed(53)
    eo = -torch.sort(torch.rand(10, generator=g, dtype=torch.float64))[0] - 0.5
    ev = torch.sort(torch.rand(30, generator=g, dtype=torch.float64))[0] + 0.1
    B = tt.ao_to_mo_transform(eri.cuda(), Co.cuda(), Cv.cuda())
    e = tt.mp2_energy(B, eo.cuda(), ev.cuda())
    B_ref = cpu_ref.ao_to_mo_transform(eri, Co, Cv)
    assert normwise(B, B_ref) <= 1e-12
    assert rel(e, cpu_ref.mp2_energy(B_ref, eo, ev)) <= 1e-10


def test_config3_scale_full_transform(hip):
    """nbasis=512, naux=1536 (config 3) with nocc=64, nvir=320, against the two-step oracle."""
    g = torch.Generator().manual_seed(0)
    Co = torch.linalg.qr(torch.randn(512, 64, generator=g, dtype=torch.float64))[0].contiguous()
    Cv = torch.linalg.qr(torch.randn(512, 320, generator=g, dtype=torch.float64))[0].contiguous()
    eri = torch.randn(512, 512, 1536, generator=g, dtype=torch.float64) * 0.05
    got = tt.ao_to_mo_transform(eri.cuda(), Co.cuda(), Cv.cuda())
    ref = cpu_ref.ao_to_mo_two_step(eri, Co, Cv)
    assert normwise(got, ref) <= 1e-12


def test_shape_errors_match_reference(hip):
    eri, Co, Cv = torch.randn(6, 6, 8), torch.randn(6, 2), torch.randn(6, 3)
    with pytest.raises(ValueError, match="must be 3D"):
        tt.ao_to_mo_transform(torch.randn(6, 6), Co, Cv)
    with pytest.raises(ValueError, match="first two dims must match"):
        tt.ao_to_mo_transform(torch.randn(6, 7, 8), Co, Cv)
    with pytest.raises(ValueError, match="C_occ"):
        tt.ao_to_mo_transform(eri, torch.randn(5, 2), Cv)
    with pytest.raises(ValueError, match="C_vir"):
        tt.ao_to_mo_transform(eri, Co, torch.randn(7, 3))
