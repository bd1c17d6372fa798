"""The reference-side ctypes stubs of the integration guide run as written:
the guide's python block that defines them is executed with the library path
pointed at the in-tree build, and each stub is checked against the oracle."""

import os
import re

import pytest
import torch

from oracle import cpu_ref
from tests.util import normwise, rel
from trntensor_amd.hip import _lib

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def stubs():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```python\n(.*?)```", text, re.S)
    block = next(b for b in blocks if "def nki_matmul" in b)
    assert 'ctypes.CDLL("libtrntensor_hip.so")' in block
    ns: dict = {}
    exec(compile(block.replace('"libtrntensor_hip.so"', repr(_lib.LIB_PATH)), "INTEGRATION.md", "exec"), ns)
    return ns


def test_nki_matmul_stub(hip, stubs):
    g = torch.Generator().manual_seed(0)
    A, B = torch.randn(130, 70, generator=g, dtype=torch.float64), torch.randn(70, 90, generator=g, dtype=torch.float64)
    got = stubs["nki_matmul"](A, B)
    assert got.device.type == "cpu" and normwise(got, A @ B) <= 1e-12


def test_nki_batched_matmul_stub(hip, stubs):
    g = torch.Generator().manual_seed(1)
    A, B = torch.randn(3, 40, 50, generator=g), torch.randn(3, 50, 60, generator=g)
    assert normwise(stubs["nki_batched_matmul"](A, B), torch.bmm(A, B)) <= 1e-5


def test_nki_mp2_energy_stub(hip, stubs):
    g = torch.Generator().manual_seed(2)
    B = torch.randn(5, 70, 48, generator=g, dtype=torch.float64) * 0.1
    eo = torch.sort(-20 + 19.7 * torch.rand(5, generator=g, dtype=torch.float64))[0]
    ev = torch.sort(0.1 + 4.9 * torch.rand(70, generator=g, dtype=torch.float64))[0]
    assert rel(stubs["_nki_mp2_energy"](B, eo, ev), cpu_ref.mp2_energy(B, eo, ev)) <= 1e-10


def test_nki_ao_to_mo_transform_stub(hip, stubs):
    g = torch.Generator().manual_seed(3)
    eri = torch.randn(40, 40, 24, generator=g, dtype=torch.float64)
    co, cv = torch.randn(40, 6, generator=g, dtype=torch.float64), torch.randn(40, 15, generator=g, dtype=torch.float64)
    got = stubs["_nki_ao_to_mo_transform"](eri, co, cv)
    assert normwise(got, cpu_ref.ao_to_mo_two_step(eri, co, cv)) <= 1e-12
