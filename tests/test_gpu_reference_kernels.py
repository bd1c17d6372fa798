"""The reference's on-hardware kernel tests (tests/test_nki_kernels.py:35-376),
run on the HIP kernels with the same shapes, seeds and assertions.

The reference checks its NKI kernels against torch on the CPU with
atol=1e-3, rtol=1e-4 (fp32). Those assertions are kept verbatim, and each
case is also held to this build's bar: normwise 1e-5 in fp32 against the
float64 product of the same inputs, and MP2 energies within 1e-5 relative of
the reference CPU loop (oracle/cpu_ref.mp2_energy). The reference's
size-limit test (test_oversize_raises) becomes a test that the same shape
computes, since these kernels have no nvir/naux <= 128 limit.
"""


import pytest
import torch

import trntensor_amd as trntensor
from oracle import cpu_ref
from tests.util import normwise, rel

pytestmark = pytest.mark.gpu

ATOL = 1e-3
RTOL = 1e-4


def check(out, ref, exact):
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)
    assert normwise(out.double(), exact) <= 1e-5


class TestHipMatmul:
    def test_aligned_shapes(self, hip):
        torch.manual_seed(0)
        A = torch.randn(128, 128)
        B = torch.randn(128, 256)
        check(trntensor.einsum("ij,jk->ik", A, B), A @ B, A.double() @ B.double())

    def test_unpadded_K_and_N(self, hip):
        torch.manual_seed(1)
        A = torch.randn(100, 70)
        B = torch.randn(70, 200)
        check(trntensor.einsum("ij,jk->ik", A, B), A @ B, A.double() @ B.double())

    def test_transA(self, hip):
        torch.manual_seed(2)
        A = torch.randn(128, 64)
        B = torch.randn(128, 256)
        check(trntensor.einsum("ji,jk->ik", A, B), A.T @ B, A.double().T @ B.double())

    def test_both_transposed(self, hip):
        torch.manual_seed(3)
        A = torch.randn(128, 64)
        B = torch.randn(256, 128)
        check(trntensor.einsum("ji,kj->ik", A, B), A.T @ B.T, A.double().T @ B.double().T)

    def test_large_N_requires_n_tiling(self, hip):
        torch.manual_seed(4)
        A = torch.randn(128, 128)
        B = torch.randn(128, 1024)
        check(trntensor.einsum("ij,jk->ik", A, B), A @ B, A.double() @ B.double())

    def test_df_mp2_pair_pattern(self, hip):
        torch.manual_seed(5)
        nvir, naux = 19, 72
        Bi = torch.randn(nvir, naux)
        Bj = torch.randn(nvir, naux)
        check(trntensor.einsum("ap,bp->ab", Bi, Bj), Bi @ Bj.T, Bi.double() @ Bj.double().T)


class TestHipBatchedMatmul:
    def test_aligned_batch(self, hip):
        torch.manual_seed(10)
        A = torch.randn(4, 128, 128)
        B = torch.randn(4, 128, 256)
        check(trntensor.einsum("bij,bjk->bik", A, B), torch.bmm(A, B), torch.bmm(A.double(), B.double()))

    def test_unpadded_inner(self, hip):
        torch.manual_seed(11)
        A = torch.randn(3, 100, 70)
        B = torch.randn(3, 70, 200)
        check(trntensor.einsum("bij,bjk->bik", A, B), torch.bmm(A, B), torch.bmm(A.double(), B.double()))

    def test_large_N(self, hip):
        torch.manual_seed(12)
        A = torch.randn(2, 128, 128)
        B = torch.randn(2, 128, 1024)
        check(trntensor.einsum("bij,bjk->bik", A, B), torch.bmm(A, B), torch.bmm(A.double(), B.double()))


def _orbital_energies(nocc, nvir):
    eps_occ = -torch.sort(torch.rand(nocc))[0] - 0.5
    eps_vir = torch.sort(torch.rand(nvir))[0] + 0.1
    return eps_occ, eps_vir


class TestMp2Energy:
    def test_demo_shape(self, hip):
        torch.manual_seed(42)
        nocc, nvir, naux = 5, 19, 72
        B = torch.randn(nocc, nvir, naux) * 0.1
        eps_occ, eps_vir = _orbital_energies(nocc, nvir)
        e = trntensor.mp2_energy(B, eps_occ, eps_vir)
        e_ref = cpu_ref.mp2_energy(B, eps_occ, eps_vir)
        torch.testing.assert_close(e, e_ref, atol=1e-3, rtol=1e-4)
        assert rel(e, e_ref) <= 1e-5

    def test_medium_shape(self, hip):
        torch.manual_seed(43)
        nocc, nvir, naux = 8, 32, 128
        B = torch.randn(nocc, nvir, naux) * 0.1
        eps_occ, eps_vir = _orbital_energies(nocc, nvir)
        e = trntensor.mp2_energy(B, eps_occ, eps_vir)
        e_ref = cpu_ref.mp2_energy(B, eps_occ, eps_vir)
        torch.testing.assert_close(e, e_ref, atol=1e-3, rtol=1e-4)
        assert rel(e, e_ref) <= 1e-5

    def test_ao_to_mo_transform_composes(self, hip):
        torch.manual_seed(42)
        nbasis, nocc, nvir, naux = 32, 5, 10, 16
        eri = torch.randn(nbasis, nbasis, naux) * 0.1
        C_occ = torch.randn(nbasis, nocc)
        C_vir = torch.randn(nbasis, nvir)
        eps_occ, eps_vir = _orbital_energies(nocc, nvir)
        B = trntensor.ao_to_mo_transform(eri, C_occ, C_vir)
        B_ref = torch.einsum("mi,na,mnP->iaP", C_occ, C_vir, eri)
        check(B, B_ref, torch.einsum("mi,na,mnP->iaP", C_occ.double(), C_vir.double(), eri.double()))
        e = trntensor.mp2_energy(B, eps_occ, eps_vir)
        e_ref = cpu_ref.mp2_energy(B_ref, eps_occ, eps_vir)
        torch.testing.assert_close(e, e_ref, atol=1e-3, rtol=1e-4)


class TestAoToMoTransformKTiling:
    def _case(self, seed, nbasis, nocc, nvir, naux):
        torch.manual_seed(seed)
        eri = torch.randn(nbasis, nbasis, naux) * 0.1
        C_occ = torch.randn(nbasis, nocc)
        C_vir = torch.randn(nbasis, nvir)
        B = trntensor.ao_to_mo_transform(eri, C_occ, C_vir)
        B_ref = torch.einsum("mi,na,mnP->iaP", C_occ, C_vir, eri)
        check(B, B_ref, torch.einsum("mi,na,mnP->iaP", C_occ.double(), C_vir.double(), eri.double()))
        return B, B_ref

    def test_nbasis_256_single_tile_k(self, hip):
        self._case(50, 256, 16, 32, 32)

    def test_nbasis_non_multiple_pads_correctly(self, hip):
        self._case(51, 200, 10, 20, 24)

    def test_df_mp2_pipeline_cc_pvtz_shape(self, hip):
        B, B_ref = self._case(52, 256, 10, 30, 32)
        eps_occ, eps_vir = _orbital_energies(10, 30)
        e = trntensor.mp2_energy(B, eps_occ, eps_vir)
        e_ref = cpu_ref.mp2_energy(B_ref, eps_occ, eps_vir)
        torch.testing.assert_close(e, e_ref, atol=1e-3, rtol=1e-4)

    def test_oversize_computes(self, hip):
        """Reference: nvir > 128 raises NotImplementedError (test_oversize_raises).
        Here the same shape computes and matches the reference CPU loop."""
        torch.manual_seed(53)
        B = torch.randn(2, 200, 50) * 0.1
        eps_occ, eps_vir = _orbital_energies(2, 200)
        e = trntensor.mp2_energy(B, eps_occ, eps_vir)
        assert rel(e, cpu_ref.mp2_energy(B, eps_occ, eps_vir)) <= 1e-5


class TestResidency:
    def test_matmul_stays_on_device(self, hip):
        torch.manual_seed(0)
        A = trntensor.to_xla(torch.randn(128, 128))
        B = trntensor.to_xla(torch.randn(128, 256))
        out = trntensor.einsum("ij,jk->ik", A, B)
        assert out.device.type == "cuda", f"expected the HIP device, got {out.device}"
        out_cpu = trntensor.from_xla(out)
        ref = trntensor.from_xla(A) @ trntensor.from_xla(B)
        torch.testing.assert_close(out_cpu, ref, atol=ATOL, rtol=RTOL)

    def test_pipeline_composition(self, hip):
        """Skipped on the reference's trn1 (a compiler issue); runs here: every
        operand pre-pinned, the intermediate B never leaves the device."""
        torch.manual_seed(7)
        nbasis, nocc, nvir, naux = 32, 5, 10, 16
        eri = torch.randn(nbasis, nbasis, naux) * 0.1
        C_occ = torch.randn(nbasis, nocc)
        C_vir = torch.randn(nbasis, nvir)
        eps_occ, eps_vir = _orbital_energies(nocc, nvir)
        args = [trntensor.to_xla(t) for t in (eri, C_occ, C_vir, eps_occ, eps_vir)]
        B_x = trntensor.ao_to_mo_transform(*args[:3])
        assert B_x.device.type == "cuda"
        E = trntensor.from_xla(trntensor.mp2_energy(B_x, *args[3:]))
        B_ref = torch.einsum("mi,na,mnP->iaP", C_occ, C_vir, eri)
        E_ref = cpu_ref.mp2_energy(B_ref, eps_occ, eps_vir)
        torch.testing.assert_close(E, E_ref, atol=1e-3, rtol=1e-4)

    def test_residency(self, hip):
        """The reference's residency test (tests/test_nki_kernels.py) times
        host-operand calls against device-resident ones and asserts a 3x
        speedup. A wall-clock bar in the parity suite can fail on a loaded box
        with no numerical fault, so the timing is a bench field
        (c1_einsum_loop_fp32.residency_speedup_2048) and this test asserts what
        residency changes: where the result lives, and that its values do not."""
        torch.manual_seed(0)
        A = torch.randn(2048, 2048)
        B = torch.randn(2048, 2048)
        cold = trntensor.einsum("ij,jk->ik", A, B)
        assert cold.device.type == "cpu"
        A_x, B_x = trntensor.to_xla(A), trntensor.to_xla(B)
        hot = trntensor.einsum("ij,jk->ik", A_x, B_x)
        assert hot.device.type == "cuda"
        assert torch.equal(trntensor.from_xla(hot), cold)
        assert normwise(cold, cpu_ref.einsum("ij,jk->ik", A.double(), B.double()).float()) <= 1e-5
