"""precision="dd": double-double accumulation on the GPU (tt_gemm / tt_strided_contract
with dtype TT_F64_DD).

The reference declares precision="dd" but raises NotImplementedError
(trntensor/einsum.py:112-116), so there is no reference result: the oracle is
exact rational arithmetic (oracle/brute.einsum_exact) rounded once to float64,
and the bar is the published error bound of the Dot2 algorithm the kernels
implement (Ogita, Rump & Oishi 2005, Prop. 5.5):
    |res - exact| <= u |exact| + gamma_n^2 sum|term|,  u = 2^-53,
    gamma_n = n u / (1 - n u),
plus one rounding of alpha * res and one of + beta * C where those apply.
Ill-conditioned inputs (condition numbers 1e18-1e22, where float64
accumulation returns no correct digit) show the bound is met by the kernels,
not by easy data.
"""

import numpy as np
import pytest
import torch

import trntensor_amd as trntensor
from oracle import brute

pytestmark = pytest.mark.gpu

U = 2.0**-53


def gamma(n):
    return n * U / (1 - n * U)


def check_bound(got, exact, scale, n, alpha=1.0, extra=None):
    """got (tensor) against the exact result under the Dot2 bound."""
    got = got.detach().cpu().double().numpy()
    bound = abs(alpha) * (U * np.abs(exact) + gamma(n) ** 2 * scale)
    if alpha != 1.0:
        bound = bound + U * np.abs(alpha * exact)
    if extra is not None:
        bound = bound + extra
    err = np.abs(got - alpha * exact)
    assert np.all(err <= bound + 1e-300), float(np.max(err - bound))


def rand(gen, *shape, dt=torch.float64):
    return torch.randn(*shape, generator=gen, dtype=torch.float64).to(dt)


class TestGemm:
    @pytest.mark.parametrize(
        "sub,ashape,bshape",
        [
            ("ij,jk->ik", (37, 70), (70, 29)),
            ("ji,jk->ik", (70, 37), (70, 29)),
            ("ij,kj->ik", (37, 70), (29, 70)),
            ("ji,kj->ik", (70, 37), (29, 70)),
            ("ij,jk->ik", (65, 17), (17, 66)),  # edges in both tile dimensions
        ],
    )
    def test_layouts_vs_exact(self, hip, sub, ashape, bshape):
        gen = torch.Generator().manual_seed(len(sub) + ashape[0])
        A, B = rand(gen, *ashape), rand(gen, *bshape)
        got = trntensor.einsum(sub, A.cuda(), B.cuda(), precision="dd")
        exact, scale, n = brute.einsum_exact(sub, A.numpy(), B.numpy())
        assert got.dtype == torch.float64
        check_bound(got, exact, scale, n)

    def test_batched(self, hip):
        gen = torch.Generator().manual_seed(5)
        A, B = rand(gen, 3, 20, 33), rand(gen, 3, 33, 18)
        got = trntensor.einsum("bij,bjk->bik", A.cuda(), B.cuda(), precision="dd")
        exact, scale, n = brute.einsum_exact("bij,bjk->bik", A.numpy(), B.numpy())
        check_bound(got, exact, scale, n)

    def test_ill_conditioned_rows(self, hip):
        """Rows of A against columns of B built to cancel (condition ~1e20):
        float64 MFMA loses every digit, double-double meets the bound."""
        rng = np.random.default_rng(3)
        K, R = 200, 6
        xs, ys = zip(*[brute.ill_conditioned_dot(K, 20, rng) for _ in range(R)])
        A = torch.tensor(np.stack(xs))  # (R, K)
        B = torch.tensor(np.stack(ys)).T.contiguous()  # (K, R)
        exact, scale, n = brute.einsum_exact("ij,jk->ik", A.numpy(), B.numpy())
        dd = trntensor.einsum("ij,jk->ik", A.cuda(), B.cuda(), precision="dd")
        check_bound(dd, exact, scale, n)
        fast = trntensor.einsum("ij,jk->ik", A.cuda(), B.cuda()).cpu().numpy()
        diag = np.arange(R)
        rel_fast = np.abs(fast[diag, diag] - exact[diag, diag]) / np.abs(exact[diag, diag])
        rel_dd = np.abs(dd.cpu().numpy()[diag, diag] - exact[diag, diag]) / np.abs(exact[diag, diag])
        assert np.max(rel_fast) > 1e-3  # the data really defeats float64 accumulation
        assert np.max(rel_dd) < 1e-6

    def test_alpha_beta_out(self, hip):
        gen = torch.Generator().manual_seed(9)
        A, B, C = rand(gen, 30, 41), rand(gen, 41, 22), rand(gen, 30, 22)
        got = trntensor.einsum("ij,jk->ik", A.cuda(), B.cuda(), alpha=1.5, beta=-0.25, out=C.cuda(), precision="dd")
        exact, scale, n = brute.einsum_exact("ij,jk->ik", A.numpy(), B.numpy())
        want = 1.5 * exact - 0.25 * C.numpy()
        err = np.abs(got.cpu().numpy() - want)
        bound = 1.5 * (U * np.abs(exact) + gamma(n) ** 2 * scale) + 2 * U * (np.abs(1.5 * exact) + np.abs(want))
        assert np.all(err <= bound)

    def test_d_aliases_c(self, hip):
        """D may alias C exactly (header contract): all of a thread's C values
        are read before its first store, so D = alpha * AB + beta * D holds."""
        from trntensor_amd.hip import engine

        gen = torch.Generator().manual_seed(11)
        A, B, C = rand(gen, 70, 45), rand(gen, 45, 66), rand(gen, 70, 66)
        Cd = C.cuda()
        with engine.accumulation("dd"):
            engine.gemm(False, False, 70, 66, 45, A.cuda(), 45, 0, B.cuda(), 66, 0, Cd, 66, 0, 1, 1.5, -0.25, Cd, 66, 0)
        torch.cuda.synchronize()
        exact, scale, n = brute.einsum_exact("ij,jk->ik", A.numpy(), B.numpy())
        want = 1.5 * exact - 0.25 * C.numpy()
        err = np.abs(Cd.cpu().numpy() - want)
        bound = 1.5 * (U * np.abs(exact) + gamma(n) ** 2 * scale) + 2 * U * (np.abs(1.5 * exact) + np.abs(want))
        assert np.all(err <= bound)

    def test_float32_operands(self, hip):
        """float32 inputs: exact products of their float64 values, result rounded
        to float64 and then to float32 (within one float32 ulp of the exact value)."""
        gen = torch.Generator().manual_seed(11)
        A, B = rand(gen, 25, 60, dt=torch.float32), rand(gen, 60, 19, dt=torch.float32)
        got = trntensor.einsum("ij,jk->ik", A.cuda(), B.cuda(), precision="dd")
        assert got.dtype == torch.float32
        exact, _, _ = brute.einsum_exact("ij,jk->ik", A.double().numpy(), B.double().numpy())
        ulp32 = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
        assert np.all(np.abs(got.cpu().double().numpy() - exact) <= ulp32)

    def test_long_k_not_split(self, hip):
        """M x N = 4 x 4 with K = 20000 would be K-split on the float64 path;
        under dd it runs unsplit (one rounding): meets the bound on
        ill-conditioned rows where split partials rounded to float64 would not."""
        rng = np.random.default_rng(21)
        K, R = 20000, 4
        xs, ys = zip(*[brute.ill_conditioned_dot(K, 18, rng) for _ in range(R)])
        A = torch.tensor(np.stack(xs))
        B = torch.tensor(np.stack(ys))  # (R, K): 'ik,jk->ij'
        exact = np.array([[float(sum_exact(xs[i], ys[j])) for j in range(R)] for i in range(R)])
        scale = np.abs(np.stack(xs)) @ np.abs(np.stack(ys)).T
        dd = trntensor.einsum("ik,jk->ij", A.cuda(), B.cuda(), precision="dd")
        # scale is itself rounded (relative 1e-12 is ample for the bound's second term)
        check_bound(dd, exact, scale * (1 + 1e-12), K)
        diag = np.arange(R)
        assert np.max(np.abs(dd.cpu().numpy()[diag, diag] - exact[diag, diag]) / np.abs(exact[diag, diag])) < 1e-6

    def test_large_agrees_with_float64(self, hip):
        """1024^3: dd and the float64 MFMA GEMM agree to float64 accuracy on
        well-conditioned data (a size-independent sanity check)."""
        gen = torch.Generator().manual_seed(2)
        A, B = rand(gen, 1024, 1024).cuda(), rand(gen, 1024, 1024).cuda()
        dd = trntensor.einsum("ij,jk->ik", A, B, precision="dd")
        f64 = trntensor.einsum("ij,jk->ik", A, B)
        assert float((dd - f64).norm() / f64.norm()) < 1e-14


def sum_exact(x, y):
    from fractions import Fraction

    return sum((Fraction(float(a)) * Fraction(float(b)) for a, b in zip(x, y)), Fraction(0))


class TestStrided:
    def test_ill_conditioned_dot(self, hip):
        """'i,i->' with n = 20000: one output, many workgroups (per-block
        schedule, partial pairs merged in a second kernel)."""
        rng = np.random.default_rng(1)
        x, y = brute.ill_conditioned_dot(20000, 22, rng)
        exact = float(sum_exact(x, y))
        scale = float(np.sum(np.abs(x * y)))
        got = trntensor.einsum("i,i->", torch.tensor(x).cuda(), torch.tensor(y).cuda(), precision="dd")
        check_bound(got, np.array(exact), np.array(scale * (1 + 1e-12)), 20000)
        assert abs(float(got) - exact) / abs(exact) < 1e-6

    def test_outer_and_trace(self, hip):
        gen = torch.Generator().manual_seed(4)
        a, b = rand(gen, 13), rand(gen, 17)
        got = trntensor.einsum("i,j->ij", a.cuda(), b.cuda(), precision="dd")
        assert torch.equal(got.cpu(), torch.outer(a, b))  # one exact product, rounded once
        M = rand(gen, 300, 300)
        tr = trntensor.einsum("ii->", M.cuda(), precision="dd")
        exact, scale, n = brute.einsum_exact("ii->", M.numpy())
        check_bound(tr, exact, scale, n)

    def test_sum_with_cancellation(self, hip):
        """'ij->i' rows like [1e16, 1, -1e16, 1]: summed left to right in float64
        the small terms vanish; double-double keeps them in any order."""
        rows = torch.tensor([[1e16, 1.0, -1e16, 1.0] * 64, [3.0, 1e-17, -3.0, 1e-17] * 64], dtype=torch.float64)
        got = trntensor.einsum("ij->i", rows.cuda(), precision="dd")
        exact, scale, n = brute.einsum_exact("ij->i", rows.numpy())
        check_bound(got, exact, scale, n)
        assert np.all(np.abs(got.cpu().numpy() - exact) <= 1e-6 * np.abs(exact))

    def test_path(self, hip):
        """Three operands: each pairwise step accumulates in double-double and
        rounds once, so on well-conditioned data the result is within a few
        float64 ulps of the exact one."""
        gen = torch.Generator().manual_seed(6)
        ops = [rand(gen, 9, 14), rand(gen, 14, 11), rand(gen, 11, 7)]
        got = trntensor.einsum("ij,jk,kl->il", *[o.cuda() for o in ops], precision="dd")
        exact, scale, _ = brute.einsum_exact("ij,jk,kl->il", *[o.numpy() for o in ops])
        assert np.all(np.abs(got.cpu().numpy() - exact) <= 64 * U * scale)
