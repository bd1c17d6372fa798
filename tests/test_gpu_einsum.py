"""GPU parity of trntensor_amd.einsum / multi_einsum against the CPU oracle.

The first classes port the reference's own einsum tests
(tests/test_einsum.py:10-342) onto the HIP path: same inputs, same
assertions, with the oracle (oracle/cpu_ref.py, the reference's CPU path
restated) as the expected value and normwise bars of 1e-12 (float64) /
1e-5 (float32). The config classes run BASELINE.json's shapes.
"""

import importlib

import numpy as np
import pytest
import torch

import trntensor_amd as trntensor
from oracle import brute, cpu_ref
from tests.util import normwise, rel

pytestmark = pytest.mark.gpu


def close(got, ref, dt=None):
    dt = dt or ref.dtype
    bar = 1e-12 if dt == torch.float64 else 1e-5
    assert got.dtype == ref.dtype, (got.dtype, ref.dtype)
    assert tuple(got.shape) == tuple(ref.shape)
    assert normwise(got, ref) <= bar


class TestEinsumReferenceCases:
    """tests/test_einsum.py:10-84 on the HIP path (CPU operands staged through the GPU)."""

    @pytest.mark.parametrize(
        "sub,shapes",
        [
            ("ij,jk->ik", [(4, 3), (3, 5)]),
            ("ji,jk->ik", [(3, 4), (3, 5)]),
            ("ij,kj->ik", [(4, 3), (5, 3)]),
            ("ji,kj->ik", [(3, 4), (5, 3)]),
            ("i,i->", [(10,), (10,)]),
            ("i,j->ij", [(3,), (4,)]),
            ("ii->", [(5, 5)]),
            ("bij,bjk->bik", [(8, 4, 3), (8, 3, 5)]),
            ("ap,bp->ab", [(5, 10), (5, 10)]),
            ("mi,mnP->inP", [(6, 2), (6, 6, 8)]),
            ("ijk,jkl->il", [(3, 4, 5), (4, 5, 6)]),
            ("ij,jk->ik", [(4, 1), (1, 5)]),
            ("ij,jk,kl->il", [(5, 8), (8, 6), (6, 4)]),
            ("ij,jk,kl,lm->im", [(3, 5), (5, 4), (4, 6), (6, 2)]),
            ("ij,ik,il->jkl", [(4, 3), (4, 5), (4, 2)]),
        ],
    )
    @pytest.mark.parametrize("dt", [torch.float32, torch.float64])
    def test_matches_oracle(self, hip, sub, shapes, dt):
        g = torch.Generator().manual_seed(len(sub))
        ops = [torch.randn(*s, generator=g, dtype=dt) for s in shapes]
        got = trntensor.einsum(sub, *ops)
        assert got.device.type == "cpu"
        close(got, cpu_ref.einsum(sub, *ops))

    def test_device_operands_stay_on_device(self, hip):
        A, B = torch.randn(64, 48, device="cuda"), torch.randn(48, 80, device="cuda")
        out = trntensor.einsum("ij,jk->ik", A, B)
        assert out.device.type == "cuda"
        close(out.cpu(), cpu_ref.einsum("ij,jk->ik", A.cpu(), B.cpu()))


class TestMisplannedPatterns:
    """Index orders the reference's matmul/bmm executors mishandle
    (trntensor/plan.py:284-305): the product computes the einsum itself."""

    @pytest.mark.parametrize(
        "sub,shapes",
        [
            ("ij,jk->ki", [(30, 20), (20, 40)]),
            ("ij,jk->i", [(30, 20), (20, 40)]),
            ("bji,bjk->bik", [(3, 20, 30), (3, 20, 40)]),
            ("iap,ibp->iab", [(3, 20, 30), (3, 25, 30)]),
            ("ibj,bjk->bik", [(20, 3, 30), (3, 30, 40)]),
        ],
    )
    def test_einsum_semantics(self, hip, sub, shapes):
        g = torch.Generator().manual_seed(7)
        ops = [torch.randn(*s, generator=g, dtype=torch.float64) for s in shapes]
        assert cpu_ref.misplanned_by_reference(sub, *ops)
        got = trntensor.einsum(sub, *ops)
        ref = torch.from_numpy(np.asarray(brute.einsum_f64(sub, *[o.numpy() for o in ops])))
        close(got, ref)


class TestRandomFrontEnd:
    """Random calls of the public einsum: one to three operands, letters
    repeated within a term (diagonals) and across terms, implicit and
    explicit outputs, extents 1-6, fp32 and fp64, non-contiguous views and
    CPU operands, alpha/beta with an `out` of the result's shape in the same
    or a wider dtype. Expected value: alpha * numpy's float64 einsum + beta *
    out (an implementation independent of the oracle's torch calls, so the
    patterns the reference's matmul/bmm executors mishandle are covered
    too). Bar per element: the recursive-summation bound
    gamma_(n+3) * (|alpha| einsum(|ops|) + |beta out|) for n terms per
    output, doubled per pairwise step of a path, plus one rounding of the
    result to its dtype; dtype and shape as result.add(out, alpha=beta)
    (trntensor/einsum.py:99-102)."""

    @staticmethod
    def _operand(rng, gen, shape, dt, on_cpu):
        x = torch.randn(*shape, generator=gen, dtype=torch.float64).to(dt)
        if len(shape) >= 2 and rng.random() < 0.3:
            perm = list(range(len(shape)))
            rng.shuffle(perm)
            inv = [perm.index(k) for k in range(len(shape))]
            x = x.permute(*perm).contiguous().permute(*inv)  # same values, non-contiguous strides
        return x if on_cpu else x.cuda()

    @pytest.mark.parametrize(
        "ncases,letters,lo,hi,seed",
        [(200, "abcde", 1, 6, 2024), (60, "abcd", 6, 40, 7)],
        ids=["small-extents", "gemm-sized"],
    )
    def test_random_calls(self, hip, ncases, letters, lo, hi, seed):
        import random

        rng = random.Random(seed)
        gen = torch.Generator().manual_seed(seed)
        for case in range(ncases):
            ext = {c: rng.randint(lo, hi) for c in letters}
            nops = rng.choice([1, 2, 2, 2, 3, 3])
            terms = ["".join(rng.choice(letters) for _ in range(rng.randint(1, 3))) for _ in range(nops)]
            seen = sorted(set("".join(terms)))
            if rng.random() < 0.2:
                sub = ",".join(terms)
            else:
                out_letters = "".join(c for c in rng.sample(seen, len(seen)) if rng.random() < 0.5)
                sub = ",".join(terms) + "->" + out_letters
            dt = rng.choice([torch.float32, torch.float64])
            on_cpu = rng.random() < 0.15  # CPU operands are staged through the GPU
            ops = [self._operand(rng, gen, [ext[c] for c in t], dt, on_cpu) for t in terms]
            ref = brute.einsum_f64(sub, *[o.cpu().numpy() for o in ops])
            scale = np.abs(brute.einsum_f64(sub, *[np.abs(o.cpu().numpy()) for o in ops]))
            kw = {}
            res_dt = dt
            out_part = np.zeros_like(ref)
            alpha = 1.0
            if rng.random() < 0.4:
                alpha = rng.choice([0.5, -1.25, 2.0])
                beta = rng.choice([0.0, 0.75, -0.5])
                out_dt = dt if rng.random() < 0.7 else torch.float64
                out = torch.randn(tuple(np.shape(ref)), generator=gen, dtype=torch.float64).to(out_dt)
                kw = dict(alpha=alpha, beta=beta, out=out.cuda() if ops[0].is_cuda else out)
                res_dt = torch.promote_types(dt, out_dt)
                out_part = beta * out.double().numpy()
            print(f"random case {case}: {sub} {dt} {kw.get('alpha', 1.0)} {kw.get('beta', 0.0)}", flush=True)
            got = trntensor.einsum(sub, *ops, **kw)
            assert got.dtype == res_dt and tuple(got.shape) == tuple(np.shape(ref)), (sub, got.dtype, got.shape)
            want = alpha * ref + out_part
            out_str = cpu_ref.parse_subscripts(sub)[1]
            n_terms = int(np.prod([ext[c] for c in set("".join(terms)) if c not in out_str]))
            u = 2.0**-53 if dt == torch.float64 else 2.0**-24
            steps = max(1, nops - 1)
            bar = 2**steps * (n_terms + 3) * u / (1 - (n_terms + 3) * u) * (abs(alpha) * scale + np.abs(out_part))
            bar = bar + (2.0**-53 if res_dt == torch.float64 else 2.0**-24) * np.abs(want) + 1e-300
            err = np.abs(got.cpu().double().numpy() - want)
            assert np.all(err <= bar), (case, sub, dt, float(np.max(err / bar)))


class TestMultiEinsum:
    """tests/test_einsum.py:87-150."""

    def test_multiple_and_shared(self, hip):
        g = torch.Generator().manual_seed(1)
        A, B, C = (torch.randn(*s, generator=g) for s in [(4, 3), (3, 5), (5, 2)])
        r = trntensor.multi_einsum(("ij,jk->ik", A, B), ("ij,jk->ik", B, C), ("ij,jk,kl->il", A, B, C), ("ij,ij->", A, A))
        assert len(r) == 4 and all(x.device.type == "cpu" for x in r)
        close(r[0], A @ B)
        close(r[1], B @ C)
        close(r[2], cpu_ref.einsum("ij,jk,kl->il", A, B, C))
        close(r[3], cpu_ref.einsum("ij,ij->", A, A))

    def test_shared_operand_views(self, hip):
        g = torch.Generator().manual_seed(2)
        Bt = torch.randn(3, 5, 8, generator=g)
        r = trntensor.multi_einsum(("ap,bp->ab", Bt[0], Bt[1]), ("ap,bp->ab", Bt[1], Bt[0]))
        close(r[0], cpu_ref.einsum("ap,bp->ab", Bt[0], Bt[1]))
        close(r[1], cpu_ref.einsum("ap,bp->ab", Bt[1], Bt[0]))


class TestAlphaBetaDtypePrecision:
    """tests/test_einsum.py:216-342."""

    @pytest.mark.parametrize("alpha,beta", [(2.0, 0.0), (1.0, 0.5), (2.0, 0.5), (1.5, 0.5)])
    @pytest.mark.parametrize("dt", [torch.float32, torch.float64])
    def test_alpha_beta(self, hip, alpha, beta, dt):
        g = torch.Generator().manual_seed(3)
        A, B, C = (torch.randn(*s, generator=g, dtype=dt) for s in [(40, 30), (30, 50), (40, 50)])
        got = trntensor.einsum("ij,jk->ik", A, B, alpha=alpha, beta=beta, out=C)
        close(got, cpu_ref.einsum("ij,jk->ik", A, B, alpha=alpha, beta=beta, out=C))
        assert torch.equal(C, C.clone())  # out is read, not written

    def test_alpha_beta_through_permute_and_path(self, hip):
        g = torch.Generator().manual_seed(4)
        A, B, C = (torch.randn(*s, generator=g, dtype=torch.float64) for s in [(20, 30), (30, 40), (40, 20)])
        close(trntensor.einsum("ij,jk->ki", A, B, alpha=1.5, beta=0.5, out=C), 1.5 * (A @ B).T + 0.5 * C)
        D = torch.randn(40, 7, generator=g, dtype=torch.float64)
        O = torch.randn(20, 7, generator=g, dtype=torch.float64)
        close(trntensor.einsum("ij,jk,kl->il", A, B, D, alpha=-2.0, beta=3.0, out=O), -2.0 * (A @ B @ D) + 3.0 * O)

    @pytest.mark.parametrize("name,dt", [("bf16", torch.bfloat16), ("fp16", torch.float16), ("f64", torch.float64)])
    def test_dtype_strings(self, hip, name, dt):
        torch.manual_seed(0)
        A, B = torch.randn(8, 6), torch.randn(6, 10)
        got = trntensor.einsum("ij,jk->ik", A, B, dtype=name)
        assert got.dtype == dt
        np.testing.assert_allclose(got.float().numpy(), (A @ B).numpy(), atol=0.05)

    def test_dtype_invalid_raises(self, hip):
        with pytest.raises(ValueError, match="unknown dtype"):
            trntensor.einsum("ij,jk->ik", torch.randn(4, 3), torch.randn(3, 5), dtype="foo")

    def test_kahan(self, hip):
        torch.manual_seed(42)
        large = torch.full((1, 512), 1e6)
        small = torch.randn(512, 1) * 1e-3
        ref = torch.einsum("ij,jk->ik", large.double(), small.double()).float()
        fast = trntensor.einsum("ij,jk->ik", large, small, precision="fast")
        kahan = trntensor.einsum("ij,jk->ik", large, small, precision="kahan")
        assert kahan.dtype == torch.float32
        assert abs(float(kahan) - float(ref)) <= abs(float(fast) - float(ref)) + 1e-3

    @pytest.mark.parametrize("sub,shapes", [("ij,jk->ik", [(4096, 4096), (4096, 4096)]),
                                            ("bij,bjk->bik", [(64, 512, 512), (64, 512, 512)])])
    def test_kahan_config2_scale(self, hip, sub, shapes):
        """precision="kahan" on config-2 float32 operands: float64 contraction on
        the device, rounded once to float32, against the oracle's kahan branch
        (float64 torch on the CPU, cast once)."""
        g = torch.Generator().manual_seed(0)
        A, B = (torch.randn(*s, generator=g, dtype=torch.float64).float() for s in shapes)
        got = trntensor.einsum(sub, A.cuda(), B.cuda(), precision="kahan")
        ref = cpu_ref.einsum(sub, A, B, precision="kahan")
        assert got.dtype == ref.dtype == torch.float32
        assert normwise(got, ref) <= 2e-7
        fast = cpu_ref.einsum(sub, A, B)
        print(f"kahan {sub}: normwise vs oracle {normwise(got, ref):.2e}; fp32 CPU path {normwise(fast, ref):.2e}")

    def test_dd_computes(self, hip):
        """The reference raises NotImplementedError for precision='dd'
        (tests/test_einsum.py:328-333); this build computes it (double-double
        accumulation, tests/test_gpu_dd.py) and returns the first operand's dtype."""
        A, B = torch.randn(4, 3), torch.randn(3, 5)
        got = trntensor.einsum("ij,jk->ik", A, B, precision="dd")
        assert got.dtype == torch.float32 and got.device.type == "cpu"
        close(got, (A.double() @ B.double()).float())

    def test_fast_equals_default(self, hip):
        torch.manual_seed(0)
        A, B = torch.randn(8, 6), torch.randn(6, 10)
        assert torch.equal(trntensor.einsum("ij,jk->ik", A, B), trntensor.einsum("ij,jk->ik", A, B, precision="fast"))


class TestOutPromotionBroadcast:
    """`out` of another dtype or shape: the reference returns
    result.add(out, alpha=beta) (trntensor/einsum.py:101-102), so the result
    takes torch's promoted dtype and broadcast shape. Checked against the
    oracle (the same add) for dtype, shape and value; the value bar is that
    of the contraction's own dtype, whose rounding the reference keeps."""

    @staticmethod
    def check(sub, shapes, dt, out_shape, out_dt, alpha=1.5, beta=0.5, device="cuda", seed=11):
        g = torch.Generator().manual_seed(seed)
        ops = [torch.randn(*s, generator=g, dtype=torch.float64).to(dt) for s in shapes]
        out = torch.randn(*out_shape, generator=g, dtype=torch.float64).to(out_dt)
        ref = cpu_ref.einsum(sub, *ops, alpha=alpha, beta=beta, out=out)
        got = trntensor.einsum(sub, *[o.to(device) for o in ops], alpha=alpha, beta=beta, out=out.to(device))
        assert got.dtype == ref.dtype, (got.dtype, ref.dtype)
        assert tuple(got.shape) == tuple(ref.shape), (tuple(got.shape), tuple(ref.shape))
        assert got.device.type == torch.device(device).type
        bar = {torch.float64: 1e-12, torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-3}[dt]
        assert normwise(got.float() if got.dtype in (torch.bfloat16, torch.float16) else got, ref.to(got.dtype)) <= bar

    def test_fp32_operands_fp64_out(self, hip):
        self.check("ij,jk->ik", [(70, 50), (50, 90)], torch.float32, (70, 90), torch.float64)

    def test_fp64_operands_fp32_out(self, hip):
        # promotes to the contraction's dtype: fused epilogue, float64 result
        self.check("ij,jk->ik", [(70, 50), (50, 90)], torch.float64, (70, 90), torch.float32)

    def test_fp32_bmm_fp64_out_cpu_operands(self, hip):
        self.check("bij,bjk->bik", [(3, 40, 30), (3, 30, 20)], torch.float32, (3, 40, 20), torch.float64, device="cpu")

    def test_out_broadcasts_into_result(self, hip):
        self.check("ij,jk->ik", [(33, 17), (17, 45)], torch.float64, (1, 45), torch.float64)
        self.check("ij,jk->ik", [(33, 17), (17, 45)], torch.float32, (45,), torch.float32)

    def test_out_larger_than_result(self, hip):
        self.check("ij,jk->ik", [(33, 17), (17, 45)], torch.float64, (4, 33, 45), torch.float64)
        self.check("ij,jk->ik", [(33, 17), (17, 45)], torch.float32, (2, 33, 1), torch.float64)

    def test_scalar_result_vector_out(self, hip):
        self.check("i,i->", [(300,), (300,)], torch.float64, (5,), torch.float64)
        self.check("ij,jk,kl->", [(6, 7), (7, 8), (8, 9)], torch.float32, (3, 1), torch.float64)

    def test_path_fp32_operands_fp64_out(self, hip):
        self.check("ij,jk,kl->il", [(20, 30), (30, 40), (40, 10)], torch.float32, (20, 10), torch.float64)

    def test_bf16_operands_fp32_out(self, hip):
        self.check("ij,jk->ik", [(64, 64), (64, 96)], torch.bfloat16, (64, 96), torch.float32, alpha=1.0)

    def test_kahan_fp32_with_fp64_out(self, hip):
        g = torch.Generator().manual_seed(12)
        A, B = (torch.randn(*s, generator=g) for s in [(30, 40), (40, 20)])
        out = torch.randn(30, 20, generator=g, dtype=torch.float64)
        ref = cpu_ref.einsum("ij,jk->ik", A, B, alpha=2.0, beta=0.25, out=out, precision="kahan")
        got = trntensor.einsum("ij,jk->ik", A.cuda(), B.cuda(), alpha=2.0, beta=0.25, out=out.cuda(), precision="kahan")
        assert got.dtype == ref.dtype == torch.float64
        assert normwise(got, ref) <= 1e-7

    def test_unbroadcastable_out_raises(self, hip):
        A, B = torch.randn(4, 3), torch.randn(3, 5)
        with pytest.raises(RuntimeError):
            trntensor.einsum("ij,jk->ik", A, B, beta=1.0, out=torch.randn(4, 4))
        with pytest.raises(RuntimeError):
            cpu_ref.einsum("ij,jk->ik", A, B, beta=1.0, out=torch.randn(4, 4))

    def test_out_not_written(self, hip):
        out = torch.randn(2, 8, 6, dtype=torch.float64, device="cuda")
        keep = out.clone()
        trntensor.einsum("ij,jk->ik", torch.randn(8, 5, device="cuda"), torch.randn(5, 6, device="cuda"), beta=2.0, out=out)
        assert torch.equal(out, keep)


class TestBackendOnDevice:
    def test_plan_backend_is_hip(self, hip):
        trntensor.clear_plan_cache()
        for sub, shapes in [("ij,jk->ik", [(2048, 2048), (2048, 2048)]), ("ij,jk->ik", [(4, 3), (3, 5)]), ("ij,jk,kl->il", [(3, 4), (4, 5), (5, 2)])]:
            p = trntensor.plan_contraction(sub, *[torch.empty(s) for s in shapes])
            assert p.backend == "hip"

    def test_pytorch_backend_refuses_to_compute(self, hip):
        trntensor.set_backend("pytorch")
        try:
            with pytest.raises(RuntimeError, match="HIP kernels"):
                trntensor.einsum("ij,jk->ik", torch.randn(4, 3), torch.randn(3, 5))
        finally:
            trntensor.set_backend("auto")

    def test_to_device_roundtrip(self, hip):
        t = torch.randn(3, 4)
        d = trntensor.to_xla(t)
        assert d.device.type == "cuda"
        assert trntensor.from_xla(d).equal(t)


# ---------------------------------------------------------------------------
# BASELINE.json configurations
# ---------------------------------------------------------------------------
class TestConfig1:
    def test_df_mp2_einsum_loop(self, hip):
        """examples/df_mp2_einsum.py:25-46 at config 1 (fp32, seed 0) with trntensor_amd.einsum."""
        g = torch.Generator().manual_seed(0)
        B = torch.randn(8, 32, 96, generator=g) * 0.1
        eo = torch.sort(-20 + 19.7 * torch.rand(8, generator=g))[0]
        ev = torch.sort(0.1 + 4.9 * torch.rand(32, generator=g))[0]
        e = 0.0
        for i in range(8):
            for j in range(8):
                T = trntensor.einsum("ap,bp->ab", B[i], B[j])
                denom = eo[i] + eo[j] - ev.unsqueeze(1) - ev.unsqueeze(0)
                e += (T * (2 * T - T.T) / denom).sum().item()
        ref = cpu_ref.df_mp2_einsum_loop(B, eo, ev)
        assert rel(e, ref) <= 1e-5
        assert rel(trntensor.mp2_energy(B, eo, ev), ref) <= 1e-5


class TestConfig2:
    @pytest.mark.parametrize("dt", [torch.float32, torch.float64])
    def test_gemm_4096(self, hip, dt):
        g = torch.Generator().manual_seed(0)
        A, B, C = (torch.randn(4096, 4096, generator=g, dtype=torch.float64).to(dt) for _ in range(3))
        got = trntensor.einsum("ij,jk->ik", A.cuda(), B.cuda(), alpha=1.5, beta=0.5, out=C.cuda())
        close(got.cpu(), cpu_ref.einsum("ij,jk->ik", A, B, alpha=1.5, beta=0.5, out=C))

    @pytest.mark.parametrize("dt", [torch.float32, torch.float64])
    def test_bmm_64x512(self, hip, dt):
        g = torch.Generator().manual_seed(0)
        A, B, C = (torch.randn(64, 512, 512, generator=g, dtype=torch.float64).to(dt) for _ in range(3))
        got = trntensor.einsum("bij,bjk->bik", A.cuda(), B.cuda(), alpha=1.5, beta=0.5, out=C.cuda())
        close(got.cpu(), cpu_ref.einsum("bij,bjk->bik", A, B, alpha=1.5, beta=0.5, out=C))


def config3_inputs():
    g = torch.Generator().manual_seed(0)
    C = torch.linalg.qr(torch.randn(512, 64, generator=g, dtype=torch.float64))[0]
    E = torch.randn(512, 512, 1536, generator=g, dtype=torch.float64)
    eri = (E + E.permute(1, 0, 2)) * (0.05 / 2**0.5)
    return C.contiguous(), eri.contiguous()


class TestConfig3:
    def test_ao_to_mo_half(self, hip):
        C, eri = config3_inputs()
        got = trntensor.einsum("mi,mnP->inP", C.cuda(), eri.cuda())
        assert trntensor.plan_contraction("mi,mnP->inP", C, eri).strategy == "torch"
        close(got.cpu(), cpu_ref.ao_to_mo_half(eri, C))

    def test_orthonormal_projection(self, hip):
        """X = C^T eri; C X = C C^T eri is the projection of eri onto span(C)."""
        C, eri = config3_inputs()
        Cd, ed = C.cuda(), eri.cuda()
        X = trntensor.einsum("mi,mnP->inP", Cd, ed)
        back = trntensor.einsum("mi,inP->mnP", Cd, X)
        proj = trntensor.einsum("mi,inP->mnP", Cd, trntensor.einsum("mi,mnP->inP", Cd, back))
        assert normwise(proj, back) <= 1e-12


class TestConfig5:
    def test_greedy_path_scalar(self, hip):
        g = torch.Generator().manual_seed(0)
        A = torch.randn(128, 400, generator=g, dtype=torch.float64) * 0.1
        B = torch.randn(128, 400, generator=g, dtype=torch.float64) * 0.1
        W = torch.randn(400, 400, 800, generator=g, dtype=torch.float64) * 0.01
        V = torch.randn(128, 128, 800, generator=g, dtype=torch.float64) * 0.1
        plan = trntensor.plan_contraction("ia,jb,abP,ijP->", A, B, W, V)
        assert plan.strategy == "path" and plan.contraction_path == [(0, 1), (0, 1), (0, 1)]
        got = trntensor.einsum("ia,jb,abP,ijP->", A.cuda(), B.cuda(), W.cuda(), V.cuda())
        # Cheap-order oracle: (ia,abP->ibP), (ibP,jb->ijP), (ijP,ijP->) in float64 on the CPU.
        ibP = torch.einsum("ia,abP->ibP", A, W)
        ijP = torch.einsum("ibP,jb->ijP", ibP, B)
        ref = torch.einsum("ijP,ijP->", ijP, V)
        scale = torch.einsum("ijP,ijP->", torch.einsum("ibP,jb->ijP", torch.einsum("ia,abP->ibP", A.abs(), W.abs()), B.abs()), V.abs())
        kappa = float(scale) / abs(float(ref))
        err = abs(float(got) - float(ref))
        print(f"config 5: E={float(got):.17g} ref={float(ref):.17g} kappa={kappa:.3e} "
              f"rel={err / abs(float(ref)):.3e} cond-aware={err / float(scale):.3e}")
        # Both bars of the north star: relative 1e-12, and 1e-14 against the
        # same contraction over absolute values (kappa is about 1.1e6 here;
        # float64 orderings of the CPU oracle agree to 1.4e-13 relative).
        assert err / abs(float(ref)) <= 1e-12
        assert err / float(scale) <= 1e-14
        assert got.shape == () and got.dtype == torch.float64


class TestPathFusion:
    """A final full dot fused into the producing GEMM's epilogue (tt_gemm_dot):
    results equal the reference's path executor (oracle) up to summation order,
    bounded by the same contraction over absolute values."""

    @staticmethod
    def check(sub, shapes, dt=torch.float64, seed=0, **kw):
        g = torch.Generator().manual_seed(seed)
        ops = [torch.randn(*s, generator=g, dtype=torch.float64).to(dt) for s in shapes]
        got = trntensor.einsum(sub, *[o.cuda() for o in ops], **kw)
        ref = cpu_ref.einsum(sub, *[o.double() for o in ops], **kw)
        scale = abs(float(torch.einsum(sub, *[o.double().abs() for o in ops]))) + abs(float(kw.get("out", torch.zeros(())))) + 1e-300
        bar = 1e-14 if dt == torch.float64 else 1e-5
        assert got.shape == () and got.dtype == dt
        assert abs(float(got) - float(ref)) / scale <= bar, (float(got), float(ref))

    def test_lazy_outer_product(self, hip):
        self.check("ia,jb,abP,ijP->", [(6, 7), (5, 9), (7, 9, 11), (6, 5, 11)])

    def test_lazy_outer_product_fp32(self, hip):
        self.check("ia,jb,abP,ijP->", [(6, 7), (5, 9), (7, 9, 11), (6, 5, 11)], dt=torch.float32, seed=1)

    def test_materialised_partner(self, hip):
        self.check("ij,jk,ik->", [(70, 33), (33, 90), (70, 90)], seed=2)

    def test_batch_letter(self, hip):
        self.check("bij,bjk,bik->", [(3, 20, 17), (3, 17, 25), (3, 20, 25)], seed=3)

    def test_alpha_beta_out(self, hip):
        self.check("ij,jk,ik->", [(40, 30), (30, 50), (40, 50)], seed=4, alpha=1.5, beta=0.5, out=torch.tensor(2.0, dtype=torch.float64))

    def test_unsupported_geometry_falls_back(self, hip):
        # three letters in the M group: not decodable by the fused epilogue
        self.check("abcK,Kde,abcde->", [(3, 4, 5, 6), (6, 7, 2), (3, 4, 5, 7, 2)], seed=5)

    def test_plan_shape(self, hip):
        from trntensor_amd.einsum import _fusion_plan, _path_names

        path = [(0, 1), (0, 1), (0, 1)]
        names = _path_names(["ia", "jb", "abP", "ijP"], "", path)
        assert _fusion_plan(["ia", "jb", "abP", "ijP"], "", path, names) == (1, 0)


class TestOptimalPath:
    """einsum(optimize="optimal"): the opt-in fewest-multiply-add order gives the
    reference path executor's value (oracle, greedy order) within a bar scaled
    by the same contraction over absolute values."""

    @staticmethod
    def check(sub, shapes, dt=torch.float64, seed=0):
        g = torch.Generator().manual_seed(seed)
        ops = [torch.randn(*s, generator=g, dtype=torch.float64).to(dt) for s in shapes]
        got = trntensor.einsum(sub, *[o.cuda() for o in ops], optimize="optimal")
        ref = cpu_ref.einsum(sub, *[o.double() for o in ops])
        scale = torch.einsum(sub, *[o.double().abs() for o in ops])
        bar = 1e-13 if dt == torch.float64 else 1e-5
        assert got.dtype == dt and tuple(got.shape) == tuple(ref.shape)
        err = (got.cpu().double() - ref).abs()
        assert bool((err <= bar * (scale + 1e-300)).all()), float((err / (scale + 1e-300)).max())

    def test_config5_small(self, hip):
        self.check("ia,jb,abP,ijP->", [(12, 20), (10, 20), (20, 20, 30), (12, 10, 30)])

    def test_chain(self, hip):
        self.check("ij,jk,kl,lm->im", [(30, 200), (200, 5), (5, 150), (150, 40)], seed=1)

    def test_chain_fp32(self, hip):
        self.check("ij,jk,kl,lm->im", [(30, 200), (200, 5), (5, 150), (150, 40)], dt=torch.float32, seed=2)

    def test_mp2_like(self, hip):
        self.check("iaP,jbP,ia,jb->ij", [(6, 24, 40), (6, 24, 40), (6, 24), (6, 24)], seed=3)

    def test_config5_full(self, hip):
        """BASELINE config 5 at full size: optimal order needs 2.16e10 multiply-adds
        instead of 2.1e12; checked against the fp64 greedy-order result on the GPU
        (the oracle takes minutes at this size)."""
        g = torch.Generator().manual_seed(0)
        A = (torch.randn(128, 400, generator=g, dtype=torch.float64) * 0.1).cuda()
        B = (torch.randn(128, 400, generator=g, dtype=torch.float64) * 0.1).cuda()
        W = (torch.randn(400, 400, 800, generator=g, dtype=torch.float64) * 0.01).cuda()
        V = (torch.randn(128, 128, 800, generator=g, dtype=torch.float64) * 0.1).cuda()
        plan = trntensor.plan_contraction("ia,jb,abP,ijP->", A, B, W, V, optimize="optimal")
        assert plan.contraction_path == [(1, 2), (1, 2), (0, 1)]
        fast = trntensor.einsum("ia,jb,abP,ijP->", A, B, W, V, optimize="optimal")
        slow = trntensor.einsum("ia,jb,abP,ijP->", A, B, W, V)
        # |sum| bound: the same contraction over absolute values, via the cheap order
        scale = trntensor.einsum("ia,jb,abP,ijP->", A.abs(), B.abs(), W.abs(), V.abs(), optimize="optimal")
        assert abs(float(fast) - float(slow)) <= 1e-13 * float(scale)


class TestIntegerAndComplex:
    """Non-floating operands, which the reference hands to torch.einsum /
    torch.matmul (trntensor/einsum.py:117-118, nki/dispatch.py:195-196).
    Integers: int64 accumulation with wraparound on the strided kernel,
    truncated to the operands' dtype: equal element for element to the
    oracle's int64 contraction truncated the same way, and to the oracle
    itself wherever torch keeps the narrow dtype (torch promotes some
    narrow-integer reductions to int64 through torch.sum, depending on the
    pattern and the extents). Complex: real contractions of the parts on the
    MFMA core; normwise bars of the parts' dtype."""

    PATTERNS = [
        ("ij,jk->ik", [(37, 50), (50, 29)]),
        ("ij,kj->ik", [(37, 50), (29, 50)]),
        ("bij,bjk->bik", [(3, 20, 30), (3, 30, 10)]),
        ("mi,mnP->inP", [(12, 5), (12, 12, 7)]),
        ("ii->", [(9, 9)]),
        ("i,j->ij", [(6,), (8,)]),
        ("ijk->k", [(5, 6, 70)]),
        ("ij,jk,kl->il", [(5, 8), (8, 6), (6, 4)]),
        ("ia,jb,abP,ijP->", [(4, 5), (3, 6), (5, 6, 7), (4, 3, 7)]),
    ]

    @pytest.mark.parametrize("dt", [torch.int64, torch.int32, torch.int16, torch.int8, torch.uint8])
    @pytest.mark.parametrize("sub,shapes", PATTERNS)
    def test_integers_equal_oracle(self, hip, dt, sub, shapes):
        g = torch.Generator().manual_seed(len(sub) + len(shapes))
        lo, hi = (0, 256) if dt == torch.uint8 else (-120, 120)
        if dt == torch.int64:
            lo, hi = -(1 << 40), 1 << 40  # products and sums wrap modulo 2^64
        ops = [torch.randint(lo, hi, s, generator=g, dtype=torch.int64).to(dt) for s in shapes]
        want = cpu_ref.einsum(sub, *[o.to(torch.int64) for o in ops]).to(dt)
        got = trntensor.einsum(sub, *[o.cuda() for o in ops])
        assert got.dtype == dt and got.device.type == "cuda"
        assert torch.equal(got.cpu(), want), (got.cpu().long() - want.long()).abs().max()
        ref = cpu_ref.einsum(sub, *ops)
        if ref.dtype == dt:
            assert torch.equal(got.cpu(), ref)

    def test_integer_alpha_beta_semantics(self, hip):
        g = torch.Generator().manual_seed(3)
        A, B = (torch.randint(-50, 50, s, generator=g) for s in [(20, 30), (30, 10)])
        out = torch.randint(-50, 50, (20, 10), generator=g)
        for kw in ({"alpha": 2}, {"alpha": 1.5}, {"beta": 3, "out": out}, {"alpha": 2, "beta": -1, "out": out},
                   {"alpha": 0.5, "beta": 2, "out": out}, {"beta": 2, "out": out.double()}):
            ref = cpu_ref.einsum("ij,jk->ik", A, B, **kw)
            got = trntensor.einsum("ij,jk->ik", A.cuda(), B.cuda(), **{k: (v.cuda() if torch.is_tensor(v) else v) for k, v in kw.items()})
            assert got.dtype == ref.dtype, kw
            assert torch.equal(got.cpu(), ref), kw
        # an integral result takes only an integral beta (torch's rule)
        with pytest.raises(RuntimeError, match="integral"):
            cpu_ref.einsum("ij,jk->ik", A, B, beta=0.5, out=out)
        with pytest.raises(RuntimeError, match="integral"):
            trntensor.einsum("ij,jk->ik", A.cuda(), B.cuda(), beta=0.5, out=out.cuda())

    @pytest.mark.parametrize("dt", [torch.complex128, torch.complex64])
    @pytest.mark.parametrize("sub,shapes", PATTERNS)
    def test_complex_matches_oracle(self, hip, dt, sub, shapes):
        g = torch.Generator().manual_seed(len(sub) * 3 + len(shapes))
        ops = [torch.randn(*s, generator=g, dtype=torch.complex128).to(dt) for s in shapes]
        ref = cpu_ref.einsum(sub, *ops)
        got = trntensor.einsum(sub, *[o.cuda() for o in ops])
        assert got.dtype == ref.dtype == dt
        bar = 1e-12 if dt == torch.complex128 else 1e-5
        assert normwise(torch.view_as_real(got.cpu()), torch.view_as_real(ref)) <= bar

    @pytest.mark.parametrize("dt", [torch.complex128, torch.complex64])
    def test_complex_alpha_beta_out(self, hip, dt):
        g = torch.Generator().manual_seed(8)
        A = torch.randn(40, 30, generator=g, dtype=torch.complex128).to(dt)
        B = torch.randn(30, 20, generator=g, dtype=torch.complex128).to(dt)
        outc = torch.randn(40, 20, generator=g, dtype=torch.complex128).to(dt)
        outr = torch.randn(1, 20, generator=g, dtype=torch.float64)
        bar = 1e-12 if dt == torch.complex128 else 1e-5
        for kw in ({"alpha": 1.5}, {"alpha": 1 - 2j}, {"beta": 0.5, "out": outc}, {"alpha": 2j, "beta": 0.5 + 1j, "out": outc},
                   {"beta": -1.0, "out": outr}):
            ref = cpu_ref.einsum("ij,jk->ik", A, B, **kw)
            got = trntensor.einsum("ij,jk->ik", A.cuda(), B.cuda(), **{k: (v.cuda() if torch.is_tensor(v) else v) for k, v in kw.items()})
            assert got.dtype == ref.dtype and got.shape == ref.shape, kw
            assert normwise(torch.view_as_real(got.cpu()), torch.view_as_real(ref)) <= bar, kw

    def test_real_operands_complex_out(self, hip):
        g = torch.Generator().manual_seed(9)
        A, B = torch.randn(16, 24, generator=g), torch.randn(24, 8, generator=g)
        out = torch.randn(16, 8, generator=g, dtype=torch.complex64)
        ref = cpu_ref.einsum("ij,jk->ik", A, B, alpha=2.0, beta=1 + 1j, out=out)
        got = trntensor.einsum("ij,jk->ik", A.cuda(), B.cuda(), alpha=2.0, beta=1 + 1j, out=out.cuda())
        assert got.dtype == ref.dtype == torch.complex64
        assert normwise(torch.view_as_real(got.cpu()), torch.view_as_real(ref)) <= 1e-5

    def test_conjugate_view_operand(self, hip):
        g = torch.Generator().manual_seed(10)
        A = torch.randn(12, 9, generator=g, dtype=torch.complex128)
        B = torch.randn(9, 7, generator=g, dtype=torch.complex128)
        ref = cpu_ref.einsum("ij,jk->ik", A.conj(), B)
        got = trntensor.einsum("ij,jk->ik", A.cuda().conj(), B.cuda())
        assert normwise(torch.view_as_real(got.cpu()), torch.view_as_real(ref)) <= 1e-12

    @pytest.mark.parametrize("dt", [torch.float32, torch.float64])
    def test_real_operands_complex_scalars(self, hip, dt):
        """A complex alpha makes a real result complex (result.mul(alpha));
        a complex beta with a real result and out raises torch's error, and is
        accepted when out or alpha makes the sum complex."""
        g = torch.Generator().manual_seed(11)
        A = torch.randn(24, 40, generator=g, dtype=torch.float64).to(dt)
        B = torch.randn(40, 16, generator=g, dtype=torch.float64).to(dt)
        outr = torch.randn(24, 16, generator=g, dtype=torch.float64).to(dt)
        bar = 1e-12 if dt == torch.float64 else 1e-5
        for kw in ({"alpha": 2j}, {"alpha": 1.5 - 0.5j, "beta": 0.5, "out": outr}, {"alpha": 2j, "beta": 1j, "out": outr},
                   {"alpha": 1 + 0j}, {"beta": 2j}):
            ref = cpu_ref.einsum("ij,jk->ik", A, B, **kw)
            got = trntensor.einsum("ij,jk->ik", A.cuda(), B.cuda(), **{k: (v.cuda() if torch.is_tensor(v) else v) for k, v in kw.items()})
            assert got.dtype == ref.dtype and got.shape == ref.shape, kw
            if ref.dtype.is_complex:
                assert normwise(torch.view_as_real(got.cpu()), torch.view_as_real(ref)) <= bar, kw
            else:
                assert normwise(got.cpu(), ref) <= bar, kw
        with pytest.raises(RuntimeError, match="complex"):
            cpu_ref.einsum("ij,jk->ik", A, B, beta=1j, out=outr)
        with pytest.raises(RuntimeError, match="complex"):
            trntensor.einsum("ij,jk->ik", A.cuda(), B.cuda(), beta=1j, out=outr.cuda())


class TestLaunchCache:
    """Repeat calls of a two-operand contraction that runs as one GEMM launch
    go through a cached launcher (one allocation, one library call). They must
    be indistinguishable from the first call: same values bitwise, a miss for
    any other shape, stride, dtype or keyword, planning again after
    clear_plan_cache, and the backend switch still honoured."""

    def _size(self):
        return importlib.import_module("trntensor_amd.einsum")._launch_cache_size()

    @pytest.mark.parametrize("sub,shapes,dt", [
        ("ap,bp->ab", [(32, 96), (32, 96)], torch.float32),
        ("ij,jk->ik", [(70, 50), (50, 130)], torch.float64),
        ("bij,bjk->bik", [(3, 40, 20), (3, 20, 64)], torch.float32),
        ("ij,kj->ik", [(64, 48), (80, 48)], torch.bfloat16),
    ])
    def test_repeat_calls_bitwise(self, hip, sub, shapes, dt):
        g = torch.Generator().manual_seed(4)
        ops = [torch.randn(*s, generator=g).to(dt).cuda() for s in shapes]
        trntensor.clear_plan_cache()
        first = trntensor.einsum(sub, *ops)
        assert self._size() == 1
        for alpha in (1.0, 2.5, 3):
            again = trntensor.einsum(sub, *ops, alpha=alpha)
            ref = trntensor.einsum(sub, *ops, alpha=alpha, beta=0.0, out=torch.zeros_like(first))  # planned path
            assert again.dtype == first.dtype and again.shape == first.shape and again.device == first.device
            assert torch.equal(again, ref)
        assert torch.equal(trntensor.einsum(sub, *ops), first)
        want = cpu_ref.einsum(sub, *[o.cpu().double() for o in ops])
        assert normwise(first.cpu().double(), want) <= (1e-2 if dt == torch.bfloat16 else {torch.float32: 1e-5, torch.float64: 1e-12}[dt])

    def test_misses_and_clear(self, hip):
        g = torch.Generator().manual_seed(5)
        B = torch.randn(8, 32, 96, generator=g).cuda()
        trntensor.clear_plan_cache()
        trntensor.einsum("ap,bp->ab", B[0], B[1])
        trntensor.einsum("ap,bp->ab", B[2], B[3])  # same shapes and strides: a hit
        assert self._size() == 1
        Bt = B.transpose(1, 2).contiguous().transpose(1, 2)  # same shape, other strides
        got = trntensor.einsum("ap,bp->ab", Bt[0], Bt[1])
        assert torch.equal(got, trntensor.einsum("ap,bp->ab", B[0], B[1]))
        assert self._size() == 2
        trntensor.einsum("ap,bp->ab", B[0].double(), B[1].double())
        assert self._size() == 3
        trntensor.clear_plan_cache()
        assert self._size() == 0 and trntensor.plan_cache_info()["size"] == 0
        trntensor.einsum("ap,bp->ab", B[0], B[1])
        assert trntensor.plan_cache_info()["size"] == 1

    def test_repeat_calls_use_the_native_launch_table(self, hip):
        """On the GPU the recorded launches live in the C++ table
        (tt_fastpath.so), not in Python launchers."""
        from trntensor_amd import plan
        from trntensor_amd.hip import _fastpath

        E = importlib.import_module("trntensor_amd.einsum")
        B = torch.randn(4, 32, 96).cuda()
        trntensor.clear_plan_cache()
        first = trntensor.einsum("ap,bp->ab", B[0], B[1])
        assert E._fast is not None, _fastpath.error()
        assert type(E._fast).__name__ == "LaunchTable" and len(E._fast) == 1 and len(plan._LAUNCH_CACHE) == 0
        assert torch.equal(trntensor.einsum("ap,bp->ab", B[0], B[1]), first)
        planned = trntensor.einsum("ap,bp->ab", B[2], B[3], beta=0.0, out=torch.zeros(32, 32).cuda())
        assert torch.equal(trntensor.einsum("ap,bp->ab", B[2], B[3]), planned)
        trntensor.clear_plan_cache()
        assert len(E._fast) == 0

    @pytest.mark.parametrize("dt", [torch.float32, torch.float64])
    def test_host_operands_repeat_bitwise(self, hip, dt):
        """Small contiguous CPU operands: repeat calls are staged by the C++
        table (one pinned upload, one launch, one download) and return CPU
        tensors bitwise equal to the planned path's; non-contiguous and
        large host operands are not recorded and stay on the planned path."""
        E = importlib.import_module("trntensor_amd.einsum")
        g = torch.Generator().manual_seed(7)
        B = (torch.randn(8, 32, 96, generator=g) * 0.1).to(dt)
        trntensor.clear_plan_cache()
        first = trntensor.einsum("ap,bp->ab", B[0], B[1])
        assert first.device.type == "cpu" and E._fast is not None and len(E._fast) == 1
        for i, j, alpha in ((0, 1, 1.0), (2, 5, 2.5), (7, 7, 3)):
            got = trntensor.einsum("ap,bp->ab", B[i], B[j], alpha=alpha)
            planned = trntensor.einsum("ap,bp->ab", B[i], B[j], alpha=alpha, beta=0.0, out=torch.zeros(32, 32, dtype=dt))
            assert got.device.type == "cpu" and got.dtype == dt and got.is_contiguous()
            assert torch.equal(got, planned), (i, j, alpha)
        want = cpu_ref.einsum("ap,bp->ab", B[0].double(), B[1].double())
        assert normwise(first.double(), want) <= (1e-5 if dt == torch.float32 else 1e-12)
        # 'bp,ap->ab' on the same operands runs swapped (the output is B^T A^T).
        sw = trntensor.einsum("bp,ap->ab", B[3], B[4])
        assert torch.equal(trntensor.einsum("bp,ap->ab", B[3], B[4]), sw) and len(E._fast) == 2
        assert normwise(sw.double(), trntensor.einsum("ap,bp->ab", B[4], B[3]).double()) <= 1e-12
        Bt = B.transpose(1, 2).contiguous().transpose(1, 2)  # non-contiguous views
        n = len(E._fast)
        nc = trntensor.einsum("ap,bp->ab", Bt[0], Bt[1])
        assert len(E._fast) == n and torch.equal(trntensor.einsum("ap,bp->ab", Bt[0], Bt[1]), nc)
        big = torch.randn(600, 1000, generator=g).to(dt)  # 2 x 4.8 MB operands: above the staging bound
        trntensor.einsum("ik,jk->ij", big, big)
        assert len(E._fast) == n

    def test_backend_switch_applies_to_cached_launches(self, hip):
        B = torch.randn(4, 32, 96).cuda()
        trntensor.einsum("ap,bp->ab", B[0], B[1])
        trntensor.einsum("ap,bp->ab", B[0], B[1])
        try:
            trntensor.set_backend("pytorch")
            with pytest.raises(RuntimeError, match="pytorch"):
                trntensor.einsum("ap,bp->ab", B[0], B[1])
        finally:
            trntensor.set_backend("auto")

    def test_keywords_bypass_the_cache(self, hip):
        g = torch.Generator().manual_seed(6)
        A, Bm, C = (torch.randn(40, 40, generator=g).cuda() for _ in range(3))
        plain = trntensor.einsum("ij,jk->ik", A, Bm)
        withc = trntensor.einsum("ij,jk->ik", A, Bm, alpha=2.0, beta=0.5, out=C)
        ref = cpu_ref.einsum("ij,jk->ik", A.cpu(), Bm.cpu(), alpha=2.0, beta=0.5, out=C.cpu())
        assert normwise(withc.cpu(), ref) <= 1e-5
        assert normwise(plain.cpu(), cpu_ref.einsum("ij,jk->ik", A.cpu(), Bm.cpu())) <= 1e-5
        kah = trntensor.einsum("ij,jk->ik", A, Bm, precision="kahan")
        assert normwise(kah.cpu(), cpu_ref.einsum("ij,jk->ik", A.cpu(), Bm.cpu(), precision="kahan")) <= 2e-7
