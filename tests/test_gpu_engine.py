"""The contraction engine's launch mappings on the GPU kernels.

tests/test_engine_host.py checks every mapping decision against CPU
emulations of the kernels; this file runs the same kinds of contraction on
the real tt_gemm / tt_gemm_dot / tt_strided_contract launches: broadcast
batches, general output strides, K-split GEMMs and fused dots, random letter
layouts on permuted (non-contiguous) operands. Expected values are
torch.einsum in float64 on the CPU; bars are normwise 1e-12 (float64) and
1e-5 (float32).
"""

import random

import pytest
import torch

from trntensor_amd.hip import engine
from tests.util import normwise

pytestmark = pytest.mark.gpu


def _operand(term, ext, gen, rng, dt):
    order = list(range(len(term)))
    rng.shuffle(order)
    base = torch.randn([ext[term[k]] for k in order], generator=gen, dtype=torch.float64)
    inv = [order.index(k) for k in range(len(term))]
    return base.permute(inv).to(dt)


def _run(sub, ext, dt, seed=0, alpha=1.0, beta=0.0, with_c=False, prefer_gemm=True):
    gen = torch.Generator().manual_seed(seed)
    rng = random.Random(seed)
    lhs, out = sub.split("->")
    terms = lhs.split(",")
    ops = [_operand(t, ext, gen, rng, dt) for t in terms]
    C = torch.randn([ext[c] for c in out], generator=gen, dtype=torch.float64).to(dt) if with_c else None
    got = engine.contract(terms, out, [o.cuda() for o in ops], alpha, beta, None if C is None else C.cuda(),
                          prefer_gemm=prefer_gemm)
    want = alpha * torch.einsum(sub, *[o.double() for o in ops])
    if C is not None:
        want = want + beta * C.double()
    assert tuple(got.shape) == tuple(want.shape)
    bar = 1e-12 if dt == torch.float64 else 1e-5
    assert normwise(got.cpu().double(), want) <= bar, sub


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize(
    "sub,ext",
    [
        ("jb,abP->jaP", dict(j=130, b=70, a=9, P=200)),  # broadcast batch over a
        ("jb,abP->ajP", dict(j=130, b=70, a=9, P=200)),
        ("ikj,kl->ilj", dict(i=6, k=50, j=70, l=90)),  # broadcast batch over i, swapped output
        ("ijP,ajP->ia", dict(i=40, a=50, j=64, P=800)),  # K = 51200: split
        ("ijP,ajP->ai", dict(i=70, a=33, j=8, P=700)),  # K = 5600, swapped output, split + remainder
        ("bij,bjk->ikb", dict(b=3, i=70, j=40, k=50)),  # permuting pass
        ("abc,bd->dac", dict(a=20, b=33, c=40, d=24)),
    ],
)
def test_mappings(hip, dt, sub, ext):
    _run(sub, ext, dt)
    _run(sub, ext, dt, seed=1, alpha=1.5, beta=0.5, with_c=True)


def test_random_layouts(hip):
    rng = random.Random(99)
    letters = "abcdefg"
    for n in range(120):
        pool = rng.sample(letters, rng.randint(2, 6))
        ext = {c: rng.choice([1, 2, 3, 7, 16, 33, 65]) for c in pool}
        ta = "".join(rng.sample(pool, rng.randint(1, min(4, len(pool)))))
        tb = "".join(rng.sample(pool, rng.randint(1, min(4, len(pool)))))
        seen = [c for c in pool if c in ta or c in tb]
        out = "".join(c for c in rng.sample(seen, len(seen)) if rng.random() < 0.5)
        _run(f"{ta},{tb}->{out}", ext, torch.float64, seed=n, prefer_gemm=rng.random() < 0.5)


@pytest.mark.parametrize(
    "gterms,xname,shapes,factors",
    [
        (["ijP", "ajP"], "ia", [(40, 64, 800), (50, 64, 800)], [("ia", (40, 50))]),  # split fused dot
        (["jPi", "jPa"], "ia", [(16, 700, 30), (16, 700, 20)], [("ia", (30, 20))]),  # row-contiguous, remainder
        (["abP", "ijP"], "abij", [(20, 30, 64), (9, 11, 64)], [("ia", (9, 20)), ("jb", (11, 30))]),  # lazy outer
    ],
)
def test_fused_dot_mappings(hip, gterms, xname, shapes, factors):
    gen = torch.Generator().manual_seed(4)
    tens = [torch.randn(*s, generator=gen, dtype=torch.float64) for s in shapes]
    facs = [(t, torch.randn(*s, generator=gen, dtype=torch.float64)) for t, s in factors]
    C = torch.tensor(0.75, dtype=torch.float64)
    got = engine.contract_gemm_dot(gterms, xname, [t.cuda() for t in tens], [(t, f.cuda()) for t, f in facs],
                                   1.5, 0.5, C.cuda())
    assert got is not None
    X = torch.einsum(",".join(gterms) + "->" + xname, *tens)
    E = torch.einsum(",".join(t for t, _ in facs) + "->" + xname, *[f for _, f in facs])
    want = 1.5 * float((X * E).sum()) + 0.5 * 0.75
    scale = 1.5 * float((X.abs() * E.abs()).sum()) + 0.5 * 0.75
    assert abs(float(got) - want) <= 1e-13 * scale


class TestIndexRange:
    """Outputs and reductions beyond 2^31 elements: the strided kernel takes
    32-bit linear indices, so the engine splits such launches; the GEMM core
    addresses with 64-bit offsets. Checked on sampled entries."""

    def test_outer_product_beyond_2_31(self, hip):
        n = 48000  # 2.30e9 outputs, 9.2 GB in float32
        a = torch.arange(n, dtype=torch.float32, device="cuda") % 1021 - 510
        b = torch.arange(n, dtype=torch.float32, device="cuda") % 997 - 498
        out = engine.contract(["i", "j"], "ij", [a, b])
        assert out.shape == (n, n)
        idx = torch.randint(0, n, (4096, 2), generator=torch.Generator().manual_seed(0))
        got = out[idx[:, 0], idx[:, 1]].cpu()
        want = (idx[:, 0] % 1021 - 510).float() * (idx[:, 1] % 997 - 498).float()
        assert torch.equal(got, want)
        # the last row and column (the split's final chunk)
        assert float(out[n - 1, n - 1]) == float(((n - 1) % 1021 - 510) * ((n - 1) % 997 - 498))
        del out

    def test_sum_beyond_2_31(self, hip):
        n = (1 << 31) + 4097  # reduction length past 2^31, 8.6 GB of float32 ones
        x = torch.ones(n, dtype=torch.float32, device="cuda")
        # The launch is split at 2^31 and the second part accumulates onto
        # the first. Every per-thread and per-block partial is an integer
        # below 2^24 (exact in float32); only the final sum rounds (2^31 + 4097
        # is not a float32), hence the relative bar.
        got = float(engine.contract(["i"], "", [x]))
        assert abs(got - n) / n < 1e-6
        del x

    def test_gemm_output_beyond_2_31(self, hip):
        M, N = 50000, 45000  # 2.25e9 outputs, K = 2
        A = (torch.arange(M * 2, dtype=torch.float32, device="cuda") % 7 - 3).view(M, 2)
        B = (torch.arange(2 * N, dtype=torch.float32, device="cuda") % 5 - 2).view(2, N)
        D = engine.contract(["ik", "kj"], "ij", [A, B], prefer_gemm=True)
        idx_m = torch.randint(0, M, (2048,), generator=torch.Generator().manual_seed(1))
        idx_n = torch.randint(0, N, (2048,), generator=torch.Generator().manual_seed(2))
        got = D[idx_m, idx_n].cpu()
        want = (A.cpu()[idx_m] * B.cpu()[:, idx_n].T).sum(1)
        assert torch.equal(got, want)
        assert float(D[M - 1, N - 1]) == float((A[M - 1] * B[:, N - 1]).sum())
        del D
