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
