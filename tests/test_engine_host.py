"""Host logic of the contraction engine (trntensor_amd/hip/engine.py) on the CPU.

The engine maps an einsum onto tt_gemm / tt_strided_contract launches
(letter grouping, in-place layouts, broadcast batches, K-splitting, packing,
output permutation). Here both launch wrappers are replaced by CPU
emulations of the kernels' documented addressing (include/trntensor_hip.h),
so every mapping decision is checked against torch.einsum without a GPU.
"""

import random

import pytest
import torch

from trntensor_amd.hip import engine


def emu_gemm(transA, transB, M, N, K, A, lda, sA, B, ldb, sB, D, ldd, sD, batch=1, alpha=1.0, beta=0.0, C=None,
             ldc=0, sC=0, a_off=0, b_off=0):
    """tt_gemm's contract: op(A)[m,k] = A[b*sA + (transA ? k*lda + m : m*lda + k)], etc."""
    if M == 0 or N == 0 or batch == 0:
        return
    opA = torch.as_strided(A, (batch, M, K), (sA, 1, lda) if transA else (sA, lda, 1), A.storage_offset() + a_off)
    opB = torch.as_strided(B, (batch, K, N), (sB, 1, ldb) if transB else (sB, ldb, 1), B.storage_offset() + b_off)
    res = alpha * torch.bmm(opA.double(), opB.double())
    if C is not None:
        res = res + beta * torch.as_strided(C, (batch, M, N), (sC, ldc, 1), C.storage_offset()).double()
    torch.as_strided(D, (batch, M, N), (sD, ldd, 1), D.storage_offset()).copy_(res)


def emu_strided(out_dims, red_dims, A, B, D, alpha=1.0, beta=0.0, C=None, a_off=0, b_off=0):
    """tt_strided_contract's contract: D[o] = alpha sum_r A[.]B[.] (+ beta C[o]), D contiguous."""
    dims = list(out_dims) + list(red_dims)
    shape = [d[0] for d in dims]
    av = torch.as_strided(A, shape, [d[1] for d in dims], A.storage_offset() + a_off).double()
    if B is not None:
        av = av * torch.as_strided(B, shape, [d[2] for d in dims], B.storage_offset() + b_off).double()
    nred = len(red_dims)
    res = av.sum(dim=tuple(range(len(out_dims), len(dims)))) if nred else av
    res = alpha * res.reshape(-1)
    if C is not None:
        res = res + beta * C.reshape(-1).double()
    D.view(-1).copy_(res)


@pytest.fixture
def emulated(monkeypatch):
    monkeypatch.setattr(engine, "gemm", emu_gemm)
    monkeypatch.setattr(engine, "strided_contract", emu_strided)
    engine._RECIPES.clear()
    yield
    engine._RECIPES.clear()


def _operand(term, ext, gen, perm_rng):
    """A float64 tensor for `term`, often as a permuted (non-contiguous) view."""
    order = list(range(len(term)))
    perm_rng.shuffle(order)
    base = torch.randn([ext[term[k]] for k in order], generator=gen, dtype=torch.float64)
    inv = [order.index(k) for k in range(len(term))]
    return base.permute(inv)


def _check(terms, out, ops, alpha=1.0, beta=0.0, C=None, prefer_gemm=False):
    got = engine.contract(terms, out, ops, alpha, beta, C, prefer_gemm=prefer_gemm)
    want = alpha * torch.einsum(",".join(terms) + "->" + out, *ops)
    if C is not None:
        want = want + beta * C
    assert tuple(got.shape) == tuple(want.shape)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize(
    "sub,ext",
    [
        ("jb,abP->jaP", dict(j=20, b=7, a=5, P=24)),  # N letters split by K in B: batch over a
        ("jb,abP->ajP", dict(j=20, b=7, a=5, P=24)),  # batch over a, output a-major
        ("abP,jb->jaP", dict(j=20, b=7, a=5, P=24)),  # same with operands swapped
        ("ikj,kl->ilj", dict(i=4, k=9, j=17, l=19)),  # M letters split by K in A
        ("ij,jk->ik", dict(i=33, j=21, k=40)),
        ("ij,kj->ki", dict(i=33, j=21, k=40)),
        ("bij,bjk->bik", dict(b=3, i=17, j=21, k=19)),
        ("bij,bjk->ikb", dict(b=3, i=17, j=21, k=19)),  # output needs a permuting pass
        ("ijP,ajP->ia", dict(i=3, a=5, j=16, P=300)),  # K = 4800: split into 9 slices + remainder
        ("ijP,ajP->ai", dict(i=3, a=5, j=16, P=256)),  # K = 4096, swapped output, split
        ("ab,bc->ac", dict(a=1, b=5000, c=1)),  # GEMV-like, split
        ("ab,bc->ac", dict(a=0, b=5000, c=3)),  # empty output, long K
        ("ab,bc->ac", dict(a=4, b=0, c=3)),  # K = 0: beta * C only
    ],
)
def test_gemm_mappings(emulated, sub, ext):
    gen = torch.Generator().manual_seed(1)
    lhs, out = sub.split("->")
    terms = lhs.split(",")
    for seed in range(3):
        rng = random.Random(seed)
        ops = [_operand(t, ext, gen, rng) for t in terms]
        C = torch.randn([ext[c] for c in out], generator=gen, dtype=torch.float64)
        _check(terms, out, ops, prefer_gemm=True)
        _check(terms, out, ops, 1.5, 0.5, C, prefer_gemm=True)


def test_broadcast_batch_is_in_place(emulated):
    """'jb,abP->jaP' runs as one launch over a broadcast batch, with no pack."""
    ext = dict(j=20, b=7, a=5, P=24)
    A = torch.randn(20, 7, dtype=torch.float64)
    B = torch.randn(5, 7, 24, dtype=torch.float64)
    maps = list(engine._inplace_mappings(engine.Operand("jb", A), engine.Operand("abP", B), "jaP", [], ["j"], ["a", "P"], ["b"], ext))
    assert maps, "expected an in-place mapping"
    swap, ta, tb, M, N, K, lda, sA, ldb, sB, ldd, sD, nb = maps[0]
    assert (swap, M, N, K, nb) == (0, 20, 24, 7, 5)
    assert sA == 0 and sB == 7 * 24 and sD == 24 and ldd == 5 * 24


def test_split_k_choice():
    assert engine.split_k(128, 400, 102400, 1) == 128
    assert engine.split_k(4096, 4096, 4096, 1) == 1  # enough tiles
    assert engine.split_k(128, 128, 4095, 1) == 1  # short K
    assert engine.split_k(128, 128, 8192, 2) == 1  # batched
    assert engine.split_k(1, 1, 5000, 1) == 9
    assert engine.split_k(0, 7, 8192, 1) == 1  # empty output


def test_random_two_operand_contractions(emulated):
    """Random letter layouts (permuted views, summed free letters, diagonals excluded)."""
    rng = random.Random(2024)
    gen = torch.Generator().manual_seed(7)
    letters = "abcdefgh"
    for _ in range(300):
        pool = rng.sample(letters, rng.randint(2, 6))
        ext = {c: rng.choice([1, 2, 3, 5, 8, 17, 33]) for c in pool}
        ta = "".join(rng.sample(pool, rng.randint(1, min(4, len(pool)))))
        tb = "".join(rng.sample(pool, rng.randint(1, min(4, len(pool)))))
        seen = [c for c in pool if c in ta or c in tb]
        out = "".join(c for c in rng.sample(seen, len(seen)) if rng.random() < 0.5)
        ops = [_operand(ta, ext, gen, rng), _operand(tb, ext, gen, rng)]
        _check([ta, tb], out, ops, prefer_gemm=rng.random() < 0.5)


def emu_gemm_dot(transA, transB, M, N, K, A, lda, sA, B, ldb, sB, batch, m_lo_extent, n_lo_extent, E1, e1s, E2, e2s,
                 alpha, beta, C, out, a_off=0, b_off=0):
    """tt_gemm_dot's contract (include/trntensor_hip.h): out = alpha sum X.*E (+ beta C[0]),
    E(b,m,n) = E1[o(e1s)] * E2[o(e2s)], o(s) = m_hi s0 + m_lo s1 + n_hi s2 + n_lo s3 + b s4."""
    opA = torch.as_strided(A, (batch, M, K), (sA, 1, lda) if transA else (sA, lda, 1), A.storage_offset() + a_off)
    opB = torch.as_strided(B, (batch, K, N), (sB, 1, ldb) if transB else (sB, ldb, 1), B.storage_offset() + b_off)
    X = torch.bmm(opA.double(), opB.double())
    b = torch.arange(batch).view(-1, 1, 1)
    m = torch.arange(M).view(1, -1, 1)
    n = torch.arange(N).view(1, 1, -1)

    def gather(E, s):
        off = (m // m_lo_extent) * s[0] + (m % m_lo_extent) * s[1] + (n // n_lo_extent) * s[2] + (n % n_lo_extent) * s[3] + b * s[4]
        return _flat(E)[off]

    E = gather(E1, e1s)
    if E2 is not None:
        E = E * gather(E2, e2s)
    v = alpha * float((X * E.double()).sum())
    if C is not None:
        v += beta * float(C.reshape(-1)[0])
    out.fill_(v)


def _flat(E):
    """Element view of E's storage from its first element (strides are element offsets)."""
    return torch.as_strided(E, (E.untyped_storage().nbytes() // E.element_size() - E.storage_offset(),), (1,), E.storage_offset())


@pytest.mark.parametrize(
    "gterms,xname,shapes,factors",
    [
        # config-5 shape: abP,ijP -> abij dotted with the outer product ia x jb
        (["abP", "ijP"], "abij", [(5, 6, 7), (3, 4, 7)], [("ia", (3, 5)), ("jb", (4, 6))]),
        # optimal-order shape with a long K: split into slices with E batch stride 0
        (["ijP", "ajP"], "ia", [(3, 16, 300), (5, 16, 300)], [("ia", (3, 5))]),
        # the same with row-contiguous operands (k-step = leading dimension)
        (["jPi", "jPa"], "ia", [(16, 300, 3), (16, 300, 5)], [("ia", (3, 5))]),
        # batch letter
        (["bij", "bjk"], "bik", [(3, 7, 9), (3, 9, 5)], [("bik", (3, 7, 5))]),
        # partner in another letter order than the product
        (["ij", "jk"], "ik", [(6, 8), (8, 9)], [("ki", (9, 6))]),
    ],
)
def test_gemm_dot_mappings(monkeypatch, gterms, xname, shapes, factors):
    monkeypatch.setattr(engine, "gemm", emu_gemm)
    monkeypatch.setattr(engine, "strided_contract", emu_strided)
    monkeypatch.setattr(engine, "gemm_dot", emu_gemm_dot)
    gen = torch.Generator().manual_seed(3)
    tens = [torch.randn(*s, generator=gen, dtype=torch.float64) for s in shapes]
    facs = [(t, torch.randn(*s, generator=gen, dtype=torch.float64)) for t, s in factors]
    C = torch.tensor(0.75, dtype=torch.float64)
    got = engine.contract_gemm_dot(gterms, xname, tens, facs, 1.5, 0.5, C)
    assert got is not None
    X = torch.einsum(",".join(gterms) + "->" + xname, *tens)
    E = torch.einsum(",".join(t for t, _ in facs) + "->" + xname, *[f for _, f in facs])
    want = 1.5 * float((X * E).sum()) + 0.5 * 0.75
    assert abs(float(got) - want) <= 1e-12 * (1 + abs(want))
