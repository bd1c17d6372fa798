"""GPU parity of the C-ABI kernels, called through the ctypes binding.

tt_gemm is checked against float64 torch matmul on the CPU (the reference's
CPU executor for the matmul/bmm strategies, trntensor/nki/dispatch.py:195-196,
347-348) over every transpose combination, ragged edges, batching, strided
leading dimensions and the alpha/beta epilogue. tt_strided_contract is checked
against numpy's float64 einsum.
"""

import numpy as np
import pytest
import torch

from oracle import brute
from tests.util import normwise

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-12, torch.float32: 1e-5}


def _gemm_case(hip, dt, ta, tb, M, N, K, batch, alpha, beta, with_c, pad=0, seed=0, alias=False, ld_align=0):
    """tt_gemm through engine.gemm against float64 torch. Leading dimensions
    are the stored widths plus `pad`, or (ld_align > 0) each width rounded up
    to a multiple of ld_align."""
    from trntensor_amd.hip import engine

    g = torch.Generator().manual_seed(seed)
    dev = torch.device("cuda")
    # Stored shapes (row-major) with optional extra columns to exercise ld > width.
    a_rows, a_cols = (K, M) if ta else (M, K)
    b_rows, b_cols = (N, K) if tb else (K, N)
    lda = a_cols + (-a_cols % ld_align if ld_align else pad)
    ldb = b_cols + (-b_cols % ld_align if ld_align else pad)
    A = torch.randn(batch, a_rows, lda, generator=g, dtype=torch.float64)
    B = torch.randn(batch, b_rows, ldb, generator=g, dtype=torch.float64)
    C = torch.randn(batch, M, N, generator=g, dtype=torch.float64)
    opA = A[:, :, :a_cols].transpose(1, 2) if ta else A[:, :, :a_cols]
    opB = B[:, :, :b_cols].transpose(1, 2) if tb else B[:, :, :b_cols]
    ref = alpha * torch.bmm(opA, opB)
    if with_c:
        ref = ref + beta * C
    Ad, Bd, Cd = A.to(dev, dt), B.to(dev, dt), C.to(dev, dt)
    D = Cd if alias else torch.full((batch, M, N), float("nan"), dtype=dt, device=dev)
    engine.gemm(
        ta, tb, M, N, K,
        Ad, lda, a_rows * lda,
        Bd, ldb, b_rows * ldb,
        D, N, M * N, batch, alpha, beta,
        Cd if with_c else None, N, M * N,
    )
    torch.cuda.synchronize()
    return normwise(D, ref)


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("M,N,K", [(130, 130, 130), (131, 131, 131), (128, 128, 131), (131, 128, 128), (128, 131, 128),
                                   (70, 33, 131)])
def test_gemm_aligned_ld_straddling_pieces(hip, dt, ta, tb, M, N, K):
    """Leading dimensions rounded up to multiples of 8 (16-byte vector path on)
    with M, N or K not multiples of the vector width: edge tiles mix whole
    vector pieces, pieces outside (zero, no load) and pieces that straddle
    the edge (element loads)."""
    assert _gemm_case(hip, dt, ta, tb, M, N, K, 1, 1.0, 0.0, False, ld_align=8, seed=M + N + K) <= TOL[dt]
    assert _gemm_case(hip, dt, ta, tb, M, N, K, 2, 1.5, -0.5, True, ld_align=8, seed=M + 7) <= TOL[dt]


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize(
    "M,N,K",
    [(1, 1, 1), (7, 5, 3), (64, 64, 16), (100, 70, 200), (129, 257, 33), (300, 40, 77), (33, 600, 130), (256, 256, 256)],
)
def test_gemm_layouts_and_edges(hip, dt, ta, tb, M, N, K):
    assert _gemm_case(hip, dt, ta, tb, M, N, K, 1, 1.0, 0.0, False) <= TOL[dt]


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize("pad", [0, 1, 3])
def test_gemm_batched_alpha_beta_ld(hip, dt, pad):
    # odd leading dimensions disable the 16-byte vector path
    assert _gemm_case(hip, dt, False, True, 70, 90, 50, 3, 1.5, 0.5, True, pad=pad, seed=1) <= TOL[dt]
    assert _gemm_case(hip, dt, True, False, 130, 65, 40, 2, -0.75, 2.0, True, pad=pad, seed=2) <= TOL[dt]


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize(
    "ta,tb,M,N,K,batch",
    [
        (False, False, 64, 300, 70, 2),  # 64 x 128 tiles (M <= 64)
        (True, False, 200, 150, 40, 3),  # 64 x 128 (fp64 batched, K <= 1024; small grid)
        (False, True, 300, 50, 90, 1),  # 256 x 64 tiles (N <= 64)
        (True, True, 257, 300, 129, 1),  # 64 x 128 tiles (small grid), ragged edges
        (False, True, 2700, 2700, 40, 1),  # 128 x 128 tiles (484 of them), ragged edges
        (False, False, 200, 512, 48, 2),  # direct-B, 16-byte C pieces of two row blocks at a time, ragged M
        (True, False, 512, 768, 64, 3),  # direct-B, the batched shape family of config 2
        (False, False, 4096, 4096, 1024, 1),  # fp32: the 256 x 256 LDS tile (with C: K >= 1024)
        (False, False, 512, 512, 1024, 64),  # fp32: the 256 x 256 LDS tile, batched, with C
    ],
)
def test_gemm_d_aliases_c(hip, dt, ta, tb, M, N, K, batch):
    """D may alias C exactly (header contract): D = alpha * op(A) op(B) + beta * D.
    Each row block's C values are loaded before its stores, so every element is
    read before it is overwritten."""
    assert _gemm_case(hip, dt, ta, tb, M, N, K, batch, 1.5, 0.5, True, seed=M + N, alias=True) <= TOL[dt]


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize(
    "ta,M,N,K,batch,alpha,beta,with_c,ldd_pad",
    [
        (True, 64, 1024, 512, 1, 1.0, 0.0, False, 0),  # the AO->MO half transform's shape family
        (True, 64, 2048, 64, 1, 1.5, 0.5, True, 0),
        (True, 64, 512, 16, 3, 1.0, 0.25, True, 0),
        (True, 64, 1024, 160, 2, -2.0, 1.0, True, 1),  # odd ldc/ldd: element stores
        (True, 50, 1024, 500, 1, 1.0, 0.0, False, 0),  # M < 64, K tail
        (True, 33, 1152, 7, 2, 0.5, 2.0, True, 1),  # one partial stage only
        (True, 1, 256, 31, 1, 1.0, 0.0, False, 0),
        (True, 64, 1030, 48, 1, 1.0, 0.5, True, 0),  # fp64: partial last column tile; fp32: LDS-staged in both runs
        (False, 200, 300, 100, 2, 1.5, 0.5, True, 1),  # fp64: partial last column tile, ragged M
        (False, 130, 2, 33, 1, 1.0, 0.0, False, 0),  # fp64: one tile of two columns
        # batched, B cached (64-row slabs of A, either layout)
        (False, 512, 512, 512, 4, 1.5, 0.5, True, 0),  # the 64 x 512^3 batch's shape
        (True, 512, 512, 512, 3, 1.0, 0.0, False, 0),
        (True, 320, 1536, 512, 2, 1.0, 0.0, False, 0),  # the AO->MO transform's second GEMM
        (False, 200, 256, 333, 3, -1.0, 1.0, True, 1),  # ragged M and K
        (True, 70, 384, 1000, 2, 2.0, 0.0, False, 0),
        # more than 64 row tiles: rows in groups of 16 slabs sweeping every column tile
        (False, 4160, 512, 48, 1, 1.5, 0.5, True, 0),
        (True, 4200, 768, 40, 2, 1.0, 0.0, False, 1),  # ragged last group and rows
        # fp32, whole 256 x 256 tiles, one per CU: the LDS-staged 256 x 256 tile kernel
        (False, 4096, 4096, 1024, 1, 1.5, 0.5, True, 0),
        (False, 2048, 8192, 32, 1, 1.0, 0.0, False, 0),  # one 32-k stage
        (False, 512, 512, 512, 64, 1.0, 0.0, False, 0),  # batched, one tile per CU, no C
        (False, 1024, 1024, 1024, 16, 1.5, 0.5, True, 0),  # batched with C, K >= 1024
    ],
)
def test_gemm_direct_b_matches_lds_tile(hip, dt, ta, M, N, K, batch, alpha, beta, with_c, ldd_pad):
    """B row-major, N even (fp64) or a multiple of 256 (fp32): the kernel that
    loads B straight into the MFMA registers, or, for fp32 problems of whole
    256 x 256 tiles filling the chip, the 256 x 256 tile. Checked against
    float64 torch, and bitwise against the LDS-staged tiles, which the same
    problem takes when B's leading dimension breaks 16-byte alignment (no
    vector path)."""
    from trntensor_amd.hip import engine

    g = torch.Generator().manual_seed(M + N + K + batch + int(ta))
    dev = torch.device("cuda")
    V = 16 // torch.tensor([], dtype=dt).element_size()  # elements per 16 bytes
    up = lambda n: n + (-n) % V  # noqa: E731
    ldb_odd = N + 1 if (N + 1) % 2 else N + 2
    a_rows, a_cols = (K, M) if ta else (M, K)
    lda = up(a_cols)  # A's 16-byte vector path
    ldb_even = up(N)
    A = torch.randn(batch, a_rows, lda, generator=g, dtype=torch.float64)
    B = torch.randn(batch, K, max(ldb_odd, ldb_even), generator=g, dtype=torch.float64)
    ld = up(N + 1) + 1 if ldd_pad else up(N + 1)  # unaligned (element stores) or aligned, above N
    C = torch.randn(batch, M, ld, generator=g, dtype=torch.float64)
    opA = A[:, :, :a_cols].transpose(1, 2) if ta else A[:, :, :a_cols]
    ref = alpha * torch.bmm(opA, B[:, :, :N])
    if with_c:
        ref = ref + beta * C[:, :, :N]
    Ad, Cd = A.to(dev, dt), C.to(dev, dt)
    Bn = B[:, :, :ldb_even].contiguous().to(dev, dt)  # aligned ldb: the direct-B kernel
    Bo = B[:, :, :ldb_odd].contiguous().to(dev, dt)  # odd ldb: the LDS-staged tiles only
    outs = []
    for Bd, ldb in ((Bn, ldb_even), (Bo, ldb_odd)):
        D = torch.full((batch, M, ld), float("nan"), dtype=dt, device=dev)
        engine.gemm(ta, False, M, N, K, Ad, lda, a_rows * lda, Bd, ldb, K * ldb, D, ld, M * ld, batch, alpha, beta,
                    Cd if with_c else None, ld, M * ld)
        outs.append(D)
    torch.cuda.synchronize()
    direct, staged = outs[0][:, :, :N], outs[1][:, :, :N]
    assert normwise(direct.cpu().double(), ref) <= TOL[dt]
    assert torch.equal(direct, staged)
    assert torch.isnan(outs[0][:, :, N:]).all()  # nothing stored past column N


@pytest.mark.parametrize(
    "ta,M,N,K,batch,alpha,beta,with_c,ldd_pad",
    [
        (False, 256, 512, 800, 1, 1.0, 0.0, False, 0),  # NT, the fused config-5 GEMM's shape family
        (True, 64, 1024, 512, 1, 1.0, 0.0, False, 0),  # TT, M <= 64: non-temporal B loads
        (False, 50, 256, 37, 2, 1.5, 0.5, True, 1),  # M < 64, K tail, element stores
        (True, 200, 384, 333, 3, -1.0, 1.0, True, 0),  # ragged M and K, batched
        (False, 33, 128, 7, 2, 0.5, 2.0, True, 1),  # one partial stage only
        (True, 128, 256, 16, 1, 1.0, 0.25, True, 0),  # one full stage only
        (False, 192, 200, 64, 1, 1.0, 0.0, False, 0),  # partial last column tile
        (True, 70, 1030, 100, 2, 1.5, 0.5, True, 1),  # partial last column tile, ragged M
    ],
)
def test_gemm_direct_b_k_contiguous_matches_lds_tile(hip, ta, M, N, K, batch, alpha, beta, with_c, ldd_pad):
    """fp64 with B stored [n][k] (k-contiguous), N even: the
    direct-B kernel with 16-byte k pieces. Checked against float64 torch, and
    bitwise against the LDS-staged tiles (reached with an odd ldb)."""
    from trntensor_amd.hip import engine

    dt = torch.float64
    g = torch.Generator().manual_seed(7 * M + N + K + batch + int(ta))
    dev = torch.device("cuda")
    a_rows, a_cols = (K, M) if ta else (M, K)
    lda = a_cols + a_cols % 2
    ldb_even = K + K % 2
    ldb_odd = K + 1 if K % 2 == 0 else K
    A = torch.randn(batch, a_rows, lda, generator=g, dtype=dt)
    B = torch.randn(batch, N, max(ldb_even, ldb_odd), generator=g, dtype=dt)
    ld = N + 1 if ldd_pad else N
    C = torch.randn(batch, M, ld, generator=g, dtype=dt)
    opA = A[:, :, :a_cols].transpose(1, 2) if ta else A[:, :, :a_cols]
    ref = alpha * torch.bmm(opA, B[:, :, :K].transpose(1, 2).contiguous())
    if with_c:
        ref = ref + beta * C[:, :, :N]
    Ad, Cd = A.to(dev), C.to(dev)
    outs = []
    for ldb in (ldb_even, ldb_odd):
        Bd = B[:, :, :ldb].contiguous().to(dev)
        assert Bd.shape == (batch, N, ldb) and ldb >= K  # rows of K elements, N of them per batch entry
        D = torch.full((batch, M, ld), float("nan"), dtype=dt, device=dev)
        engine.gemm(ta, True, M, N, K, Ad, lda, a_rows * lda, Bd, ldb, N * ldb, D, ld, M * ld, batch, alpha, beta,
                    Cd if with_c else None, ld, M * ld)
        outs.append(D)
    torch.cuda.synchronize()
    direct, staged = outs[0][:, :, :N], outs[1][:, :, :N]
    assert normwise(direct.cpu(), ref) <= TOL[dt]
    assert torch.equal(direct, staged)
    if ld > N:
        assert torch.isnan(outs[0][:, :, N:]).all()  # nothing stored past column N


@pytest.mark.parametrize(
    "ta,tb,M,N,K,batch,with_e2",
    [
        (False, True, 256, 512, 800, 1, True),  # the fused config-5 dot GEMM's shape family
        (False, True, 64, 256, 100, 2, False),  # M = 64: non-temporal B loads
        (True, False, 128, 384, 37, 3, True),  # K tail, B row-major
        (True, True, 192, 128, 16, 1, False),
        (False, True, 4224, 256, 64, 1, True),  # 66 row tiles: the grouped row order of config 5's GEMM
        (False, True, 400, 256, 800, 1, True),  # ragged M: config 5's optimal-order dot GEMM, transposed
        (True, False, 200, 384, 37, 2, False),  # ragged M and K tail, B row-major
        (False, False, 33, 128, 16, 1, True),  # one partial row tile
    ],
)
def test_gemm_dot_direct_b_matches_lds_tile(hip, ta, tb, M, N, K, batch, with_e2):
    """fp64 dot GEMM (sum of op(A) op(B) .* E1 .* E2) with N a multiple of 128
    (any M; rows past M are left out of the sum): the direct-B kernel's dot
    epilogue. Against float64 torch, and
    against the LDS-staged tiles (odd ldb) to 1e-13 relative: the per-tile sums
    are added in another order."""
    from trntensor_amd.hip import engine

    dt = torch.float64
    g = torch.Generator().manual_seed(M + 3 * N + K + batch)
    dev = torch.device("cuda")
    a_rows, a_cols = (K, M) if ta else (M, K)
    b_rows, b_cols = (N, K) if tb else (K, N)
    lda = a_cols + a_cols % 2
    ldb_even = b_cols + b_cols % 2
    ldb_odd = b_cols + 1 if b_cols % 2 == 0 else b_cols
    A = torch.randn(batch, a_rows, lda, generator=g, dtype=dt)
    B = torch.randn(batch, b_rows, max(ldb_even, ldb_odd), generator=g, dtype=dt)
    E1 = torch.randn(batch, M, N, generator=g, dtype=dt)
    E2 = torch.randn(batch, M, N, generator=g, dtype=dt) if with_e2 else None
    opA = A[:, :, :a_cols].transpose(1, 2) if ta else A[:, :, :a_cols]
    opB = B[:, :, :b_cols].transpose(1, 2) if tb else B[:, :, :b_cols]
    X = torch.bmm(opA.contiguous(), opB.contiguous())
    ref = float((X * E1 * (E2 if with_e2 else 1.0)).sum())
    es = [0, N, 0, 1, M * N]  # E[b, m, n]: m_lo extent M, n_lo extent N
    outs = []
    for ldb in (ldb_even, ldb_odd):
        Bd = B[:, :, :ldb].contiguous().to(dev)
        assert Bd.shape == (batch, b_rows, ldb) and ldb >= b_cols
        out = torch.zeros(1, dtype=dt, device=dev)
        engine.gemm_dot(ta, tb, M, N, K, A.to(dev), lda, a_rows * lda, Bd, ldb, b_rows * ldb, batch, M, N, E1.to(dev), es,
                        E2.to(dev) if with_e2 else None, es if with_e2 else None, 1.0, 0.0, None, out)
        outs.append(float(out.cpu()))
    direct, staged = outs
    scale = float((X.abs() * E1.abs() * (E2.abs() if with_e2 else 1.0)).sum())
    assert abs(direct - ref) <= 1e-13 * scale
    assert abs(direct - staged) <= 1e-13 * scale


def test_gemm_k_zero_is_beta_c(hip):
    assert _gemm_case(hip, torch.float64, False, False, 9, 11, 0, 2, 1.5, 0.5, True) == 0.0


def test_gemm_rejects_bad_arguments(hip):
    from trntensor_amd.hip import engine

    A = torch.zeros(4, 4, dtype=torch.float64, device="cuda")
    with pytest.raises(ValueError, match="leading dimension"):
        engine.gemm(False, False, 4, 4, 4, A, 2, 0, A, 4, 0, A, 4, 0)
    with pytest.raises(NotImplementedError, match="float32/float64"):
        engine.gemm(False, False, 2, 2, 2, A.int(), 2, 0, A.int(), 2, 0, A.int(), 2, 0)


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize(
    "sub,shapes",
    [
        ("ii->", [(37, 37)]),
        ("ij->ji", [(33, 65)]),
        ("ijk->kj", [(5, 7, 9)]),
        ("i,i->", [(100003,), (100003,)]),
        ("i,j->ij", [(130,), (70,)]),
        ("ij,ij->ij", [(40, 50), (40, 50)]),
        ("ij,jk->i", [(20, 30), (30, 10)]),
        ("bij,bjk->bik", [(3, 4, 5), (3, 5, 6)]),
        ("iajb,abij->", [(6, 5, 7, 4), (5, 4, 6, 7)]),
    ],
)
def test_strided_contract_vs_numpy(hip, dt, sub, shapes):
    from trntensor_amd.hip import engine

    g = torch.Generator().manual_seed(3)
    ops = [torch.randn(*s, generator=g, dtype=torch.float64) for s in shapes]
    ref = torch.from_numpy(np.asarray(brute.einsum_f64(sub, *[o.numpy() for o in ops])))
    lhs, out = sub.split("->")
    res = engine.contract(lhs.split(","), out, [o.to("cuda", dt) for o in ops])
    torch.cuda.synchronize()
    assert normwise(res, ref) <= (1e-12 if dt == torch.float64 else 1e-5)


def test_strided_split_reduction_matches_single_pass(hip):
    """A reduction long enough to use partials agrees with float64 numpy."""
    from trntensor_amd.hip import engine

    g = torch.Generator().manual_seed(4)
    x = torch.randn(3, 2_000_000, generator=g, dtype=torch.float64)
    y = torch.randn(3, 2_000_000, generator=g, dtype=torch.float64)
    res = engine.contract(["ij", "ij"], "i", [x.cuda(), y.cuda()])
    ref = (x * y).sum(1)
    assert normwise(res, ref) <= 1e-12


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize(
    "sub,shapes",
    [
        # column tiles: the output's innermost letter is the operands' contiguous one
        ("ijk->k", [(70, 300, 129)]),
        ("ijk->jk", [(500, 33, 260)]),
        ("ijk,ijk->k", [(40, 300, 77), (40, 300, 77)]),
        ("ij,ij->j", [(5000, 3)]),
        # transpose tiles: permutations whose innermost output letter is strided
        ("ij->ji", [(1000, 333)]),
        ("ijk->kji", [(70, 65, 130)]),
        ("abcd->dbca", [(9, 70, 5, 66)]),
        ("abc->bca", [(130, 3, 200)]),
    ],
)
def test_strided_schedules(hip, dt, sub, shapes):
    """The column-tile and transpose-tile schedules against float64 numpy,
    with and without the alpha/beta epilogue."""
    from trntensor_amd.hip import engine

    g = torch.Generator().manual_seed(7)
    lhs, out = sub.split("->")
    terms = lhs.split(",")
    if len(terms) == 2 and len(shapes) == 1:
        shapes = shapes * 2
    ops = [torch.randn(*s, generator=g, dtype=torch.float64) for s in shapes]
    ref = torch.from_numpy(np.asarray(brute.einsum_f64(sub, *[o.numpy() for o in ops])))
    res = engine.contract(terms, out, [o.to("cuda", dt) for o in ops])
    assert normwise(res, ref) <= (1e-12 if dt == torch.float64 else 1e-5)
    C = torch.randn(*ref.shape, generator=g, dtype=torch.float64)
    res = engine.contract(terms, out, [o.to("cuda", dt) for o in ops], 1.5, -0.5, C.to("cuda", dt))
    assert normwise(res, 1.5 * ref - 0.5 * C) <= (1e-12 if dt == torch.float64 else 1e-5)


def test_coltile_double_double(hip):
    """'ijk->k' through the column-tile schedule with double-double partials:
    sums that cancel to a few units are exact, where float64 partials are not."""
    from trntensor_amd.hip import engine

    n = 1 << 16
    base = torch.tensor([1e16, 1.0, -1e16, 1.0], dtype=torch.float64)
    x = base.repeat(n // 4)[:, None].expand(n, 96).contiguous().view(n // 64, 64, 96)
    with engine.accumulation("dd"):
        got = engine.contract(["ijk"], "k", [x.cuda()])
    assert torch.equal(got.cpu(), torch.full((96,), float(n // 2), dtype=torch.float64))


@pytest.mark.parametrize(
    "code,dt,expected_per_iter,tol",
    [
        # Lane 0 holds rows {0,4,8,12} (f64) or {0,1,2,3} (f32, 16-bit) of
        # column 0 in each of 8 identical chains; operand of lane l is
        # ((l & 7) + 1) * s and ((l >> 3 & 7) + 1) * s, s = 1e-6 (1e-3 for
        # 16-bit), so per iteration D[i][0] = ((i & 7) + 1) * (1+3+5+7) s^2
        # (times 8 for the 32-deep 16-bit MFMA).
        (1, torch.float64, 8 * 12 * 16e-12, 1e-12),
        (0, torch.float32, 8 * 10 * 16e-12, 1e-4),
        (3, torch.bfloat16, 8 * 10 * 128e-6, 2e-2),
        (4, torch.float16, 8 * 10 * 128e-6, 2e-2),
    ],
)
def test_mfma_rate_probe_closed_form(hip, code, dt, expected_per_iter, tol):
    """The measurement probe really issues `iters` rounds of its MFMA chains:
    workgroup 0's value against the closed form of the operand pattern."""
    from trntensor_amd.hip import _lib

    lib = _lib.load()
    out = torch.zeros(4, dtype=dt, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.tt_mfma_rate_probe(code, 4, 100, out.data_ptr(), st), "tt_mfma_rate_probe")
    torch.cuda.synchronize()
    got = out.double().cpu()
    want = 100 * expected_per_iter
    assert abs(got[0].item() - want) <= tol * want
    assert torch.equal(got, got[:1].expand(4))
    with pytest.raises(ValueError):
        _lib.check(lib.tt_mfma_rate_probe(code, 0, 1, out.data_ptr(), st), "tt_mfma_rate_probe")
    with pytest.raises(NotImplementedError):
        _lib.check(lib.tt_mfma_rate_probe(2, 1, 1, out.data_ptr(), st), "tt_mfma_rate_probe")


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize("M,ntiles,K,batch,alpha", [
    (64, 3104, 512, 1, 1.0),           # the AO->MO half transform's shape class (B streamed, M <= 64)
    (64, 3100, 16, 1, 1.5),            # one k-stage per tile
    (128, 3120, 48, 1, 1.0),           # two row tiles per column tile
    (192, 3120, 64, 8, -0.5),          # batched, three row tiles: tiles cross batch entries
    (64, 3105, 64, 1, 1.0),            # N not a multiple of 256: fp64 keeps the 64 x 128 kernel
    (64, 3104, 32, 2, 2.0),            # fp64 streaming kernel, batched: tiles cross batch entries
])
def test_gemm_persistent_matches_per_tile_kernel(hip, dt, M, ntiles, K, batch, alpha):
    """A transposed, B row-major, no C, three or more rounds of 64-row tiles:
    the persistent direct-B kernel (each workgroup walks a list of tiles, the
    next tile's first stage loaded during the current tile's last MFMAs), or
    for fp64 with at most two row tiles and N a multiple of 256 its streaming
    variant (64 x 256 tiles, two workgroups per CU).
    Bitwise equal to the per-tile direct-B kernel, which the same columns take
    in a launch of fewer tiles (the two keep one MFMA order per output), and
    checked against float64 torch on sampled columns."""
    from trntensor_amd.hip import engine

    dev = torch.device("cuda")
    BN = 128 if dt == torch.float64 else 256
    nb = ntiles // ((M // 64) * batch)  # column tiles per batch entry
    N = nb * BN
    assert (M // 64) * nb * batch >= 3 * 1024  # three rounds on a 256-CU device
    g = torch.Generator(device=dev).manual_seed(M + K + batch)
    A = torch.randn(batch, K, M, generator=g, device=dev, dtype=torch.float64).to(dt)  # stored [k][m]
    B = torch.randn(batch, K, N, generator=g, device=dev, dtype=torch.float64).to(dt)
    D = torch.full((batch, M, N), float("nan"), dtype=dt, device=dev)
    engine.gemm(True, False, M, N, K, A, M, K * M, B, N, K * N, D, N, M * N, batch, alpha)
    # The same columns in launches of 16 column tiles (per-tile kernel),
    # reading B and writing D in place through offsets (ldb = ldd = N).
    P = torch.full_like(D, float("nan"))
    for c0 in list(range(0, min(N, 4 * 16 * BN), 16 * BN)) + [N - 16 * BN]:
        engine.gemm(True, False, M, 16 * BN, K, A, M, K * M, B, N, K * N, P, N, M * N, batch, alpha,
                    b_off=c0, d_off=c0)
    torch.cuda.synchronize()
    cols = torch.cat([torch.arange(0, min(N, 4 * 16 * BN)), torch.arange(N - 16 * BN, N)]).to(dev)
    assert torch.equal(D[:, :, cols], P[:, :, cols])
    ref = alpha * torch.bmm(A[:, :, :].transpose(1, 2).double().cpu(), B[:, :, cols].double().cpu())
    assert normwise(D[:, :, cols].cpu(), ref) <= TOL[dt]
    assert not torch.isnan(D).any()


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize("M,N,K,batch", [(32, 32, 96, 1), (32, 32, 128, 3), (17, 29, 64, 2), (1, 32, 5, 1),
                                         (32, 7, 33, 5), (32, 32, 64, 1), (30, 31, 127, 1)])
@pytest.mark.parametrize("alpha,beta,with_c", [(1.0, 0.0, False), (1.5, 0.5, True)])
def test_gemm_small_tile_matches_wide_tiles(hip, dt, M, N, K, batch, alpha, beta, with_c):
    """M, N <= 32 with both operands k-contiguous and K within one deep stage
    (config 1's 'ap,bp->ab', 32 x 32 x 96): the 32 x 32 single-stage tile.
    Checked against float64 torch, and bitwise against the same outputs as
    part of a wider problem (M = 40 takes the 64-row tiles; the extra rows
    do not change the first M), which keeps the k order per output."""
    from trntensor_amd.hip import engine

    g = torch.Generator().manual_seed(M * 7 + N + K + batch)
    dev = torch.device("cuda")
    Mw = 40
    A = torch.randn(batch, Mw, K, generator=g, dtype=torch.float64)
    B = torch.randn(batch, N, K, generator=g, dtype=torch.float64)
    C = torch.randn(batch, Mw, N, generator=g, dtype=torch.float64)
    ref = alpha * torch.bmm(A[:, :M], B.transpose(1, 2).contiguous())
    if with_c:
        ref = ref + beta * C[:, :M]
    Ad, Bd, Cd = A.to(dev, dt), B.to(dev, dt), C.to(dev, dt)
    outs = []
    for m in (M, Mw):
        D = torch.full((batch, Mw, N), float("nan"), dtype=dt, device=dev)
        engine.gemm(False, True, m, N, K, Ad, K, Mw * K, Bd, K, N * K, D, N, Mw * N, batch, alpha, beta,
                    Cd if with_c else None, N, Mw * N)
        outs.append(D[:, :M])
    torch.cuda.synchronize()
    assert normwise(outs[0], ref) <= TOL[dt]
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("with_c", [False, True])
def test_gemm_big_tile_broadcast_b(hip, with_c):
    """fp32 batched products sharing one B (batch stride 0, the engine's
    broadcast of an unbatched operand), whole 256 x 256 tiles filling the
    chip: the 256 x 256 LDS tile (with C only for K >= 1024). Checked against
    float64 torch, and bitwise against the LDS-staged tiles, which take the
    same problem when B's leading dimension breaks 16-byte alignment."""
    from trntensor_amd.hip import engine

    dev = torch.device("cuda")
    batch, M, N = 64, 512, 512
    K = 1024 if with_c else 512
    g = torch.Generator().manual_seed(K + batch)
    A = torch.randn(batch, M, K, generator=g, dtype=torch.float64)
    B = torch.randn(K, N + 1, generator=g, dtype=torch.float64)
    C = torch.randn(batch, M, N, generator=g, dtype=torch.float64)
    ref = 1.5 * torch.matmul(A, B[:, :N])
    if with_c:
        ref = ref + 0.5 * C
    Ad, Cd = A.to(dev, torch.float32), C.to(dev, torch.float32)
    Bn = B[:, :N].contiguous().to(dev, torch.float32)  # ldb = N: the 256 x 256 tile
    Bo = B.contiguous().to(dev, torch.float32)  # ldb = N + 1: the LDS-staged tiles
    outs = []
    for Bd, ldb in ((Bn, N), (Bo, N + 1)):
        D = torch.full((batch, M, N), float("nan"), dtype=torch.float32, device=dev)
        engine.gemm(False, False, M, N, K, Ad, K, M * K, Bd, ldb, 0, D, N, M * N, batch, 1.5, 0.5,
                    Cd if with_c else None, N, M * N)
        outs.append(D)
    torch.cuda.synchronize()
    assert normwise(outs[0].cpu().double(), ref) <= TOL[torch.float32]
    assert torch.equal(outs[0], outs[1])
