"""bfloat16 / float16 contractions: GEMM shapes run on the 16-bit MFMA GEMM
(tt_gemm with TT_BF16 / TT_F16: fp32 products and sums, alpha/beta in fp32,
one rounding at the store); every other shape is widened to float32.

The reference computes these in torch on the CPU in the 16-bit dtype
(trntensor/einsum.py:94-103 with dtype="bf16"), whose rounding of partial
results is torch's own. The expected value here is the float32 product of the
same 16-bit inputs (exact widening), rounded once to the 16-bit dtype; the
bar is normwise 1e-2 (bf16, 8-bit mantissa) and 2e-3 (fp16), i.e. a few
16-bit ulps plus fp32 summation-order differences.
"""

import pytest
import torch

import trntensor_amd as trntensor
from tests.util import normwise
from trntensor_amd.hip import engine

pytestmark = pytest.mark.gpu

BAR = {torch.bfloat16: 1e-2, torch.float16: 2e-3}


def _native_used(dt):
    return any(k[7] == dt for k in engine._RECIPES)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(
    "sub,shapes",
    [
        ("ij,jk->ik", [(256, 192), (192, 384)]),
        ("ij,jk->ik", [(200, 150), (150, 130)]),  # ragged tiles and K
        ("ji,jk->ik", [(150, 200), (150, 130)]),
        ("ij,kj->ik", [(200, 150), (130, 150)]),
        ("ji,kj->ik", [(150, 200), (130, 150)]),
        ("ij,jk->ki", [(200, 150), (150, 130)]),  # swapped output
        ("bij,bjk->bik", [(3, 130, 70), (3, 70, 140)]),
        ("ap,bp->ab", [(320, 1200), (320, 1200)]),  # DF-MP2 pair block
    ],
)
def test_gemm_shapes_native(hip, dt, sub, shapes):
    g = torch.Generator().manual_seed(5)
    ops = [torch.randn(*s, generator=g).to(dt) for s in shapes]
    engine._RECIPES.clear()
    got = trntensor.einsum(sub, *[o.cuda() for o in ops])
    assert got.dtype == dt
    assert _native_used(dt)
    want = torch.einsum(sub, *[o.float() for o in ops]).to(dt)
    assert normwise(got.float(), want.float()) <= BAR[dt]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_alpha_beta_out(hip, dt):
    g = torch.Generator().manual_seed(6)
    A, B, C = (torch.randn(*s, generator=g).to(dt) for s in ((130, 90), (90, 150), (130, 150)))
    got = trntensor.einsum("ij,jk->ik", A.cuda(), B.cuda(), alpha=1.5, beta=-0.5, out=C.cuda())
    want = (1.5 * (A.float() @ B.float()) - 0.5 * C.float()).to(dt)
    assert normwise(got.float(), want.float()) <= BAR[dt]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(
    "sub,shapes",
    [
        ("ij,ij->", [(64, 80), (64, 80)]),  # no GEMM shape: widened
        ("ijk,jk->i", [(40, 30, 20), (30, 20)]),  # K over two letters in place
        ("iaj,jb->iab", [(20, 30, 40), (40, 50)]),
    ],
)
def test_other_shapes(hip, dt, sub, shapes):
    g = torch.Generator().manual_seed(7)
    ops = [torch.randn(*s, generator=g).to(dt) for s in shapes]
    got = trntensor.einsum(sub, *[o.cuda() for o in ops])
    assert got.dtype == dt
    want = torch.einsum(sub, *[o.float() for o in ops]).to(dt)
    assert normwise(got.float(), want.float()) <= BAR[dt]


def test_dtype_string_bf16_large(hip):
    """einsum(dtype="bf16") on fp32 inputs at 2048^3: cast, native GEMM, bf16 result."""
    g = torch.Generator().manual_seed(8)
    A = torch.randn(2048, 2048, generator=g).cuda()
    B = torch.randn(2048, 2048, generator=g).cuda()
    got = trntensor.einsum("ij,jk->ik", A, B, dtype="bf16")
    assert got.dtype == torch.bfloat16
    want = (A.bfloat16().float() @ B.bfloat16().float()).bfloat16()
    assert normwise(got.float(), want.float()) <= 1e-2


def _gemm16_case(dt, ta, tb, M, N, K, batch, alpha, beta, with_c, pad=0, alias=False, seed=0, ld_align=0):
    """tt_gemm with TT_BF16/TT_F16 through engine.gemm against the float64
    product of the same 16-bit inputs, rounded once to the 16-bit dtype.
    Leading dimensions are the widths plus `pad`, or (ld_align > 0) each width
    rounded up to a multiple of ld_align."""
    g = torch.Generator().manual_seed(seed)
    dev = torch.device("cuda")
    a_rows, a_cols = (K, M) if ta else (M, K)
    b_rows, b_cols = (N, K) if tb else (K, N)
    if ld_align:
        pa, pb, pc = -a_cols % ld_align, -b_cols % ld_align, -N % ld_align
    else:
        pa = pb = pc = pad
    A = torch.randn(batch, a_rows, a_cols + pa, generator=g).to(dt)
    B = torch.randn(batch, b_rows, b_cols + pb, generator=g).to(dt)
    C = torch.randn(batch, M, N + pc, generator=g).to(dt)
    opA = A[:, :, :a_cols].double().transpose(1, 2) if ta else A[:, :, :a_cols].double()
    opB = B[:, :, :b_cols].double().transpose(1, 2) if tb else B[:, :, :b_cols].double()
    ref = alpha * torch.bmm(opA, opB)
    if with_c:
        ref = ref + beta * C[:, :, :N].double()
    ref = ref.to(dt)
    Ad, Bd, Cd = A.to(dev), B.to(dev), C.to(dev)
    D = Cd if alias else torch.full((batch, M, N + pc), float("nan"), dtype=dt, device=dev)
    engine.gemm(
        ta, tb, M, N, K,
        Ad, a_cols + pa, a_rows * (a_cols + pa),
        Bd, b_cols + pb, b_rows * (b_cols + pb),
        D, N + pc, M * (N + pc), batch, alpha, beta,
        Cd if with_c else None, N + pc, M * (N + pc),
    )
    torch.cuda.synchronize()
    return normwise(D[:, :, :N].float().cpu(), ref.float())


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize(
    "M,N,K,batch,pad",
    [
        (1, 1, 1, 1, 0),
        (130, 136, 72, 1, 0),
        (264, 272, 96, 2, 0),
        (200, 150, 70, 2, 0),
        (96, 88, 40, 3, 3),
        (300, 520, 100, 2, 0),
        (512, 512, 512, 2, 0),
        (264, 300, 129, 1, 3),
        (520, 264, 1056, 1, 0),
        (256, 512, 1024, 2, 0),
        (256, 256, 256, 2, 0),
        (384, 256, 512, 1, 0),
        (256, 256, 2560, 1, 0),
        (200, 300, 512, 2, 0),
        (256, 512, 256, 64, 0),
        (1032, 1024, 256, 16, 0),
        (256, 512, 256, 16, 0),
        (2056, 1024, 256, 1, 0),
        (256, 512, 2560, 128, 0),
    ],
)
def test_gemm16_epilogue_alpha_beta(hip, dt, ta, tb, M, N, K, batch, pad):
    """Aligned leading dimensions (multiples of 8) take the 16-byte epilogue,
    odd ones (pad 3) and ragged column blocks the element-wise one. M, N >= 256
    with aligned operands, K a multiple of 32 of at least 256, at least 64
    whole tiles and ragged strips of at most 1/64 of the outputs run whole
    tiles on the direct-load kernel and the strips on the register-staged one
    (16 x 1032 x 1024 x 256, 2056 x 1024 x 256). Its tiles are 128 x 256
    (64 x 256 x 512 x 256, 16 x 1032 x 1024 x 256), 256 x 256 for NT beyond
    K = 2048 (128 x 256 x 512 x 2560), and 128 x 128 when fewer than 256
    tiles of 128 x 256 exist (16 x 256 x 512 x 256, 2056 x 1024 x 256). The
    smaller shapes run on the register-staged kernel alone."""
    assert _gemm16_case(dt, ta, tb, M, N, K, batch, 1.5, -0.5, True, pad=pad, seed=M) <= BAR[dt]
    assert _gemm16_case(dt, ta, tb, M, N, K, batch, 1.0, 0.0, False, pad=pad, seed=M + 1) <= BAR[dt]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("M,N,K", [(130, 130, 130), (131, 133, 129), (128, 128, 131), (70, 33, 131)])
def test_gemm16_aligned_ld_straddling_pieces(hip, dt, ta, tb, M, N, K):
    """Leading dimensions rounded up to multiples of 8 (16-byte pieces on) with
    M, N or K not multiples of 8: edge tiles mix whole pieces, pieces outside
    and pieces straddling the edge."""
    assert _gemm16_case(dt, ta, tb, M, N, K, 1, 1.0, 0.0, False, ld_align=8, seed=M + N) <= BAR[dt]
    assert _gemm16_case(dt, ta, tb, M, N, K, 2, 1.5, -0.5, True, ld_align=8, seed=K) <= BAR[dt]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_gemm16_d_aliases_c(hip, dt):
    """D may alias C exactly (header contract): D = alpha * AB + beta * D."""
    assert _gemm16_case(dt, False, True, 136, 264, 64, 2, 0.5, 2.0, True, alias=True, seed=3) <= BAR[dt]
    assert _gemm16_case(dt, True, False, 100, 90, 33, 1, 0.5, 2.0, True, pad=1, alias=True, seed=4) <= BAR[dt]
    assert _gemm16_case(dt, False, False, 256, 512, 1024, 2, 0.5, 2.0, True, alias=True, seed=5) <= BAR[dt]
    assert _gemm16_case(dt, True, True, 520, 264, 1056, 1, 0.5, 2.0, True, alias=True, seed=6) <= BAR[dt]
    # the direct-load kernel (whole tiles) and its ragged strips
    assert _gemm16_case(dt, False, True, 256, 512, 256, 64, 0.5, 2.0, True, alias=True, seed=7) <= BAR[dt]
    assert _gemm16_case(dt, True, False, 1032, 1024, 256, 16, 0.5, 2.0, True, alias=True, seed=8) <= BAR[dt]
    assert _gemm16_case(dt, True, True, 2056, 1024, 256, 1, 0.5, 2.0, True, alias=True, seed=9) <= BAR[dt]
