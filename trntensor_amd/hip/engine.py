"""Contraction engine: maps any one- or two-operand einsum onto the HIP kernels.

Every contraction on the path ends up in one of two kernels of
libtrntensor_hip.so:

- ``tt_gemm`` (MFMA core) when the contraction has a GEMM shape: letters
  shared by both operands and the output form the batch, letters of one
  operand and the output form M (of A) or N (of B), letters shared by both
  operands but absent from the output form K. Each group must collapse to one
  (extent, stride) pair in the operand and either K or the row group must be
  unit-stride; otherwise the operand is first packed contiguously by
  ``tt_strided_contract``. The output is written in place when its letter
  order is batch+M+N (or batch+N+M, by swapping the operands), else through a
  packed temporary and one permuting pass.
- ``tt_strided_contract`` for everything without a GEMM shape: outer
  products, elementwise products, traces, dots, permutations, letters summed
  away, tiny matrix dimensions.

The mapping is derived from letter positions and strides, never from the
reference planner's strategy label, so index orders the reference's
matmul/bmm executors mishandle (output order, summed free letters, bmm index
positions; reference trntensor/plan.py:284-305) are computed as einsum
defines them.
"""

from __future__ import annotations

import contextlib
import contextvars
import ctypes

import torch

from . import _lib

_MAX_INDEX = (1 << 31) - 1

# Accumulation of float64 launches: "native" (float64) or "dd" (double-double,
# dtype code TT_F64_DD). Set for a block of calls with `accumulation(...)`.
_ACCUMULATION: contextvars.ContextVar[str] = contextvars.ContextVar("tt_accumulation", default="native")


@contextlib.contextmanager
def accumulation(mode: str):
    """Run the enclosed float64 launches with `mode` accumulation ("native" | "dd")."""
    if mode not in ("native", "dd"):
        raise ValueError(f"accumulation mode {mode!r}")
    token = _ACCUMULATION.set(mode)
    try:
        yield
    finally:
        _ACCUMULATION.reset(token)


def dtype_code(dt: torch.dtype) -> int:
    """Library dtype code of a launch on `dt` data (bfloat16/float16: tt_gemm only)."""
    if dt == torch.float64:
        return _lib.TT_F64_DD if _ACCUMULATION.get() == "dd" else _lib.TT_F64
    if dt == torch.float32:
        if _ACCUMULATION.get() == "dd":
            raise NotImplementedError("double-double accumulation needs float64 data")
        return _lib.TT_F32
    if dt == torch.bfloat16:
        return _lib.TT_BF16
    if dt == torch.float16:
        return _lib.TT_F16
    if dt == torch.int64:
        return _lib.TT_I64
    raise NotImplementedError(f"HIP kernels compute in float32/float64 (bfloat16/float16 GEMMs, int64 strided), not {dt}")


# Raw handle of torch's current stream on a device index (what
# torch.cuda.current_stream(device).cuda_stream returns, without building a
# Stream object: a few microseconds per launch on small contractions).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_ptr(device: torch.device) -> int:
    """torch's current stream on `device`, the stream every launch is enqueued on."""
    if _raw_stream is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    """Device address of `t` (ctypes passes an int for a void* argument), or NULL."""
    return None if t is None else t.data_ptr()


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------
# letter bookkeeping
# ---------------------------------------------------------------------------
class Operand:
    """A tensor view with one letter per dimension (no repeats)."""

    __slots__ = ("t", "letters", "ext", "strd")

    def __init__(self, term: str, t: torch.Tensor):
        # Repeated letters select a diagonal: one dimension whose stride is the
        # sum of the repeated dimensions' strides (a view, no data movement).
        letters: list[str] = []
        ext: list[int] = []
        strd: list[int] = []
        for c, n, s in zip(term, t.shape, t.stride()):
            if c in letters:
                strd[letters.index(c)] += s
            else:
                letters.append(c)
                ext.append(int(n))
                strd.append(int(s))
        self.t = t
        self.letters = letters
        self.ext = dict(zip(letters, ext))
        self.strd = dict(zip(letters, strd))


def _merge(op: Operand, letters: list[str]) -> tuple[int, int] | None:
    """Collapse `letters` (outer to inner) of `op` into one (extent, stride), or None."""
    extent, stride = 1, 0
    for c in reversed(letters):
        n, s = op.ext[c], op.strd[c]
        if n == 1:
            continue
        if extent == 1:
            extent, stride = n, s
        elif s == stride * extent:
            extent *= n
        else:
            return None
    return extent, stride


def _numel(exts) -> int:
    r = 1
    for n in exts:
        r *= int(n)
    return r


# ---------------------------------------------------------------------------
# strided multiply-reduce
# ---------------------------------------------------------------------------
def _merge_dims(dims: list[tuple[int, int, int]]) -> list[tuple[int, int, int]]:
    """Merge adjacent (extent, a_stride, b_stride) dims that are jointly contiguous;
    drop extent-1 dims. Used for output dims (the output itself is row-major in
    this order, so its strides always merge) and reduction dims."""
    out: list[list[int]] = []
    for n, sa, sb in dims:
        if n == 1:
            continue
        if out:
            pn, psa, psb = out[-1]
            if psa == sa * n and psb == sb * n:
                out[-1] = [pn * n, sa, sb]
                continue
        out.append([n, sa, sb])
    return [tuple(d) for d in out]


def strided_contract(
    out_dims: list[tuple[int, int, int]],
    red_dims: list[tuple[int, int, int]],
    A: torch.Tensor,
    B: torch.Tensor | None,
    D: torch.Tensor,
    alpha: float = 1.0,
    beta: float = 0.0,
    C: torch.Tensor | None = None,
    a_off: int = 0,
    b_off: int = 0,
) -> None:
    """D (contiguous, out_dims order) = alpha * sum_red A*B (+ beta*C), via tt_strided_contract.

    Dims are (extent, stride in A, stride in B), element strides relative to
    A/B's first element (``data_ptr()``) plus a_off/b_off. Launches are split so every index
    range stays below 2^31.
    """
    lib = _lib.load()
    out_dims = _merge_dims(out_dims)
    red_dims = _merge_dims(red_dims)
    n_out = _numel(d[0] for d in out_dims)
    n_red = _numel(d[0] for d in red_dims)
    if n_out == 0:
        return
    if len(out_dims) > _lib.TT_MAX_DIMS or len(red_dims) > _lib.TT_MAX_DIMS:
        raise NotImplementedError("contraction with more than 8 independent strided dimensions")

    # Split the outermost output dim while the output range reaches 2^31.
    if n_out > _MAX_INDEX:
        n0, sa0, sb0 = out_dims[0]
        inner = n_out // n0
        if inner > _MAX_INDEX:
            raise NotImplementedError("output with more than 2^31 elements per outer index")
        chunk = max(1, _MAX_INDEX // inner)
        Dflat = D.view(-1)
        Cflat = C.view(-1) if C is not None else None
        for s in range(0, n0, chunk):
            e = min(n0, s + chunk)
            strided_contract(
                [(e - s, sa0, sb0)] + out_dims[1:],
                red_dims,
                A,
                B,
                Dflat[s * inner : e * inner],
                alpha,
                beta,
                None if Cflat is None else Cflat[s * inner : e * inner],
                a_off + s * sa0,
                b_off + s * sb0,
            )
        return
    # Split the outermost reduction dim while the reduction range reaches 2^31;
    # later chunks accumulate onto D (beta = 1, C = D).
    if n_red > _MAX_INDEX:
        n0, sa0, sb0 = red_dims[0]
        inner = n_red // n0
        if inner > _MAX_INDEX:
            raise NotImplementedError("reduction with more than 2^31 elements per outer index")
        chunk = max(1, _MAX_INDEX // inner)
        first = True
        for s in range(0, n0, chunk):
            e = min(n0, s + chunk)
            strided_contract(
                out_dims,
                [(e - s, sa0, sb0)] + red_dims[1:],
                A,
                B,
                D,
                alpha,
                beta if first else 1.0,
                C if first else D,
                a_off + s * sa0,
                b_off + s * sb0,
            )
            first = False
        return

    code = dtype_code(D.dtype)
    es = D.element_size()
    oshape = _lib.i64_array(d[0] for d in out_dims)
    oa = _lib.i64_array(d[1] for d in out_dims)
    ob = _lib.i64_array(d[2] for d in out_dims)
    rshape = _lib.i64_array(d[0] for d in red_dims)
    ra = _lib.i64_array(d[1] for d in red_dims)
    rb = _lib.i64_array(d[2] for d in red_dims)
    wsb = lib.tt_strided_contract_workspace_bytes(code, len(out_dims), oshape, len(red_dims), rshape)
    ws = _workspace(wsb, D.device)
    a_ptr = A.data_ptr() + a_off * es
    b_ptr = None if B is None else B.data_ptr() + b_off * es
    st = lib.tt_strided_contract(
        code,
        len(out_dims),
        oshape,
        oa,
        ob,
        len(red_dims),
        rshape,
        ra,
        rb,
        a_ptr,
        b_ptr,
        float(alpha),
        float(beta),
        _ptr(C),
        _ptr(D),
        _ptr(ws),
        wsb,
        _stream_ptr(D.device),
    )
    _lib.check(st, "tt_strided_contract")


def pack(op: Operand, order: list[str]) -> torch.Tensor:
    """Copy `op` into a new contiguous tensor with dims in `order`."""
    D = torch.empty([op.ext[c] for c in order], dtype=op.t.dtype, device=op.t.device)
    dims = [(op.ext[c], op.strd[c], 0) for c in order]
    strided_contract(dims, [], op.t, None, D)
    return D


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------
def gemm(
    transA: bool,
    transB: bool,
    M: int,
    N: int,
    K: int,
    A: torch.Tensor,
    lda: int,
    sA: int,
    B: torch.Tensor,
    ldb: int,
    sB: int,
    D: torch.Tensor,
    ldd: int,
    sD: int,
    batch: int = 1,
    alpha: float = 1.0,
    beta: float = 0.0,
    C: torch.Tensor | None = None,
    ldc: int = 0,
    sC: int = 0,
    a_off: int = 0,
    b_off: int = 0,
    d_off: int = 0,
) -> None:
    """tt_gemm on torch tensors (pointers taken at the given element offsets)."""
    lib = _lib.load()
    es = D.element_size()
    st = lib.tt_gemm(
        dtype_code(D.dtype),
        int(transA),
        int(transB),
        M,
        N,
        K,
        float(alpha),
        A.data_ptr() + a_off * es,
        lda,
        sA,
        B.data_ptr() + b_off * es,
        ldb,
        sB,
        float(beta),
        _ptr(C),
        ldc,
        sC,
        D.data_ptr() + d_off * es,
        ldd,
        sD,
        batch,
        _stream_ptr(D.device),
    )
    _lib.check(st, "tt_gemm")


def split_k(M: int, N: int, K: int, batch: int) -> int:
    """K-slices for a GEMM whose output tiles cannot fill the chip.

    A launch with fewer than ~200 128x128 output tiles leaves most of the
    256 CUs idle however long K is; slicing K (each slice >= 512 deep) into
    batch entries gives ~512 workgroups. Only unbatched GEMMs with K >= 4096
    are split.
    """
    if batch > 1 or K < 4096 or M == 0 or N == 0:
        return 1
    tiles = (-(-M // 128)) * (-(-N // 128))
    if tiles >= 192:
        return 1
    return max(1, min(-(-512 // tiles), K // 512))


def _slice_depth(K: int, split: int) -> int:
    """K per slice: ceil(K / split) rounded up to the kernels' 16-deep stage,
    so slice offsets keep 16-byte alignment and slices end on full stages."""
    kc = -(-K // split)
    return -(-kc // 16) * 16


def _k_step(k_contiguous: bool, ld: int) -> int:
    """Element distance between consecutive k of an operand viewed rows x K."""
    return 1 if k_contiguous else ld


def gemm_dot(
    transA: bool,
    transB: bool,
    M: int,
    N: int,
    K: int,
    A: torch.Tensor,
    lda: int,
    sA: int,
    B: torch.Tensor,
    ldb: int,
    sB: int,
    batch: int,
    m_lo_extent: int,
    n_lo_extent: int,
    E1: torch.Tensor,
    e1_strides: list[int],
    E2: torch.Tensor | None,
    e2_strides: list[int] | None,
    alpha: float,
    beta: float,
    C: torch.Tensor | None,
    out: torch.Tensor,
    a_off: int = 0,
    b_off: int = 0,
) -> None:
    """tt_gemm_dot on torch tensors: out = alpha * sum (op(A) op(B)) .* E (+ beta * C[0])."""
    lib = _lib.load()
    code = dtype_code(A.dtype)
    es = A.element_size()
    wsb = lib.tt_gemm_dot_workspace_bytes(code, M, N, batch)
    ws = _workspace(wsb, A.device)
    st = lib.tt_gemm_dot(
        code, int(transA), int(transB), M, N, K,
        ctypes.c_void_p(A.data_ptr() + a_off * es), lda, sA,
        ctypes.c_void_p(B.data_ptr() + b_off * es), ldb, sB, batch,
        m_lo_extent, n_lo_extent,
        _ptr(E1), _lib.i64_array(e1_strides), _ptr(E2), None if E2 is None else _lib.i64_array(e2_strides),
        float(alpha), float(beta), _ptr(C), _ptr(out), _ptr(ws), wsb, _stream_ptr(A.device),
    )
    _lib.check(st, "tt_gemm_dot")


class _GemmRecipe:
    """Launch parameters of a contraction that maps onto tt_gemm with both
    operands in place; `swap` means the output is computed as B^T A^T.

    split > 1 slices K into `split` batch entries of a [split, M, N]
    temporary (slice s reads k in [s*kc, (s+1)*kc), a last shorter slice goes
    in a second launch), summed in slice order into D by one strided pass
    that also applies alpha/beta. D is then [M][N] contiguous."""

    __slots__ = ("swap", "ta", "tb", "M", "N", "K", "lda", "sA", "ldb", "sB", "ldd", "sD", "batch", "shape", "dt",
                 "split")

    def __init__(self, swap, ta, tb, M, N, K, lda, sA, ldb, sB, ldd, sD, batch, shape, dt, split=1):
        self.swap, self.ta, self.tb = swap, ta, tb
        self.M, self.N, self.K = M, N, K
        self.lda, self.sA, self.ldb, self.sB, self.ldd, self.sD = lda, sA, ldb, sB, ldd, sD
        self.batch, self.shape, self.dt = batch, shape, dt
        self.split = split

    def run(self, At, Bt, alpha, beta, C):
        D = torch.empty(tuple(self.shape), dtype=self.dt, device=At.device)
        X, Y = (Bt, At) if self.swap else (At, Bt)
        # K-slices would each round to float64: double-double runs unsplit.
        if self.split <= 1 or _ACCUMULATION.get() == "dd":
            gemm(self.ta, self.tb, self.M, self.N, self.K, X, self.lda, self.sA, Y, self.ldb, self.sB, D,
                 self.ldd, self.sD, self.batch, alpha, beta, C, self.ldd, self.sD)
            return D
        M, N, K = self.M, self.N, self.K
        kc = _slice_depth(K, self.split)
        full, rem = K // kc, K % kc
        ka = _k_step(not self.ta, self.lda)  # X[m*lda + k] unless transposed
        kb = _k_step(self.tb, self.ldb)  # Y[n*ldb + k] when transposed
        T = torch.empty((full + (rem > 0), M, N), dtype=self.dt, device=At.device)
        gemm(self.ta, self.tb, M, N, kc, X, self.lda, kc * ka, Y, self.ldb, kc * kb, T, N, M * N, full)
        if rem:
            gemm(self.ta, self.tb, M, N, rem, X, self.lda, 0, Y, self.ldb, 0, T[full], N, 0, 1,
                 a_off=full * kc * ka, b_off=full * kc * kb)
        strided_contract([(M, N, 0), (N, 1, 0)], [(T.shape[0], M * N, 0)], T, None, D, alpha, beta, C)
        return D


    def packed_params(self) -> list[int] | None:
        """tt_gemm_packed's parameter block for this recipe's one tt_gemm
        launch (no C), or None if the recipe needs more than one launch (K
        split) or its dtype has no packed launch."""
        if self.split > 1 or self.dt not in (torch.float32, torch.float64, torch.bfloat16, torch.float16):
            return None
        return [dtype_code(self.dt), int(self.ta), int(self.tb), self.M, self.N, self.K, self.lda, self.sA, self.ldb,
                self.sB, 0, 0, self.ldd, self.sD, self.batch]

    def launcher(self, device: torch.device):
        """A callable (A, B, alpha) -> D that repeats this recipe's one
        tt_gemm launch (no C) through tt_gemm_packed, with the integer launch
        parameters kept in one array; None if the recipe needs more than one
        launch (K split). For callers that have checked the operands against
        the recipe's key (shapes, strides, dtype, device)."""
        pl = self.packed_params()
        if pl is None:
            return None
        lib = _lib.load()
        fn = lib.tt_gemm_packed
        params = (ctypes.c_int64 * 15)(*pl)
        pp = ctypes.addressof(params)
        shape, dt, swap = tuple(self.shape), self.dt, self.swap
        strides = _contiguous_strides(shape)
        idx = device.index if device.index is not None else torch.cuda.current_device()
        # torch.empty_strided with tuples parses in a third of the time of
        # torch.empty with a list (1.4 against 4.2 us on a host core).
        empty, raw, acc = torch.empty_strided, _raw_stream, _ACCUMULATION
        if raw is None:
            return None

        def run(a, b, alpha):
            if acc.get() != "native":
                return None
            D = empty(shape, strides, dtype=dt, device=device)
            x, y = (b, a) if swap else (a, b)
            st = fn(pp, alpha, 0.0, x.data_ptr(), y.data_ptr(), None, D.data_ptr(), raw(idx))
            if st:
                _lib.check(st, "tt_gemm")
            return D

        run.params = params  # keeps the array alive with the callable
        return run


def _contiguous_strides(shape: tuple) -> tuple:
    """Row-major strides of `shape` (torch's, for extents of 0 or 1 included)."""
    st, acc = [], 1
    for n in reversed(shape):
        st.append(acc)
        acc *= max(n, 1)
    return tuple(reversed(st))


# Recipes keyed by (terms, out, shapes, strides, dtype, prefer_gemm); bounded.
_RECIPES: dict[tuple, _GemmRecipe] = {}
_RECIPES_MAX = 4096


def cached_recipe(ta: str, tb: str, out: str, a: torch.Tensor, b: torch.Tensor, prefer_gemm: bool):
    """The cached in-place recipe of this two-operand contraction, or None."""
    return _RECIPES.get((ta, tb, out, a.shape, a.stride(), b.shape, b.stride(), a.dtype, prefer_gemm))



def _gemm_layout(op: Operand, rows: list[str], ks: list[str]):
    """(k_contiguous, ld) for an operand viewed as rows x K, or None."""
    r = _merge(op, rows)
    k = _merge(op, ks)
    if r is None or k is None:
        return None
    (nr, sr), (nk, sk) = r, k
    if nk == 1 or sk == 1:
        ld = sr if nr > 1 else max(nk, 1)
        if nr > 1 and ld < nk:
            return None
        return True, ld
    if nr == 1 or sr == 1:
        ld = sk
        if ld < nr:
            return None
        return False, ld
    return None


def _merge_strides(ext: dict, strd: dict, letters: list[str]) -> tuple[int, int] | None:
    """_merge on plain extent/stride maps (letters absent from `strd` have stride 0)."""
    extent, stride = 1, 0
    for c in reversed(letters):
        n, s = ext[c], strd.get(c, 0)
        if n == 1:
            continue
        if extent == 1:
            extent, stride = n, s
        elif s == stride * extent:
            extent *= n
        else:
            return None
    return extent, stride


def _inplace_mappings(A: Operand, B: Operand, out: str, batch, ml, nl, kl, ext):
    """Yield GEMM mappings that use both operands and the output in place.

    The output is contiguous in `out` order. Each candidate assigns letters to
    (batch, M, N); a mapping is kept when A's M and K groups, B's N and K
    groups and every group of the output each collapse to one stride, and
    the output has N (direct) or M (swapped) unit-stride. Besides the plain
    grouping, an unbatched contraction may move one M letter (or N letter)
    into the batch, read with stride 0 by the other operand: a broadcast
    batch, which replaces packing an operand whose M or N letters are split
    by a K letter (e.g. 'jb,abP->jaP' runs as a batch over a).
    Yields (swap, ta, tb, M, N, K, lda, sA, ldb, sB, ldd, sD, nb).
    """
    dstrd: dict[str, int] = {}
    acc = 1
    for c in reversed(out):
        dstrd[c] = acc
        acc *= ext[c]
    cands = [(batch, ml, nl)]
    if not batch:
        # a peel must not leave a sliver M or N (MFMA tiles are 64+ wide)
        M0, N0 = _numel(ext[c] for c in ml), _numel(ext[c] for c in nl)
        cands += [([x], [c for c in ml if c != x], nl) for x in ml
                  if ext[x] > 1 and M0 // ext[x] >= min(16, M0)]
        cands += [([x], ml, [c for c in nl if c != x]) for x in nl
                  if ext[x] > 1 and N0 // ext[x] >= min(16, N0)]
    K = _numel(ext[c] for c in kl)
    for bl, m_, n_ in cands:
        la = _gemm_layout(A, m_, kl)
        lb = _gemm_layout(B, n_, kl)
        if la is None or lb is None:
            continue
        nb = _numel(ext[c] for c in bl)
        ga = _merge_strides(ext, A.strd, bl)
        gb = _merge_strides(ext, B.strd, bl)
        gd = _merge_strides(ext, dstrd, bl)
        dm = _merge_strides(ext, dstrd, m_)
        dn = _merge_strides(ext, dstrd, n_)
        if None in (ga, gb, gd, dm, dn):
            continue
        sA, sB, sD = (ga[1], gb[1], gd[1]) if nb > 1 else (0, 0, 0)
        M = _numel(ext[c] for c in m_)
        N = _numel(ext[c] for c in n_)
        if N == 1 or dn[1] == 1:
            ldd = dm[1] if M > 1 else max(N, 1)
            if M <= 1 or ldd >= N:
                yield (0, not la[0], lb[0], M, N, K, la[1], sA, lb[1], sB, ldd, sD, nb)
        if M == 1 or dm[1] == 1:
            ldd = dn[1] if N > 1 else max(M, 1)
            if N <= 1 or ldd >= M:
                yield (1, not lb[0], la[0], N, M, K, lb[1], sB, la[1], sA, ldd, sD, nb)


def _inplace_recipe(A, B, out, batch, ml, nl, kl, ext, dt) -> _GemmRecipe | None:
    """The first in-place mapping (see _inplace_mappings) as a recipe, with
    K split when the output alone cannot fill the chip."""
    shape = [ext[c] for c in out]
    for swap, ta, tb, M, N, K, lda, sA, ldb, sB, ldd, sD, nb in _inplace_mappings(A, B, out, batch, ml, nl, kl, ext):
        split = split_k(M, N, K, nb) if ldd == max(N, 1) else 1
        return _GemmRecipe(swap, ta, tb, M, N, K, lda, sA, ldb, sB, ldd, sD, nb, shape, dt, split)
    return None


def contract_gemm(
    A: Operand,
    B: Operand,
    out: str,
    batch: list[str],
    ml: list[str],
    nl: list[str],
    kl: list[str],
    alpha: float,
    beta: float,
    C: torch.Tensor | None,
    recipe_key: tuple | None = None,
) -> torch.Tensor:
    """Contraction with a GEMM shape through tt_gemm (operands packed only if needed).

    When both operands are used in place and the output is written directly,
    the launch parameters are cached under `recipe_key`.
    """
    dev, dt = A.t.device, A.t.dtype
    ext = {**A.ext, **B.ext}
    rec = _inplace_recipe(A, B, out, batch, ml, nl, kl, ext, dt)
    if rec is not None:
        if recipe_key is not None:
            _RECIPES[recipe_key] = rec
        return rec.run(A.t, B.t, alpha, beta, C)

    nb = _numel(ext[c] for c in batch)
    M = _numel(ext[c] for c in ml)
    N = _numel(ext[c] for c in nl)
    K = _numel(ext[c] for c in kl)

    packed = False
    la = _gemm_layout(A, ml, kl)
    gba = _merge(A, batch)
    if la is None or gba is None:
        A = Operand("".join(batch + ml + kl), pack(A, batch + ml + kl))
        la, gba = (True, max(K, 1)), (nb, M * K)
        packed = True
    lb = _gemm_layout(B, nl, kl)
    gbb = _merge(B, batch)
    if lb is None or gbb is None:
        B = Operand("".join(batch + kl + nl), pack(B, batch + kl + nl))
        lb, gbb = (False, max(N, 1)), (nb, K * N)
        packed = True
    sA = gba[1] if nb > 1 else 0
    sB = gbb[1] if nb > 1 else 0

    direct = "".join(batch + ml + nl) == out
    swapped = (not direct) and "".join(batch + nl + ml) == out
    shape = [ext[c] for c in out]
    if direct or swapped:
        if direct:
            # A rows m: k-contiguous -> not transposed. B rows n: k-contiguous -> transposed.
            rec = _GemmRecipe(0, not la[0], lb[0], M, N, K, la[1], sA, lb[1], sB, max(N, 1), M * N, nb, shape, dt)
        else:
            rec = _GemmRecipe(1, not lb[0], la[0], N, M, K, lb[1], sB, la[1], sA, max(M, 1), M * N, nb, shape, dt)
        if recipe_key is not None and not packed:
            _RECIPES[recipe_key] = rec
        return rec.run(A.t, B.t, alpha, beta, C)
    # Packed [batch, M, N] temporary, then one permuting pass into the output order.
    T = torch.empty([ext[c] for c in batch + ml + nl], dtype=dt, device=dev)
    gemm(not la[0], lb[0], M, N, K, A.t, la[1], sA, B.t, lb[1], sB, T, max(N, 1), M * N, nb,
         1.0, 0.0, None, 0, 0)
    Top = Operand("".join(batch + ml + nl), T)
    D = torch.empty(shape, dtype=dt, device=dev)
    strided_contract([(Top.ext[c], Top.strd[c], 0) for c in out], [], T, None, D, alpha, beta, C)
    return D


# ---------------------------------------------------------------------------
# public entry: one or two operands
# ---------------------------------------------------------------------------
_HALF = (torch.bfloat16, torch.float16)


def _contract_half(terms, out, tensors, alpha, beta, C, prefer_gemm, key):
    """The in-place GEMM mapping of a 16-bit two-operand contraction, run on
    the 16-bit MFMA GEMM, or None when the contraction needs anything else
    (packing, a permuting pass, summed one-sided letters, K-splitting)."""
    if len(tensors) != 2 or len(set(out)) != len(out):
        return None
    A, B = (Operand(t, x) for t, x in zip(terms, tensors))
    la, lb, lo = set(A.letters), set(B.letters), set(out)
    if any(c not in la and c not in lb for c in lo):
        return None
    if any(c not in lb and c not in lo for c in la) or any(c not in la and c not in lo for c in lb):
        return None
    kl = [c for c in A.letters if c in lb and c not in lo]
    batch = [c for c in out if c in la and c in lb]
    ml = [c for c in out if c in la and c not in lb]
    nl = [c for c in out if c in lb and c not in la]
    ext = {**A.ext, **B.ext}
    M, N = _numel(ext[c] for c in ml), _numel(ext[c] for c in nl)
    if not kl or not (prefer_gemm or (M >= 16 and N >= 16)):
        return None
    kl.sort(key=lambda c: -A.strd[c])
    rec = _inplace_recipe(A, B, out, batch, ml, nl, kl, ext, tensors[0].dtype)
    if rec is None:
        return None
    rec.split = 1  # slices would need a 16-bit reduction pass
    if key is not None:
        _RECIPES[key] = rec
    return rec.run(A.t, B.t, alpha, beta, C)


def contract(
    terms: list[str],
    out: str,
    tensors: list[torch.Tensor],
    alpha: float = 1.0,
    beta: float = 0.0,
    C: torch.Tensor | None = None,
    prefer_gemm: bool = False,
) -> torch.Tensor:
    """einsum of one or two device tensors (same dtype: float32/float64, or
    bfloat16/float16 for contractions that map onto the GEMM in place).

    C (if given) is contiguous in the output's shape and enters as beta*C.
    16-bit operands run on the 16-bit MFMA GEMM (fp32 accumulation) when the
    contraction maps onto it without packing; otherwise they are widened to
    float32 (exactly) and the result is rounded back to their dtype.
    """
    if tensors[0].is_complex():
        return _contract_complex(terms, out, tensors, alpha, beta, C, prefer_gemm)
    key = None
    if len(tensors) == 2:
        a, b = tensors
        key = (terms[0], terms[1], out, a.shape, a.stride(), b.shape, b.stride(), a.dtype, prefer_gemm)
        rec = _RECIPES.get(key)
        if rec is not None:
            return rec.run(a, b, alpha, beta, C)
        if len(_RECIPES) >= _RECIPES_MAX:
            _RECIPES.clear()
    if tensors[0].dtype in _HALF:
        res = _contract_half(terms, out, tensors, alpha, beta, C, prefer_gemm, key)
        if res is not None:
            return res
        wide = contract(terms, out, [t.float() for t in tensors], alpha, beta, None if C is None else C.float(),
                        prefer_gemm)
        return wide.to(tensors[0].dtype)
    ops = [Operand(t, x) for t, x in zip(terms, tensors)]
    present = set().union(*[set(o.letters) for o in ops])
    if len(set(out)) != len(out):
        raise RuntimeError(f"einsum(): output subscript {out!r} includes a letter more than once")
    missing = [c for c in out if c not in present]
    if missing:
        raise RuntimeError(f"einsum(): output subscript {missing[0]} does not appear in the equation for any input operand")
    ext: dict[str, int] = {}
    for o in ops:
        ext.update(o.ext)
    shape = [ext[c] for c in out]
    dt, dev = tensors[0].dtype, tensors[0].device
    dtype_code(dt)

    if len(ops) == 2:
        A, B = ops
        la, lb, lo = set(A.letters), set(B.letters), set(out)
        kl = [c for c in A.letters if c in lb and c not in lo]
        batch = [c for c in out if c in la and c in lb]
        ml = [c for c in out if c in la and c not in lb]
        nl = [c for c in out if c in lb and c not in la]
        # Under double-double accumulation a pre-reduced operand would be
        # rounded to float64 before the GEMM; such contractions take the
        # strided kernel, which accumulates the whole reduction in one pair.
        one_sided = any(c not in lb and c not in lo for c in la) or any(c not in la and c not in lo for c in lb)
        # Integer contractions take the strided kernel (int64, wrapping sums).
        if kl and not (one_sided and _ACCUMULATION.get() == "dd") and dt != torch.int64:
            M = _numel(ext[c] for c in ml)
            N = _numel(ext[c] for c in nl)
            if prefer_gemm or (M >= 16 and N >= 16):
                # Letters of one operand that are summed away are reduced first.
                for idx, (op, other) in enumerate(((A, lb), (B, la))):
                    gone = [c for c in op.letters if c not in other and c not in lo]
                    if gone:
                        keep = [c for c in op.letters if c not in gone]
                        R = torch.empty([op.ext[c] for c in keep], dtype=dt, device=dev)
                        strided_contract(
                            [(op.ext[c], op.strd[c], 0) for c in keep],
                            [(op.ext[c], op.strd[c], 0) for c in gone],
                            op.t,
                            None,
                            R,
                        )
                        ops[idx] = Operand("".join(keep), R)
                A, B = ops
                # K letters ordered by A's strides (outer first) so A's K group collapses.
                kl.sort(key=lambda c: -A.strd[c])
                pre_reduced = A.t is not tensors[0] or B.t is not tensors[1]
                return contract_gemm(A, B, out, batch, ml, nl, kl, alpha, beta, C, None if pre_reduced else key)

    # Strided multiply-reduce over the whole contraction.
    A = ops[0]
    B = ops[1] if len(ops) == 2 else None

    def s(op, c):
        return 0 if op is None or c not in op.ext else op.strd[c]

    red = [c for c in sorted(present - set(out))]
    red.sort(key=lambda c: (-s(A, c), -s(B, c)))
    D = torch.empty(shape, dtype=dt, device=dev)
    strided_contract(
        [(ext[c], s(A, c), s(B, c)) for c in out],
        [(ext[c], s(A, c), s(B, c)) for c in red],
        A.t,
        None if B is None else B.t,
        D,
        alpha,
        beta,
        C,
    )
    return D


# ---------------------------------------------------------------------------
# complex operands: real contractions on the parts
# ---------------------------------------------------------------------------
def complex_parts(z: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(real, imaginary) parts of a complex tensor as contiguous real tensors
    (one strided copy each, on the device)."""
    v = torch.view_as_real(z.resolve_conj())
    parts = []
    for k in (0, 1):
        P = torch.empty(z.shape, dtype=v.dtype, device=z.device)
        strided_contract([(n, s, 0) for n, s in zip(z.shape, v.stride()[:-1])], [], v, None, P, a_off=k)
        parts.append(P)
    return parts[0], parts[1]


def _contract_complex(terms, out, tensors, alpha, beta, C, prefer_gemm):
    """A complex contraction as real ones: one operand contracts each part;
    two operands give Re = ArBr - AiBi and Im = ArBi + AiBr, the second
    product of each added through the first's beta epilogue. alpha and beta
    are real here (complex scalars are applied by the caller); C (complex,
    contiguous in the output's shape) enters as beta * C."""
    if isinstance(alpha, complex) or isinstance(beta, complex):
        raise NotImplementedError("complex alpha/beta are applied outside the engine")
    parts = [complex_parts(t) for t in tensors]
    Cr, Ci = complex_parts(C) if C is not None else (None, None)
    if len(tensors) == 1:
        (ar, ai), = parts
        re = contract(terms, out, [ar], alpha, beta, Cr)
        im = contract(terms, out, [ai], alpha, beta, Ci)
    else:
        (ar, ai), (br, bi) = parts
        re = contract(terms, out, [ar, br], alpha, beta, Cr, prefer_gemm)
        re = contract(terms, out, [ai, bi], -alpha, 1.0, re, prefer_gemm)
        im = contract(terms, out, [ar, bi], alpha, beta, Ci, prefer_gemm)
        im = contract(terms, out, [ai, br], alpha, 1.0, im, prefer_gemm)
    return torch.complex(re, im)


# ---------------------------------------------------------------------------
# GEMM with a dot epilogue (a product contracted with E on the spot)
# ---------------------------------------------------------------------------
def contract_gemm_dot(
    terms: list[str],
    xname: str,
    tensors: list[torch.Tensor],
    factors: list[tuple[str, torch.Tensor]],
    alpha: float = 1.0,
    beta: float = 0.0,
    C: torch.Tensor | None = None,
) -> torch.Tensor | None:
    """sum over X * E with X = einsum(terms -> xname)(tensors) never stored, via tt_gemm_dot.

    E is the product of the factor tensors, whose letters together are X's
    letters (one factor: a tensor in X's letters; two: an outer product that
    is never materialised either). Returns a 0-D tensor, or None when the
    contraction has no GEMM shape or its letter groups exceed what the fused
    kernel decodes (batch <= 1 letter, M and N <= 2 letters each).
    """
    ops = [Operand(t, x) for t, x in zip(terms, tensors)]
    A, B = ops
    la, lb, lo = set(A.letters), set(B.letters), set(xname)
    kl = [c for c in A.letters if c in lb and c not in lo]
    batch = [c for c in xname if c in la and c in lb]
    ml = [c for c in xname if c in la and c not in lb]
    nl = [c for c in xname if c in lb and c not in la]
    facs = [Operand(t, x) for t, x in factors]
    if not kl or len(batch) > 1 or len(ml) > 2 or len(nl) > 2 or not 1 <= len(facs) <= 2:
        return None
    if set().union(*[set(f.letters) for f in facs]) != lo or len(xname) != len(lo):
        return None
    dt, dev = A.t.dtype, A.t.device
    dtype_code(dt)  # raises for dtypes the kernels do not compute in
    for idx, (op, other) in enumerate(((A, lb), (B, la))):
        gone = [c for c in op.letters if c not in other and c not in lo]
        if gone:
            keep = [c for c in op.letters if c not in gone]
            R = torch.empty([op.ext[c] for c in keep], dtype=dt, device=dev)
            strided_contract([(op.ext[c], op.strd[c], 0) for c in keep], [(op.ext[c], op.strd[c], 0) for c in gone], op.t, None, R)
            ops[idx] = Operand("".join(keep), R)
    A, B = ops
    ext = {**A.ext, **B.ext}
    # The fp64 direct-B dot kernel needs whole 128-column tiles (any M): with
    # N ragged and M whole, the product is formed transposed (X^T = B^T A^T,
    # E read with the row and column letters exchanged). Config 5's
    # optimal-order dot GEMM (16384 x 400 x 800): 400 x 16384 runs on the
    # direct-B kernel with 448 padded rows instead of 512 padded columns.
    if dt == torch.float64 and _numel(ext[c] for c in nl) % 128 and not _numel(ext[c] for c in ml) % 128:
        A, B, ml, nl = B, A, nl, ml
    kl.sort(key=lambda c: -A.strd[c])
    nb = _numel(ext[c] for c in batch)
    M = _numel(ext[c] for c in ml)
    N = _numel(ext[c] for c in nl)
    K = _numel(ext[c] for c in kl)
    la_ = _gemm_layout(A, ml, kl)
    gba = _merge(A, batch)
    if la_ is None or gba is None:
        A = Operand("".join(batch + ml + kl), pack(A, batch + ml + kl))
        la_, gba = (True, max(K, 1)), (nb, M * K)
    lb_ = _gemm_layout(B, nl, kl)
    gbb = _merge(B, batch)
    if lb_ is None or gbb is None:
        B = Operand("".join(batch + kl + nl), pack(B, batch + kl + nl))
        lb_, gbb = (False, max(N, 1)), (nb, K * N)
    sA = gba[1] if nb > 1 else 0
    sB = gbb[1] if nb > 1 else 0

    m_hi = ml[0] if len(ml) == 2 else None
    m_lo = ml[-1] if ml else None
    n_hi = nl[0] if len(nl) == 2 else None
    n_lo = nl[-1] if nl else None
    b_l = batch[0] if batch and nb > 1 else None  # K-slices reuse the batch index with E stride 0

    def strides(f: Operand):
        return [0 if c is None else f.strd.get(c, 0) for c in (m_hi, m_lo, n_hi, n_lo, b_l)]

    e1 = facs[0]
    e2 = facs[1] if len(facs) == 2 else None
    out = torch.empty((), dtype=dt, device=dev)
    m_ext = ext[m_lo] if m_lo else 1
    n_ext = ext[n_lo] if n_lo else 1

    def launch(kk, nbat, sa, sb, a_off, b_off, beta_, C_):
        gemm_dot(not la_[0], lb_[0], M, N, kk, A.t, la_[1], sa, B.t, lb_[1], sb, nbat, m_ext, n_ext,
                 e1.t, strides(e1), None if e2 is None else e2.t, None if e2 is None else strides(e2),
                 alpha, beta_, C_, out, a_off, b_off)

    split = split_k(M, N, K, nb)
    if split <= 1:
        launch(K, nb, sA, sB, 0, 0, beta, C)
        return out
    # The dot is linear in the product, so K-slices (batch entries whose E
    # batch stride is 0) each contribute partials to the same sum; a last
    # shorter slice adds its share onto the first launch's result.
    kc = _slice_depth(K, split)
    full, rem = K // kc, K % kc
    ka = _k_step(la_[0], la_[1])
    kb = _k_step(lb_[0], lb_[1])
    launch(kc, full, kc * ka, kc * kb, 0, 0, beta, C)
    if rem:
        launch(rem, 1, 0, 0, full * kc * ka, full * kc * kb, 1.0, out)
    return out
