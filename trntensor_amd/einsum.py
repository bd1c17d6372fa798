"""einsum front-end: dtype cast, planning, execution on the HIP kernels, and
the alpha/beta epilogue fused into the last kernel's store.

Mirrors trntensor/einsum.py (reference): same signature and keyword
semantics (``alpha``, ``beta``, ``out``, ``dtype``, ``precision``), same
error types, same path-executor step order. The results are what einsum
defines; every step runs on libtrntensor_hip.so.
"""

from __future__ import annotations

import torch

from .hip import _fastpath
from .hip import dispatch
from .hip import engine
from .plan import (_CLEAR_HOOKS, _LAUNCH_CACHE, _LAUNCH_CACHE_MAX, _PLAN_CACHE, ContractionPlan, _parse_subscripts,
                   _shape_key, plan_contraction)

_DTYPE_MAP: dict[str, torch.dtype] = {
    "bf16": torch.bfloat16,
    "bfloat16": torch.bfloat16,
    "fp16": torch.float16,
    "float16": torch.float16,
    "f32": torch.float32,
    "float32": torch.float32,
    "f64": torch.float64,
    "float64": torch.float64,
}


def _resolve_dtype(dtype: str | torch.dtype | None) -> torch.dtype | None:
    """``None``, a ``torch.dtype``, or one of the strings above (case-insensitive);
    anything else raises ``ValueError`` (reference trntensor/einsum.py:39-48)."""
    if dtype is None or isinstance(dtype, torch.dtype):
        return dtype
    found = _DTYPE_MAP.get(dtype.lower())
    if found is None:
        raise ValueError(f"unknown dtype {dtype!r}; valid strings: {sorted(_DTYPE_MAP)}")
    return found


def einsum(
    subscripts: str,
    *operands: torch.Tensor,
    alpha: float = 1.0,
    beta: float = 0.0,
    out: torch.Tensor | None = None,
    dtype: str | torch.dtype | None = None,
    precision: str = "fast",
    optimize: str = "greedy",
) -> torch.Tensor:
    """Einstein summation with contraction planning, executed on MI355X.

    Returns ``alpha * contract(operands) + beta * out`` (``out`` is read, never
    written; the result is a new tensor, as in the reference). ``dtype`` casts
    every operand first and the result comes back in that dtype.
    ``precision="kahan"`` contracts in float64 and returns the first operand's
    dtype; ``"dd"`` forms every product exactly and sums in double-double,
    rounding once per pairwise step (the reference raises
    ``NotImplementedError`` for it). The result lives on the
    first operand's device: CPU operands are staged through the GPU.
    ``optimize`` selects the path search for 3+ operands: ``"greedy"`` (the
    reference's order, default) or ``"optimal"`` (fewest multiply-adds; opt-in).

    Examples::

        einsum("ij,jk->ik", A, B)
        einsum("ij,jk->ik", A, B, alpha=2.0, beta=0.5, out=C)
        einsum("ap,bp->ab", B[i], B[j])          # DF-MP2 pair block
        einsum("mi,mnP->inP", C_occ, eri)        # AO->MO half transform
        einsum("ia,jb,abP,ijP->", A, B, W, V)    # greedy path
    """
    # Repeat call of a two-operand contraction that runs as one GEMM launch:
    # the launch recorded on its first call (plan cached, same shapes,
    # strides, dtypes and devices), one allocation and one library call, in
    # the C++ launch table when it is built, else through a cached ctypes
    # launcher.
    plain = (len(operands) == 2 and out is None and dtype is None and precision == "fast" and optimize == "greedy"
             and type(alpha) in (float, int))
    if plain:
        a, b = operands
        fast = _fast
        if fast is not None:
            if dispatch._use_hip() and engine._ACCUMULATION.get() == "native":
                try:
                    res = fast.run(subscripts, a, b, float(alpha))
                except TypeError:  # not tensors: planning reports it
                    res = None
                if res is not None:
                    return res
        else:
            run = _LAUNCH_CACHE.get(_launch_key(subscripts, a, b))
            if run is not None and dispatch._use_hip():
                res = run(a, b, float(alpha))
                if res is not None:
                    return res
    target = _resolve_dtype(dtype)
    if target is not None:
        operands = tuple(op.to(target) for op in operands)
    plan = plan_contraction(subscripts, *operands, precision=precision, optimize=optimize)
    res = _execute_contraction(subscripts, operands, plan, alpha=alpha, beta=beta, out=out)
    if plain:
        _remember_launch(subscripts, plan, a, b)
    return res


_FAST_DTYPES = (torch.float32, torch.float64, torch.bfloat16, torch.float16)

# The C++ launch table (hip/_fastpath.py) once the first launch has been
# recorded, if it is built; None while launches go through _LAUNCH_CACHE.
_fast = None


def _launch_key(subscripts, a, b) -> tuple:
    return (subscripts, a.shape, a.stride(), b.shape, b.stride(), a.dtype, b.dtype, a.device, b.device)


def _launch_cache_size() -> int:
    """Recorded launches (the C++ table's, or the ctypes launchers')."""
    return len(_fast) if _fast is not None else len(_LAUNCH_CACHE)


def _clear_launches() -> None:
    if _fast is not None:
        _fast.clear()


def _remember_launch(subscripts, plan, a, b) -> None:
    """Record the launch of a just-run two-operand contraction when both
    operands are on one HIP device (or both on the host) in one real dtype
    and the engine ran it as one in-place GEMM launch (its recipe is
    cached). Host operands are recorded only in the C++ table, which stages
    small contiguous ones through pinned memory."""
    global _fast
    host = a.device.type == "cpu" and b.device.type == "cpu"
    if (plan.strategy == "path" or not (host or a.device.type == "cuda") or b.device != a.device
            or a.dtype != b.dtype or a.dtype not in _FAST_DTYPES
            or _PLAN_CACHE.get(_shape_key(subscripts, (a, b))) is not plan):
        return
    lhs, out_str = _parse_subscripts(subscripts)
    ta, tb = lhs.split(",")
    rec = engine.cached_recipe(ta, tb, out_str, a, b, plan.strategy in ("matmul", "bmm"))
    if rec is None:
        return
    if _fast is None:
        _fast = _fastpath.table(_LAUNCH_CACHE_MAX)
        if _fast is not None:
            _LAUNCH_CACHE.clear()
            _CLEAR_HOOKS.append(_clear_launches)
    if _fast is not None:
        params = rec.packed_params()
        if params is not None:
            if host:
                _fast.add_host(subscripts, a, b, params, list(rec.shape), bool(rec.swap), dispatch._device().index or 0)
            else:
                _fast.add(subscripts, a, b, params, list(rec.shape), bool(rec.swap))
        return
    if host:
        return
    run = rec.launcher(a.device)
    if run is not None:
        if len(_LAUNCH_CACHE) >= _LAUNCH_CACHE_MAX:
            _LAUNCH_CACHE.clear()
        _LAUNCH_CACHE[_launch_key(subscripts, a, b)] = run


def _execute_contraction(
    subscripts: str,
    operands: tuple,
    plan: ContractionPlan,
    alpha: float = 1.0,
    beta: float = 0.0,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Run a plan (reference trntensor/einsum.py:106-126).

    "kahan" contracts in float64 and casts back to the first operand's dtype.
    "dd" (which the reference rejects with NotImplementedError) contracts
    float64 copies with every product exact and every sum in double-double,
    rounded to float64 once per pairwise step, then casts back. Otherwise
    the strategy selects the executor: matmul and bmm go to the GEMM core,
    "torch" to the general engine, "path" to the pairwise executor.
    """
    if plan.precision == "dd":
        with engine.accumulation("dd"):
            return _run(subscripts, operands, plan, alpha, beta, out, torch.float64)
    return _run(subscripts, operands, plan, alpha, beta, out, None)


def _run(subscripts, operands, plan, alpha, beta, out, cd_override):
    dispatch.require_hip()
    devs, orig = dispatch.place(*operands, *([out] if out is not None else []))
    ops = devs[: len(operands)]
    out_dev = devs[-1] if out is not None else None
    dts = {o.dtype for o in ops}
    if len(dts) > 1:
        raise RuntimeError(f"einsum(): operands must share one dtype, got {sorted(str(d) for d in dts)}")
    res_dtype = ops[0].dtype
    if cd_override is not None:
        cd = cd_override
    elif plan.precision == "kahan":
        cd = torch.float64
    elif res_dtype in (torch.bfloat16, torch.float16) and len(ops) == 2 and plan.strategy != "path":
        cd = res_dtype  # the engine runs GEMM shapes on the 16-bit MFMA and widens the rest
    else:
        cd = dispatch.compute_dtype(res_dtype)
    ops = [o if o.dtype == cd else o.to(cd) for o in ops]
    lhs, out_str = _parse_subscripts(subscripts)
    terms = lhs.split(",")

    prefer_gemm = plan.strategy in ("matmul", "bmm")
    if res_dtype.is_complex or not res_dtype.is_floating_point or isinstance(alpha, complex) or isinstance(beta, complex):
        # Integer and complex results, and complex scalars: the contraction
        # alone on the kernels, then the reference's two scalar passes
        # (trntensor/einsum.py:99-102) under torch's promotion rules: an
        # integer result times a float alpha becomes float32, a complex alpha
        # makes a real result complex, complex scalars rotate the parts, an
        # integral result takes only an integral beta and a real one only a
        # real beta.
        res = _contract(terms, out_str, ops, plan, 1.0, 0.0, None, prefer_gemm)
        if res.dtype != res_dtype:
            res = res.to(res_dtype)
        res = _scalar_epilogue(res, alpha, beta, out_dev)
        return res if res.device == orig else res.to(orig)

    # The reference finishes with result.add(out, alpha=beta)
    # (trntensor/einsum.py:101-102): torch's type promotion and broadcasting.
    # When `out` promotes to the contraction's dtype and broadcasts to its
    # shape, beta*out is fused into the last kernel's store; otherwise the
    # contraction (with alpha) is rounded to its own dtype first and a
    # second pass adds beta*out in the promoted dtype and broadcast shape.
    C = None
    post = None
    if out_dev is not None:
        shape = _result_shape(terms, out_str, ops)
        final_dtype = torch.promote_types(res_dtype, out_dev.dtype)
        final_shape = list(torch.broadcast_shapes(tuple(shape), tuple(out_dev.shape)))
        if final_dtype == res_dtype and final_shape == shape:
            C = out_dev.to(cd).expand(shape).contiguous()
        else:
            dispatch.compute_dtype(final_dtype)  # raises for dtypes the kernels do not compute in
            post = (final_dtype, final_shape)

    kb, kc = (beta, C) if post is None else (0.0, None)
    res = _contract(terms, out_str, ops, plan, alpha, kb, kc, prefer_gemm)
    if res.dtype != res_dtype:
        res = res.to(res_dtype)
    if post is not None:
        res = _scalar_epilogue(res, 1.0, beta, out_dev)
    return res if res.device == orig else res.to(orig)


def _contract(terms, out_str, ops, plan, alpha, beta, C, prefer_gemm):
    if plan.strategy == "path":
        return _execute_path(terms, out_str, ops, plan.contraction_path, alpha, beta, C)
    return engine.contract(terms, out_str, ops, alpha, beta, C, prefer_gemm=prefer_gemm)


def _scalar_epilogue(res: torch.Tensor, alpha, beta, out: torch.Tensor | None) -> torch.Tensor:
    """result.mul(alpha) if alpha != 1, then result.add(out, alpha=beta), with
    torch's dtype rules (trntensor/einsum.py:99-102), on the device kernels."""
    if alpha != 1.0:
        res = _mul_scalar(res, alpha)
    if out is None:
        return res
    dtype = torch.promote_types(res.dtype, out.dtype)
    if not (dtype.is_floating_point or dtype.is_complex) and isinstance(beta, float):
        raise RuntimeError("For integral input tensors, argument alpha must not be a floating point number.")
    if not dtype.is_complex and isinstance(beta, complex):
        raise RuntimeError("For non-complex input tensors, argument alpha must not be a complex number.")
    shape = list(torch.broadcast_shapes(tuple(res.shape), tuple(out.shape)))
    return _add_out(res, out, beta, dtype, shape)


def _mul_scalar(res: torch.Tensor, alpha) -> torch.Tensor:
    """res * alpha in torch.result_type(res, alpha), one strided pass per part."""
    dtype = torch.result_type(res, alpha)
    if dtype.is_complex:
        re, im = engine.complex_parts(res.to(dtype).resolve_conj())
        a = complex(alpha)
        if a.imag == 0:
            re2, im2 = _axpby(re, a.real), _axpby(im, a.real)
        else:
            # (re + i im)(ar + i ai) = (ar re - ai im) + i (ar im + ai re)
            re2, im2 = _axpby(re, a.real, im, -a.imag), _axpby(im, a.real, re, a.imag)
        return torch.complex(re2, im2)
    cd = dispatch.compute_dtype(dtype)
    r = res.to(cd).contiguous()
    out = _axpby(r, int(alpha) if cd == torch.int64 else float(alpha))
    return out if cd == dtype else out.to(dtype)


def _axpby(x: torch.Tensor, a, y: torch.Tensor | None = None, b=0.0) -> torch.Tensor:
    """a * x (+ b * y) for contiguous real tensors of one shape (one strided pass)."""
    D = torch.empty_like(x)
    engine.strided_contract([(n, s, 0) for n, s in zip(x.shape, x.stride())], [], x, None, D, a, b, y)
    return D


def _add_out(res: torch.Tensor, out: torch.Tensor, beta, dtype: torch.dtype, shape: list[int]) -> torch.Tensor:
    """res + beta * out in `dtype`, broadcast to `shape` (one strided pass on the
    device per real part; 16-bit results are computed in float32 and rounded
    once; integers in int64 with wraparound)."""
    if dtype.is_complex:
        rr, ri = engine.complex_parts(res.to(dtype).resolve_conj())
        orr, ori = engine.complex_parts(out.to(dtype).resolve_conj())
        b = complex(beta)
        re = _add_real(rr, orr, b.real, shape)
        im = _add_real(ri, ori, b.real, shape)
        if b.imag != 0:
            re = _add_real(re, ori, -b.imag, shape)
            im = _add_real(im, orr, b.imag, shape)
        return torch.complex(re, im)
    cd = dispatch.compute_dtype(dtype)
    D = _add_real(res.to(cd), out.to(cd), int(beta) if cd == torch.int64 else beta, shape)
    return D if cd == dtype else D.to(dtype)


def _add_real(r: torch.Tensor, o: torch.Tensor, beta, shape: list[int]) -> torch.Tensor:
    """r + beta * o, both broadcast to `shape`, in their (common, real) dtype."""
    lead = len(shape) - r.dim()
    strides = [0] * lead + [0 if n == 1 and m != 1 else s for n, m, s in zip(r.shape, shape[lead:], r.stride())]
    C = o.expand(shape).contiguous()
    D = torch.empty(shape, dtype=r.dtype, device=r.device)
    engine.strided_contract([(n, s, 0) for n, s in zip(shape, strides)], [], r, None, D, 1.0, beta, C)
    return D


def _result_shape(terms, out_str, ops) -> list[int]:
    ext: dict[str, int] = {}
    for term, op in zip(terms, ops):
        ext.update((c, int(n)) for c, n in zip(term, op.shape))
    return [ext[c] for c in out_str]


def _step_output(terms: list[str], i: int, j: int, out: str) -> str:
    """Intermediate letters of a path step (reference trntensor/einsum.py:171-185):
    free letters of terms[i] then terms[j] in first-seen order, minus letters
    no later operand or the output needs."""
    keep = set(out)
    for k, term in enumerate(terms):
        if k != i and k != j:
            keep.update(term)
    gone = (set(terms[i]) | set(terms[j])) - keep
    seen: list[str] = []
    for c in terms[i] + terms[j]:
        if c not in gone and c not in seen:
            seen.append(c)
    return "".join(seen)


def _path_names(terms: list[str], out: str, path: list[tuple[int, int]]) -> list[str]:
    """Letter order of every intermediate.

    Starts from the reference's naming. An intermediate's letter order is not
    observable (only the final output's is), so it is chosen for the step
    that consumes it: the letters summed in that step must form one run in
    the partner operand's order, or the GEMM would first pack the
    intermediate. When they do not, the intermediate keeps its other letters
    in order and takes the summed letters last, in the partner's order. This
    covers a full or elementwise dot (every letter summed: the intermediate
    takes the partner's order and the step streams both tensors
    contiguously). When both operands of a step are intermediates, the one
    produced earlier is reordered. Each intermediate is consumed exactly
    once, so steps are visited from the last to the first.
    """
    names: list[str] = []
    cur = list(terms)
    entries: list[tuple[str, int]] = [("in", k) for k in range(len(terms))]
    step_ops = []
    for s, (i, j) in enumerate(path):
        step_ops.append((entries[i], entries[j]))
        name = out if s == len(path) - 1 else _step_output(cur, i, j, out)
        names.append(name)
        cur = [t for k, t in enumerate(cur) if k != i and k != j] + [name]
        entries = [e for k, e in enumerate(entries) if k != i and k != j] + [("st", s)]

    def name_of(e):
        return terms[e[1]] if e[0] == "in" else names[e[1]]

    for t in reversed(range(len(path))):
        ei, ej = step_ops[t]
        inter = [e for e in (ei, ej) if e[0] == "st"]
        if not inter:
            continue
        x = min(inter, key=lambda e: e[1])
        partner = ej if x is ei else ei
        xn, pn = name_of(x), name_of(partner)
        if len(set(pn)) != len(pn):
            continue
        summed = (set(xn) & set(pn)) - set(names[t])
        if not summed:
            continue
        order = "".join(c for c in pn if c in summed)
        if order in (xn[: len(order)], xn[len(xn) - len(order):]):
            continue  # already one run, in the partner's order, at an end
        names[x[1]] = "".join(c for c in xn if c not in summed) + order
    return names


def _fusion_plan(terms: list[str], out: str, path: list[tuple[int, int]], names: list[str]):
    """Steps whose results are never materialised, or None.

    When the path ends in a full dot (scalar output) of two tensors with the
    same letters and one of them is produced by a GEMM-shaped step, that
    step's product is contracted in the GEMM epilogue instead of stored. If
    the dot's other operand is produced by an outer-product step (no shared
    letters), it stays unevaluated too: its two factors multiply in the same
    epilogue. Returns (gemm_step, lazy_step or None).
    """
    if out != "" or len(path) < 2:
        return None
    entries: list[tuple[str, tuple]] = [(t, ("in", k)) for k, t in enumerate(terms)]
    step_ops = []
    for s, (i, j) in enumerate(path):
        step_ops.append((entries[i], entries[j]))
        entries = [e for k, e in enumerate(entries) if k != i and k != j] + [(names[s], ("st", s))]
    (ta, oa), (tb, ob) = step_ops[-1]
    if set(ta) != set(tb) or len(set(ta)) != len(ta) or len(set(tb)) != len(tb):
        return None

    def gemm_shaped(s):
        (t1, _), (t2, _) = step_ops[s]
        return bool((set(t1) & set(t2)) - set(names[s]))

    def outer(s):
        (t1, _), (t2, _) = step_ops[s]
        return not (set(t1) & set(t2)) and set(names[s]) == set(t1) | set(t2)

    cands = [(o, other) for o, other in ((oa, ob), (ob, oa)) if o[0] == "st" and gemm_shaped(o[1])]
    if not cands:
        return None
    g_origin, other = max(cands, key=lambda c: c[0][1])
    lazy = other[1] if other[0] == "st" and outer(other[1]) else None
    return g_origin[1], lazy


def _execute_path(
    terms: list[str],
    out: str,
    ops: list[torch.Tensor],
    path: list[tuple[int, int]],
    alpha: float,
    beta: float,
    C: torch.Tensor | None,
) -> torch.Tensor:
    """Pairwise execution of a greedy path (reference trntensor/einsum.py:151-193).

    Each step contracts ``ops[i]`` and ``ops[j]`` on the HIP engine, removes
    both and appends the result; the last step produces ``out`` and carries
    the alpha/beta epilogue. A final full dot is fused into the GEMM that
    produces one of its operands (see ``_fusion_plan``): the 21 GB product and
    outer product of 'ia,jb,abP,ijP->' are never written.
    """
    names = _path_names(terms, out, path)
    # The fused dot epilogue covers real float32/float64 products with native accumulation.
    fusable = engine._ACCUMULATION.get() != "dd" and ops[0].dtype in (torch.float32, torch.float64)
    plan = _fusion_plan(terms, out, path, names) if fusable else None
    deferred = set() if plan is None else {s for s in plan if s is not None}
    cur_terms = list(terms)
    cur: list = list(ops)
    for s, (i, j) in enumerate(path):
        last = s == len(path) - 1
        ti, tj = cur_terms[i], cur_terms[j]
        if s in deferred:
            res = ("deferred", s, [ti, tj], [cur[i], cur[j]])
        elif last and plan is not None:
            res = _fused_dot(names, plan, ti, cur[i], tj, cur[j], alpha, beta, C)
        else:
            res = engine.contract(
                [ti, tj],
                names[s],
                [_materialise(names, cur[i]), _materialise(names, cur[j])],
                alpha if last else 1.0,
                beta if last else 0.0,
                C if last else None,
            )
        cur = [t for k, t in enumerate(cur) if k != i and k != j] + [res]
        cur_terms = [t for k, t in enumerate(cur_terms) if k != i and k != j] + [names[s]]
    return cur[0]


def _materialise(names, x):
    """A deferred step's result as a tensor (computed now)."""
    if isinstance(x, tuple):
        _, s, tt, tensors = x
        return engine.contract(tt, names[s], [_materialise(names, t) for t in tensors])
    return x


def _fused_dot(names, plan, ti, xi, tj, xj, alpha, beta, C):
    """Final full dot with one operand produced by the deferred GEMM step."""
    gs, lazy = plan
    g, other, t_other = (xi, xj, tj) if isinstance(xi, tuple) and xi[1] == gs else (xj, xi, ti)
    _, _, gterms, gtensors = g
    gtensors = [_materialise(names, t) for t in gtensors]
    if isinstance(other, tuple) and other[1] == lazy:
        factors = list(zip(other[2], [_materialise(names, t) for t in other[3]]))
    else:
        factors = [(t_other, _materialise(names, other))]
    res = engine.contract_gemm_dot(gterms, names[gs], gtensors, factors, alpha, beta, C)
    if res is not None:
        return res
    return engine.contract([ti, tj], "", [_materialise(names, xi), _materialise(names, xj)], alpha, beta, C)


def multi_einsum(*contractions: tuple) -> list[torch.Tensor]:
    """Several contractions in one call; each entry is ``(subscripts, *operands)``.

    Operands that appear (by identity) in two or more contractions are copied
    to the device once and reused; each result comes back on the device of
    its contraction's first original operand (reference
    trntensor/einsum.py:196-241).
    """
    counts: dict[int, int] = {}
    keep: dict[int, torch.Tensor] = {}
    for c in contractions:
        for op in c[1:]:
            counts[id(op)] = counts.get(id(op), 0) + 1
            keep[id(op)] = op
    pinned: dict[int, torch.Tensor] = {}
    if dispatch.HAS_HIP and dispatch._use_hip():
        pinned = {k: dispatch.to_device(keep[k]) for k, n in counts.items() if n > 1 and keep[k].device.type == "cpu"}
    results = []
    for c in contractions:
        subs, originals = c[0], c[1:]
        ops = tuple(pinned.get(id(op), op) for op in originals)
        res = einsum(subs, *ops)
        if originals and res.device != originals[0].device:
            res = res.to(originals[0].device)
        results.append(res)
    return results
