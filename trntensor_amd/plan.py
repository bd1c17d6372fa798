"""Contraction planner: subscript validation, binary strategy labels, greedy
path search for 3+ operands, and the plan cache.

Mirrors trntensor/plan.py (reference): the same ``ContractionPlan`` fields,
the same strategy labels ("matmul" | "bmm" | "torch" | "path"), the same
greedy pair choices and intermediate naming, the same cache key and the same
``ValueError`` messages. The labels describe the contraction's shape only;
on this build every strategy executes on the HIP kernels (see
``trntensor_amd.hip.dispatch``), so ``backend`` reports ``"hip"`` whenever the
HIP runtime will run the call.
"""

from __future__ import annotations

import re
from collections import Counter
from dataclasses import dataclass, field

import torch

_SUBSCRIPT_RE = re.compile(r"[a-zA-Z,]+(->[a-zA-Z]*)?")


@dataclass
class ContractionPlan:
    """Execution plan for a tensor contraction (reference trntensor/plan.py:22-39).

    ``strategy`` is the reference's label for the contraction's shape;
    ``backend`` names the executor ("hip" on a gfx950 device, "pytorch" when
    no HIP runtime is present, in which case execution raises).
    ``contraction_path`` lists (i, j) pairs in the opt_einsum convention:
    indices into the current operand list, the result appended at the end.
    """

    subscripts: str
    strategy: str
    backend: str = "pytorch"
    transA: bool = False
    transB: bool = False
    contraction_indices: list[str] = field(default_factory=list)
    batch_indices: list[str] = field(default_factory=list)
    output_indices: list[str] = field(default_factory=list)
    estimated_flops: int = 0
    contraction_path: list[tuple[int, int]] = field(default_factory=list)
    precision: str = "fast"


def _parse_subscripts(subscripts: str) -> tuple[str, str]:
    """Split ``'ij,jk->ik'`` into ``('ij,jk', 'ik')``.

    Without ``->`` the output is every letter that occurs exactly once,
    in sorted order (reference trntensor/plan.py:246-258).
    """
    if "->" in subscripts:
        lhs, rhs = subscripts.split("->")
        return lhs, rhs
    counts = Counter(ch for ch in subscripts if ch.isalpha())
    return subscripts, "".join(sorted(ch for ch, n in counts.items() if n == 1))


def _validate_subscripts(subscripts: str, operands: tuple) -> None:
    """Raise ``ValueError`` for a malformed call (reference trntensor/plan.py:68-112).

    Checked in order: allowed characters, number of terms vs operands,
    each term's length vs its operand's ndim, one size per index letter.
    """
    if not _SUBSCRIPT_RE.fullmatch(subscripts):
        raise ValueError(
            f"einsum subscript {subscripts!r} contains invalid characters; "
            "only a-zA-Z, commas, and '->' are allowed"
        )
    terms = _parse_subscripts(subscripts)[0].split(",")
    if len(terms) != len(operands):
        raise ValueError(
            f"einsum subscript {subscripts!r} has {len(terms)} operand term(s) "
            f"but {len(operands)} operand(s) were given"
        )
    first_seen: dict[str, tuple[int, int]] = {}
    for pos, (term, op) in enumerate(zip(terms, operands)):
        if len(term) != op.ndim:
            raise ValueError(
                f"einsum operand {pos} has shape {tuple(op.shape)} (ndim={op.ndim}) "
                f"but subscript term {term!r} has {len(term)} indices"
            )
        for letter, extent in zip(term, op.shape):
            extent = int(extent)
            prev = first_seen.get(letter)
            if prev is None:
                first_seen[letter] = (extent, pos)
            elif prev[0] != extent:
                raise ValueError(
                    f"einsum index {letter!r} is size {prev[0]} in operand {prev[1]} "
                    f"but size {extent} in operand {pos}"
                )


_PLAN_CACHE: dict[tuple, ContractionPlan] = {}
# Launchers of two-operand contractions whose plan is cached and which run as
# one GEMM launch, keyed by subscripts and both operands' shapes, strides,
# dtypes and devices (filled and read by the einsum front-end; emptied with
# the plan cache, so a call after clear_plan_cache plans again).
_LAUNCH_CACHE: dict[tuple, object] = {}
_LAUNCH_CACHE_MAX = 4096
# Called by clear_plan_cache (the einsum front-end registers the clearing of
# its C++ launch table here).
_CLEAR_HOOKS: list = []

# Path searches for 3+ operands. "greedy" is the reference's rule and the
# default; "optimal" is opt-in (no counterpart in the reference).
PATH_SEARCHES = ("greedy", "optimal")


def _shape_key(subscripts: str, operands: tuple, precision: str = "fast", optimize: str = "greedy") -> tuple:
    """Cache key: subscripts, operand shapes, precision (reference plan.py:119-123).

    dtype and device are not part of the key, as in the reference. A
    non-default path search is appended, so default keys keep the
    reference's form.
    """
    key = (subscripts, tuple(tuple(op.shape) for op in operands), precision)
    return key if optimize == "greedy" else key + (optimize,)


def clear_plan_cache() -> None:
    """Discard all cached contraction plans."""
    _PLAN_CACHE.clear()
    _LAUNCH_CACHE.clear()
    for hook in _CLEAR_HOOKS:
        hook()


def plan_cache_info() -> dict[str, int]:
    """Cache statistics: ``{"size": number of cached plans}``."""
    return {"size": len(_PLAN_CACHE)}


def _backend_for(strategy: str, operands: tuple) -> str:
    """Executor that will run the plan (reference trntensor/plan.py:42-65).

    The reference reports "nki" only for matmul/bmm above a dispatch-latency
    threshold. A HIP launch costs microseconds and every strategy has a HIP
    executor, so here the answer depends only on whether the HIP runtime is
    active.
    """
    from .hip.dispatch import HAS_HIP, _use_hip

    return "hip" if (HAS_HIP and _use_hip()) else "pytorch"


def plan_contraction(
    subscripts: str, *operands: torch.Tensor, precision: str = "fast", optimize: str = "greedy"
) -> ContractionPlan:
    """Validate, then return the (cached) plan for this subscript/shape/precision.

    An unknown ``precision`` or ``optimize`` raises ``ValueError`` on every
    call. The subscripts are validated against the operands when the plan is
    not cached: the outcome depends only on the subscripts and the operand
    shapes, which the cache key holds, so a cached plan means an identical
    call already passed (the reference validates before its lookup; the
    errors raised are the same). Two operands get a binary strategy,
    three or more a path, one operand the "torch" label
    (reference trntensor/plan.py:140-185).

    ``optimize`` picks the path search for 3+ operands: ``"greedy"`` (default)
    is the reference's rule, so ``contraction_path`` matches the reference;
    ``"optimal"`` returns the order with the fewest total multiply-adds under
    the same per-step cost (see ``_optimal_path_search``). It changes only the
    order of pairwise steps, never the result beyond rounding.
    """
    if precision not in ("fast", "kahan", "dd") or optimize not in PATH_SEARCHES:
        _validate_subscripts(subscripts, operands)  # its errors come first, as in the reference
        if precision not in ("fast", "kahan", "dd"):
            raise ValueError(f"precision must be 'fast', 'kahan', or 'dd', got {precision!r}")
        raise ValueError(f"optimize must be one of {PATH_SEARCHES}, got {optimize!r}")
    key = _shape_key(subscripts, operands, precision, optimize)
    hit = _PLAN_CACHE.get(key)
    if hit is not None:
        return hit
    _validate_subscripts(subscripts, operands)

    lhs, out = _parse_subscripts(subscripts)
    terms = lhs.split(",")
    if len(operands) == 2:
        plan = _plan_binary(subscripts, terms, out, operands)
    elif len(operands) >= 3:
        extents: dict[str, int] = {}
        for term, op in zip(terms, operands):
            extents.update((c, int(n)) for c, n in zip(term, op.shape))
        search = _optimal_path_search if optimize == "optimal" else _greedy_path_search
        plan = ContractionPlan(
            subscripts=subscripts,
            strategy="path",
            contraction_path=search(terms, out, extents),
        )
    else:
        plan = ContractionPlan(subscripts=subscripts, strategy="torch")
    plan.backend = _backend_for(plan.strategy, operands)
    plan.precision = precision
    _PLAN_CACHE[key] = plan
    return plan


def _survivors(terms: list[str], i: int, j: int, out: str) -> set[str]:
    """Letters that must outlive a step contracting terms i and j."""
    keep = set(out)
    for k, term in enumerate(terms):
        if k != i and k != j:
            keep.update(term)
    return keep


def _greedy_path_search(input_list: list[str], output_str: str, size_map: dict[str, int]) -> list[tuple[int, int]]:
    """Greedy pairwise order for 3+ operands (reference trntensor/plan.py:188-243).

    Each step takes the pair whose letter union has the smallest product of
    extents (first pair wins ties, scanning i < j in order); the intermediate
    is named by its surviving letters in sorted order and appended to the
    list; the path ends with (0, 1).
    """
    terms = list(input_list)
    path: list[tuple[int, int]] = []
    while len(terms) > 2:
        best_cost = None
        best = (0, 1, "")
        for i in range(len(terms) - 1):
            for j in range(i + 1, len(terms)):
                union = set(terms[i]) | set(terms[j])
                cost = 1
                for letter in union:
                    cost *= size_map.get(letter, 1)
                if best_cost is None or cost < best_cost:
                    best_cost = cost
                    inter = union & _survivors(terms, i, j, output_str)
                    best = (i, j, "".join(sorted(inter)))
        i, j, name = best
        path.append((i, j))
        terms = [t for k, t in enumerate(terms) if k != i and k != j] + [name]
    path.append((0, 1))
    return path


def path_cost(input_list: list[str], output_str: str, size_map: dict[str, int], path: list[tuple[int, int]]) -> int:
    """Total multiply-adds of a pairwise path under the greedy search's step
    cost (product of the extents of every letter either operand carries).
    Intermediates carry the letters that a later operand or the output needs."""
    terms = list(input_list)
    total = 0
    for i, j in path:
        union = set(terms[i]) | set(terms[j])
        cost = 1
        for letter in union:
            cost *= size_map.get(letter, 1)
        total += cost
        name = "".join(sorted(union & _survivors(terms, i, j, output_str)))
        terms = [t for k, t in enumerate(terms) if k != i and k != j] + [name]
    return total


OPTIMAL_MAX_OPERANDS = 10


def _optimal_path_search(input_list: list[str], output_str: str, size_map: dict[str, int]) -> list[tuple[int, int]]:
    """Pairwise order with the fewest total multiply-adds (opt-in; the
    reference has only the greedy rule).

    Dynamic programming over operand subsets: the intermediate of a subset S
    carries the letters of S that an operand outside S or the output needs
    (an input keeps its own letters); contracting S1 with S2 costs the product
    of the extents of their letters, as in the greedy rule; best(S) is the
    minimum over splits S = S1 + S2 of best(S1) + best(S2) + that cost. The
    search is O(3^n), so above OPTIMAL_MAX_OPERANDS operands it returns the
    cheaper of the reference greedy path and a greedy path that picks the pair
    whose intermediate shrinks the working set most (ties: fewer
    multiply-adds, then first pair). The returned path uses the reference's
    convention: (i, j) index the current list, the result is appended, the
    last step is (0, 1).
    """
    n = len(input_list)
    if n > OPTIMAL_MAX_OPERANDS:
        cands = [_greedy_path_search(input_list, output_str, size_map), _shrink_path_search(input_list, output_str, size_map)]
        return min(cands, key=lambda p: path_cost(input_list, output_str, size_map, p))

    full = (1 << n) - 1
    letters = [set(t) for t in input_list]
    out = set(output_str)
    sub_letters: dict[int, set] = {}
    for s in range(1, full + 1):
        acc: set = set()
        for k in range(n):
            if s >> k & 1:
                acc |= letters[k]
        sub_letters[s] = acc

    def carried(s: int) -> set:
        if s & (s - 1) == 0:
            return letters[s.bit_length() - 1]
        rest = sub_letters[full & ~s] if s != full else set()
        return sub_letters[s] & (rest | out)

    inter = {s: carried(s) for s in range(1, full + 1)}
    best: dict[int, tuple[int, int]] = {1 << k: (0, 0) for k in range(n)}
    for s in sorted(range(1, full + 1), key=lambda x: bin(x).count("1")):
        if s & (s - 1) == 0:
            continue
        low = s & -s
        choice = None
        sub = (s - 1) & s
        while sub:
            if sub & low:  # each split once: S1 holds the lowest operand
                other = s ^ sub
                cost = 1
                for letter in inter[sub] | inter[other]:
                    cost *= size_map.get(letter, 1)
                total = best[sub][0] + best[other][0] + cost
                if choice is None or total < choice[0] or (total == choice[0] and sub < choice[1]):
                    choice = (total, sub)
            sub = (sub - 1) & s
        best[s] = choice

    cur = [1 << k for k in range(n)]
    path: list[tuple[int, int]] = []

    def emit(s: int) -> None:
        if s & (s - 1) == 0:
            return
        s1 = best[s][1]
        s2 = s ^ s1
        emit(s1)
        emit(s2)
        i, j = sorted((cur.index(s1), cur.index(s2)))
        path.append((i, j))
        del cur[j], cur[i]
        cur.append(s)

    emit(full)
    return path


def _shrink_path_search(input_list: list[str], output_str: str, size_map: dict[str, int]) -> list[tuple[int, int]]:
    """Greedy order by working-set size: each step takes the pair minimising
    size(intermediate) - size(a) - size(b), ties by step multiply-adds, then
    first pair (i < j scan)."""

    def size(letters) -> int:
        v = 1
        for c in letters:
            v *= size_map.get(c, 1)
        return v

    terms = list(input_list)
    path: list[tuple[int, int]] = []
    while len(terms) > 2:
        best = None
        for i in range(len(terms) - 1):
            for j in range(i + 1, len(terms)):
                union = set(terms[i]) | set(terms[j])
                inter = union & _survivors(terms, i, j, output_str)
                score = (size(inter) - size(terms[i]) - size(terms[j]), size(union))
                if best is None or score < best[0]:
                    best = (score, i, j, "".join(sorted(inter)))
        _, i, j, name = best
        path.append((i, j))
        terms = [t for k, t in enumerate(terms) if k != i and k != j] + [name]
    path.append((0, 1))
    return path


def _plan_binary(subscripts: str, input_indices: list[str], output_str: str, operands: tuple) -> ContractionPlan:
    """Reference strategy label for two operands (trntensor/plan.py:261-314).

    "matmul": one shared letter summed, no batch letter, both 2-D; transA is
    set when the summed letter leads A, transB when it trails B.
    "bmm": one summed letter and one batch letter, both 3-D. Otherwise "torch".
    The label does not decide the numerics: the HIP executor derives its GEMM
    mapping from letter positions, so every label computes the einsum.
    """
    ta, tb = input_indices[0], input_indices[1]
    out = list(output_str)
    shared = set(ta) & set(tb)
    contracted = shared - set(out)
    batch = shared & set(out)
    A, B = operands
    if len(contracted) == 1 and not batch and A.dim() == 2 and B.dim() == 2:
        c = next(iter(contracted))
        return ContractionPlan(
            subscripts=subscripts,
            strategy="matmul",
            transA=ta.index(c) == 0,
            transB=tb.index(c) == 1,
            contraction_indices=[c],
            output_indices=out,
        )
    strategy = "bmm" if (len(contracted) == 1 and len(batch) == 1 and A.dim() == 3 and B.dim() == 3) else "torch"
    return ContractionPlan(
        subscripts=subscripts,
        strategy=strategy,
        contraction_indices=list(contracted),
        batch_indices=list(batch),
        output_indices=out,
    )


def estimate_flops(subscripts: str, *operands: torch.Tensor) -> int:
    """Multiply-add count estimate: product of every distinct letter's extent
    (reference trntensor/plan.py:317-332)."""
    lhs, _ = _parse_subscripts(subscripts)
    extents: dict[str, int] = {}
    for term, op in zip(lhs.split(","), operands):
        for c, n in zip(term, op.shape):
            extents[c] = n
    total = 1
    for letter in {ch for ch in lhs if ch.isalpha()}:
        total *= extents.get(letter, 1)
    return total
