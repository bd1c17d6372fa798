"""CPU oracle: a restatement of trntensor's CPU torch path.

TEST INFRASTRUCTURE ONLY. Nothing in ``trntensor_amd`` imports this module;
it is imported by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, where it is the checker (and the timed
CPU baseline), never the thing measured or shipped.

The reference (trntensor 0.4.0) is pure Python over torch: with no NKI
runtime every contraction on the hot path is a fixed sequence of torch CPU
ops. This module performs the same ops in the same order, so on the same
torch build it reproduces the reference's CPU results bitwise. Each function
cites the reference file:line it follows (paths relative to the reference
repository root).

Pins (how each function is checked independently of itself) are listed in
``tests/test_oracle.py``; the numbers they rest on are in ``tests/golden/``.
"""

from __future__ import annotations

import re
from collections import Counter
from dataclasses import dataclass, field

import torch

# --------------------------------------------------------------------------
# dtype strings  (trntensor/einsum.py:27-48)
# --------------------------------------------------------------------------
DTYPE_MAP = {
    "bf16": torch.bfloat16,
    "bfloat16": torch.bfloat16,
    "fp16": torch.float16,
    "float16": torch.float16,
    "f32": torch.float32,
    "float32": torch.float32,
    "f64": torch.float64,
    "float64": torch.float64,
}


def resolve_dtype(dtype):
    """trntensor/einsum.py:39-48."""
    if dtype is None or isinstance(dtype, torch.dtype):
        return dtype
    key = dtype.lower()
    if key not in DTYPE_MAP:
        raise ValueError(f"unknown dtype {dtype!r}; valid strings: {sorted(DTYPE_MAP)}")
    return DTYPE_MAP[key]


# --------------------------------------------------------------------------
# planner  (trntensor/plan.py)
# --------------------------------------------------------------------------
@dataclass
class Plan:
    """Field set of ContractionPlan, trntensor/plan.py:22-39."""

    subscripts: str
    strategy: str
    backend: str = "pytorch"
    transA: bool = False
    transB: bool = False
    contraction_indices: list = field(default_factory=list)
    batch_indices: list = field(default_factory=list)
    output_indices: list = field(default_factory=list)
    estimated_flops: int = 0
    contraction_path: list = field(default_factory=list)
    precision: str = "fast"


def parse_subscripts(subscripts):
    """trntensor/plan.py:246-258: implicit output = letters seen once, sorted."""
    if "->" in subscripts:
        lhs, rhs = subscripts.split("->")
        return lhs, rhs
    letters = [c for c in subscripts if c.isalpha()]
    once = sorted(c for c, n in Counter(letters).items() if n == 1)
    return subscripts, "".join(once)


def validate_subscripts(subscripts, operands):
    """trntensor/plan.py:68-112 (same checks, same order, same messages)."""
    if not re.fullmatch(r"[a-zA-Z,]+(->[a-zA-Z]*)?", subscripts):
        raise ValueError(
            f"einsum subscript {subscripts!r} contains invalid characters; "
            "only a-zA-Z, commas, and '->' are allowed"
        )
    terms = parse_subscripts(subscripts)[0].split(",")
    if len(terms) != len(operands):
        raise ValueError(
            f"einsum subscript {subscripts!r} has {len(terms)} operand term(s) "
            f"but {len(operands)} operand(s) were given"
        )
    seen = {}
    for k, (term, op) in enumerate(zip(terms, operands)):
        if len(term) != op.ndim:
            raise ValueError(
                f"einsum operand {k} has shape {tuple(op.shape)} (ndim={op.ndim}) "
                f"but subscript term {term!r} has {len(term)} indices"
            )
        for c, n in zip(term, op.shape):
            n = int(n)
            if c in seen and seen[c][0] != n:
                raise ValueError(
                    f"einsum index {c!r} is size {seen[c][0]} in operand {seen[c][1]} "
                    f"but size {n} in operand {k}"
                )
            seen.setdefault(c, (n, k))


def plan_binary(subscripts, terms, out, operands):
    """trntensor/plan.py:261-314."""
    ta, tb = terms[0], terms[1]
    contracted = (set(ta) & set(tb)) - set(out)
    batch = set(ta) & set(tb) & set(out)
    A, B = operands
    if len(contracted) == 1 and not batch and A.dim() == 2 and B.dim() == 2:
        c = next(iter(contracted))
        return Plan(
            subscripts,
            "matmul",
            transA=ta.index(c) == 0,
            transB=tb.index(c) == 1,
            contraction_indices=[c],
            output_indices=list(out),
        )
    if len(contracted) == 1 and len(batch) == 1 and A.dim() == 3 and B.dim() == 3:
        return Plan(
            subscripts,
            "bmm",
            contraction_indices=list(contracted),
            batch_indices=list(batch),
            output_indices=list(out),
        )
    return Plan(
        subscripts,
        "torch",
        contraction_indices=list(contracted),
        batch_indices=list(batch),
        output_indices=list(out),
    )


def greedy_path(terms, out, sizes):
    """trntensor/plan.py:188-243: cost = product of sizes over the pair's union,
    first strict minimum wins, intermediate named by its sorted letters,
    a final (0, 1) closes the path."""
    terms = list(terms)
    path = []
    while len(terms) > 2:
        best = None
        for i in range(len(terms)):
            for j in range(i + 1, len(terms)):
                keep = set(out)
                for k, t in enumerate(terms):
                    if k not in (i, j):
                        keep |= set(t)
                union = set(terms[i]) | set(terms[j])
                cost = 1
                for c in union:
                    cost *= sizes.get(c, 1)
                if best is None or cost < best[0]:
                    best = (cost, i, j, union & keep)
        _, i, j, inter = best
        path.append((i, j))
        terms = [t for k, t in enumerate(terms) if k not in (i, j)] + ["".join(sorted(inter))]
    path.append((0, 1))
    return path


def plan_contraction(subscripts, *operands, precision="fast"):
    """trntensor/plan.py:140-185 without the cache (no NKI: backend 'pytorch')."""
    validate_subscripts(subscripts, operands)
    if precision not in ("fast", "kahan", "dd"):
        raise ValueError(f"precision must be 'fast', 'kahan', or 'dd', got {precision!r}")
    lhs, out = parse_subscripts(subscripts)
    terms = lhs.split(",")
    if len(operands) == 2:
        plan = plan_binary(subscripts, terms, out, operands)
    elif len(operands) >= 3:
        sizes = {}
        for t, op in zip(terms, operands):
            for c, n in zip(t, op.shape):
                sizes[c] = int(n)
        plan = Plan(subscripts, "path", contraction_path=greedy_path(terms, out, sizes))
    else:
        plan = Plan(subscripts, "torch")
    plan.precision = precision
    return plan


def estimate_flops(subscripts, *operands):
    """trntensor/plan.py:317-332: product of every distinct index size (MACs)."""
    lhs, _ = parse_subscripts(subscripts)
    sizes = {}
    for t, op in zip(lhs.split(","), operands):
        for c, n in zip(t, op.shape):
            sizes[c] = n
    total = 1
    for c in set(ch for ch in lhs if ch.isalpha()):
        total *= sizes.get(c, 1)
    return total


# --------------------------------------------------------------------------
# executors  (trntensor/einsum.py:106-193, nki/dispatch.py:195-196,347-348)
# --------------------------------------------------------------------------
def path_step_output(terms, i, j, out):
    """Intermediate naming of the path executor, trntensor/einsum.py:171-185:
    free letters of terms[i] then terms[j], first occurrence kept."""
    keep = set(out)
    for k, t in enumerate(terms):
        if k not in (i, j):
            keep |= set(t)
    dropped = (set(terms[i]) | set(terms[j])) - keep
    inter = []
    for c in terms[i] + terms[j]:
        if c not in dropped and c not in inter:
            inter.append(c)
    return "".join(inter)


def execute_path(subscripts, operands, plan):
    """trntensor/einsum.py:151-193: each binary step is a torch.einsum call."""
    lhs, out = parse_subscripts(subscripts)
    terms = lhs.split(",")
    ops = list(operands)
    steps = plan.contraction_path
    for s, (i, j) in enumerate(steps):
        inter = out if s == len(steps) - 1 else path_step_output(terms, i, j, out)
        res = torch.einsum(f"{terms[i]},{terms[j]}->{inter}", ops[i], ops[j])
        ops = [o for k, o in enumerate(ops) if k not in (i, j)] + [res]
        terms = [t for k, t in enumerate(terms) if k not in (i, j)] + [inter]
    return ops[0]


def execute(subscripts, operands, plan):
    """trntensor/einsum.py:106-148 (CPU branches of the NKI dispatchers)."""
    if plan.precision == "kahan":
        dt = operands[0].dtype if operands else torch.float32
        return torch.einsum(subscripts, *(o.to(torch.float64) for o in operands)).to(dt)
    if plan.precision == "dd":
        raise NotImplementedError(
            "precision='dd' requires double-double GEMM kernels; "
            "use precision='kahan' (fp64 accumulation) as an alternative."
        )
    if plan.strategy == "matmul":
        A, B = operands
        return torch.matmul(A.T if plan.transA else A, B.T if plan.transB else B)
    if plan.strategy == "bmm":
        return torch.bmm(*operands)
    if plan.strategy == "path":
        return execute_path(subscripts, operands, plan)
    return torch.einsum(subscripts, *operands)


def einsum(subscripts, *operands, alpha=1.0, beta=0.0, out=None, dtype=None, precision="fast"):
    """trntensor/einsum.py:51-103: cast, plan, execute, then the two separate
    epilogue passes (result*alpha, then result + beta*out as a new tensor)."""
    target = resolve_dtype(dtype)
    if target is not None:
        operands = tuple(o.to(target) for o in operands)
    plan = plan_contraction(subscripts, *operands, precision=precision)
    res = execute(subscripts, operands, plan)
    if alpha != 1.0:
        res = res.mul(alpha)
    if out is not None:
        res = res.add(out, alpha=beta)
    return res


def multi_einsum(*contractions):
    """trntensor/einsum.py:196-241 with no device runtime: a loop of einsum."""
    return [einsum(c[0], *c[1:]) for c in contractions]


def misplanned_by_reference(subscripts, *operands):
    """True where the reference's matmul/bmm executor disagrees with einsum
    semantics (trntensor/plan.py:284-305 checks neither output order, nor
    free letters summed away, nor bmm index positions). The reference returns
    ``A@B`` / ``bmm(A,B)`` for these; the product computes the einsum."""
    plan = plan_contraction(subscripts, *operands)
    lhs, out = parse_subscripts(subscripts)
    ta, tb = (lhs.split(",") + ["", ""])[:2]
    if plan.strategy == "matmul":
        m = ta[1] if plan.transA else ta[0]
        n = tb[0] if plan.transB else tb[1]
        return out != m + n
    if plan.strategy == "bmm":
        b = plan.batch_indices[0]
        c = plan.contraction_indices[0]
        if ta[0] != b or tb[0] != b or ta[2] != c or tb[1] != c:
            return True
        return out != b + ta[1] + tb[2]
    return False


# --------------------------------------------------------------------------
# quantum primitives  (trntensor/quantum.py)
# --------------------------------------------------------------------------
def mp2_energy(B, eps_occ, eps_vir):
    """_cpu_mp2_energy, trntensor/quantum.py:87-100: all nocc^2 ordered pairs,
    per pair one 'ap,bp->ab' einsum, denominator ((e_i+e_j)-e_a)-e_b, term
    T*(2T-T.T)/denom summed, accumulated in a 0-D tensor of B.dtype."""
    e = B.new_zeros(())
    ev_col = eps_vir.unsqueeze(1)
    ev_row = eps_vir.unsqueeze(0)
    for i in range(B.shape[0]):
        for j in range(B.shape[0]):
            T = torch.einsum("ap,bp->ab", B[i], B[j])
            denom = eps_occ[i] + eps_occ[j] - ev_col - ev_row
            e = e + (T * (2 * T - T.T) / denom).sum()
    return e


def mp2_energy_pairs(B, eps_occ, eps_vir, pairs):
    """The same per-pair arithmetic as mp2_energy over an explicit list of
    (i, j) pairs; used to time a bounded sample of the full loop."""
    e = B.new_zeros(())
    ev_col = eps_vir.unsqueeze(1)
    ev_row = eps_vir.unsqueeze(0)
    for i, j in pairs:
        T = torch.einsum("ap,bp->ab", B[i], B[j])
        denom = eps_occ[i] + eps_occ[j] - ev_col - ev_row
        e = e + (T * (2 * T - T.T) / denom).sum()
    return e


def df_mp2_einsum_loop(B, eps_occ, eps_vir):
    """examples/df_mp2_einsum.py:25-46: the config-1 harness. Same loop, each
    pair through einsum (matmul strategy, transB), Python-float accumulation."""
    e = 0.0
    for i in range(B.shape[0]):
        for j in range(B.shape[0]):
            T = einsum("ap,bp->ab", B[i], B[j])
            denom = eps_occ[i] + eps_occ[j] - eps_vir.unsqueeze(1) - eps_vir.unsqueeze(0)
            e += (T * (2 * T - T.T) / denom).sum().item()
    return e


def ao_to_mo_transform(eri, C_occ, C_vir):
    """_cpu_ao_to_mo_transform, trntensor/quantum.py:188-194."""
    return torch.einsum("mi,na,mnP->iaP", C_occ, C_vir, eri)


def ao_to_mo_two_step(eri, C_occ, C_vir):
    """The decomposed form the reference's own test checks against
    (tests/test_quantum.py:72-74); scales to large nbasis, unlike the
    3-operand einsum, which materialises an (m,i,n,a) product."""
    X = torch.einsum("mi,mnP->inP", C_occ, eri)
    return torch.einsum("na,inP->iaP", C_vir, X)


def ao_to_mo_half(eri, C_occ):
    """Config-3 contraction 'mi,mnP->inP': planned "torch" by the reference
    (trntensor/plan.py:307-314) and run as torch.einsum (einsum.py:117-118)."""
    return torch.einsum("mi,mnP->inP", C_occ, eri)
