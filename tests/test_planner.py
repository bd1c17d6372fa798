"""Planner host logic on any host: the reference's own assertions
(tests/test_plan.py:10-273, tests/test_einsum.py:190-213) applied to the
product planner (trntensor_amd.plan) and to the oracle's restatement, the
config-5 closed form, and a differential check of the two on random
expressions.
"""

import random

import pytest
import torch

import trntensor_amd as trntensor
from oracle import cpu_ref
from trntensor_amd.plan import _greedy_path_search, _parse_subscripts, _validate_subscripts


@pytest.fixture(params=["product", "oracle"])
def impl(request):
    if request.param == "product":
        return {
            "parse": _parse_subscripts,
            "validate": _validate_subscripts,
            "greedy": _greedy_path_search,
            "plan": trntensor.plan_contraction,
            "flops": trntensor.estimate_flops,
        }
    return {
        "parse": cpu_ref.parse_subscripts,
        "validate": cpu_ref.validate_subscripts,
        "greedy": cpu_ref.greedy_path,
        "plan": cpu_ref.plan_contraction,
        "flops": cpu_ref.estimate_flops,
    }


def t(*shape):
    return torch.empty(*shape)


class TestParse:
    def test_cases(self, impl):
        p = impl["parse"]
        assert p("ij,jk->ik") == ("ij,jk", "ik")
        assert p("ij,jk") == ("ij,jk", "ik")
        assert p("i,i")[1] == ""
        assert p("i,j")[1] == "ij"
        assert p("ba,cb")[1] == "ac"


class TestStrategy:
    def test_matmul_flags(self, impl):
        plan = impl["plan"]
        p = plan("ji,kj->ik", t(3, 4), t(5, 3))
        assert (p.strategy, p.transA, p.transB) == ("matmul", True, True)
        p = plan("ij,jk->ik", t(4, 3), t(3, 5))
        assert (p.strategy, p.transA, p.transB) == ("matmul", False, False)
        p = plan("ap,bp->ab", t(32, 96), t(32, 96))
        assert (p.strategy, p.transA, p.transB) == ("matmul", False, True)

    def test_bmm_torch_path(self, impl):
        plan = impl["plan"]
        p = plan("bij,bjk->bik", t(2, 3, 4), t(2, 4, 5))
        assert p.strategy == "bmm" and "j" in p.contraction_indices and "b" in p.batch_indices
        assert plan("ijk,jkl->il", t(3, 4, 5), t(4, 5, 6)).strategy == "torch"
        assert plan("mi,mnP->inP", t(8, 2), t(8, 8, 4)).strategy == "torch"
        assert plan("ii->", t(5, 5)).strategy == "torch"
        p = plan("ij,jk,kl->il", t(3, 4), t(4, 5), t(5, 2))
        assert p.strategy == "path" and len(p.contraction_path) == 2
        p = plan("ij,jk,kl,lm->im", t(3, 4), t(4, 5), t(5, 6), t(6, 2))
        assert p.strategy == "path" and len(p.contraction_path) == 3

    def test_estimated_flops_field_unset(self, impl):
        # reference plan.py:34: the field exists and is never populated
        assert impl["plan"]("ij,jk->ik", t(4, 3), t(3, 5)).estimated_flops == 0


class TestEstimateFlops:
    def test_values(self, impl):
        f = impl["flops"]
        assert f("ij,jk->ik", t(10, 20), t(20, 30)) == 10 * 20 * 30
        assert f("ij,jk->ik", t(4, 10), t(10, 6)) == 2 * f("ij,jk->ik", t(4, 5), t(5, 6))
        assert f("bij,bjk->bik", t(7, 3, 4), t(7, 4, 5)) == 7 * 3 * 4 * 5


class TestGreedy:
    def test_reference_pair_choices(self, impl):
        g = impl["greedy"]
        assert g(["ij", "jk", "kl"], "il", {"i": 100, "j": 200, "k": 5, "l": 50})[0] == (1, 2)
        assert g(["ij", "jk", "kl", "lm"], "im", {"i": 100, "j": 200, "k": 5, "l": 50, "m": 3})[0] == (2, 3)
        for n in range(3, 7):
            terms = [f"{chr(97 + k)}{chr(98 + k)}" for k in range(n)]
            sizes = {chr(97 + k): 4 for k in range(n + 1)}
            assert len(g(terms, "a" + chr(97 + n), sizes)) == n - 1

    def test_config5_path_closed_form(self, impl):
        """Pair costs over ['ia','jb','abP','ijP'] (rule of trntensor/plan.py:226-231):
        (0,1) = 128*400*128*400 = 2.62144e9 is the minimum; then all three pairs
        of ['abP','ijP','abij'] cost 400*400*128*128*800 = 2.097152e12 and the
        first wins; the path closes with (0,1)."""
        sizes = {"i": 128, "a": 400, "j": 128, "b": 400, "P": 800}
        assert 128 * 400 * 128 * 400 == 2_621_440_000
        assert impl["greedy"](["ia", "jb", "abP", "ijP"], "", sizes) == [(0, 1), (0, 1), (0, 1)]
        p = impl["plan"]("ia,jb,abP,ijP->", t(128, 400), t(128, 400), t(400, 400, 800), t(128, 128, 800))
        assert p.strategy == "path" and p.contraction_path == [(0, 1), (0, 1), (0, 1)]


class TestValidation:
    """tests/test_plan.py:178-210 error messages."""

    def test_messages(self, impl):
        v = impl["validate"]
        with pytest.raises(ValueError, match="2 operand term"):
            v("ij,jk->ik", (t(4, 3), t(3, 5), t(5, 2)))
        with pytest.raises(ValueError, match="operand 1"):
            v("ij,jkl->ikl", (t(4, 3), t(3, 5)))
        with pytest.raises(ValueError, match="index 'j'"):
            v("ij,jk->ik", (t(4, 3), t(5, 6)))
        with pytest.raises(ValueError, match="invalid characters"):
            v("i j,jk->ik", (t(4, 3), t(3, 5)))
        with pytest.raises(ValueError, match="invalid characters"):
            v("...i,i->", (t(4, 3), t(3)))
        v("ij,jk->ik", (t(4, 3), t(3, 5)))
        with pytest.raises(ValueError, match="index 'j'"):
            impl["plan"]("ij,jk->ik", t(4, 3), t(5, 6))
        with pytest.raises(ValueError, match="precision must be"):
            impl["plan"]("ij,jk->ik", t(4, 3), t(3, 5), precision="super")


class TestPlanCache:
    """tests/test_plan.py:213-273 (product planner only: the oracle has no cache)."""

    def setup_method(self):
        trntensor.clear_plan_cache()

    def test_errors_around_a_cached_plan(self):
        """Validation runs on cache misses only; a call that would fail never
        matches a cached key (same subscripts and shapes), so every error
        still surfaces, in the reference's precedence."""
        A, B = t(4, 3), t(3, 5)
        trntensor.plan_contraction("ij,jk->ik", A, B)
        with pytest.raises(ValueError, match="index 'j'"):
            trntensor.plan_contraction("ij,jk->ik", A, t(5, 6))
        with pytest.raises(ValueError, match="2 operand term"):
            trntensor.plan_contraction("ij,jk->ik", A, B, t(5, 2))
        with pytest.raises(ValueError, match="precision must be"):
            trntensor.plan_contraction("ij,jk->ik", A, B, precision="super")
        with pytest.raises(ValueError, match="optimize must be"):
            trntensor.plan_contraction("ij,jk->ik", A, B, optimize="fastest")
        # subscript errors take precedence over a bad keyword
        with pytest.raises(ValueError, match="index 'j'"):
            trntensor.plan_contraction("ij,jk->ik", A, t(5, 6), precision="super")
        assert trntensor.plan_cache_info()["size"] == 1

    def test_hit_miss_clear_and_precision_key(self):
        A, B = t(4, 3), t(3, 5)
        p1 = trntensor.plan_contraction("ij,jk->ik", A, B)
        p2 = trntensor.plan_contraction("ij,jk->ik", A, B)
        assert p1 is p2 and trntensor.plan_cache_info()["size"] == 1
        trntensor.plan_contraction("ij,jk->ik", t(6, 3), t(3, 5))
        assert trntensor.plan_cache_info()["size"] == 2
        p3 = trntensor.plan_contraction("ij,jk->ik", A, B, precision="kahan")
        assert p3.precision == "kahan" and trntensor.plan_cache_info()["size"] == 3
        trntensor.clear_plan_cache()
        assert trntensor.plan_cache_info()["size"] == 0

    def test_validation_runs_on_cache_hit(self):
        trntensor.plan_contraction("ij,jk->ik", t(4, 3), t(3, 5))
        with pytest.raises(ValueError, match="precision must be"):
            trntensor.plan_contraction("ij,jk->ik", t(4, 3), t(3, 5), precision="bogus")

    def test_config5_cached_identity(self):
        ops = (t(128, 400), t(128, 400), t(400, 400, 800), t(128, 128, 800))
        assert trntensor.plan_contraction("ia,jb,abP,ijP->", *ops) is trntensor.plan_contraction("ia,jb,abP,ijP->", *ops)
        assert trntensor.plan_cache_info()["size"] == 1


def _random_expression(rng):
    letters = "abcdefghijklmnopqrstuvwxyzABCDEFGHIJ"
    nops = rng.choice([1, 2, 2, 2, 3, 4, 5])
    pool = rng.sample(letters, rng.randint(2, 7))
    sizes = {c: rng.randint(1, 9) for c in pool}
    terms = ["".join(rng.sample(pool, rng.randint(1, min(4, len(pool))))) for _ in range(nops)]
    seen = "".join(terms)
    out = "".join(c for c in pool if c in seen and rng.random() < 0.4)
    sub = ",".join(terms) + ("->" + out if rng.random() < 0.8 else "")
    return sub, [t(*[sizes[c] for c in term]) for term in terms]


def test_product_planner_matches_oracle_on_random_expressions():
    rng = random.Random(1234)
    fields = ("strategy", "transA", "transB", "contraction_path", "precision")
    for _ in range(3000):
        sub, ops = _random_expression(rng)
        trntensor.clear_plan_cache()
        a = trntensor.plan_contraction(sub, *ops)
        b = cpu_ref.plan_contraction(sub, *ops)
        for f in fields:
            assert getattr(a, f) == getattr(b, f), (sub, f)
        assert sorted(a.contraction_indices) == sorted(b.contraction_indices), sub
        assert sorted(a.batch_indices) == sorted(b.batch_indices), sub
        assert a.output_indices == b.output_indices, sub
        assert trntensor.estimate_flops(sub, *ops) == cpu_ref.estimate_flops(sub, *ops)


def test_path_layout_choice_config5():
    """The product names config 5's first intermediate 'abij' (not the reference's
    'iajb') so the final dot streams both tensors in the same order; the letter
    sets, and so the arithmetic, are those of the reference's path."""
    from trntensor_amd.einsum import _path_names, _step_output

    path = [(0, 1), (0, 1), (0, 1)]
    names = _path_names(["ia", "jb", "abP", "ijP"], "", path)
    assert names == ["abij", "abij", ""]
    assert _step_output(["ia", "jb", "abP", "ijP"], 0, 1, "") == "iajb"
    # chains keep the reference's names
    assert _path_names(["ij", "jk", "kl"], "il", [(1, 2), (0, 1)]) == ["jl", "il"]


class TestOptimalPath:
    """optimize="optimal" (opt-in; no counterpart in the reference): the DP path
    is pinned against brute force over every pairwise order, checked to be a
    valid path by executing it on the CPU, and never costs more than greedy."""

    @staticmethod
    def _all_paths(n):
        if n <= 2:
            yield [(0, 1)]
            return
        for i in range(n - 1):
            for j in range(i + 1, n):
                for rest in TestOptimalPath._all_paths(n - 1):
                    yield [(i, j)] + rest

    @staticmethod
    def _sizes(terms, ops):
        return {c: int(n) for term, op in zip(terms, ops) for c, n in zip(term, op.shape)}

    def test_config5_closed_form(self):
        from trntensor_amd.plan import _optimal_path_search, path_cost

        terms, sizes = ["ia", "jb", "abP", "ijP"], dict(i=128, j=128, a=400, b=400, P=800)
        path = _optimal_path_search(terms, "", sizes)
        # jb.abP -> ajP (i a b P... = 128*400*400*800), ijP.ajP -> ia (128*128*800*400), ia.ia -> ''
        assert path == [(1, 2), (1, 2), (0, 1)]
        assert path_cost(terms, "", sizes, path) == 128 * 400 * 400 * 800 + 128 * 128 * 800 * 400 + 128 * 400
        greedy = _greedy_path_search(terms, "", sizes)
        # ia.jb -> abij, abP.ijP -> abij, abij.abij -> ''
        assert path_cost(terms, "", sizes, greedy) == 2 * 128 * 400 * 128 * 400 + 128 * 128 * 400 * 400 * 800

    def test_matches_brute_force(self):
        from trntensor_amd.plan import _optimal_path_search, path_cost

        rng = random.Random(7)
        checked = 0
        while checked < 150:
            sub, ops = _random_expression(rng)
            lhs, out = _parse_subscripts(sub)
            terms = lhs.split(",")
            if not 3 <= len(terms) <= 5:
                continue
            sizes = self._sizes(terms, ops)
            path = _optimal_path_search(terms, out, sizes)
            assert len(path) == len(terms) - 1 and path[-1] == (0, 1), sub
            best = min(path_cost(terms, out, sizes, p) for p in self._all_paths(len(terms)))
            assert path_cost(terms, out, sizes, path) == best, sub
            assert best <= path_cost(terms, out, sizes, _greedy_path_search(terms, out, sizes)), sub
            checked += 1

    def test_path_executes_to_einsum(self):
        """The optimal path, run by the oracle's pairwise executor, gives einsum's value."""
        rng = random.Random(11)
        gen = torch.Generator().manual_seed(3)
        checked = 0
        while checked < 60:
            sub, ops = _random_expression(rng)
            if len(ops) < 3:
                continue
            ops = [torch.randn(*o.shape, generator=gen, dtype=torch.float64) for o in ops]
            trntensor.clear_plan_cache()
            plan = trntensor.plan_contraction(sub, *ops, optimize="optimal")
            ref_plan = cpu_ref.plan_contraction(sub, *ops)
            ref_plan.contraction_path = plan.contraction_path
            got = cpu_ref.execute_path(sub, ops, ref_plan)
            want = torch.einsum(sub, *ops)
            assert torch.allclose(got, want, rtol=1e-10, atol=1e-10), sub
            checked += 1

    def test_large_operand_count_falls_back(self):
        from trntensor_amd.plan import OPTIMAL_MAX_OPERANDS, _optimal_path_search, path_cost

        rng = random.Random(5)
        n = OPTIMAL_MAX_OPERANDS + 2
        letters = "abcdefghijklmn"
        terms = [letters[k] + letters[k + 1] for k in range(n)]  # a matrix chain
        sizes = {c: rng.randint(2, 60) for c in letters}
        out = letters[0] + letters[n]
        path = _optimal_path_search(terms, out, sizes)
        assert len(path) == n - 1 and path[-1] == (0, 1)
        assert path_cost(terms, out, sizes, path) <= path_cost(terms, out, sizes, _greedy_path_search(terms, out, sizes))

    def test_default_and_cache(self):
        ops = (t(128, 400), t(128, 400), t(400, 400, 800), t(128, 128, 800))
        trntensor.clear_plan_cache()
        g = trntensor.plan_contraction("ia,jb,abP,ijP->", *ops)
        o = trntensor.plan_contraction("ia,jb,abP,ijP->", *ops, optimize="optimal")
        assert g.contraction_path == [(0, 1), (0, 1), (0, 1)]
        assert o.contraction_path == [(1, 2), (1, 2), (0, 1)]
        assert trntensor.plan_cache_info()["size"] == 2
        assert trntensor.plan_contraction("ia,jb,abP,ijP->", *ops, optimize="optimal") is o
        # two operands: the label does not depend on the search
        assert trntensor.plan_contraction("ij,jk->ik", t(4, 3), t(3, 5), optimize="optimal").strategy == "matmul"
        with pytest.raises(ValueError, match="optimize must be"):
            trntensor.plan_contraction("ij,jk->ik", t(4, 3), t(3, 5), optimize="dp")
