"""Pins for the CPU oracle (oracle/cpu_ref.py), on any host.

Each oracle function is checked against something it does not share code
with: the reference's tutorial known answer, the golden fixtures (explicit
loops / numpy float64), closed forms and invariances. The planted-mistake
tests show the pins reject a dropped exchange term, a wrong sign, a
transposed operand and a wrong denominator order.
"""

import os

import numpy as np
import pytest
import torch

from oracle import brute, cpu_ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


# ---------------------------------------------------------------------------
# MP2
# ---------------------------------------------------------------------------
def test_tutorial_known_answer():
    """docs/tutorial_df_mp2.md:23-28,75-77 / examples/df_mp2_einsum.py:64-67:
    E = -50.5432928801 for nocc,nvir,naux = 5,19,72, seed 42."""
    torch.manual_seed(42)
    B = torch.randn(5, 19, 72) * 0.1
    eo = -torch.sort(torch.rand(5))[0] - 0.5
    ev = torch.sort(torch.rand(19))[0] + 0.1
    e = cpu_ref.df_mp2_einsum_loop(B, eo, ev)
    assert abs(e - (-50.5432928801)) <= 5e-11
    assert abs(float(cpu_ref.mp2_energy(B, eo, ev)) - e) <= 1e-4


def test_mp2_matches_golden_loops():
    g = load("mp2_small.npz")
    k = 0
    while f"B{k}" in g:
        B, eo, ev = (torch.from_numpy(g[n + str(k)]) for n in ("B", "eo", "ev"))
        e = float(cpu_ref.mp2_energy(B, eo, ev))
        assert abs(e - float(g[f"E_loops{k}"])) <= 1e-12 * max(1.0, abs(e))
        assert abs(e - float(g[f"E_4index{k}"])) <= 1e-12 * max(1.0, abs(e))
        k += 1
    assert k == 5


def test_mp2_matches_reference_unrolled_formula():
    """tests/test_quantum.py:11-33: the loop equals the 4-index einsum formula."""
    torch.manual_seed(0)
    B = torch.randn(2, 3, 5) * 0.1
    eo = torch.tensor([-0.5, -0.4])
    ev = torch.tensor([0.1, 0.2, 0.3])
    T = torch.einsum("iap,jbp->ijab", B, B)
    denom = eo.view(-1, 1, 1, 1) + eo.view(1, -1, 1, 1) - ev.view(1, 1, -1, 1) - ev.view(1, 1, 1, -1)
    expected = (T * (2 * T - T.transpose(-1, -2)) / denom).sum()
    torch.testing.assert_close(cpu_ref.mp2_energy(B, eo, ev), expected, atol=1e-6, rtol=1e-6)


def test_mp2_rank1_closed_form():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4, generator=g, dtype=torch.float64)
    y = torch.randn(6, generator=g, dtype=torch.float64)
    eo = torch.sort(-20 + 19.7 * torch.rand(4, generator=g, dtype=torch.float64))[0]
    ev = torch.sort(0.1 + 4.9 * torch.rand(6, generator=g, dtype=torch.float64))[0]
    B = (x[:, None] * y[None, :])[:, :, None]
    e = float(cpu_ref.mp2_energy(B, eo, ev))
    assert abs(e - brute.mp2_energy_rank1(x, y, eo, ev)) <= 1e-13 * abs(e)


def test_mp2_invariants():
    g = torch.Generator().manual_seed(6)
    B = torch.randn(3, 7, 9, generator=g, dtype=torch.float64) * 0.1
    eo = torch.sort(-20 + 19.7 * torch.rand(3, generator=g, dtype=torch.float64))[0]
    ev = torch.sort(0.1 + 4.9 * torch.rand(7, generator=g, dtype=torch.float64))[0]
    e = float(cpu_ref.mp2_energy(B, eo, ev))
    assert e < 0
    assert abs(float(cpu_ref.mp2_energy(B, eo + 0.5, ev + 0.5)) - e) <= 1e-12 * abs(e)
    assert abs(float(cpu_ref.mp2_energy(3.0 * B, eo, ev)) - 81.0 * e) <= 1e-12 * 81 * abs(e)
    perm = torch.randperm(7, generator=g)
    assert abs(float(cpu_ref.mp2_energy(B[:, perm], eo, ev[perm])) - e) <= 1e-12 * abs(e)
    assert float(cpu_ref.mp2_energy(torch.zeros_like(B), eo, ev)) == 0.0


def _mutant(kind):
    """Oracle loop with one planted mistake (CPU only)."""

    def run(B, eo, ev):
        e = B.new_zeros(())
        for i in range(B.shape[0]):
            for j in range(B.shape[0]):
                Bj = B[j] if kind != "transposed" else B[i]
                T = torch.einsum("ap,bp->ab", B[i], Bj)
                if kind == "denominator":
                    d = eo[i] + eo[j] - ev.unsqueeze(1) + ev.unsqueeze(0)
                else:
                    d = eo[i] + eo[j] - ev.unsqueeze(1) - ev.unsqueeze(0)
                if kind == "no_exchange":
                    num = T * (2 * T)
                elif kind == "sign":
                    num = T * (2 * T + T.T)
                else:
                    num = T * (2 * T - T.T)
                e = e + (num / d).sum()
        return e

    return run


@pytest.mark.parametrize("kind", ["no_exchange", "sign", "transposed", "denominator"])
def test_planted_mistakes_fail_the_golden_pin(kind):
    g = load("mp2_small.npz")
    worst = 0.0
    for k in range(1, 5):
        B, eo, ev = (torch.from_numpy(g[n + str(k)]) for n in ("B", "eo", "ev"))
        ref = float(g[f"E_loops{k}"])
        worst = max(worst, abs(float(_mutant(kind)(B, eo, ev)) - ref) / abs(ref))
    assert worst > 1e-6


# ---------------------------------------------------------------------------
# AO -> MO
# ---------------------------------------------------------------------------
def test_ao_to_mo_matches_golden_and_two_step():
    g = load("ao2mo_small.npz")
    for k in range(2):
        eri, Co, Cv = (torch.from_numpy(g[n + str(k)]) for n in ("eri", "Co", "Cv"))
        ref = g[f"B{k}"]
        np.testing.assert_allclose(cpu_ref.ao_to_mo_transform(eri, Co, Cv).numpy(), ref, rtol=0, atol=1e-13)
        np.testing.assert_allclose(cpu_ref.ao_to_mo_two_step(eri, Co, Cv).numpy(), ref, rtol=0, atol=1e-13)
        X = cpu_ref.ao_to_mo_half(eri, Co)
        np.testing.assert_allclose(X.numpy(), np.einsum("mi,mnP->inP", g[f"Co{k}"], g[f"eri{k}"]), atol=1e-13)


# ---------------------------------------------------------------------------
# einsum and the executors
# ---------------------------------------------------------------------------
def test_einsum_matches_golden_numpy():
    g = load("einsum_small.npz")
    k = 0
    while f"sub{k}" in g:
        sub = str(g[f"sub{k}"])
        ops, m = [], 0
        while f"op{k}_{m}" in g:
            ops.append(torch.from_numpy(g[f"op{k}_{m}"]))
            m += 1
        got = cpu_ref.einsum(sub, *ops)
        np.testing.assert_allclose(got.numpy(), g[f"out{k}"], rtol=1e-12, atol=1e-12)
        k += 1
    assert k == 9


def test_alpha_beta_closed_form():
    g = torch.Generator().manual_seed(1)
    A, B, C = (torch.randn(*s, generator=g, dtype=torch.float64) for s in [(4, 3), (3, 5), (4, 5)])
    got = cpu_ref.einsum("ij,jk->ik", A, B, alpha=2.0, beta=0.5, out=C)
    torch.testing.assert_close(got, 2.0 * (A @ B) + 0.5 * C)


def test_dtype_and_precision_semantics():
    A, B = torch.randn(4, 3), torch.randn(3, 5)
    assert cpu_ref.einsum("ij,jk->ik", A, B, dtype="bf16").dtype == torch.bfloat16
    assert cpu_ref.einsum("ij,jk->ik", A, B, precision="kahan").dtype == torch.float32
    with pytest.raises(ValueError, match="unknown dtype"):
        cpu_ref.einsum("ij,jk->ik", A, B, dtype="fp64")
    with pytest.raises(NotImplementedError, match="kahan"):
        cpu_ref.einsum("ij,jk->ik", A, B, precision="dd")


KAHAN_CASES = [
    ("ij,jk->ik", [(40, 300), (300, 30)]),
    ("bij,bjk->bik", [(3, 20, 200), (3, 200, 10)]),
    ("mi,mnP->inP", [(30, 4), (30, 30, 12)]),
    ("ij,jk,kl->il", [(10, 200), (200, 50), (50, 7)]),
    ("i,i->", [(5000,), (5000,)]),
]


@pytest.mark.parametrize("sub,shapes", KAHAN_CASES)
def test_kahan_branch_is_float64_rounded_once(sub, shapes):
    """precision="kahan" (trntensor/einsum.py:108-111): the float64 contraction
    of the float32 operands, cast once. Pinned against numpy's float64 einsum
    cast once to float32: every element within one float32 rounding (the two
    float64 sums differ only in order, which can move a value across a float32
    rounding boundary). Data with large and small magnitudes, so that float32
    accumulation (the planted mistake) misses the bar."""
    g = torch.Generator().manual_seed(len(sub))
    ops = []
    for k, s in enumerate(shapes):
        x = torch.randn(*s, generator=g, dtype=torch.float64)
        if k == 0:
            x = x * torch.where(torch.rand(*s, generator=g) < 0.1, 1e4, 1e-2)
        ops.append(x.float())
    got = cpu_ref.einsum(sub, *ops, precision="kahan")
    assert got.dtype == torch.float32
    want = np.einsum(sub, *[o.double().numpy() for o in ops]).astype(np.float32)
    ulp = np.spacing(np.abs(want)).astype(np.float64)
    diff = np.abs(got.numpy().astype(np.float64) - want.astype(np.float64))
    assert np.all(diff <= ulp), float((diff / np.maximum(ulp, 1e-45)).max())
    fast = cpu_ref.einsum(sub, *ops).numpy().astype(np.float64)
    assert np.any(np.abs(fast - want.astype(np.float64)) > ulp), "data must tell fp32 accumulation apart"


@pytest.mark.parametrize(
    "dt,out_dt,out_shape,want_dt,want_shape",
    [
        (torch.float32, torch.float64, (6, 5), torch.float64, (6, 5)),
        (torch.float64, torch.float32, (6, 5), torch.float64, (6, 5)),
        (torch.float32, torch.float32, (5,), torch.float32, (6, 5)),
        (torch.float64, torch.float64, (3, 6, 5), torch.float64, (3, 6, 5)),
        (torch.float32, torch.float64, (2, 6, 1), torch.float64, (2, 6, 5)),
        (torch.bfloat16, torch.float32, (6, 5), torch.float32, (6, 5)),
        (torch.float32, torch.int64, (6, 5), torch.float32, (6, 5)),
    ],
)
def test_out_promotion_and_broadcast(dt, out_dt, out_shape, want_dt, want_shape):
    """trntensor/einsum.py:99-102: alpha scales the result in its own dtype, then
    result.add(out, alpha=beta) promotes and broadcasts. Pinned by dtype and
    shape tables (numpy's float promotion agrees) and a float64 closed form."""
    g = torch.Generator().manual_seed(5)
    A, B = (torch.randn(*s, generator=g, dtype=torch.float64).to(dt) for s in [(6, 4), (4, 5)])
    out = (torch.randn(*out_shape, generator=g, dtype=torch.float64) * 10).to(out_dt)
    got = cpu_ref.einsum("ij,jk->ik", A, B, alpha=1.5, beta=0.5, out=out)
    assert got.dtype == want_dt and tuple(got.shape) == want_shape
    if dt != torch.bfloat16 and out_dt != torch.int64:
        np_dt = np.result_type(torch.empty(0, dtype=dt).numpy().dtype, torch.empty(0, dtype=out_dt).numpy().dtype)
        assert np_dt == torch.empty(0, dtype=want_dt).numpy().dtype
    want = 1.5 * (A.double() @ B.double()) + 0.5 * out.double()
    bar = 1e-2 if dt == torch.bfloat16 else (1e-6 if torch.float32 in (dt, want_dt) else 1e-13)
    assert (got.double() - want).abs().max() <= bar * want.abs().max()


def test_path_step_naming():
    """trntensor/einsum.py:171-185 on the config-5 expression: 'iajb' then 'abij'."""
    terms = ["ia", "jb", "abP", "ijP"]
    assert cpu_ref.path_step_output(terms, 0, 1, "") == "iajb"
    assert cpu_ref.path_step_output(["abP", "ijP", "iajb"], 0, 1, "") == "abij"


def test_misplanned_detection():
    A, B = torch.randn(3, 4), torch.randn(4, 5)
    assert not cpu_ref.misplanned_by_reference("ij,jk->ik", A, B)
    assert cpu_ref.misplanned_by_reference("ij,jk->ki", A, B)
    assert cpu_ref.misplanned_by_reference("ij,jk->i", A, B)
    assert not cpu_ref.misplanned_by_reference("bij,bjk->bik", torch.randn(2, 3, 4), torch.randn(2, 4, 5))
    assert cpu_ref.misplanned_by_reference("iap,ibp->iab", torch.randn(2, 3, 4), torch.randn(2, 5, 4))
    # the reference's own result differs from einsum semantics here
    res = cpu_ref.einsum("ij,jk->ki", torch.eye(3) * 2, torch.arange(9.0).view(3, 3))
    assert not torch.equal(res, torch.einsum("ij,jk->ki", torch.eye(3) * 2, torch.arange(9.0).view(3, 3)))


def test_pairs_sampler_equals_full_loop():
    """mp2_energy_pairs over every ordered pair is the reference loop itself."""
    g = torch.Generator().manual_seed(8)
    B = torch.randn(3, 6, 7, generator=g, dtype=torch.float64) * 0.1
    eo = torch.sort(-20 + 19.7 * torch.rand(3, generator=g, dtype=torch.float64))[0]
    ev = torch.sort(0.1 + 4.9 * torch.rand(6, generator=g, dtype=torch.float64))[0]
    pairs = [(i, j) for i in range(3) for j in range(3)]
    assert torch.equal(cpu_ref.mp2_energy_pairs(B, eo, ev, pairs), cpu_ref.mp2_energy(B, eo, ev))


def test_multi_einsum_is_a_loop_of_einsum():
    g = torch.Generator().manual_seed(9)
    A, B, C = (torch.randn(*s, generator=g, dtype=torch.float64) for s in [(4, 3), (3, 5), (5, 2)])
    r = cpu_ref.multi_einsum(("ij,jk->ik", A, B), ("ij,jk,kl->il", A, B, C), ("ij,ij->", A, A))
    np.testing.assert_allclose(r[0].numpy(), brute.einsum_f64("ij,jk->ik", A, B), rtol=1e-13)
    np.testing.assert_allclose(r[1].numpy(), brute.einsum_f64("ij,jk,kl->il", A, B, C), rtol=1e-12)
    np.testing.assert_allclose(float(r[2]), float(brute.einsum_f64("ij,ij->", A, A)), rtol=1e-13)


class TestExactEinsum:
    """Pins of oracle/brute.einsum_exact and ill_conditioned_dot (the dd oracle)."""

    def test_matches_float64_on_easy_data(self):
        g = torch.Generator().manual_seed(0)
        A, B = torch.randn(7, 9, generator=g, dtype=torch.float64), torch.randn(9, 5, generator=g, dtype=torch.float64)
        exact, scale, n = brute.einsum_exact("ij,jk->ik", A.numpy(), B.numpy())
        assert n == 9
        np.testing.assert_allclose(exact, (A @ B).numpy(), rtol=1e-14, atol=1e-14)
        np.testing.assert_allclose(scale, (A.abs() @ B.abs()).numpy(), rtol=1e-14)

    def test_closed_forms(self):
        # cancellation float64 cannot see
        r, _, _ = brute.einsum_exact("i->", np.array([1e16, 1.0, -1e16, 1.0]))
        assert float(r) == 2.0
        # one product is the correctly rounded float64 product
        x, y = np.array([0.1]), np.array([0.3])
        r, _, _ = brute.einsum_exact("i,i->", x, y)
        assert float(r) == 0.1 * 0.3
        # trace and outer product
        M = np.arange(9.0).reshape(3, 3)
        assert float(brute.einsum_exact("ii->", M)[0]) == 12.0
        np.testing.assert_array_equal(brute.einsum_exact("i,j->ij", np.array([1.0, 2.0]), np.array([3.0]))[0], [[3.0], [6.0]])

    def test_rounding_is_nearest(self):
        # 1 + 2^-53 + 2^-80: exact sum rounds up to 1 + 2^-52 (above the tie)
        r, _, _ = brute.einsum_exact("i->", np.array([1.0, 2.0**-53, 2.0**-80]))
        assert float(r) == 1.0 + 2.0**-52
        r, _, _ = brute.einsum_exact("i->", np.array([1.0, 2.0**-53]))  # tie: to even
        assert float(r) == 1.0

    def test_ill_conditioned_generator(self):
        from fractions import Fraction

        rng = np.random.default_rng(5)
        for logc in (12, 20, 28):
            x, y = brute.ill_conditioned_dot(200, logc, rng)
            exact = sum((Fraction(float(a)) * Fraction(float(b)) for a, b in zip(x, y)), Fraction(0))
            cond = 2 * float(np.sum(np.abs(x * y))) / abs(float(exact))
            assert 10 ** (logc - 3) <= cond <= 10 ** (logc + 4), (logc, cond)


def test_integer_einsum_wraps_like_int64_truncated():
    """The integer path computes in int64 (wrapping) and truncates to the
    operands' dtype. Pinned: the oracle's (torch's) int8 and int32 einsums
    equal the int64 contraction reduced modulo 2^8 / 2^32, including sums
    that overflow the narrow type."""
    g = torch.Generator().manual_seed(4)
    for dt, bits in ((torch.int8, 8), (torch.int32, 32)):
        lo, hi = (-128, 128) if bits == 8 else (-(1 << 31), 1 << 31)
        A = torch.randint(lo, hi, (20, 300), generator=g, dtype=torch.int64)
        B = torch.randint(lo, hi, (300, 10), generator=g, dtype=torch.int64)
        wide = np.einsum("ij,jk->ik", A.numpy().astype(object), B.numpy().astype(object))
        want = np.vectorize(lambda v: ((v + (1 << (bits - 1))) % (1 << bits)) - (1 << (bits - 1)))(wide).astype(np.int64)
        got = cpu_ref.einsum("ij,jk->ik", A.to(dt), B.to(dt))
        assert got.dtype == dt
        assert np.array_equal(got.to(torch.int64).numpy(), want)
        assert np.abs(wide).max() >= (1 << (bits - 1)), "the data must overflow the narrow type"


@pytest.mark.parametrize("sub,shapes", [("ij,jk->ik", [(7, 9), (9, 5)]), ("bij,bjk->bik", [(2, 4, 6), (2, 6, 3)]),
                                        ("ij,jk,kl->il", [(3, 4), (4, 5), (5, 2)]), ("ii->", [(6, 6)]),
                                        ("mi,mnP->inP", [(5, 2), (5, 5, 3)])])
def test_complex_einsum_matches_numpy(sub, shapes):
    """The oracle's complex contractions (torch on the CPU) against numpy's
    complex128 einsum, an independent implementation, plus a complex alpha
    and beta with a real out (promotion to complex)."""
    g = np.random.default_rng(len(sub))
    ops = [g.standard_normal(s) + 1j * g.standard_normal(s) for s in shapes]
    got = cpu_ref.einsum(sub, *[torch.from_numpy(o) for o in ops])
    want = np.einsum(sub, *ops)
    assert got.dtype == torch.complex128
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-12, atol=1e-12)
    out = g.standard_normal(np.shape(want))
    got = cpu_ref.einsum(sub, *[torch.from_numpy(o) for o in ops], alpha=1 - 2j, beta=0.5j, out=torch.from_numpy(out))
    np.testing.assert_allclose(got.numpy(), (1 - 2j) * want + 0.5j * out, rtol=1e-12, atol=1e-12)
