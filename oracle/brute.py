"""Independent pins for the CPU oracle: numpy float64 formulas that share no
code with ``oracle/cpu_ref.py``.

TEST INFRASTRUCTURE ONLY (imported by ``tests/`` and nothing else).

They check the oracle against what the mathematics fixes: the explicit
four-index MP2 sum, closed forms and invariances, and textbook linear algebra.
"""

from __future__ import annotations

import numpy as np


def mp2_energy_4index(B, eps_occ, eps_vir):
    """E = sum_ijab T_ijab (2 T_ijab - T_ijba) / (e_i + e_j - e_a - e_b) with
    T_ijab = sum_P B_iaP B_jbP, built as an explicit 4-index array in float64
    (the formula of trntensor/quantum.py:28-35 and tests/test_quantum.py:21-33)."""
    B = np.asarray(B, dtype=np.float64)
    eo = np.asarray(eps_occ, dtype=np.float64)
    ev = np.asarray(eps_vir, dtype=np.float64)
    T = np.einsum("iap,jbp->ijab", B, B, optimize=False)
    D = eo[:, None, None, None] + eo[None, :, None, None] - ev[None, None, :, None] - ev[None, None, None, :]
    return float(np.sum(T * (2.0 * T - T.transpose(0, 1, 3, 2)) / D))


def mp2_energy_loops(B, eps_occ, eps_vir):
    """The same sum by plain Python loops over (i, j, a, b, P): for tiny inputs
    only; shares nothing with either einsum formulation."""
    B = np.asarray(B, dtype=np.float64)
    nocc, nvir, naux = B.shape
    e = 0.0
    for i in range(nocc):
        for j in range(nocc):
            for a in range(nvir):
                for b in range(nvir):
                    tab = sum(B[i, a, p] * B[j, b, p] for p in range(naux))
                    tba = sum(B[i, b, p] * B[j, a, p] for p in range(naux))
                    d = eps_occ[i] + eps_occ[j] - eps_vir[a] - eps_vir[b]
                    e += tab * (2.0 * tab - tba) / d
    return e


def mp2_energy_rank1(x, y, eps_occ, eps_vir):
    """Closed form for naux = 1 with B_ia = x_i y_a:
    T_ijab = x_i x_j y_a y_b is symmetric in (a, b), so
    E = sum_ijab (x_i x_j y_a y_b)^2 / (e_i + e_j - e_a - e_b)."""
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    eo = np.asarray(eps_occ, dtype=np.float64)
    ev = np.asarray(eps_vir, dtype=np.float64)
    num = (x[:, None] * x[None, :]) ** 2
    num = num[:, :, None, None] * ((y[:, None] * y[None, :]) ** 2)[None, None]
    den = eo[:, None, None, None] + eo[None, :, None, None] - ev[None, None, :, None] - ev[None, None, None, :]
    return float(np.sum(num / den))


def ao_to_mo_loops(eri, C_occ, C_vir):
    """B[i,a,P] = sum_{mu,nu} C_occ[mu,i] C_vir[nu,a] eri[mu,nu,P] as two
    matrix products per P (textbook C_occ^T eri[:,:,P] C_vir) in float64."""
    eri = np.asarray(eri, dtype=np.float64)
    Co = np.asarray(C_occ, dtype=np.float64)
    Cv = np.asarray(C_vir, dtype=np.float64)
    out = np.empty((Co.shape[1], Cv.shape[1], eri.shape[2]))
    for P in range(eri.shape[2]):
        out[:, :, P] = Co.T @ eri[:, :, P] @ Cv
    return out


def einsum_f64(subscripts, *ops):
    """numpy's einsum in float64 (an independent implementation of the
    contraction semantics the reference hands to torch.einsum)."""
    return np.einsum(subscripts, *[np.asarray(o, dtype=np.float64) for o in ops], optimize=False)


def einsum_exact(subscripts, *ops):
    """Exact einsum of float inputs: every product and sum in rational
    arithmetic (fractions.Fraction holds each float exactly), each output
    rounded to the nearest float64 once (int / int true division rounds
    correctly). Also returns, per output, sum |term| as a float64 array: the
    scale that bounds a double-double (Dot2) result's error,
    |res - exact| <= u |exact| + gamma_n^2 sum|term| (Ogita-Rump-Oishi 2005,
    Prop. 5.5, u = 2^-53, gamma_n = n u / (1 - n u)). For small inputs only:
    pure Python loops over every index combination.

    Returns (rounded float64 array, sum |term| float64 array, n terms per output).
    """
    from fractions import Fraction
    from itertools import product

    lhs, out = subscripts.split("->")
    terms = lhs.split(",")
    ext = {}
    vals = []
    for t, x in zip(terms, ops):
        a = np.asarray(x, dtype=np.float64)
        for c, n in zip(t, a.shape):
            ext[c] = n
        vals.append(a)
    red = sorted({c for t in terms for c in t} - set(out))
    res = np.zeros([ext[c] for c in out], dtype=np.float64)
    scale = np.zeros_like(res)
    nterms = 1
    for c in red:
        nterms *= ext[c]
    for oidx in product(*[range(ext[c]) for c in out]):
        env = dict(zip(out, oidx))
        acc = Fraction(0)
        mag = Fraction(0)
        for ridx in product(*[range(ext[c]) for c in red]):
            env.update(zip(red, ridx))
            term = Fraction(1)
            for t, a in zip(terms, vals):
                term *= Fraction(float(a[tuple(env[c] for c in t)]))
            acc += term
            mag += abs(term)
        res[oidx] = acc.numerator / acc.denominator
        scale[oidx] = mag.numerator / mag.denominator
    return res, scale, nterms


def ill_conditioned_dot(n, log10_cond, rng):
    """Vectors x, y whose dot product has condition number about
    10**log10_cond (2 sum|x_i y_i| / |x.y|), after Ogita-Rump-Oishi 2005,
    Algorithm 6.1 (GenDot): the first half carries exponents spread over
    0..b = log2 cond / 2, the second half is chosen so that the running exact
    dot product cancels towards exponents that fall linearly to 0. Returns
    float64 numpy arrays."""
    from fractions import Fraction

    b = log10_cond * np.log2(10.0) / 2.0
    n2 = n // 2
    x = np.zeros(n)
    y = np.zeros(n)
    e = np.rint(rng.uniform(0, b, n2)).astype(int)
    e[0] = int(round(b)) + 1
    e[-1] = 0
    x[:n2] = (2 * rng.uniform(size=n2) - 1) * np.exp2(e)
    y[:n2] = (2 * rng.uniform(size=n2) - 1) * np.exp2(e)
    exact = sum((Fraction(float(x[i])) * Fraction(float(y[i])) for i in range(n2)), Fraction(0))
    e2 = np.rint(np.linspace(b, 0, n - n2)).astype(int)
    for k, i in enumerate(range(n2, n)):
        x[i] = (2 * rng.uniform() - 1) * 2.0 ** e2[k]
        y[i] = float(((2 * rng.uniform() - 1) * 2.0 ** e2[k] - float(exact)) / x[i])
        exact += Fraction(float(x[i])) * Fraction(float(y[i]))
    perm = rng.permutation(n)
    return x[perm], y[perm]
