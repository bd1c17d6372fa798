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
