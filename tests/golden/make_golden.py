"""Write the golden fixtures in this directory.

Run from the repository root:  python tests/golden/make_golden.py

The reference stores no golden vectors (its tests compare against torch
computed inside each test). These fixtures hold small seeded inputs and
float64 expected values from formulas independent of the oracle:
- mp2_small.npz: MP2 energies by explicit Python loops over (i, j, a, b, P)
  (oracle.brute.mp2_energy_loops) and by the explicit 4-index array;
- ao2mo_small.npz: AO->MO by per-P textbook matrix products
  (oracle.brute.ao_to_mo_loops);
- einsum_small.npz: contractions by numpy.einsum in float64.
The tutorial's known answer (docs/tutorial_df_mp2.md:75-77) is a literal in
the tests, not a fixture.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import brute  # noqa: E402

MP2_SHAPES = [(1, 1, 1), (2, 3, 5), (2, 4, 3), (3, 2, 4), (3, 5, 1)]
EINSUM_CASES = [
    ("ij,jk->ik", [(4, 3), (3, 5)]),
    ("ji,kj->ik", [(3, 4), (5, 3)]),
    ("bij,bjk->bik", [(3, 4, 3), (3, 3, 5)]),
    ("mi,mnP->inP", [(6, 2), (6, 6, 8)]),
    ("ijk,jkl->il", [(3, 4, 5), (4, 5, 6)]),
    ("ii->", [(5, 5)]),
    ("i,j->ij", [(3,), (4,)]),
    ("ij,jk,kl->il", [(5, 8), (8, 6), (6, 4)]),
    ("ia,jb,abP,ijP->", [(3, 4), (2, 5), (4, 5, 6), (3, 2, 6)]),
]


def main() -> None:
    rng = np.random.default_rng(20260501)
    mp2 = {}
    for k, (no, nv, na) in enumerate(MP2_SHAPES):
        B = rng.standard_normal((no, nv, na)) * 0.1
        eo = np.sort(rng.uniform(-20.0, -0.3, no))
        ev = np.sort(rng.uniform(0.1, 5.0, nv))
        mp2[f"B{k}"] = B
        mp2[f"eo{k}"] = eo
        mp2[f"ev{k}"] = ev
        mp2[f"E_loops{k}"] = np.array(brute.mp2_energy_loops(B, eo, ev))
        mp2[f"E_4index{k}"] = np.array(brute.mp2_energy_4index(B, eo, ev))
    np.savez(os.path.join(HERE, "mp2_small.npz"), **mp2)

    ao = {}
    for k, (nb, no, nv, na) in enumerate([(4, 2, 3, 5), (6, 3, 2, 4)]):
        eri = rng.standard_normal((nb, nb, na)) * 0.1
        Co = rng.standard_normal((nb, no))
        Cv = rng.standard_normal((nb, nv))
        ao[f"eri{k}"] = eri
        ao[f"Co{k}"] = Co
        ao[f"Cv{k}"] = Cv
        ao[f"B{k}"] = brute.ao_to_mo_loops(eri, Co, Cv)
    np.savez(os.path.join(HERE, "ao2mo_small.npz"), **ao)

    es = {}
    for k, (sub, shapes) in enumerate(EINSUM_CASES):
        ops = [rng.standard_normal(s) for s in shapes]
        es[f"sub{k}"] = np.array(sub)
        for m, o in enumerate(ops):
            es[f"op{k}_{m}"] = o
        es[f"out{k}"] = np.asarray(brute.einsum_f64(sub, *ops))
    np.savez(os.path.join(HERE, "einsum_small.npz"), **es)


if __name__ == "__main__":
    main()
