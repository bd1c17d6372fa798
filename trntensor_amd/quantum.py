"""Quantum-chemistry primitives on fused HIP kernels: DF-MP2 energy and the
AO->MO integral transform.

Mirrors trntensor/quantum.py (reference): same signatures, same validation
messages, same return shapes and dtypes. Both routes go straight to the HIP
library; the reference's NKI size limits (nvir, naux <= 128 for MP2;
nbasis <= 512, nocc <= 128, nvir <= 512 for AO->MO) do not apply.
"""

from __future__ import annotations

import torch

from .hip import dispatch


def mp2_energy(B: torch.Tensor, eps_occ: torch.Tensor, eps_vir: torch.Tensor) -> torch.Tensor:
    """Density-fitted MP2 correlation energy.

        E_MP2 = sum_{ijab} T_ijab (2 T_ijab - T_ijba) / (e_i + e_j - e_a - e_b),
        T_ijab = sum_P B[i,a,P] B[j,b,P]

    One fused kernel (tt_mp2_energy): T is formed block by block on MFMA and
    never written to memory; the denominator and exchange term are applied in
    registers and each workgroup contributes one partial sum.

    Parameters: B (nocc, nvir, naux); eps_occ (nocc,); eps_vir (nvir,).
    Returns a 0-D tensor on B's device whose dtype is torch's promotion of
    the three inputs' dtypes, as the reference loop's result
    (trntensor/quantum.py:21-84, 94-99); with one dtype throughout that is
    B's dtype.

    Device memory: when naux is not a multiple of 16 the call also takes a
    row-padded copy of B (as large as B) for its duration, which makes it
    5-7% faster; if the device cannot hold the copy, the call runs on B as
    given with only the per-work-unit partials as workspace.
    """
    if B.dim() != 3:
        raise ValueError(f"B must be 3D (nocc, nvir, naux); got shape {tuple(B.shape)}")
    nocc, nvir, _naux = B.shape
    if eps_occ.shape != (nocc,):
        raise ValueError(f"eps_occ must have shape ({nocc},); got {tuple(eps_occ.shape)}")
    if eps_vir.shape != (nvir,):
        raise ValueError(f"eps_vir must have shape ({nvir},); got {tuple(eps_vir.shape)}")
    return dispatch._hip_mp2_energy(B, eps_occ, eps_vir)


def mp2_energy_shard(B: torch.Tensor, eps_occ: torch.Tensor, eps_vir: torch.Tensor, rank: int,
                     world_size: int) -> torch.Tensor:
    """One GPU's share of :func:`mp2_energy` for a run sharded over
    ``world_size`` GPUs (no counterpart in the reference).

    The energy is a sum over independent work units (occupied pair i <= j,
    pair of 64-row virtual blocks); shard ``rank`` takes a contiguous,
    balanced range of them. With B and the orbital energies on every GPU,
    ``torch.distributed.all_reduce`` of the shards' values (one scalar)
    gives the energy::

        e = trntensor.mp2_energy_shard(B, eo, ev, rank, world_size)
        torch.distributed.all_reduce(e)        # e == mp2_energy(B, eo, ev)

    Same validation and dtype as :func:`mp2_energy`.
    """
    if B.dim() != 3:
        raise ValueError(f"B must be 3D (nocc, nvir, naux); got shape {tuple(B.shape)}")
    nocc, nvir, _naux = B.shape
    if eps_occ.shape != (nocc,):
        raise ValueError(f"eps_occ must have shape ({nocc},); got {tuple(eps_occ.shape)}")
    if eps_vir.shape != (nvir,):
        raise ValueError(f"eps_vir must have shape ({nvir},); got {tuple(eps_vir.shape)}")
    return dispatch._hip_mp2_energy_shard(B, eps_occ, eps_vir, rank, world_size)


def ao_to_mo_transform(eri: torch.Tensor, C_occ: torch.Tensor, C_vir: torch.Tensor) -> torch.Tensor:
    """Four-index AO->MO transform of density-fitted integrals.

        B[i, a, P] = sum_{mu, nu} C_occ[mu, i] C_vir[nu, a] eri[mu, nu, P]

    Two MFMA GEMMs with P-contiguous loads (tt_ao_to_mo_transform). Composes
    with :func:`mp2_energy`; B stays on the device when eri is there.

    Parameters: eri (nbasis, nbasis, naux); C_occ (nbasis, nocc);
    C_vir (nbasis, nvir). Returns (nocc, nvir, naux)
    (reference trntensor/quantum.py:103-185).
    """
    if eri.dim() != 3:
        raise ValueError(f"eri must be 3D (nbasis, nbasis, naux); got shape {tuple(eri.shape)}")
    nbasis_mu, nbasis_nu, _naux = eri.shape
    if nbasis_mu != nbasis_nu:
        raise ValueError(f"eri first two dims must match (nbasis, nbasis); got ({nbasis_mu}, {nbasis_nu})")
    nbasis = nbasis_mu
    if C_occ.dim() != 2 or C_occ.shape[0] != nbasis:
        raise ValueError(f"C_occ must have shape ({nbasis}, nocc); got {tuple(C_occ.shape)}")
    if C_vir.dim() != 2 or C_vir.shape[0] != nbasis:
        raise ValueError(f"C_vir must have shape ({nbasis}, nvir); got {tuple(C_vir.shape)}")
    return dispatch._hip_ao_to_mo_transform(eri, C_occ, C_vir)
