"""HIP dispatch for the fused-contraction path: backend control, device
placement, and the entry points that replace the reference's NKI dispatchers.

Reference counterpart: trntensor/nki/dispatch.py. Differences by design:

- Every contraction strategy executes on the HIP kernels; there is no FLOP
  threshold (a HIP launch costs microseconds, not the NKI path's ~0.67 ms)
  and no zero-padding (the kernels mask edge tiles).
- There is no silent fallback to torch. A kernel error raises (ValueError /
  NotImplementedError / RuntimeError by status code), which is what the
  reference does under TRNTENSOR_REQUIRE_NKI=1; that variable and
  TRNTENSOR_REQUIRE_HIP are accepted and change nothing. With no usable HIP
  device, or with the "pytorch" backend selected, contraction calls raise
  RuntimeError instead of computing on the host.
- Residency: CPU operands are copied to the current HIP device, the kernels
  run there, and the result is copied back to the first operand's device
  (reference _to_xla / .to(orig), dispatch.py:127-149, 232). Operands already
  on the device keep the result on the device.
"""

from __future__ import annotations

import os

import torch

from . import _lib, engine

# ---------------------------------------------------------------------------
# availability and backend selection (reference dispatch.py:28-120)
# ---------------------------------------------------------------------------
_ARCH = "gfx950"


def _probe() -> tuple[bool, str]:
    if _lib.load() is None:
        return False, _lib.load_error() or "library not loaded"
    try:
        if not torch.cuda.is_available():
            return False, "no HIP device visible to torch"
        arch = torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName
    except Exception as exc:  # noqa: BLE001 - any runtime failure means unavailable
        return False, f"HIP runtime error: {exc}"
    if not arch.startswith(_ARCH):
        return False, f"device arch {arch} is not {_ARCH}"
    return True, ""


HAS_HIP, _UNAVAILABLE_REASON = _probe()
# Name kept for drop-in compatibility with code that tests trntensor.HAS_NKI.
HAS_NKI = False

_TRUTHY = ("1", "true", "yes")
# Accepted for compatibility; errors always propagate in this build.
_REQUIRE_HIP = os.environ.get("TRNTENSOR_REQUIRE_HIP", os.environ.get("TRNTENSOR_REQUIRE_NKI", "")).lower() in _TRUTHY

_BACKENDS = ("auto", "pytorch", "hip", "nki")
_backend = "auto"


def set_backend(backend: str) -> None:
    """Select "auto" (HIP when available), "hip" ("nki" is an alias), or "pytorch".

    Unknown names raise AssertionError (the reference asserts, dispatch.py:96;
    this check also survives ``python -O``). Selecting "hip" without a usable
    gfx950 device raises RuntimeError and leaves the backend unchanged.
    """
    global _backend
    if backend not in _BACKENDS:
        raise AssertionError(f"backend must be one of {_BACKENDS}, got {backend!r}")
    if backend in ("hip", "nki") and not HAS_HIP:
        raise RuntimeError(f"HIP backend requires libtrntensor_hip and a {_ARCH} device: {_UNAVAILABLE_REASON}")
    _backend = "hip" if backend == "nki" else backend


def get_backend() -> str:
    return _backend


# TRNTENSOR_FORCE_BACKEND is read on every call, as the reference does. On
# CPython, os.environ keeps its encoded entries in a dict (`_data`), which
# the lookup below reads directly: the same value os.environ.get returns, at
# a tenth of the cost (0.08 against 0.65 us), which counts on the per-call
# path of small contractions.
_FORCE_VAR = "TRNTENSOR_FORCE_BACKEND"
_ENV_DATA = getattr(os.environ, "_data", None)
try:
    _FORCE_KEY = os.environ.encodekey(_FORCE_VAR)  # type: ignore[attr-defined]
    _decode = os.environ.decodevalue  # type: ignore[attr-defined]
except AttributeError:
    _ENV_DATA = None


def _forced_backend() -> str:
    if isinstance(_ENV_DATA, dict):
        v = _ENV_DATA.get(_FORCE_KEY)
        return "" if v is None else _decode(v).lower()
    return os.environ.get(_FORCE_VAR, "").lower()


def _use_hip() -> bool:
    """TRNTENSOR_FORCE_BACKEND > set_backend > availability (reference dispatch.py:108-120)."""
    forced = _forced_backend()
    if forced in ("hip", "nki"):
        return True
    if forced == "pytorch":
        return False
    if _backend == "hip":
        return True
    if _backend == "pytorch":
        return False
    return HAS_HIP


def require_hip() -> None:
    """Raise unless contractions will run on the HIP kernels."""
    if HAS_HIP and not _use_hip():
        raise RuntimeError(
            "trntensor_amd computes contractions only on its HIP kernels and the 'pytorch' "
            "backend is selected; call torch.einsum directly for a host computation"
        )
    if not HAS_HIP:
        raise RuntimeError(f"trntensor_amd HIP runtime unavailable: {_UNAVAILABLE_REASON}")


# ---------------------------------------------------------------------------
# residency (reference dispatch.py:127-184)
# ---------------------------------------------------------------------------
def _device() -> torch.device:
    return torch.device("cuda", torch.cuda.current_device())


def to_device(tensor: torch.Tensor) -> torch.Tensor:
    """Move a tensor to the HIP device (no-op if already there).

    Raises RuntimeError when no HIP runtime is available (reference
    ``to_xla``, dispatch.py:152-177).
    """
    if tensor.device.type == "cuda":
        return tensor
    if not HAS_HIP:
        raise RuntimeError(f"to_device requires the HIP runtime on a {_ARCH} device: {_UNAVAILABLE_REASON}")
    return tensor.to(_device())


def from_device(tensor: torch.Tensor) -> torch.Tensor:
    """Move a tensor back to the CPU; no-op for CPU tensors."""
    if tensor.device.type == "cpu":
        return tensor
    return tensor.to("cpu")


# Drop-in names of the reference's residency helpers.
to_xla = to_device
from_xla = from_device


def place(*tensors: torch.Tensor) -> tuple[list[torch.Tensor], torch.device]:
    """Operands on one HIP device, plus the device the result goes back to."""
    orig = tensors[0].device if tensors else _device()
    cuda = [t.device for t in tensors if t.device.type == "cuda"]
    dev = cuda[0] if cuda else _device()
    if any(d != dev for d in cuda):
        raise RuntimeError(f"operands on different devices: {sorted({str(d) for d in cuda})}")
    # When the result goes back to the host, the caller's blocking copy of the
    # result orders after these uploads on the same stream, so they need not
    # block on their own (pageable sources are staged by the runtime before
    # the call returns). A device-resident result keeps blocking uploads.
    nb = orig.type == "cpu"
    return [t if t.device == dev else t.to(dev, non_blocking=nb) for t in tensors], orig


_WIDEN = {torch.bfloat16: torch.float32, torch.float16: torch.float32}
_INTS = (torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8)


def compute_dtype(dt: torch.dtype) -> torch.dtype:
    """Kernel dtype for an operand dtype: fp32/fp64 and complex64/complex128 as
    is (complex contractions run as real ones on their parts), bf16/fp16
    widened to fp32 (exact; products of 8/11-bit mantissas are exact in fp32
    accumulation), integers widened to int64 (sums wrap modulo 2^64, so
    truncating back gives each type's own wrapping result)."""
    if dt in (torch.float32, torch.float64, torch.complex64, torch.complex128):
        return dt
    if dt in _WIDEN:
        return _WIDEN[dt]
    if dt in _INTS:
        return torch.int64
    raise NotImplementedError(f"trntensor_amd HIP kernels do not compute in {dt}")


# ---------------------------------------------------------------------------
# entry points replacing the reference's NKI dispatchers
# ---------------------------------------------------------------------------
def _mp2_workspace(lib, code: int, nocc: int, nvir: int, naux: int, device: torch.device,
                   _alloc=None) -> tuple[torch.Tensor, int]:
    """Workspace for tt_mp2_energy: (tensor, bytes).

    When naux is not a multiple of 16 the full query includes a row-padded
    copy of B (as many bytes as B itself, rounded up), which makes the call
    5-7% faster with the same energy bitwise. If the device cannot hold that
    copy, the call runs on B as given with a workspace of the partials only
    (the query for naux rounded up to 16). `_alloc` replaces torch.empty in
    tests.
    """
    alloc = _alloc or (lambda n: torch.empty(n, dtype=torch.uint8, device=device))
    full = int(lib.tt_mp2_energy_workspace_bytes(code, nocc, nvir, naux))
    part = int(lib.tt_mp2_energy_workspace_bytes(code, nocc, nvir, (naux + 15) // 16 * 16))
    if full > part:
        try:
            return alloc(full), full
        except torch.OutOfMemoryError:
            pass
    return alloc(max(part, 1)), part


def _hip_mp2_energy(B: torch.Tensor, eps_occ: torch.Tensor, eps_vir: torch.Tensor, deterministic: bool = True) -> torch.Tensor:
    """Fused DF-MP2 energy on tt_mp2_energy (reference _nki_mp2_energy, dispatch.py:240-283).

    Returns a 0-D tensor on B's device in the dtype the reference's loop
    returns: torch's promotion of B's and the orbital energies' dtypes
    (trntensor/quantum.py:94-99). Mixed dtypes are computed in that promoted
    dtype; the reference forms T in B's dtype and the denominators in the
    orbital energies' dtype, so its result carries the lower precision's
    rounding (the tests bound the difference at the float32 bar).
    """
    require_hip()
    lib = _lib.load()
    (b, eo, ev), orig = place(B, eps_occ, eps_vir)
    res_dtype = torch.promote_types(torch.promote_types(b.dtype, eo.dtype), ev.dtype)
    cd = compute_dtype(res_dtype)
    b = b.to(cd).contiguous()
    eo = eo.to(cd).contiguous()
    ev = ev.to(cd).contiguous()
    nocc, nvir, naux = b.shape
    code = engine.dtype_code(cd)
    ws, wsb = _mp2_workspace(lib, code, nocc, nvir, naux, b.device)
    e = torch.empty((), dtype=cd, device=b.device)
    st = lib.tt_mp2_energy(
        code,
        nocc,
        nvir,
        naux,
        engine._ptr(b),
        engine._ptr(eo),
        engine._ptr(ev),
        engine._ptr(e),
        engine._ptr(ws),
        wsb,
        int(bool(deterministic)),
        engine._stream_ptr(b.device),
    )
    _lib.check(st, "tt_mp2_energy")
    return e.to(res_dtype).to(orig)


def _hip_mp2_energy_shard(B: torch.Tensor, eps_occ: torch.Tensor, eps_vir: torch.Tensor, rank: int, world_size: int,
                          deterministic: bool = True) -> torch.Tensor:
    """Contribution of shard `rank` of `world_size` (a contiguous, balanced
    range of work units, tt_mp2_energy_shard) to the MP2 energy; the shards'
    values sum to the whole energy. 0-D tensor in the promoted dtype on B's
    device."""
    require_hip()
    if not 0 <= rank < world_size:
        raise ValueError(f"rank {rank} outside world_size {world_size}")
    lib = _lib.load()
    (b, eo, ev), orig = place(B, eps_occ, eps_vir)
    res_dtype = torch.promote_types(torch.promote_types(b.dtype, eo.dtype), ev.dtype)
    cd = compute_dtype(res_dtype)
    b, eo, ev = (x.to(cd).contiguous() for x in (b, eo, ev))
    nocc, nvir, naux = b.shape
    total = lib.tt_mp2_energy_unit_count(nocc, nvir)
    first = total * rank // world_size
    count = total * (rank + 1) // world_size - first
    code = engine.dtype_code(cd)
    # The partials only (the size for naux rounded up to a multiple of 16):
    # a shard makes no row-padded copy of B, which would cost each shard's
    # call as much as it saves on that shard's share of the work.
    wsb = lib.tt_mp2_energy_workspace_bytes(code, nocc, nvir, (naux + 15) // 16 * 16)
    ws = torch.empty(max(int(wsb), 1), dtype=torch.uint8, device=b.device)
    e = torch.empty((), dtype=cd, device=b.device)
    st = lib.tt_mp2_energy_shard(
        code, nocc, nvir, naux, engine._ptr(b), engine._ptr(eo), engine._ptr(ev), first, count,
        engine._ptr(e), engine._ptr(ws), wsb, int(bool(deterministic)), engine._stream_ptr(b.device),
    )
    _lib.check(st, "tt_mp2_energy_shard")
    return e.to(res_dtype).to(orig)


def _hip_ao_to_mo_transform(eri: torch.Tensor, C_occ: torch.Tensor, C_vir: torch.Tensor) -> torch.Tensor:
    """Full AO->MO transform on tt_ao_to_mo_transform (reference
    _nki_ao_to_mo_transform, dispatch.py:286-336). Result on eri's device."""
    require_hip()
    lib = _lib.load()
    (e, co, cv), orig = place(eri, C_occ, C_vir)
    if not (e.dtype == co.dtype == cv.dtype):
        raise RuntimeError(f"expected one dtype, got {e.dtype}, {co.dtype}, {cv.dtype}")
    cd = compute_dtype(e.dtype)
    e = e.to(cd).contiguous()
    co = co.to(cd).contiguous()
    cv = cv.to(cd).contiguous()
    nbasis, _, naux = e.shape
    nocc, nvir = co.shape[1], cv.shape[1]
    code = engine.dtype_code(cd)
    wsb = lib.tt_ao_to_mo_workspace_bytes(code, nbasis, nocc, nvir, naux)
    ws = torch.empty(max(int(wsb), 1), dtype=torch.uint8, device=e.device)
    out = torch.empty((nocc, nvir, naux), dtype=cd, device=e.device)
    st = lib.tt_ao_to_mo_transform(
        code,
        nbasis,
        nocc,
        nvir,
        naux,
        engine._ptr(e),
        engine._ptr(co),
        engine._ptr(cv),
        engine._ptr(out),
        engine._ptr(ws),
        wsb,
        engine._stream_ptr(e.device),
    )
    _lib.check(st, "tt_ao_to_mo_transform")
    return out.to(eri.dtype).to(orig)
