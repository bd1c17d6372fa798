"""ctypes binding of libtrntensor_hip.so (the C ABI in include/trntensor_hip.h).

The library is built in-tree by ``trntensor_amd/csrc/build.py`` into
``trntensor_amd/_lib/``. torch is imported first so that the library binds to
the HIP runtime torch already loaded (one runtime, shared streams).
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads torch's HIP runtime before the library)

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_lib", "libtrntensor_hip.so")

TT_OK, TT_INVALID, TT_UNSUPPORTED, TT_HIP_ERROR = 0, 1, 2, 3
TT_F32, TT_F64, TT_F64_DD, TT_BF16, TT_F16, TT_I64 = 0, 1, 2, 3, 4, 5
TT_MAX_DIMS = 8
ABI_VERSION = 4

# Every symbol include/trntensor_hip.h declares, with its ctypes signature.
_i64 = ctypes.c_int64
_int = ctypes.c_int
_dbl = ctypes.c_double
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_i64p = ctypes.POINTER(ctypes.c_int64)

SIGNATURES = {
    "tt_abi_version": (_int, []),
    "tt_status_string": (ctypes.c_char_p, [_int]),
    "tt_last_error": (ctypes.c_char_p, []),
    "tt_gemm": (
        _int,
        [_int, _int, _int, _i64, _i64, _i64, _dbl, _vp, _i64, _i64, _vp, _i64, _i64, _dbl, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _vp],
    ),
    "tt_gemm_packed": (_int, [_vp, _dbl, _dbl, _vp, _vp, _vp, _vp, _vp]),
    "tt_gemm_dot_workspace_bytes": (_sz, [_int, _i64, _i64, _i64]),
    "tt_gemm_dot": (
        _int,
        [_int, _int, _int, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _i64p, _vp, _i64p,
         _dbl, _dbl, _vp, _vp, _vp, _sz, _vp],
    ),
    "tt_mp2_energy_workspace_bytes": (_sz, [_int, _i64, _i64, _i64]),
    "tt_mp2_energy": (_int, [_int, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _sz, _int, _vp]),
    "tt_mp2_energy_noalloc": (_int, [_int, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _int, _vp]),
    "tt_mp2_energy_unit_count": (_i64, [_i64, _i64]),
    "tt_mp2_energy_shard": (_int, [_int, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _sz, _int, _vp]),
    "tt_ao_to_mo_workspace_bytes": (_sz, [_int, _i64, _i64, _i64, _i64]),
    "tt_ao_to_mo_transform": (_int, [_int, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "tt_mfma_rate_probe": (_int, [_int, _i64, _i64, _vp, _vp]),
    "tt_hbm_probe": (_int, [_int, _vp, _vp, _i64, _i64, _vp, _vp]),
    "tt_strided_contract_workspace_bytes": (_sz, [_int, _int, _i64p, _int, _i64p]),
    "tt_strided_contract": (
        _int,
        [_int, _int, _i64p, _i64p, _i64p, _int, _i64p, _i64p, _i64p, _vp, _vp, _dbl, _dbl, _vp, _vp, _vp, _sz, _vp],
    ),
}

_lib = None
_load_error: str | None = None


def load():
    """Load (once) and return the library handle, or None with the reason kept."""
    global _lib, _load_error
    if _lib is not None or _load_error is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        _load_error = f"{LIB_PATH} is not built (run trntensor_amd/csrc/build.py)"
        return None
    try:
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.tt_abi_version() != ABI_VERSION:
            raise OSError(f"ABI version {lib.tt_abi_version()} != {ABI_VERSION}")
    except (OSError, AttributeError) as exc:  # AttributeError: a symbol the header declares is missing
        _load_error = f"cannot load {LIB_PATH}: {exc}"
        return None
    _lib = lib
    return _lib


def load_error() -> str | None:
    load()
    return _load_error


def check(status: int, what: str) -> None:
    """Map a library status code to the reference's exception classes."""
    if status == TT_OK:
        return
    detail = _lib.tt_last_error().decode(errors="replace") if _lib is not None else ""
    msg = f"{what}: {detail or _lib.tt_status_string(status).decode()}"
    if status == TT_INVALID:
        raise ValueError(msg)
    if status == TT_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def i64_array(values) -> ctypes.Array:
    vals = list(values) or [0]
    return (ctypes.c_int64 * len(vals))(*vals)
