"""Loader of the host launch table (``csrc/tt_fastpath.cpp``).

The table keeps, per (subscripts, operand sizes, strides, dtype, device), the
tt_gemm_packed parameter block of a two-operand contraction that runs as one
GEMM launch, so a repeat einsum call costs one lookup, one allocation and one
library call in C++. It calls the entry point of the already loaded
libtrntensor_hip.so by address. When the table is not built (or cannot be
loaded), einsum keeps its launchers in a Python dict instead: the same
launches through ctypes, a few microseconds more per call.
"""

from __future__ import annotations

import ctypes
import importlib.util
import os

from . import _lib

PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_lib", "fastpath", "tt_fastpath.so")

_table = None
_error: str | None = None
_tried = False


def table(max_entries: int):
    """The process's LaunchTable (created on first use), or None with the reason in error()."""
    global _table, _error, _tried
    if _tried:
        return _table
    _tried = True
    lib = _lib.load()
    if lib is None:
        _error = _lib.load_error()
        return None
    if not os.path.exists(PATH):
        _error = f"{PATH} is not built"
        return None
    try:
        spec = importlib.util.spec_from_file_location("tt_fastpath", PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)

        def addr(fn) -> int:
            return ctypes.cast(fn, ctypes.c_void_p).value

        _table = mod.LaunchTable(addr(lib.tt_gemm_packed), addr(lib.tt_last_error), addr(lib.tt_status_string),
                                 max_entries)
    except (ImportError, OSError, AttributeError) as exc:
        _error = f"cannot load {PATH}: {exc}"
        _table = None
    return _table


def error() -> str | None:
    return _error
