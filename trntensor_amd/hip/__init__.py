"""HIP module for gfx950: replaces the reference's trntensor/nki package.

``HAS_HIP`` reports whether libtrntensor_hip.so loaded and a gfx950 device is
visible; ``set_backend`` / ``get_backend`` select the executor.
"""

from .dispatch import HAS_HIP, HAS_NKI, get_backend, set_backend

__all__ = ["HAS_HIP", "HAS_NKI", "set_backend", "get_backend"]
