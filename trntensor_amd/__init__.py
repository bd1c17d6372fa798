"""trntensor_amd — trntensor's fused tensor-contraction path on AMD MI355X.

Drop-in for the contraction API of trntensor 0.4.0 (``import trntensor_amd as
trntensor``): einsum with alpha/beta/out/dtype/precision, multi_einsum, the
contraction planner with its cache and greedy path search, and the DF-MP2
energy / AO->MO transform primitives. Every contraction executes on
hand-written gfx950 HIP kernels (libtrntensor_hip.so, C ABI in
include/trntensor_hip.h) loaded into PyTorch-ROCm through ctypes.
The reference's tensor decompositions (CP/Tucker/TT) are not part of this
package.
"""

__version__ = "0.4.0+mi355x"

from .einsum import einsum, multi_einsum
from .hip import HAS_HIP, HAS_NKI, get_backend, set_backend
from .hip.dispatch import from_device, from_xla, to_device, to_xla
from .plan import (
    ContractionPlan,
    clear_plan_cache,
    estimate_flops,
    plan_cache_info,
    plan_contraction,
)
from .quantum import ao_to_mo_transform, mp2_energy, mp2_energy_shard

__all__ = [
    "einsum",
    "multi_einsum",
    "ContractionPlan",
    "plan_contraction",
    "estimate_flops",
    "clear_plan_cache",
    "plan_cache_info",
    "HAS_HIP",
    "HAS_NKI",
    "set_backend",
    "get_backend",
    "to_device",
    "from_device",
    "to_xla",
    "from_xla",
    "mp2_energy",
    "mp2_energy_shard",
    "ao_to_mo_transform",
]
