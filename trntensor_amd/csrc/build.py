"""Build libtrntensor_hip.so for gfx950 from the HIP sources in this directory.

Usage: python trntensor_amd/csrc/build.py [--jobs N] [--no-fastpath]

Each source is compiled to an object with hipcc in parallel, then linked
into ``trntensor_amd/_lib/libtrntensor_hip.so`` (in-tree, so it travels
with the source tree). Packed-FP32 instruction selection is disabled for all
device code. Then the host launch table (tt_fastpath.cpp, a torch C++
extension) is built into ``trntensor_amd/_lib/fastpath/``.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
OUT_DIR = os.path.join(PKG, "_lib")
LIB = os.path.join(OUT_DIR, "libtrntensor_hip.so")
SOURCES = [
    "tt_abi.hip",
    "tt_dd.hip",
    "tt_gemm.hip",
    "tt_gemm16.hip",
    "tt_gemm16_dma.hip",
    "tt_gemm_big.hip",
    "tt_mp2.hip",
    "tt_probe.hip",
    "tt_strided.hip",
]
# Sources whose MFMA accumulators belong in AGPRs (256 fp32 per lane): built
# without the VGPR-accumulator option below.
AGPR_SOURCES = {"tt_gemm16_dma.hip", "tt_gemm_big.hip"}
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    # keep MFMA accumulators in VGPRs (no per-iteration AGPR<->VGPR copies)
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
    "-Wall",
    "-Wno-unused-result",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP library needs ROCm's hipcc")
    return path


def build(jobs: int = 4, verbose: bool = False, extra: list[str] | None = None) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    obj_dir = os.path.join(OUT_DIR, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    cc = hipcc()
    flags = HIPCC_FLAGS + list(extra or [])

    def compile_one(src: str) -> str:
        obj = os.path.join(obj_dir, src.replace(".hip", ".o"))
        fl = list(flags)
        if src in AGPR_SOURCES:
            i = fl.index("-amdgpu-mfma-vgpr-form")
            del fl[i - 1 : i + 1]
        cmd = [cc, *fl, "-c", os.path.join(HERE, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
        if verbose and res.stderr:
            print(res.stderr, file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


FASTPATH_DIR = os.path.join(OUT_DIR, "fastpath")
FASTPATH = os.path.join(FASTPATH_DIR, "tt_fastpath.so")


def build_fastpath(verbose: bool = False) -> str:
    """Compile tt_fastpath.cpp (host C++ against torch's headers, no device
    code) into ``_lib/fastpath/tt_fastpath.so``, from scratch each time."""
    import torch.utils.cpp_extension as ce

    os.makedirs(FASTPATH_DIR, exist_ok=True)
    for f in os.listdir(FASTPATH_DIR):
        if f.endswith((".so", ".o")) or f in ("build.ninja", ".ninja_deps", ".ninja_log"):
            os.remove(os.path.join(FASTPATH_DIR, f))
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    ce.load(
        "tt_fastpath",
        [os.path.join(HERE, "tt_fastpath.cpp")],
        build_directory=FASTPATH_DIR,
        extra_cflags=["-O2", "-D__HIP_PLATFORM_AMD__", f"-I{rocm}/include", f"-I{os.path.join(os.path.dirname(PKG), 'include')}"],
        extra_ldflags=["-lc10_hip", f"-L{rocm}/lib", "-lamdhip64"],
        with_cuda=False,
        verbose=verbose,
    )
    if not os.path.exists(FASTPATH):
        raise RuntimeError(f"tt_fastpath build produced no {FASTPATH}")
    return FASTPATH


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--no-fastpath", action="store_true", help="skip the host C++ launch table")
    args, rest = ap.parse_known_args()
    print(build(args.jobs, args.verbose, rest))
    if not args.no_fastpath:
        print(build_fastpath(args.verbose))
