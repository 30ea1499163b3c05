"""Build recipe for libvoid_amd.so (gfx950 HIP kernels + C ABI).

Run ``python -m void_amd.build`` (or ``__graft_entry__.build()``).  The
library is built in-tree next to this file so that it travels with the
repository snapshot; nothing is installed.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
SRC_DIR = PKG_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
LIB_PATH = PKG_DIR / "libvoid_amd.so"
ARCH = "gfx950"

SOURCES = [SRC_DIR / "void_spmm.hip", SRC_DIR / "void_quant.hip", SRC_DIR / "void_format.hip", SRC_DIR / "void_sddmm.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-shared",
    "-fPIC",
    # Exact control of rounding: every fused multiply-add in the kernels is
    # an explicit fmaf, so the ROW_MEAN epilogue keeps separate mul / add.
    "-ffp-contract=off",
    # Packed fp32 VALU forms are kept out of generated code on this pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    # The column-group kernel's first five argument dwords (work-list address
    # and the packed grid layout) arrive preloaded in SGPRs, so that its first
    # work-item read does not wait for a kernel-argument load.
    "-mllvm", "-amdgpu-kernarg-preload-count=5",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the gfx950 library cannot be built")
    return path


# Instrumented variant for clock measurements (bench.py --op clock): every
# SpMM workgroup records real-time and shader-clock stamps at its start and
# end into a buffer set with void_debug_set_trace.  Not used by the product.
CLOCK_LIB_PATH = PKG_DIR / "libvoid_amd_clock.so"
CLOCK_FLAGS = ["-DVOID_TRACE", "-DVOID_TRACE_CLK"]
# Instrumented variant for phase timelines (bench.py --op phases): every SpMM
# workgroup records s_memrealtime at its phase boundaries.  Not used by the
# product.
PHASE_LIB_PATH = PKG_DIR / "libvoid_amd_phase.so"
PHASE_FLAGS = ["-DVOID_TRACE"]


def build(verbose: bool = False, clock_probe: bool = False, phase_probe: bool = False) -> Path:
    """Compile every HIP source into ``void_amd/libvoid_amd.so`` (or the
    instrumented ``libvoid_amd_clock.so`` with clock_probe,
    ``libvoid_amd_phase.so`` with phase_probe)."""
    out = CLOCK_LIB_PATH if clock_probe else PHASE_LIB_PATH if phase_probe else LIB_PATH
    tmp = out.with_suffix(".so.tmp")
    extra = CLOCK_FLAGS if clock_probe else PHASE_FLAGS if phase_probe else []
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, f"-I{INCLUDE_DIR}", *map(str, SOURCES), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True, clock_probe="--clock-probe" in sys.argv[1:], phase_probe="--phase-probe" in sys.argv[1:]))
