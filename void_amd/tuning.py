"""Fixed gfx950 launch configuration (replaces the reference's autotuner).

The reference searches TILE_N x num_warps x num_stages at run time and keeps
a JSON cache (void/autotune.py:39-104, 345-381).  On MI355X the kernel shape
is fixed by the hardware instead:

* one workgroup = 4 wave64s, one 32-row block-row x 128-column panel of C,
  each wave owning 32 columns; the LDS-DMA column-group kernel uses 40 KB of
  LDS and about 100 registers per lane -> 4 workgroups per CU;
* 256 CUs in 8 XCDs -> 1024 resident workgroups;
* the only shape-dependent knob is the Stream-K chunk: the most tiles one
  work item may take before its block-row is split.  The column-group
  kernel takes items of at most 64 tiles (an item's block columns and
  scales sit one per lane), and a split row pays a partial-tile round trip
  through L2 (coherent 16-byte stores, an atomic, coherent loads):
  - every block-row fits in 64 tiles: chunk 64, nothing is split;
  - some block-row is longer: 1.3 times the average work per resident
    workgroup slot, clamped to [32, 64].  Plans with split rows run the
    two-ring kernel (8-wave workgroups, 2 per CU), so a slot is 1/512 of
    the chip.  Measured on the power-law config (Zipf rows up to 512 tiles,
    cold): two-ring kernel at chunk 32 / 46 / 64: 33.4-33.9 / 29.5-30.0 /
    27.8-28.1 us; the one-ring kernel at 32 / 46 / 64: 30.9-31.0 / 29.4-29.5
    / 28.5-28.7 us.
"""

from __future__ import annotations

import math

GFX950_CUS = 256
GFX950_XCDS = 8
WAVES_PER_WORKGROUP = 4
WORKGROUPS_PER_CU = 4
PANEL_COLUMNS = 128
TILE = 32

MIN_SPLIT_CHUNK = 32

# (name, longest item of the column-group kernel, factor on the per-slot average)
CHUNK_TABLE = {
    "int8": (64, 1.3),
    "fp8": (64, 1.3),
}


# Longest work item of the kernels that stage fp32 B slabs (the float SpMM
# and the E4M3 x fp32 SpMM): they hold an item's block columns one per lane.
FP32_B_MAX_CHUNK = 64


def resident_workgroups() -> int:
    return GFX950_CUS * WORKGROUPS_PER_CU


# Workgroups per CU of the two-ring kernel that plans with split rows run.
SPLIT_WORKGROUPS_PER_CU = 2


def n_panels(N: int) -> int:
    return (N + PANEL_COLUMNS - 1) // PANEL_COLUMNS


def select_chunk(kind: str, n_blocks: int, N: int, max_row: int = 0) -> int:
    """Stream-K chunk (max tiles per work item) for a problem whose longest
    block-row has max_row tiles."""
    cg_max, factor = CHUNK_TABLE[kind]
    if max_row <= cg_max:
        return cg_max
    per_slot = n_blocks * n_panels(max(N, 1)) / (GFX950_CUS * SPLIT_WORKGROUPS_PER_CU)
    return min(cg_max, max(MIN_SPLIT_CHUNK, int(math.ceil(per_slot * factor))))


# A column-major B (X.t() of token-major activations) runs the register-staged
# column-group loop, whose 16-byte loads from one column each use a quarter
# of a 128-byte line; the LDS-DMA ring reads row-major B in whole lines.  When
# the slabs gathered (32 N bytes per tile) exceed 32 times B itself, a
# row-major copy of B (one pass over it) pays for itself: on the FFN config
# the SpMM with GELU took 183 us with B column-major against 91 us
# row-major.  VOID_AMD_BT=0 / 1 forces the copy off / on.
COL_MAJOR_COPY_RATIO = 32


def copy_col_major_b(n_blocks: int, K: int) -> bool:
    import os
    env = os.environ.get("VOID_AMD_BT")
    if env in ("0", "1"):
        return env == "1"
    return 32 * n_blocks >= COL_MAJOR_COPY_RATIO * max(K, 1)
