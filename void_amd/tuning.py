"""Fixed gfx950 launch configuration (replaces the reference's autotuner).

The reference searches TILE_N x num_warps x num_stages at run time and keeps
a JSON cache (void/autotune.py:39-104, 345-381).  On MI355X the kernel shape
is fixed by the hardware instead:

* one workgroup = 4 wave64s, one 32-row block-row x 128-column panel of C,
  each wave owning 32 columns; 48 KB of LDS (shared A tiles, per-wave B
  slabs) and at most 256 registers per lane -> 2 workgroups per CU;
* 256 CUs in 8 XCDs -> 512 resident workgroups;
* the only shape-dependent knob is the Stream-K chunk: the most tiles one
  work item may take before its block-row is split.  A split row pays for
  a partial-tile round trip through memory (coherent stores, an atomic,
  coherent loads: several microseconds), so the chunk is the larger of a
  floor of 64 tiles and the average work per resident workgroup slot (only
  rows far longer than the typical item are split), capped at the 64 tiles
  whose block columns and scales the column-group kernel holds in one
  register per lane (a longer chunk runs on the general kernel).
"""

from __future__ import annotations

import math

GFX950_CUS = 256
GFX950_XCDS = 8
WAVES_PER_WORKGROUP = 4
WORKGROUPS_PER_CU = 2
PANEL_COLUMNS = 128
TILE = 32

# (name, floor on the chunk, factor on the per-slot average, cap)
CHUNK_TABLE = {
    "int8": (64, 1.0, 64),
    "fp8": (64, 1.0, 64),
}


def resident_workgroups() -> int:
    return GFX950_CUS * WORKGROUPS_PER_CU


def n_panels(N: int) -> int:
    return (N + PANEL_COLUMNS - 1) // PANEL_COLUMNS


def select_chunk(kind: str, n_blocks: int, N: int) -> int:
    """Stream-K chunk (max tiles per work item) for a problem."""
    floor, factor, cap = CHUNK_TABLE[kind]
    per_slot = n_blocks * n_panels(max(N, 1)) / resident_workgroups()
    return min(cap, max(floor, int(math.ceil(per_slot * factor))))
