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
  coherent loads: several microseconds), so rows are split only when they
  are far longer than the typical item:
  - every block-row fits in 64 tiles: chunk 64, nothing is split, and the
    column-group kernel runs (it holds an item's block columns and scales
    in one register per lane, so it takes items of at most 64 tiles);
  - some block-row is longer: the chunk is the larger of 65 and 1.3 times
    the average work per resident workgroup slot, and the general kernel
    runs, whose four waves share an item's tiles (a quarter of the
    dependent chain of the column-group kernel, where every wave walks all
    of them).  Measured on the power-law config (dealt work list): chunk 71
    56 us, 90 48 us, 100 52 us, 110 49 us, 128 56 us, 200 59 us; the
    column-group kernel at its 64-tile limit 80 us.
"""

from __future__ import annotations

import math

GFX950_CUS = 256
GFX950_XCDS = 8
WAVES_PER_WORKGROUP = 4
WORKGROUPS_PER_CU = 2
PANEL_COLUMNS = 128
TILE = 32

# (name, longest item of the column-group kernel, factor on the per-slot average)
CHUNK_TABLE = {
    "int8": (64, 1.3),
    "fp8": (64, 1.3),
}


def resident_workgroups() -> int:
    return GFX950_CUS * WORKGROUPS_PER_CU


def n_panels(N: int) -> int:
    return (N + PANEL_COLUMNS - 1) // PANEL_COLUMNS


def select_chunk(kind: str, n_blocks: int, N: int, max_row: int = 0) -> int:
    """Stream-K chunk (max tiles per work item) for a problem whose longest
    block-row has max_row tiles."""
    cg_max, factor = CHUNK_TABLE[kind]
    if max_row <= cg_max:
        return cg_max
    per_slot = n_blocks * n_panels(max(N, 1)) / resident_workgroups()
    return max(cg_max + 1, int(math.ceil(per_slot * factor)))
