"""Stream-K partition of a block-sparse SpMM over its nonzero tiles.

Mirrors ``void/stream_k.py``'s host API (StreamKWorkload,
compute_stream_k_workload, analyze_workload_balance).  The partition itself
is computed by the C planner of libvoid_amd.so (void_streamk_plan): each
block-row is one work item unless it has more tiles than the chunk size,
in which case it is cut into near-equal chunks whose partial tiles the
kernel combines in a fixed order (no spin locks, unlike the reference's
stream_k_spmm_kernel, stream_k.py:198-219).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _runtime


@dataclass
class StreamKWorkload:
    """Per-worker assignments (stream_k.py:13-33); one worker per non-empty work item."""
    worker_rows: torch.Tensor
    worker_block_start: torch.Tensor
    worker_block_end: torch.Tensor
    worker_needs_atomic: torch.Tensor
    n_workers: int
    total_work: int
    chunk_tiles: int = 0


def _row_ptr_host(void_tensor) -> np.ndarray:
    row_ptr, _ = void_tensor.get_row_block_info()
    return row_ptr.detach().cpu().numpy().astype(np.int32)


def compute_stream_k_workload(void_tensor, n_workers: Optional[int] = None,
                              max_work_per_worker: int = 16) -> StreamKWorkload:
    """Split block-rows into chunks (stream_k.py:36-110).

    Chunk size as in the reference: ceil(total / n_workers) capped at
    max_work_per_worker, n_workers defaulting to min(total, 1024).  A split
    row's chunks differ in length by at most one tile.  Workers are listed by
    row, then by position in the row; empty rows get no worker.
    """
    total = int(void_tensor.n_blocks)
    if n_workers is None:
        n_workers = min(total, 1024)
    target = (total + n_workers - 1) // n_workers if n_workers > 0 else 1
    target = max(1, min(target, max_work_per_worker))
    items, _, _ = _runtime.plan_rows(_row_ptr_host(void_tensor), target)
    items = items[items[:, 2] > items[:, 1]]
    order = np.lexsort((items[:, 1], items[:, 0]))
    items = items[order]
    dev = void_tensor.values.device if hasattr(void_tensor, "values") else void_tensor.values_fp8.device
    return StreamKWorkload(
        worker_rows=torch.from_numpy(items[:, 0].copy()).to(dev),
        worker_block_start=torch.from_numpy(items[:, 1].copy()).to(dev),
        worker_block_end=torch.from_numpy(items[:, 2].copy()).to(dev),
        worker_needs_atomic=torch.from_numpy(items[:, 3] >= 0).to(dev),
        n_workers=int(items.shape[0]),
        total_work=total,
        chunk_tiles=target,
    )


def analyze_workload_balance(void_tensor) -> dict:
    """Blocks-per-row statistics (stream_k.py:467-492)."""
    rp = _row_ptr_host(void_tensor)
    work = torch.from_numpy((rp[1:] - rp[:-1]).astype(np.float32))
    nz = work > 0
    w = work[nz]
    if len(w) == 0:
        return {"empty": True}
    return {
        "empty": False,
        "n_rows": len(work),
        "n_nonempty_rows": int(nz.sum().item()),
        "min_blocks_per_row": w.min().item(),
        "max_blocks_per_row": w.max().item(),
        "mean_blocks_per_row": w.mean().item(),
        "std_blocks_per_row": w.std().item() if len(w) > 1 else 0.0,
        "imbalance_ratio": (w.max() / w.mean()).item(),
        "coefficient_of_variation": (w.std() / w.mean()).item() if len(w) > 1 else 0.0,
    }


__all__ = ["StreamKWorkload", "compute_stream_k_workload", "analyze_workload_balance"]
