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


def workload_plan(void_tensor, workload: StreamKWorkload) -> "_runtime.DevicePlan":
    """Device work items that run exactly the workload's worker ranges,
    cached on the tensor's device view per workload object."""
    from .ops import F32_CHUNK
    # Plans depend only on the block structure, which every device copy of
    # the tiles shares: take the copy in the tiles' own dtype (the one the
    # 16-bit kernel uses for 16-bit tensors) rather than make another.
    dt = void_tensor.values.dtype
    dbsr = void_tensor.device_bsr(dt if dt in (torch.bfloat16, torch.float16) else torch.float32)
    key = ("workload", id(workload))
    cached = dbsr.plans.get(key)
    if cached is not None and cached[0] is workload:
        return cached[1]
    items, n_tiles, n_slots, longest = _runtime.plan_from_ranges(
        dbsr.row_ptr_host, dbsr.col_idx_host, workload.worker_rows.detach().cpu().numpy(),
        workload.worker_block_start.detach().cpu().numpy(), workload.worker_block_end.detach().cpu().numpy(),
        F32_CHUNK)
    plan = _runtime.DevicePlan(torch.from_numpy(items).to(dbsr.row_ptr.device), items.shape[0], n_tiles, n_slots,
                               max(longest, 1), items)
    old = [k for k in dbsr.plans if isinstance(k, tuple) and k[0] == "workload"]
    for k in old[:max(0, len(old) - 7)]:  # keep the plans of the last 8 workloads
        del dbsr.plans[k]
    dbsr.plans[key] = (workload, plan)
    return plan


def void_spmm_stream_k(a, b: torch.Tensor, workload: Optional[StreamKWorkload] = None,
                       out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Stream-K load-balanced SpMM C = A @ B for a float VOIDTensor
    (stream_k.py:233-301), on the float MFMA kernels of libvoid_amd.so (the
    16-bit one when the tiles and B share a 16-bit dtype).

    Each worker of ``workload`` (computed by compute_stream_k_workload when
    None) becomes one work item over its tile range; the partial blocks of a
    row that several workers share are summed in range order by the last of
    them to finish (a deterministic fix-up in place of the reference's
    spin-locked read-modify-write).  C has B's dtype; ``out`` is
    overwritten."""
    if b.dim() != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"B must be [K={a.shape[1]}, N], got {tuple(b.shape)}")
    _runtime.require_gpu(b, "B")
    _runtime.require_gpu(a.values, "A")
    from .ops import float_spmm
    M, N = a.shape[0], b.shape[1]
    if out is not None and tuple(out.shape) != (M, N):
        raise ValueError(f"out must be [{M}, {N}]")
    if a.n_blocks == 0:
        if out is None:
            return torch.zeros(M, N, dtype=b.dtype, device=b.device)
        return out.zero_()
    if workload is None:
        workload = compute_stream_k_workload(a)
    return float_spmm(a, b, out=out, plan=workload_plan(a, workload))


__all__ = ["StreamKWorkload", "compute_stream_k_workload", "analyze_workload_balance", "void_spmm_stream_k",
           "workload_plan"]

