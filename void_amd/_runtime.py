"""Device-side state shared by the quantized SpMM entry points.

A quantized VOID tensor gets, once per device, a ``DeviceBsr``: its tiles and
scales gathered into block-row-major order, the block-row pointer and column
indices, and a cache of Stream-K plans (work items on the device plus a
zero-initialised workspace).  ``launch`` fills the C-ABI descriptors and calls
into ``libvoid_amd.so`` on the current torch stream.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from collections import OrderedDict
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

from . import _lib, tuning
from .format import build_bsr_layout

_OUT_CODES = {
    torch.float32: _lib.DT_F32,
    torch.bfloat16: _lib.DT_BF16,
    torch.float16: _lib.DT_F16,
    torch.int32: _lib.DT_I32,
}


# Streams whose eager split-row workspaces a plan keeps (least recently used
# first out).
MAX_STREAM_WORKSPACES = 8
# Largest split-row workspace of which a plan keeps a zeroed spare for the
# next HIP graph capture.
MAX_SPARE_WORKSPACE = 64 << 20


@dataclass
class DevicePlan:
    items: torch.Tensor          # int32 [n_items, 32] on device (void_work_item)
    n_items: int
    n_split_tiles: int
    n_slots: int
    chunk: int
    host_items: np.ndarray       # int32 [n_items, 32] copy, for inspection
    workspaces: "OrderedDict[Tuple[int, int], torch.Tensor]" = field(default_factory=OrderedDict)
    capture_workspaces: List[torch.Tensor] = field(default_factory=list)
    capture_spares: Dict[int, torch.Tensor] = field(default_factory=dict)  # nbytes -> zeroed, for the next capture
    capture_by_id: Dict[Tuple[int, int, int], torch.Tensor] = field(default_factory=dict)  # (capture, stream, nbytes)
    ws_sizes: Dict[int, int] = field(default_factory=dict)  # N -> void_workspace_bytes
    _cplan: Optional["_lib.Plan"] = None

    def cplan(self) -> "_lib.Plan":
        """The C descriptor of this plan (its arrays never change: built once)."""
        if self._cplan is None:
            self._cplan = _lib.Plan(items=self.items.data_ptr(), n_items=self.n_items,
                                    n_split_tiles=self.n_split_tiles, n_slots=self.n_slots, chunk_tiles=self.chunk)
        return self._cplan

    def counter_bytes(self, N: int) -> int:
        """Bytes of split-row arrival counters at the start of the workspace
        (n_split_tiles x n_panels int32, rounded up to 256 bytes)."""
        return (self.n_split_tiles * tuning.n_panels(max(N, 1)) * 4 + 255) // 256 * 256

    def workspace(self, N: int, device: torch.device,
                  stream: Optional[int] = None) -> Tuple[Optional[torch.Tensor], int]:
        """The split-row workspace of this plan for N columns on one HIP stream.

        The workspace holds the split rows' arrival counters and partial
        blocks, so two launches that share one would mix their partials:
        each stream gets its own (launches on one stream run in order, and
        every launch leaves the counters at zero).  ``stream`` is the raw
        stream handle, torch's current stream of ``device`` by default.

        Eager launches reuse one workspace per stream, the last
        ``MAX_STREAM_WORKSPACES`` streams being kept.  Under HIP graph capture
        each (capture, stream) gets a workspace of its own, its counters zeroed
        by a fill kernel captured into the same graph before its first launch,
        so that every graph clears and owns its counters and graphs replayed on
        different streams never share them; the launches of one capture on one
        stream run in order and share it.  It is kept for the lifetime of the
        plan.  Only the counters are cleared: the partial blocks are always
        written before they are read.  The first eager launch of a size also
        prepares one spare workspace (up to MAX_SPARE_WORKSPACE bytes), zeroed
        and synchronised once, which the next capture takes as its own with no
        fill kernel in the graph."""
        nbytes = self.ws_sizes.get(N)
        if nbytes is None:
            nbytes = self.ws_sizes[N] = int(_lib.lib().void_workspace_bytes(self.n_split_tiles, self.n_slots, N))
        if nbytes == 0:
            return None, 0
        if torch.cuda.is_current_stream_capturing():
            raw = stream if stream is not None else torch.cuda.current_stream(device).cuda_stream
            cid = ctypes.c_ulonglong(0)
            _lib.check(_lib.lib().void_stream_capture_id(ctypes.c_void_p(int(raw)), ctypes.byref(cid)),
                       "void_stream_capture_id")
            key = (int(cid.value), int(raw), nbytes)
            ws = self.capture_by_id.get(key)
            if ws is None:
                ws = self.capture_spares.pop(nbytes, None)
                if ws is None:
                    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
                    ws[:self.counter_bytes(N)].zero_()
                self.capture_by_id[key] = ws
                self.capture_workspaces.append(ws)
            return ws, nbytes
        if stream is None:
            stream = torch.cuda.current_stream(device).cuda_stream
        key = (nbytes, int(stream))
        ws = self.workspaces.get(key)
        if ws is None:
            # Counters must start at zero; every launch leaves them at zero.
            # The zeroing runs on the stream that will use the workspace.
            ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
            _zero_on_stream(ws[:self.counter_bytes(N)], int(stream), device)
            self.workspaces[key] = ws
            if nbytes <= MAX_SPARE_WORKSPACE and nbytes not in self.capture_spares:
                spare = torch.empty(nbytes, dtype=torch.uint8, device=device)
                spare[:self.counter_bytes(N)].zero_()
                # Zeroed before any graph can use it, whatever stream replays it.
                torch.cuda.current_stream(device).synchronize()
                self.capture_spares[nbytes] = spare
            while len(self.workspaces) > MAX_STREAM_WORKSPACES:
                # The oldest stream's workspace is freed; the caching allocator
                # keeps its memory until the work queued on that stream is done.
                self.workspaces.popitem(last=False)
        else:
            self.workspaces.move_to_end(key)
        return ws, nbytes


def _zero_on_stream(t: torch.Tensor, stream: int, device: torch.device) -> None:
    """t.zero_() ordered before later work on the raw HIP stream ``stream``."""
    cur = torch.cuda.current_stream(device)
    if cur.cuda_stream == stream:
        t.zero_()
        return
    ext = torch.cuda.ExternalStream(stream, device=device)
    with torch.cuda.stream(ext):
        t.zero_()
    # The allocation came from the current stream's pool; keep it alive for
    # the external stream as well.
    t.record_stream(ext)


def plan_rows(row_ptr_host: np.ndarray, chunk: int,
              col_idx_host: Optional[np.ndarray] = None) -> Tuple[np.ndarray, int, int]:
    """Run the C planner on host index arrays; returns (items[n, 32] int32, n_split_tiles, n_slots)."""
    lib = _lib.lib()
    rp = np.ascontiguousarray(row_ptr_host, dtype=np.int32)
    ci = None if col_idx_host is None else np.ascontiguousarray(col_idx_host, dtype=np.int32)
    ci_ptr = None if ci is None else ci.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    n_br = rp.size - 1
    n_items = ctypes.c_int32()
    n_tiles = ctypes.c_int32()
    n_slots = ctypes.c_int32()
    rp_ptr = rp.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    cap = max(n_br, 1)
    while True:
        buf = (_lib.WorkItem * cap)()
        st = lib.void_streamk_plan(rp_ptr, ci_ptr, n_br, int(chunk), buf, cap, ctypes.byref(n_items),
                                   ctypes.byref(n_tiles), ctypes.byref(n_slots))
        if st == -5 and n_items.value > cap:
            cap = n_items.value
            continue
        _lib.check(st, "void_streamk_plan")
        break
    W = _lib.ITEM_INTS
    items = np.frombuffer(buf, dtype=np.int32, count=n_items.value * W).reshape(n_items.value, W).copy()
    return items, n_tiles.value, n_slots.value


def plan_from_ranges(row_ptr_host: np.ndarray, col_idx_host: np.ndarray, rows: np.ndarray, begins: np.ndarray,
                     ends: np.ndarray, max_chunk: int) -> Tuple[np.ndarray, int, int, int]:
    """Work items that run exactly the given tile ranges (BSR positions
    [begins[w], ends[w]) of block-row rows[w]), as the reference's Stream-K
    workers do (stream_k.py:113-222).

    Ranges longer than max_chunk are cut into near-equal pieces.  A row
    covered by more than one range becomes a split row whose partial blocks
    the kernel sums in range order; rows that no range covers get an empty
    item, so their output is written (zero, or the epilogue of zero), where
    the reference leaves its zero-filled output untouched.
    Returns (items[n, 32] int32, n_split_tiles, n_slots, longest item)."""
    rp = np.asarray(row_ptr_host, dtype=np.int64)
    n_br = rp.size - 1
    rows = np.asarray(rows, dtype=np.int64).reshape(-1)
    begins = np.asarray(begins, dtype=np.int64).reshape(-1)
    ends = np.asarray(ends, dtype=np.int64).reshape(-1)
    if not (rows.size == begins.size == ends.size):
        raise ValueError("worker_rows, worker_block_start and worker_block_end differ in length")
    if rows.size and (rows.min() < 0 or rows.max() >= n_br):
        raise ValueError(f"worker rows must lie in [0, {n_br})")
    if np.any(begins > ends) or np.any(begins < rp[rows]) or np.any(ends > rp[rows + 1]):
        raise ValueError("a worker's block range lies outside its block-row")
    pieces = []  # (row, begin, end)
    for r, b, e in zip(rows.tolist(), begins.tolist(), ends.tolist()):
        n = e - b
        if n == 0:
            continue
        k = -(-n // max_chunk)
        for c in range(k):
            pieces.append((r, b + c * n // k, b + (c + 1) * n // k))
    pieces.sort(key=lambda x: (x[0], x[1]))
    covered = np.zeros(n_br, dtype=bool)
    per_row = {}
    for pc in pieces:
        per_row.setdefault(pc[0], []).append(pc)
        covered[pc[0]] = True
    W = _lib.ITEM_INTS
    items = []
    n_tiles = n_slots = 0
    ci = np.asarray(col_idx_host, dtype=np.int32)
    for r in range(n_br):
        lst = per_row.get(r)
        if not lst:
            lst = [(r, int(rp[r]), int(rp[r]))]
        split = len(lst) > 1
        for c, (_, b, e) in enumerate(lst):
            it = np.full(W, -1, dtype=np.int32)
            it[:8] = (r, b, e, n_tiles if split else -1, len(lst), c if split else 0, n_slots if split else 0, 0)
            m = min(e - b, _lib.ITEM_INLINE_COLS)
            it[8:8 + m] = ci[b:b + m]
            items.append(it)
        if split:
            n_tiles += 1
            n_slots += len(lst)
    arr = np.stack(items).astype(np.int32)
    lengths = arr[:, 2] - arr[:, 1]
    arr = arr[np.argsort(-lengths, kind="stable")]  # longest first, as the planner orders
    return arr, n_tiles, n_slots, int(lengths.max()) if lengths.size else 0


@dataclass
class DeviceBsr:
    tiles: torch.Tensor          # uint8 [n_blocks, 32, 32] block-row-major
    scales: torch.Tensor         # float32 [n_blocks] (or [1] with per_tensor)
    row_ptr: torch.Tensor        # int32 [n_block_rows + 1]
    col_idx: torch.Tensor        # int32 [n_blocks]
    row_ptr_host: np.ndarray
    col_idx_host: np.ndarray
    per_tensor: bool
    M: int
    K: int
    n_blocks: int
    n_block_rows: int
    plans: Dict[int, DevicePlan] = field(default_factory=dict)
    _max_row: Optional[int] = None
    _desc: Optional[_lib.BsrDesc] = None
    order: Optional[torch.Tensor] = None  # BSR position -> index of the source tile
    src_key: tuple = ()                   # source_key of the tensors the arrays were gathered from

    def refresh(self, values: torch.Tensor, scales: torch.Tensor) -> None:
        """Gather the tile values and scales again from their sources into the
        existing arrays, after the sources changed in place; the block
        structure, plans and descriptor stay valid."""
        if self.order is None:
            raise RuntimeError("this device copy records no gather order; build the VOID tensor again")
        dev = self.tiles.device
        v = values.to(dev)
        if v.dtype != torch.uint8:
            v = v.view(torch.uint8)
        if self.n_blocks:
            torch.index_select(v, 0, self.order, out=self.tiles)
        sc = scales.to(device=dev, dtype=torch.float32)
        if self.per_tensor:
            self.scales.copy_(sc.reshape(-1)[:1])
        elif sc.numel():
            torch.index_select(sc, 0, self.order, out=self.scales)

    @property
    def max_row(self) -> int:
        """Tiles in the longest block-row (the structure is fixed: computed once)."""
        if self._max_row is None:
            rp = self.row_ptr_host
            self._max_row = int(np.max(np.diff(rp))) if len(rp) > 1 else 0
        return self._max_row

    def plan(self, chunk: int) -> DevicePlan:
        p = self.plans.get(chunk)
        if p is None:
            items, n_tiles, n_slots = plan_rows(self.row_ptr_host, chunk, self.col_idx_host)
            dev_items = torch.from_numpy(items).to(self.row_ptr.device)
            p = DevicePlan(dev_items, items.shape[0], n_tiles, n_slots, chunk, items)
            self.plans[chunk] = p
        return p

    def desc(self) -> _lib.BsrDesc:
        """The C descriptor of this matrix (its arrays never change: built once)."""
        if self._desc is None:
            self._desc = self._make_desc()
        return self._desc

    def _make_desc(self) -> _lib.BsrDesc:
        return _lib.BsrDesc(
            tiles=self.tiles.data_ptr() if self.n_blocks else None,
            scales=self.scales.data_ptr() if self.scales.numel() else None,
            row_ptr=self.row_ptr.data_ptr(),
            col_idx=self.col_idx.data_ptr() if self.n_blocks else None,
            M=self.M, K=self.K, n_blocks=self.n_blocks, n_block_rows=self.n_block_rows,
            per_tensor_a=int(self.per_tensor), reserved=0)


def make_device_bsr(values: torch.Tensor, scales: torch.Tensor, block_rows: torch.Tensor,
                    block_cols: torch.Tensor, shape: Tuple[int, int], tile_size: Tuple[int, int],
                    device: torch.device, per_tensor: bool, layout=None) -> DeviceBsr:
    """Gather the tiles into block-row-major order.  ``layout`` (a BsrLayout
    of the same block structure) skips the host-side ordering."""
    if tuple(tile_size) != (32, 32):
        raise NotImplementedError(f"the gfx950 kernels take 32x32 tiles, got {tile_size}")
    M, K = shape
    n_br = (M + 31) // 32
    n_bc = (K + 31) // 32
    lay = layout if layout is not None else build_bsr_layout(block_rows, block_cols, n_br, n_bc, device)
    v = values.to(device)
    if v.dtype != torch.uint8:
        v = v.view(torch.uint8)
    tiles = v.index_select(0, lay.order).contiguous() if v.shape[0] else v.contiguous()
    s = scales.to(device=device, dtype=torch.float32)
    if per_tensor:
        s = s.reshape(-1)[:1].contiguous()
    else:
        s = s.index_select(0, lay.order).contiguous() if s.numel() else s.contiguous()
    return DeviceBsr(tiles=tiles, scales=s, row_ptr=lay.row_ptr, col_idx=lay.col_idx,
                     row_ptr_host=lay.row_ptr_host, col_idx_host=lay.col_idx.cpu().numpy(),
                     per_tensor=per_tensor, M=M, K=K,
                     n_blocks=int(values.shape[0]), n_block_rows=n_br, order=lay.order)


def source_key(*tensors: torch.Tensor) -> tuple:
    """Identity and in-place version of the tensors a device copy is made
    from: the copy is stale once either changes.  Inference tensors
    (torch.inference_mode) keep no version counter, so for them only a new
    tensor is noticed."""
    return tuple((t.data_ptr(), None if t.is_inference() else t._version) for t in tensors)


def require_gpu(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{what} must be a GPU (HIP) tensor; the SpMM runs only on the gfx950 "
                           f"kernels of libvoid_amd.so (got device {t.device})")


def dense_operand(b: torch.Tensor) -> Tuple[torch.Tensor, int, bool]:
    """(tensor, ld, col_major) for B without copying when B is row- or column-major."""
    if b.stride(1) == 1 and (b.stride(0) >= b.shape[1] or b.shape[0] <= 1):
        return b, max(b.stride(0), b.shape[1]), False
    if b.stride(0) == 1 and (b.stride(1) >= b.shape[0] or b.shape[1] <= 1):
        return b, max(b.stride(1), b.shape[0]), True
    b = b.contiguous()
    return b, b.shape[1], False


def row_major_copy_b8(b: torch.Tensor, ld: int) -> torch.Tensor:
    """Row-major K x N copy of a column-major 8-bit B (N columns of K bytes,
    ld apart): void_transpose_b8 where the shape allows, torch's copy
    otherwise."""
    K, N = b.shape
    out = torch.empty(K, N, dtype=b.dtype, device=b.device)
    if K % 16 == 0 and N % 16 == 0 and ld % 16 == 0 and b.data_ptr() % 16 == 0:
        st = _lib.lib().void_transpose_b8(b.data_ptr(), ld, N, K, out.data_ptr(), N,
                                          torch.cuda.current_stream(b.device).cuda_stream)
        _lib.check(st, "void_transpose_b8")
        return out
    out.copy_(b)
    return out


def launch(kind: str, dbsr: DeviceBsr, b: torch.Tensor, *, b_scale: float = 1.0,
           b_scale_vec: Optional[torch.Tensor] = None, out: torch.Tensor, epilogue: int,
           activation: int = _lib.ACT_NONE, bias: Optional[torch.Tensor] = None,
           chunk: int) -> torch.Tensor:
    """Launch one SpMM on the current stream of out's device; returns out."""
    lib = _lib.lib()
    N = b.shape[1]
    b_t, ldb, col_major = dense_operand(b)
    if col_major and kind in ("int8", "fp8") and tuning.copy_col_major_b(dbsr.n_blocks, dbsr.K):
        b_t, ldb, col_major = row_major_copy_b8(b_t, ldb), N, False  # for the LDS-DMA ring
    target = out
    if out.stride(1) != 1 or out.stride(0) < N:
        target = torch.empty(out.shape, dtype=out.dtype, device=out.device)
    plan = dbsr.plan(chunk)
    stream = torch.cuda.current_stream(out.device).cuda_stream
    ws, ws_bytes = plan.workspace(N, out.device, stream)
    cplan = plan.cplan()
    dense = _lib.DenseArgs(
        b=b_t.data_ptr(), ldb=ldb, b_col_major=int(col_major), N=N, b_scale=float(b_scale),
        b_scale_vec=b_scale_vec.data_ptr() if b_scale_vec is not None else None,
        bias=bias.data_ptr() if bias is not None else None,
        c=target.data_ptr(), ldc=target.stride(0), out_dtype=_OUT_CODES[target.dtype],
        activation=activation)
    desc = dbsr.desc()
    ws_ptr = ws.data_ptr() if ws is not None else None
    if kind == "int8":
        st = lib.void_spmm_int8(ctypes.byref(desc), ctypes.byref(dense), epilogue, ctypes.byref(cplan),
                                ws_ptr, ws_bytes, stream)
    elif kind == "fp8":
        st = lib.void_spmm_fp8(ctypes.byref(desc), ctypes.byref(dense), ctypes.byref(cplan),
                               ws_ptr, ws_bytes, stream)
    elif kind == "fp8_f32b":
        st = lib.void_spmm_fp8_f32b(ctypes.byref(desc), ctypes.byref(dense), ctypes.byref(cplan),
                                    ws_ptr, ws_bytes, stream)
    elif kind in ("fp8_bf16b", "fp8_f16b"):
        bdt = _lib.DT_BF16 if kind == "fp8_bf16b" else _lib.DT_F16
        st = lib.void_spmm_fp8_b16(ctypes.byref(desc), ctypes.byref(dense), bdt, ctypes.byref(cplan),
                                   ws_ptr, ws_bytes, stream)
    else:
        raise ValueError(f"unknown SpMM kind {kind!r}")
    _lib.check(st, f"void_spmm_{kind}")
    if target is not out:
        out.copy_(target)
    return out


def out_code(dtype: torch.dtype) -> int:
    if dtype not in _OUT_CODES:
        raise ValueError(f"unsupported output dtype {dtype}")
    return _OUT_CODES[dtype]


def device_tile_quant_ok(values: torch.Tensor) -> bool:
    """The device quantisers take contiguous fp32 [n, 32, 32] GPU tiles."""
    return (values.is_cuda and values.dtype == torch.float32 and values.dim() == 3
            and tuple(values.shape[1:]) == (32, 32) and values.is_contiguous() and values.shape[0] > 0)


def quantize_tiles_i8(values: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(codes int8 [n,32,32], scales f32 [n]) from the gfx950 per-tile INT8 quantiser."""
    n = values.shape[0]
    q = torch.empty(values.shape, dtype=torch.int8, device=values.device)
    scales = torch.empty(n, dtype=torch.float32, device=values.device)
    st = _lib.lib().void_quantize_tiles_i8(values.data_ptr(), n, q.data_ptr(), scales.data_ptr(),
                                           torch.cuda.current_stream(values.device).cuda_stream)
    _lib.check(st, "void_quantize_tiles_i8")
    return q, scales


def quantize_tiles_fp8(values: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(codes uint8 [n,32,32], scales f32 [n], amax f32 [n]) from the gfx950 per-tile E4M3 quantiser."""
    n = values.shape[0]
    q = torch.empty(values.shape, dtype=torch.uint8, device=values.device)
    scales = torch.empty(n, dtype=torch.float32, device=values.device)
    amax = torch.empty(n, dtype=torch.float32, device=values.device)
    st = _lib.lib().void_quantize_tiles_fp8(values.data_ptr(), n, q.data_ptr(), scales.data_ptr(),
                                            amax.data_ptr(), torch.cuda.current_stream(values.device).cuda_stream)
    _lib.check(st, "void_quantize_tiles_fp8")
    return q, scales, amax


def csr_to_tiles(indptr: np.ndarray, indices: np.ndarray, data: np.ndarray, shape: Tuple[int, int],
                 device: torch.device):
    """Device CSR -> VOID tiles (void_csr_count_blocks + void_csr_to_tiles).

    Returns (values f32 [n,32,32], block_rows i32, block_cols i32, morton i64)
    in Morton order, or None when the block grid is too large for the device
    conversion.  The CSR arrays must be canonical (no duplicate entries)."""
    M, N = shape
    lib = _lib.lib()
    ws_bytes = lib.void_csr_workspace_bytes(M, N)
    if ws_bytes == 0:
        return None
    stream = torch.cuda.current_stream(device).cuda_stream
    d_indptr = torch.from_numpy(np.ascontiguousarray(indptr, dtype=np.int32)).to(device)
    d_indices = torch.from_numpy(np.ascontiguousarray(indices, dtype=np.int32)).to(device)
    d_data = torch.from_numpy(np.ascontiguousarray(data, dtype=np.float32)).to(device)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    count = torch.empty(1, dtype=torch.int64, device=device)
    idx_ptr = d_indices.data_ptr() if d_indices.numel() else d_indptr.data_ptr()
    _lib.check(lib.void_csr_count_blocks(d_indptr.data_ptr(), idx_ptr, M, N, ws.data_ptr(), ws_bytes,
                                         count.data_ptr(), stream), "void_csr_count_blocks")
    n = int(count.item())
    values = torch.empty((n, 32, 32), dtype=torch.float32, device=device)
    rows = torch.empty(n, dtype=torch.int32, device=device)
    cols = torch.empty(n, dtype=torch.int32, device=device)
    morton = torch.empty(n, dtype=torch.int64, device=device)
    if n:
        _lib.check(lib.void_csr_to_tiles(d_indptr.data_ptr(), d_indices.data_ptr(), d_data.data_ptr(), M, N,
                                         ws.data_ptr(), ws_bytes, n, values.data_ptr(), rows.data_ptr(),
                                         cols.data_ptr(), morton.data_ptr(), stream), "void_csr_to_tiles")
    return values, rows, cols, morton


def sddmm_tiles(grad_c: torch.Tensor, b: torch.Tensor, block_rows: torch.Tensor, block_cols: torch.Tensor,
                shape: Tuple[int, int], out_dtype: torch.dtype, layout=None) -> torch.Tensor:
    """[n, 32, 32] gradient of the nonzero tiles: grad_c[rows of t] @ b[cols of t]^T.

    With the tiles' BsrLayout (block-row order and the Morton index of each
    position), void_sddmm_rows_f32 shares each block-row's grad_c rows among
    its tiles (void_sddmm_rows_bf16 / _f16 when grad_c and b share a 16-bit
    dtype); without it, void_sddmm_f32 takes the tiles one by one."""
    M, K = shape
    n = int(block_rows.numel())
    N = grad_c.shape[1]
    out = torch.empty((n, 32, 32), dtype=out_dtype, device=grad_c.device)
    if n == 0:
        return out
    if N == 0:
        return out.zero_()
    stream = torch.cuda.current_stream(grad_c.device).cuda_stream
    entry16 = {torch.bfloat16: "void_sddmm_rows_bf16", torch.float16: "void_sddmm_rows_f16"}.get(grad_c.dtype)
    if layout is not None and entry16 is not None and b.dtype == grad_c.dtype:
        # 16-bit operands of one dtype on the 16-bit MFMA (16-byte rows).
        g16 = grad_c if grad_c.stride(1) == 1 else grad_c.contiguous()
        b16 = b if b.stride(1) == 1 else b.contiguous()
        if (N % 8 == 0 and g16.stride(0) % 8 == 0 and b16.stride(0) % 8 == 0 and g16.data_ptr() % 16 == 0
                and b16.data_ptr() % 16 == 0 and 32 * max(g16.stride(0), b16.stride(0)) * 2 < (1 << 31)):
            groups = layout.row_groups()
            st = getattr(_lib.lib(), entry16)(g16.data_ptr(), g16.stride(0), b16.data_ptr(), b16.stride(0),
                                              groups.data_ptr(), int(groups.shape[0]), layout.col_idx.data_ptr(),
                                              layout.order.data_ptr(), M, N, K, out.data_ptr(), out_code(out_dtype),
                                              stream)
            _lib.check(st, entry16)
            return out
    g = grad_c.to(torch.float32).contiguous()
    bb = b.to(torch.float32).contiguous()
    groups = layout.row_groups() if layout is not None else None
    # Up to 1.5 row groups per CU: the per-tile kernel, whose workgroups
    # always hold 8 tiles, outweighs the shared grad_c rows (c2, 262 groups of
    # 6.3 tiles: 33.3 against 38.6 us; c3, 461 groups of 7.1: 44.9 against
    # 40.5 us).  VOID_AMD_SDDMM=grouped / tiles forces one or the other.
    force = os.environ.get("VOID_AMD_SDDMM")
    if groups is not None and (force == "tiles" or (groups.shape[0] <= tuning.GFX950_CUS * 3 // 2
                                                    and force not in ("grouped", "rows"))):
        groups = None
    if groups is not None:
        st = _lib.lib().void_sddmm_rows_f32(g.data_ptr(), g.stride(0), bb.data_ptr(), bb.stride(0), groups.data_ptr(),
                                            int(groups.shape[0]), layout.col_idx.data_ptr(), layout.order.data_ptr(),
                                            M, N, K, out.data_ptr(), out_code(out_dtype), stream)
        _lib.check(st, "void_sddmm_rows_f32")
        return out
    rows = block_rows.to(device=g.device, dtype=torch.int32).contiguous()
    cols = block_cols.to(device=g.device, dtype=torch.int32).contiguous()
    st = _lib.lib().void_sddmm_f32(g.data_ptr(), g.stride(0), bb.data_ptr(), bb.stride(0), rows.data_ptr(),
                                   cols.data_ptr(), n, M, N, K, out.data_ptr(), out_code(out_dtype), stream)
    _lib.check(st, "void_sddmm_f32")
    return out
