"""VOID tile format: 32x32 dense tiles of a block-sparse matrix.

Mirrors ``void/format.py`` of the reference (same names, fields and
semantics) and adds the device layout the gfx950 kernels read:
``bsr_layout`` gathers the Morton-ordered tiles once into block-row-major
order (rows ascending, columns ascending within a row), so that a workgroup
streams a block-row's tiles from contiguous memory without the
``block_indices`` indirection of the reference kernels.
"""

from __future__ import annotations

import warnings
from dataclasses import dataclass, field
from typing import Optional, Tuple, Union

import numpy as np
import torch
from scipy import sparse

# format.py:12 — tile sizes below 16 were rejected by the reference's tensor-core path.
MIN_TENSOR_CORE_TILE = 16


def _spread_bits(v: np.ndarray) -> np.ndarray:
    v = v.astype(np.uint64)
    v = (v | (v << np.uint64(8))) & np.uint64(0x00FF00FF)
    v = (v | (v << np.uint64(4))) & np.uint64(0x0F0F0F0F)
    v = (v | (v << np.uint64(2))) & np.uint64(0x33333333)
    v = (v | (v << np.uint64(1))) & np.uint64(0x55555555)
    return v


def _compact_bits(v: np.ndarray) -> np.ndarray:
    v = v.astype(np.uint64) & np.uint64(0x55555555)
    v = (v | (v >> np.uint64(1))) & np.uint64(0x33333333)
    v = (v | (v >> np.uint64(2))) & np.uint64(0x0F0F0F0F)
    v = (v | (v >> np.uint64(4))) & np.uint64(0x00FF00FF)
    v = (v | (v >> np.uint64(8))) & np.uint64(0x0000FFFF)
    return v


def morton_encode(x: int, y: int) -> int:
    """Z-order code of (x, y): x bits at even, y bits at odd positions (format.py:15-25)."""
    return int(morton_encode_batch(np.array([x]), np.array([y]))[0])


def morton_decode(code: int) -> Tuple[int, int]:
    """Inverse of morton_encode for 16-bit coordinates (format.py:28-38)."""
    c = np.array([code], dtype=np.uint64)
    return int(_compact_bits(c)[0]), int(_compact_bits(c >> np.uint64(1))[0])


def morton_encode_batch(rows: np.ndarray, cols: np.ndarray) -> np.ndarray:
    """Vectorised Morton code, rows in even bits, cols in odd bits; 16-bit inputs (format.py:41-51)."""
    return _spread_bits(np.asarray(rows)) | (_spread_bits(np.asarray(cols)) << np.uint64(1))


@dataclass
class BsrLayout:
    """Device arrays of the block-row-major tile order (one per device)."""

    order: torch.Tensor     # int64 [n_blocks]: Morton index of each BSR position
    row_ptr: torch.Tensor   # int32 [n_block_rows + 1] on device
    col_idx: torch.Tensor   # int32 [n_blocks] on device
    row_ptr_host: np.ndarray  # int32 copy on the host, for the planner
    sddmm_groups: Optional[torch.Tensor] = None  # int32 [n_groups, 3], built on first use

    def row_groups(self) -> torch.Tensor:
        """(block row, first BSR position, count <= 8) per group of a row's tiles,
        the work list of void_sddmm_rows_f32."""
        if self.sddmm_groups is None:
            rp = self.row_ptr_host.astype(np.int64)
            counts = np.diff(rp)
            ng = (counts + 7) // 8
            rows = np.repeat(np.arange(len(counts)), ng)
            k = np.arange(int(ng.sum())) - np.repeat(np.cumsum(ng) - ng, ng)
            start = rp[rows] + 8 * k
            cnt = np.minimum(8, rp[rows + 1] - start)
            arr = np.stack([rows, start, cnt], axis=1).astype(np.int32).reshape(-1, 3)
            self.sddmm_groups = torch.from_numpy(arr).to(self.row_ptr.device)
        return self.sddmm_groups


def build_bsr_layout(block_rows: torch.Tensor, block_cols: torch.Tensor, n_block_rows: int,
                     n_block_cols: int, device: torch.device) -> BsrLayout:
    """Row pointer and BSR order of a tile set.

    Same ordering as get_row_block_info (format.py:201-237): tiles sorted by
    (block_row, block_col); row_ptr is the cumulative per-row tile count.
    """
    r = block_rows.detach().to("cpu", torch.int64).numpy()
    c = block_cols.detach().to("cpu", torch.int64).numpy()
    order = np.argsort(r * n_block_cols + c, kind="stable")
    counts = np.bincount(r, minlength=n_block_rows) if r.size else np.zeros(n_block_rows, np.int64)
    row_ptr = np.zeros(n_block_rows + 1, dtype=np.int32)
    np.cumsum(counts, out=row_ptr[1:])
    col_idx = c[order].astype(np.int32)
    return BsrLayout(
        order=torch.from_numpy(order).to(device),
        row_ptr=torch.from_numpy(row_ptr).to(device),
        col_idx=torch.from_numpy(col_idx).to(device),
        row_ptr_host=row_ptr,
    )


@dataclass
class VOIDTensor:
    """Block-sparse matrix as dense tiles (format.py:54-245).

    values: [n_blocks, tile_m, tile_n]; block_rows/block_cols: int32 [n_blocks];
    morton_codes: int64 [n_blocks]; tiles are Morton-ordered.
    """

    values: torch.Tensor
    block_rows: torch.Tensor
    block_cols: torch.Tensor
    morton_codes: torch.Tensor
    shape: Tuple[int, int]
    tile_size: Tuple[int, int]
    nnz_original: int
    n_blocks: int
    density: float
    dtype: torch.dtype = torch.float32
    _device_bsr: dict = field(default_factory=dict, repr=False, compare=False)
    # Block-row order of the tiles (a BsrLayout), when a caller already has it.
    _bsr_layout: object = field(default=None, repr=False, compare=False)

    def device_bsr(self, dtype: torch.dtype = torch.float32):
        """Block-row-major device copy of the tiles in ``dtype`` (fp32 for the
        fp32 kernel, bf16 / fp16 for the 16-bit one), built once per device
        and dtype and gathered again when the values change in place, since
        the reference reads them on every call."""
        from . import _runtime
        key = str(self.values.device) if dtype == torch.float32 else f"{self.values.device}/{dtype}"
        src = _runtime.source_key(self.values)
        d = self._device_bsr.get(key)
        if d is None:
            ones = torch.ones(1, dtype=torch.float32, device=self.values.device)
            d = _runtime.make_device_bsr(self.values.detach().to(dtype).contiguous(), ones, self.block_rows,
                                         self.block_cols, self.shape, self.tile_size, self.values.device, True,
                                         layout=self._bsr_layout)
            d.src_key = src
            self._device_bsr[key] = d
        elif d.src_key != src:
            d.refresh(self.values.detach().to(dtype).contiguous(), d.scales)
            d.src_key = src
        return d

    @property
    def padded_shape(self) -> Tuple[int, int]:
        tm, tn = self.tile_size
        return (((self.shape[0] + tm - 1) // tm) * tm, ((self.shape[1] + tn - 1) // tn) * tn)

    @property
    def block_grid(self) -> Tuple[int, int]:
        tm, tn = self.tile_size
        return ((self.shape[0] + tm - 1) // tm, (self.shape[1] + tn - 1) // tn)

    @property
    def sparsity(self) -> float:
        return 1.0 - self.nnz_original / (self.shape[0] * self.shape[1])

    @property
    def block_sparsity(self) -> float:
        return 1.0 - self.n_blocks / (self.block_grid[0] * self.block_grid[1])

    @property
    def overhead_ratio(self) -> float:
        return self.n_blocks * self.tile_size[0] * self.tile_size[1] / max(self.nnz_original, 1)

    def _replace(self, **kw) -> "VOIDTensor":
        fields = dict(values=self.values, block_rows=self.block_rows, block_cols=self.block_cols,
                      morton_codes=self.morton_codes, shape=self.shape, tile_size=self.tile_size,
                      nnz_original=self.nnz_original, n_blocks=self.n_blocks, density=self.density,
                      dtype=self.dtype)
        fields.update(kw)
        return VOIDTensor(**fields)

    def to(self, device: Union[str, torch.device]) -> "VOIDTensor":
        return self._replace(values=self.values.to(device), block_rows=self.block_rows.to(device),
                             block_cols=self.block_cols.to(device),
                             morton_codes=self.morton_codes.to(device))

    def cuda(self) -> "VOIDTensor":
        return self.to("cuda")

    def cpu(self) -> "VOIDTensor":
        return self.to("cpu")

    def to_dtype(self, dtype: torch.dtype) -> "VOIDTensor":
        return self._replace(values=self.values.to(dtype), dtype=dtype)

    def half(self) -> "VOIDTensor":
        return self.to_dtype(torch.float16)

    def bfloat16(self) -> "VOIDTensor":
        return self.to_dtype(torch.bfloat16)

    def float(self) -> "VOIDTensor":
        return self.to_dtype(torch.float32)

    def to_fp8(self, format: str = "e4m3", scale_mode: str = "per_block"):
        from .fp8 import void_tensor_to_fp8
        return void_tensor_to_fp8(self, format=format, scale_mode=scale_mode)

    def to_dense(self) -> torch.Tensor:
        """Dense [M, N] matrix (format.py:180-199), one scatter instead of a per-tile loop."""
        tm, tn = self.tile_size
        n_br, n_bc = self.block_grid
        grid = torch.zeros(n_br * n_bc, tm, tn, dtype=self.values.dtype, device=self.values.device)
        if self.n_blocks:
            key = self.block_rows.long() * n_bc + self.block_cols.long()
            grid[key.to(grid.device)] = self.values
        dense = grid.view(n_br, n_bc, tm, tn).permute(0, 2, 1, 3).reshape(n_br * tm, n_bc * tn)
        return dense[: self.shape[0], : self.shape[1]]

    def get_row_block_info(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """(row_ptr, block_indices) with block_indices = argsort(row * n_bc + col) (format.py:201-237)."""
        cache = getattr(self, "_row_info_cache", None)
        if cache is not None and cache[0].device == self.block_rows.device:
            return cache
        n_br, n_bc = self.block_grid
        dev = self.block_rows.device
        counts = torch.zeros(n_br, dtype=torch.int32, device=dev)
        counts.scatter_add_(0, self.block_rows.long(), torch.ones_like(self.block_rows))
        row_ptr = torch.zeros(n_br + 1, dtype=torch.int32, device=dev)
        row_ptr[1:] = torch.cumsum(counts, dim=0)
        keys = self.block_rows.long() * n_bc + self.block_cols.long()
        block_indices = torch.argsort(keys, stable=True).to(torch.int32)
        self._row_info_cache = (row_ptr, block_indices)
        return self._row_info_cache

    def __repr__(self) -> str:
        return (f"VOIDTensor(shape={self.shape}, tile_size={self.tile_size}, n_blocks={self.n_blocks}, "
                f"sparsity={self.sparsity:.1%}, block_sparsity={self.block_sparsity:.1%}, "
                f"overhead={self.overhead_ratio:.2f}x, dtype={self.dtype})")


def csr_to_void(
    matrix: Union[sparse.csr_matrix, "sparse.csr_array"],
    tile_size: int = 32,
    dtype: torch.dtype = torch.float32,
    device: str = "cpu",
    warn_small_tiles: bool = True,
) -> VOIDTensor:
    """CSR -> VOID tiles (format.py:248-349).

    Same result as the reference, whose per-nonzero Python loop
    (format.py:321-327) becomes one vectorised scatter.  Explicit zeros
    still activate their tile; values are cast to float32 first.
    """
    if warn_small_tiles and tile_size < MIN_TENSOR_CORE_TILE:
        warnings.warn(f"tile_size={tile_size} < {MIN_TENSOR_CORE_TILE}, Tensor Cores require K >= 16",
                      UserWarning)
    if not sparse.isspmatrix_csr(matrix):
        matrix = sparse.csr_matrix(matrix)
    M, N = matrix.shape
    nnz = matrix.nnz
    n_br = (M + tile_size - 1) // tile_size
    n_bc = (N + tile_size - 1) // tile_size

    dev = torch.device(device)
    if (dev.type == "cuda" and tile_size == 32 and matrix.has_canonical_format and nnz < 2 ** 31
            and M < 2 ** 31 and N < 2 ** 31):
        # Device conversion (void_csr_count_blocks / void_csr_to_tiles): same
        # tiles, order and metadata.  Inputs with duplicate entries stay on
        # the host path below, whose "last entry wins" rule needs the
        # sequential order.
        from . import _runtime
        built = _runtime.csr_to_tiles(matrix.indptr, matrix.indices, matrix.data.astype(np.float32),
                                      (M, N), dev)
        if built is not None:
            values, rows, cols, morton = built
            return VOIDTensor(values=values if dtype == torch.float32 else values.to(dtype), block_rows=rows,
                              block_cols=cols, morton_codes=morton, shape=(M, N), tile_size=(32, 32),
                              nnz_original=nnz, n_blocks=int(values.shape[0]),
                              density=values.shape[0] / (n_br * n_bc) if n_br * n_bc else 0.0, dtype=dtype)

    coo = matrix.tocoo()
    rows = np.asarray(coo.row, dtype=np.int64)
    cols = np.asarray(coo.col, dtype=np.int64)
    data = np.asarray(coo.data)
    keys = (rows // tile_size) * n_bc + (cols // tile_size)
    unique_blocks, inverse = np.unique(keys, return_inverse=True)
    n_blocks = len(unique_blocks)
    act_rows = unique_blocks // n_bc
    act_cols = unique_blocks % n_bc
    morton = morton_encode_batch(act_rows, act_cols)
    order = np.argsort(morton)
    reverse = np.empty(n_blocks, dtype=np.int64)
    reverse[order] = np.arange(n_blocks)

    values = np.zeros((n_blocks, tile_size, tile_size), dtype=np.float32)
    if nnz:
        # A later duplicate of the same position overwrites an earlier one, as
        # the reference's sequential loop does.
        values[reverse[inverse.reshape(-1)], rows % tile_size, cols % tile_size] = data.astype(np.float32)

    vt = torch.from_numpy(values).to(device)
    if dtype != torch.float32:
        vt = vt.to(dtype)
    return VOIDTensor(
        values=vt,
        block_rows=torch.from_numpy(act_rows[order].astype(np.int32)).to(device),
        block_cols=torch.from_numpy(act_cols[order].astype(np.int32)).to(device),
        morton_codes=torch.from_numpy(morton[order].astype(np.int64)).to(device),
        shape=(M, N),
        tile_size=(tile_size, tile_size),
        nnz_original=nnz,
        n_blocks=n_blocks,
        density=n_blocks / (n_br * n_bc) if n_br * n_bc else 0.0,
        dtype=dtype,
    )


def dense_to_void(matrix: torch.Tensor, tile_size: int = 32, threshold: float = 0.0) -> VOIDTensor:
    """Dense -> VOID keeping tiles whose L1 norm exceeds threshold (format.py:352-446)."""
    assert matrix.dim() == 2, "Input must be 2D tensor"
    M, N = matrix.shape
    device, dtype = matrix.device, matrix.dtype
    pad_m = (tile_size - M % tile_size) % tile_size
    pad_n = (tile_size - N % tile_size) % tile_size
    if pad_m or pad_n:
        matrix = torch.nn.functional.pad(matrix, (0, pad_n, 0, pad_m))
    n_br, n_bc = matrix.shape[0] // tile_size, matrix.shape[1] // tile_size
    tiles = matrix.reshape(n_br, tile_size, n_bc, tile_size).permute(0, 2, 1, 3)
    active = (tiles.abs().sum(dim=(2, 3)) > threshold).nonzero(as_tuple=False)
    nnz = int((matrix[:M, :N] != 0).sum().item())
    if len(active) == 0:
        return VOIDTensor(
            values=torch.empty((0, tile_size, tile_size), dtype=dtype, device=device),
            block_rows=torch.empty(0, dtype=torch.int32, device=device),
            block_cols=torch.empty(0, dtype=torch.int32, device=device),
            morton_codes=torch.empty(0, dtype=torch.int64, device=device),
            shape=(M, N), tile_size=(tile_size, tile_size), nnz_original=nnz, n_blocks=0,
            density=0.0, dtype=dtype)
    br, bc = active[:, 0], active[:, 1]
    morton = morton_encode_batch(br.cpu().numpy(), bc.cpu().numpy())
    order = np.argsort(morton)
    order_t = torch.from_numpy(order).to(device)
    sbr = br[order_t].to(torch.int32)
    sbc = bc[order_t].to(torch.int32)
    return VOIDTensor(
        values=tiles[sbr.long(), sbc.long()],
        block_rows=sbr,
        block_cols=sbc,
        morton_codes=torch.from_numpy(morton[order].astype(np.int64)).to(device),
        shape=(M, N), tile_size=(tile_size, tile_size), nnz_original=nnz, n_blocks=len(active),
        density=len(active) / (n_br * n_bc), dtype=dtype)


def void_to_csr(void_tensor: VOIDTensor) -> sparse.csr_matrix:
    """VOID -> scipy CSR through the dense matrix (format.py:449-452)."""
    return sparse.csr_matrix(void_tensor.to_dense().cpu().numpy())


__all__ = [
    "MIN_TENSOR_CORE_TILE", "VOIDTensor", "BsrLayout", "build_bsr_layout", "csr_to_void",
    "dense_to_void", "void_to_csr", "morton_encode", "morton_decode", "morton_encode_batch",
]
