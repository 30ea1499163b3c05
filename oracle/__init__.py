"""CPU oracle for the quantised block-sparse SpMM path.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and
bench.py's cpu_baseline leg may import this package, and only as the
checker.  The product package (void_amd) never imports it.

Two layers, each a restatement of the reference algorithm cited per function:
* numpy (this file): tile format, Morton order, INT8 and FP8 quantisation,
  dense construction and the BSR ordering of tiles;
* C (spmm_oracle.c, built into oracle/liboracle.so): exact int32
  accumulators, the fp32 row-mean epilogue, per-block dequantisation and the
  FP8 SpMM in double, tanh-GELU.

Pinning (tests/test_oracle.py): every function here is checked against the
reference's own known answers where they exist (test_fp8.py:51-67 FP8
limits, test_fp8.py:133-150 amax) and otherwise against an independent
computation the mathematics fixes: brute-force bit interleaving (Morton),
dense round trips (format), hand-computed quantisation cases (scale, ties,
saturation, empty tile), numpy int64 dense matmul (accumulators and per-block
dequantisation), torch's float8_e4m3fn cast over all 256 codes and on random
data (FP8 decode / encode) and torch's tanh GELU (activation).  The row-mean
epilogue is pinned by a hand-computed case and by its reduction to the
per-block result when all tile scales are equal.
"""

from __future__ import annotations

import ctypes
import os
import shutil
import subprocess
from pathlib import Path
from typing import Tuple

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB = ORACLE_DIR / "liboracle.so"
SRC = ORACLE_DIR / "spmm_oracle.c"
TILE = 32

_lib = None


def build() -> Path:
    """Compile spmm_oracle.c with gcc (OpenMP when available)."""
    gcc = shutil.which("gcc") or "gcc"
    base = [gcc, "-O2", "-fPIC", "-shared", "-ffp-contract=off", str(SRC), "-o", str(LIB) + ".tmp", "-lm"]
    proc = subprocess.run(base[:5] + ["-fopenmp"] + base[5:], capture_output=True, text=True)
    if proc.returncode != 0:
        proc = subprocess.run(base, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError("oracle build failed:\n" + proc.stderr)
    os.replace(str(LIB) + ".tmp", LIB)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists() or LIB.stat().st_mtime < SRC.stat().st_mtime:
            build()
        L = ctypes.CDLL(str(LIB))
        P = ctypes.c_void_p
        i32, i64 = ctypes.c_int32, ctypes.c_int64
        L.oracle_i8_acc.restype = ctypes.c_int
        L.oracle_i8_acc.argtypes = [P, P, P, i32, i32, i32, P, i64, i32, P, i64]
        L.oracle_row_mean.restype = None
        L.oracle_row_mean.argtypes = [P, i64, P, P, i32, i32, i32, P, P, i64]
        L.oracle_i8_per_block.restype = None
        L.oracle_i8_per_block.argtypes = [P, P, P, P, i32, i32, i32, P, i64, i32, P, P, i64]
        L.oracle_fp8_spmm.restype = ctypes.c_int
        L.oracle_fp8_spmm.argtypes = [P, P, P, P, i32, i32, i32, P, i64, i32, P, P, i64]
        L.oracle_fp8_spmm_f32b.restype = ctypes.c_int
        L.oracle_fp8_spmm_f32b.argtypes = [P, P, P, P, i32, i32, i32, P, i64, i32, P, P, i64]
        L.oracle_e4m3_decode.restype = ctypes.c_double
        L.oracle_e4m3_decode.argtypes = [ctypes.c_uint8]
        L.oracle_gelu_tanh_array.restype = None
        L.oracle_gelu_tanh_array.argtypes = [P, P, i64]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- format

def morton_encode(rows: np.ndarray, cols: np.ndarray) -> np.ndarray:
    """Z-order code, row bits at even and column bits at odd positions
    (format.py:41-51), written as a per-bit interleave of 16-bit inputs."""
    r = np.asarray(rows, dtype=np.uint64) & np.uint64(0xFFFF)
    c = np.asarray(cols, dtype=np.uint64) & np.uint64(0xFFFF)
    out = np.zeros(np.broadcast(r, c).shape, dtype=np.uint64)
    for bit in range(16):
        one = np.uint64(1)
        out |= ((r >> np.uint64(bit)) & one) << np.uint64(2 * bit)
        out |= ((c >> np.uint64(bit)) & one) << np.uint64(2 * bit + 1)
    return out


def csr_tiles(dense: np.ndarray, tile: int = TILE) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Active tiles of a dense matrix whose nonzero positions are the stored entries.

    Returns (values[n,tile,tile] float32, block_rows, block_cols) in Morton
    order, as csr_to_void (format.py:287-327) produces from a CSR matrix
    without explicit zeros.
    """
    M, N = dense.shape
    nbr, nbc = -(-M // tile), -(-N // tile)
    pad = np.zeros((nbr * tile, nbc * tile), dtype=np.float32)
    pad[:M, :N] = dense
    grid = pad.reshape(nbr, tile, nbc, tile).transpose(0, 2, 1, 3)
    nz = np.zeros((nbr * tile, nbc * tile), dtype=bool)
    nz[:M, :N] = dense != 0
    active = nz.reshape(nbr, tile, nbc, tile).any(axis=(1, 3))
    br, bc = np.nonzero(active)
    order = np.argsort(morton_encode(br, bc), kind="stable")
    br, bc = br[order], bc[order]
    return grid[br, bc].copy(), br.astype(np.int32), bc.astype(np.int32)


def bsr_order(block_rows: np.ndarray, block_cols: np.ndarray, n_block_rows: int) -> Tuple[np.ndarray, np.ndarray]:
    """(order, row_ptr): tiles sorted by (row, col) and the block-row pointer
    (get_row_block_info, format.py:201-237)."""
    br = np.asarray(block_rows, dtype=np.int64)
    bc = np.asarray(block_cols, dtype=np.int64)
    order = np.lexsort((bc, br))
    row_ptr = np.zeros(n_block_rows + 1, dtype=np.int32)
    for r in br:
        row_ptr[r + 1] += 1
    return order, np.cumsum(row_ptr).astype(np.int32)


def densify(tiles: np.ndarray, block_rows, block_cols, shape: Tuple[int, int]) -> np.ndarray:
    """Dense matrix from tiles (VOIDTensor.to_dense, format.py:180-199), tile by tile."""
    M, N = shape
    tm = tiles.shape[1]
    nbr, nbc = -(-M // tm), -(-N // tm)
    out = np.zeros((nbr * tm, nbc * tm), dtype=tiles.dtype)
    for t in range(tiles.shape[0]):
        r, c = int(block_rows[t]), int(block_cols[t])
        out[r * tm:(r + 1) * tm, c * tm:(c + 1) * tm] = tiles[t]
    return out[:M, :N]


# ---------------------------------------------------------------- INT8 quantisation

def quantize_i8_blocks(values: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Symmetric per-tile INT8 (int_quant.py:178-214, 254-305, 363-369):
    s = max(max(|min|, |max|) / 128, 1e-8) in float32; q = clamp(rint(x / s), -128, 127)."""
    v = np.asarray(values, dtype=np.float32)
    flat = v.reshape(v.shape[0], -1)
    amax = np.maximum(np.abs(flat.min(axis=1)), np.abs(flat.max(axis=1))) if flat.size else np.zeros(0, np.float32)
    scale = np.maximum((amax / np.float32(128)).astype(np.float32), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.rint(v / scale[:, None, None]), -128, 127).astype(np.int8)
    return q, scale


def quantize_i8_tensor(x: np.ndarray) -> Tuple[np.ndarray, np.float32]:
    """Per-tensor symmetric INT8 of a float matrix (int_quant.py:565-573)."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.maximum(np.abs(x.min()), np.abs(x.max()))
    s = np.maximum(np.float32(amax) / np.float32(128), np.float32(1e-8)).astype(np.float32)
    return np.clip(np.rint(x / s), -128, 127).astype(np.int8), np.float32(s)


def quantize_i8_columns(x: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Per-column symmetric INT8 of a K x N matrix: the per-tensor rule applied to each column."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.maximum(np.abs(x.min(axis=0)), np.abs(x.max(axis=0)))
    s = np.maximum((amax / np.float32(128)).astype(np.float32), np.float32(1e-8)).astype(np.float32)
    return np.clip(np.rint(x / s[None, :]), -128, 127).astype(np.int8), s


# ---------------------------------------------------------------- FP8 E4M3FN

def e4m3_table() -> np.ndarray:
    """float64 value of every E4M3FN code (NaN for 0x7F / 0xFF)."""
    L = lib()
    return np.array([L.oracle_e4m3_decode(v) for v in range(256)], dtype=np.float64)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even E4M3FN encoding of float32 values already in [-448, 448]."""
    x = np.asarray(x, dtype=np.float32)
    tab = e4m3_table()[:127]  # codes 0..126: 0 .. 448, increasing
    a = np.abs(x).astype(np.float64)
    hi = np.clip(np.searchsorted(tab, a, side="left"), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    d_lo = np.abs(a - tab[lo])
    d_hi = np.abs(tab[hi] - a)
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    return code | (np.signbit(x).astype(np.uint8) << 7)


def quantize_fp8_blocks(values: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Per-tile E4M3 with the reference's first-call scaling (fp8.py:81-105, 185-229):
    amax history of zeros -> scale = max(amax / 448, 1e-12); q = e4m3(clamp(x * (1/scale), +-448))."""
    v = np.asarray(values, dtype=np.float32)
    amax = np.abs(v.reshape(v.shape[0], -1)).max(axis=1).astype(np.float32)
    scale = np.maximum((amax / np.float32(448.0)).astype(np.float32), np.float32(1e-12)).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    scaled = np.clip((v * inv[:, None, None]).astype(np.float32), -448.0, 448.0).astype(np.float32)
    return e4m3_encode(scaled), scale


def quantize_fp8_tensor(x: np.ndarray) -> Tuple[np.ndarray, np.float32]:
    """Per-tensor E4M3 (same rule, one amax)."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.float32(np.abs(x).max())
    s = np.float32(max(np.float32(amax / np.float32(448.0)), np.float32(1e-12)))
    inv = np.float32(np.float32(1.0) / s)
    return e4m3_encode(np.clip((x * inv).astype(np.float32), -448.0, 448.0)), s


# ---------------------------------------------------------------- SpMM (C)

class Bsr:
    """Tiles in block-row-major order, as spmm_oracle.c takes them."""

    def __init__(self, tiles, scales, block_rows, block_cols, shape):
        M, K = shape
        self.M, self.K = int(M), int(K)
        self.n_block_rows = -(-self.M // TILE)
        order, self.row_ptr = bsr_order(block_rows, block_cols, self.n_block_rows)
        self.tiles = np.ascontiguousarray(np.asarray(tiles)[order])
        self.scales = np.ascontiguousarray(np.asarray(scales, dtype=np.float32).reshape(-1)[order]) \
            if np.asarray(scales).size == len(order) else np.ascontiguousarray(
                np.full(len(order), np.asarray(scales, dtype=np.float32).reshape(-1)[0], dtype=np.float32))
        self.col_idx = np.ascontiguousarray(np.asarray(block_cols, dtype=np.int32)[order])


def _sb(b_scale, N: int) -> np.ndarray:
    s = np.asarray(b_scale, dtype=np.float32).reshape(-1)
    return np.ascontiguousarray(np.full(N, s[0], np.float32) if s.size == 1 else s.astype(np.float32))


def i8_acc(A: Bsr, b: np.ndarray) -> np.ndarray:
    """int32 accumulators [M, N] of the INT8 SpMM."""
    b = np.ascontiguousarray(b, dtype=np.int8)
    N = b.shape[1]
    acc = np.zeros((A.M, N), dtype=np.int32)
    if A.M and N:
        rc = lib().oracle_i8_acc(_p(A.tiles), _p(A.row_ptr), _p(A.col_idx), A.n_block_rows, A.M, A.K,
                                 _p(b), b.shape[1], N, _p(acc), N)
        if rc != 0:
            raise OverflowError("int32 accumulator overflow")
    return acc


def row_mean(A: Bsr, acc: np.ndarray, b_scale) -> np.ndarray:
    """float32 output of the reference's row-mean epilogue."""
    N = acc.shape[1]
    out = np.zeros((A.M, N), dtype=np.float32)
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    lib().oracle_row_mean(_p(acc), N, _p(A.scales), _p(A.row_ptr), A.n_block_rows, A.M, N,
                          _p(_sb(b_scale, N)), _p(out), N)
    return out


def i8_per_block(A: Bsr, b: np.ndarray, b_scale) -> np.ndarray:
    """float64 true per-tile dequantised product."""
    b = np.ascontiguousarray(b, dtype=np.int8)
    N = b.shape[1]
    out = np.zeros((A.M, N), dtype=np.float64)
    lib().oracle_i8_per_block(_p(A.tiles), _p(A.scales), _p(A.row_ptr), _p(A.col_idx), A.n_block_rows,
                              A.M, A.K, _p(b), N, N, _p(_sb(b_scale, N)), _p(out), N)
    return out


def fp8_spmm(A: Bsr, b_codes: np.ndarray, b_scale) -> np.ndarray:
    """float64 FP8 SpMM with E4M3 codes for A tiles and B."""
    b = np.ascontiguousarray(b_codes, dtype=np.uint8)
    N = b.shape[1]
    out = np.zeros((A.M, N), dtype=np.float64)
    tiles = np.ascontiguousarray(A.tiles.view(np.uint8))
    if lib().oracle_fp8_spmm(_p(tiles), _p(A.scales), _p(A.row_ptr), _p(A.col_idx), A.n_block_rows,
                             A.M, A.K, _p(b), N, N, _p(_sb(b_scale, N)), _p(out), N) != 0:
        raise MemoryError("oracle_fp8_spmm: no memory for the decoded B")
    return out


def fp8_spmm_float_b(A: Bsr, b: np.ndarray, b_scale=1.0) -> np.ndarray:
    """float64 FP8 SpMM with E4M3 codes for the A tiles and a float32 B, the
    reference's semantics for a float B (fp8.py:624-671): sum_t s_t dec(A_t) @ B."""
    b = np.ascontiguousarray(b, dtype=np.float32)
    N = b.shape[1]
    out = np.zeros((A.M, N), dtype=np.float64)
    tiles = np.ascontiguousarray(A.tiles.view(np.uint8))
    if lib().oracle_fp8_spmm_f32b(_p(tiles), _p(A.scales), _p(A.row_ptr), _p(A.col_idx), A.n_block_rows,
                                  A.M, A.K, _p(b), N, N, _p(_sb(b_scale, N)), _p(out), N) != 0:
        raise MemoryError("oracle_fp8_spmm_f32b: no memory for the B copy")
    return out


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """tanh-form GELU (fusion.py:38-43) in float64."""
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty_like(x)
    lib().oracle_gelu_tanh_array(_p(x), _p(y), x.size)
    return y


def cpu_baseline_spmm(tiles_f32, scales, col_idx, row_of_tile, b_deq, M: int):
    """Torch-CPU path on the tile format: dequantise, batched tile matmul, scatter-add rows.

    The reported CPU baseline (dequantise then matmul on the VOID tiles);
    all arguments are torch CPU tensors.
    """
    import torch
    K, N = b_deq.shape
    kb = -(-K // TILE)
    if K % TILE:
        b_deq = torch.nn.functional.pad(b_deq, (0, 0, 0, kb * TILE - K))
    out = torch.zeros(-(-M // TILE), TILE, N, dtype=torch.float32)
    step = max(1, (1 << 26) // (TILE * max(N, 1)))  # bound the gathered B panels to 256 MB
    for s in range(0, tiles_f32.shape[0], step):
        a_deq = tiles_f32[s:s + step] * scales[s:s + step, None, None]
        panels = b_deq.view(kb, TILE, N)[col_idx[s:s + step]]
        out.index_add_(0, row_of_tile[s:s + step], torch.bmm(a_deq, panels))
    return out.view(-1, N)[:M]
