"""Seeded generators of the benchmark configurations (c1..c5) and small cases.

Every generator returns host numpy data; tests and bench.py move it to the
device themselves.  Tiles are produced in Morton order like csr_to_void.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np
import scipy.sparse as sp

TILE = 32


@dataclass
class BlockCase:
    name: str
    M: int
    K: int
    N: int
    tiles: np.ndarray        # float32 [nb, 32, 32], Morton order
    block_rows: np.ndarray   # int32 [nb]
    block_cols: np.ndarray   # int32 [nb]
    b: np.ndarray            # float32 [K, N]


def _morton(r, c):
    from void_amd.format import morton_encode_batch
    return morton_encode_batch(r, c)


def _sorted(tiles, br, bc):
    order = np.argsort(_morton(br, bc), kind="stable")
    return tiles[order], br[order].astype(np.int32), bc[order].astype(np.int32)


def uniform_blocks(M: int, K: int, N: int, n_active: int, seed: int = 0, name: str = "uniform") -> BlockCase:
    """n_active of the (M/32)(K/32) tiles chosen uniformly, entries N(0,1); B N(0,1)."""
    rng = np.random.default_rng(seed)
    nbr, nbc = -(-M // TILE), -(-K // TILE)
    pick = rng.choice(nbr * nbc, n_active, replace=False)
    br, bc = pick // nbc, pick % nbc
    tiles = rng.standard_normal((n_active, TILE, TILE), dtype=np.float32)
    # Zero the parts of edge tiles that lie outside the matrix.
    for t in np.nonzero((br == nbr - 1) | (bc == nbc - 1))[0]:
        rows_valid = min(TILE, M - br[t] * TILE)
        cols_valid = min(TILE, K - bc[t] * TILE)
        tiles[t, rows_valid:, :] = 0
        tiles[t, :, cols_valid:] = 0
    tiles, br, bc = _sorted(tiles, br, bc)
    b = rng.standard_normal((K, N), dtype=np.float32)
    return BlockCase(name, M, K, N, tiles, br, bc, b)


def c1_plumbing(seed: int = 0) -> tuple:
    """Config 1: sp.random(512, 512, density 0.1, random_state=0), B 512x128 N(0,1)."""
    A = sp.random(512, 512, density=0.1, format="csr", random_state=seed, dtype=np.float64)
    rng = np.random.default_rng(seed)
    B = rng.standard_normal((512, 128), dtype=np.float32)
    return A, B


def c2_int8(seed: int = 0) -> BlockCase:
    """Config 2: 4096^2, 1638 of 16384 tiles (90 % block sparsity), N=512."""
    return uniform_blocks(4096, 4096, 512, 1638, seed, "c2_int8_4096_90pct_n512")


def c3_fp8(seed: int = 0) -> BlockCase:
    """Config 3: 4096^2, 80 % block sparsity (3277 tiles), N=512."""
    return uniform_blocks(4096, 4096, 512, 3277, seed, "c3_fp8_4096_80pct_n512")


def c4_powerlaw(seed: int = 0) -> BlockCase:
    """Config 4: 16384^2, per-block-row tile count min(Zipf(1.5), 512), columns uniform; N=256."""
    rng = np.random.default_rng(seed)
    nbr = nbc = 512
    counts = np.minimum(rng.zipf(1.5, size=nbr), 512)
    br = np.repeat(np.arange(nbr), counts)
    bc = np.concatenate([rng.choice(nbc, c, replace=False) for c in counts])
    tiles = rng.standard_normal((len(br), TILE, TILE), dtype=np.float32)
    tiles, br, bc = _sorted(tiles, br, bc)
    b = rng.standard_normal((16384, 256), dtype=np.float32)
    return BlockCase("c4_powerlaw_16384_n256", 16384, 16384, 256, tiles, br, bc, b)


def c5_ffn(seed: int = 0, n_tokens: int = 2048) -> BlockCase:
    """Config 5: W 14336x4096 N(0,0.02) keeping the top 25 % of tiles by L1 norm; X 4096 x tokens N(0,1)."""
    rng = np.random.default_rng(seed)
    M, K = 14336, 4096
    nbr, nbc = M // TILE, K // TILE
    W = rng.standard_normal((M, K), dtype=np.float32) * np.float32(0.02)
    grid = W.reshape(nbr, TILE, nbc, TILE).transpose(0, 2, 1, 3)
    norms = np.abs(grid).sum(axis=(2, 3)).reshape(-1)
    keep = np.sort(np.argpartition(-norms, nbr * nbc // 4)[: nbr * nbc // 4])
    br, bc = keep // nbc, keep % nbc
    tiles = np.ascontiguousarray(grid[br, bc])
    del W, grid
    tiles, br, bc = _sorted(tiles, br, bc)
    x = rng.standard_normal((K, n_tokens), dtype=np.float32)
    return BlockCase(f"c5_ffn_14336x4096_75pct_n{n_tokens}", M, K, n_tokens, tiles, br, bc, x)


def make_void_tensor(case: BlockCase, device: str = "cpu"):
    """VOIDTensor over a BlockCase's tiles (Morton order kept)."""
    import torch
    from void_amd.format import VOIDTensor
    nbr, nbc = -(-case.M // TILE), -(-case.K // TILE)
    return VOIDTensor(
        values=torch.from_numpy(case.tiles).to(device),
        block_rows=torch.from_numpy(case.block_rows).to(device),
        block_cols=torch.from_numpy(case.block_cols).to(device),
        morton_codes=torch.from_numpy(_morton(case.block_rows, case.block_cols).astype(np.int64)).to(device),
        shape=(case.M, case.K), tile_size=(TILE, TILE),
        nnz_original=int(np.count_nonzero(case.tiles)), n_blocks=len(case.block_rows),
        density=len(case.block_rows) / (nbr * nbc))
