"""VOID tile format (void_amd.format) against the oracle and the reference's
format edge cases (test_advanced_features.py:837-962)."""

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import oracle
import void_amd
from void_amd.format import build_bsr_layout


def _dense(m):
    return np.asarray(m.todense(), dtype=np.float32)


def test_csr_to_void_matches_oracle_tiles():
    A = sp.random(300, 200, density=0.05, format="csr", random_state=3, dtype=np.float64)
    vt = void_amd.csr_to_void(A)
    tiles, br, bc = oracle.csr_tiles(_dense(A))
    assert vt.n_blocks == len(tiles)
    assert np.array_equal(vt.block_rows.numpy(), br) and np.array_equal(vt.block_cols.numpy(), bc)
    assert np.array_equal(vt.values.numpy(), tiles)
    assert np.array_equal(vt.morton_codes.numpy(), oracle.morton_encode(br, bc).astype(np.int64))
    assert np.array_equal(vt.to_dense().numpy(), _dense(A))


def test_morton_product_matches_oracle():
    r, c = np.meshgrid(np.arange(200), np.arange(150), indexing="ij")
    assert np.array_equal(void_amd.morton_encode_batch(r.ravel(), c.ravel()),
                          oracle.morton_encode(r.ravel(), c.ravel()))
    assert void_amd.morton_decode(void_amd.morton_encode(123, 45)) == (123, 45)


def test_c1_block_count():
    # sp.random(512, 512, density 0.1, random_state=0) activates every 32x32 tile
    A = sp.random(512, 512, density=0.1, format="csr", random_state=0)
    vt = void_amd.csr_to_void(A)
    assert vt.n_blocks == 256 and vt.nnz_original == A.nnz


def test_explicit_zero_activates_tile():
    A = sp.csr_matrix((np.array([0.0]), (np.array([40]), np.array([70]))), shape=(64, 96))
    vt = void_amd.csr_to_void(A)
    assert vt.n_blocks == 1 and (vt.block_rows[0].item(), vt.block_cols[0].item()) == (1, 2)


def test_empty_matrix():
    vt = void_amd.csr_to_void(sp.csr_matrix((100, 100), dtype=np.float32), tile_size=16, warn_small_tiles=False)
    assert vt.n_blocks == 0 and vt.nnz_original == 0 and vt.shape == (100, 100)


def test_single_block_tile16():
    m = sp.lil_matrix((64, 64), dtype=np.float32)
    m[0:16, 0:16] = 1.0
    vt = void_amd.csr_to_void(m.tocsr(), tile_size=16)
    assert vt.n_blocks == 1 and vt.shape == (64, 64)


def test_tile64_and_small_matrix():
    np.random.seed(42)
    vt = void_amd.csr_to_void(sp.random(512, 512, density=0.1, format="csr", dtype=np.float32), tile_size=64)
    assert vt.tile_size == (64, 64)
    vt = void_amd.csr_to_void(sp.random(16, 16, density=0.3, format="csr", dtype=np.float32))
    assert vt.padded_shape == (32, 32) and vt.n_blocks <= 1


@pytest.mark.parametrize("M,N", [(512, 128), (128, 512), (333, 555)])
def test_rectangular_shapes(M, N):
    np.random.seed(42)
    A = sp.random(M, N, density=0.1, format="csr", dtype=np.float32)
    vt = void_amd.csr_to_void(A)
    assert vt.shape == (M, N)
    assert vt.padded_shape[0] % 32 == 0 and vt.padded_shape[1] % 32 == 0
    assert np.array_equal(vt.to_dense().numpy(), _dense(A))


def test_extremely_sparse_and_dense():
    np.random.seed(42)
    vt = void_amd.csr_to_void(sp.random(1024, 1024, density=0.0005, format="csr", dtype=np.float32))
    assert vt.block_sparsity > 0.5 and vt.overhead_ratio >= 1.0
    vt = void_amd.csr_to_void(sp.random(256, 256, density=0.8, format="csr", dtype=np.float32))
    assert vt.block_sparsity < 0.5 and vt.overhead_ratio < 2.0


def test_get_row_block_info():
    A = sp.random(200, 300, density=0.05, format="csr", random_state=1)
    vt = void_amd.csr_to_void(A)
    row_ptr, idx = vt.get_row_block_info()
    br, bc = vt.block_rows.numpy(), vt.block_cols.numpy()
    order, rp = oracle.bsr_order(br, bc, vt.block_grid[0])
    assert np.array_equal(row_ptr.numpy(), rp) and np.array_equal(idx.numpy(), order)


def test_bsr_layout_matches_oracle():
    A = sp.random(256, 512, density=0.03, format="csr", random_state=2)
    vt = void_amd.csr_to_void(A)
    lay = build_bsr_layout(vt.block_rows, vt.block_cols, 8, 16, torch.device("cpu"))
    order, rp = oracle.bsr_order(vt.block_rows.numpy(), vt.block_cols.numpy(), 8)
    assert np.array_equal(lay.order.numpy(), order) and np.array_equal(lay.row_ptr_host, rp)
    assert np.array_equal(lay.col_idx.numpy(), vt.block_cols.numpy()[order])


def test_dense_to_void_threshold_and_roundtrip():
    rng = np.random.default_rng(0)
    d = np.where(rng.random((100, 70)) < 0.05, rng.standard_normal((100, 70)), 0).astype(np.float32)
    vt = void_amd.dense_to_void(torch.from_numpy(d))
    tiles, br, bc = oracle.csr_tiles(d)
    assert vt.n_blocks == len(tiles) and np.array_equal(vt.to_dense().numpy(), d)
    assert np.array_equal(vt.block_rows.numpy(), br)
    assert void_amd.dense_to_void(torch.zeros(40, 40)).n_blocks == 0
    csr = void_amd.void_to_csr(vt)
    assert np.array_equal(csr.toarray(), d)


def test_dtype_conversions():
    vt = void_amd.csr_to_void(sp.random(64, 64, density=0.2, format="csr", random_state=4))
    assert vt.half().values.dtype == torch.float16 and vt.bfloat16().dtype == torch.bfloat16
    assert vt.float().values.dtype == torch.float32


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_bsr_layout_row_groups(seed):
    """Work list of the row-grouped SDDMM: every block-row's tiles in runs of
    at most 8 consecutive BSR positions, in order, covering each tile once."""
    rng = np.random.default_rng(seed)
    n_br, n_bc = 40, 64
    counts = rng.integers(0, 30, size=n_br)
    counts[rng.integers(0, n_br, size=5)] = 0  # empty rows
    rows = np.repeat(np.arange(n_br), counts)
    cols = np.concatenate([np.sort(rng.choice(n_bc, c, replace=False)) for c in counts])
    lay = build_bsr_layout(torch.from_numpy(rows.astype(np.int32)), torch.from_numpy(cols.astype(np.int32)),
                           n_br, n_bc, torch.device("cpu"))
    got = lay.row_groups().numpy()
    want = []
    rp = lay.row_ptr_host
    for r in range(n_br):
        for s in range(rp[r], rp[r + 1], 8):
            want.append((r, s, min(8, rp[r + 1] - s)))
    assert got.dtype == np.int32 and got.shape == (len(want), 3)
    assert [tuple(x) for x in got.tolist()] == want
    assert got[:, 2].sum() == len(rows) and got[:, 2].max() <= 8
