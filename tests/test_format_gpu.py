"""Device-side csr_to_void (void_csr_count_blocks / void_csr_to_tiles)
against the host conversion, field by field and bit for bit."""

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import cases
import oracle
import void_amd

pytestmark = pytest.mark.gpu


def _same(dev_vt, host_vt):
    assert dev_vt.values.is_cuda
    assert dev_vt.n_blocks == host_vt.n_blocks and dev_vt.nnz_original == host_vt.nnz_original
    assert dev_vt.shape == host_vt.shape and dev_vt.density == host_vt.density
    for name in ("values", "block_rows", "block_cols", "morton_codes"):
        a, b = getattr(dev_vt, name).cpu(), getattr(host_vt, name)
        assert a.dtype == b.dtype, name
        assert torch.equal(a, b), name


# Morton code spaces up to 32768 codes rank in one workgroup; larger ones
# count per chunk of 4096 codes and rank with the chunks' offsets, summed in
# each workgroup up to 256 chunks (65536 and 2^20 codes here) and by a
# separate scan beyond (2^22 codes, the last shape).
@pytest.mark.parametrize("M,N,density,seed", [(300, 200, 0.05, 1), (2000, 70, 0.02, 2), (70, 3000, 0.02, 3),
                                              (4096, 4096, 0.002, 4), (33, 33, 0.5, 5), (1, 1000, 0.1, 6),
                                              (8192, 6000, 0.0005, 7), (20000, 64, 0.01, 8), (33000, 40, 0.001, 9)])
def test_device_csr_to_void_matches_host(gpu, M, N, density, seed):
    A = sp.random(M, N, density=density, format="csr", random_state=seed, dtype=np.float64)
    A.sort_indices()
    _same(void_amd.csr_to_void(A, device="cuda"), void_amd.csr_to_void(A))


def test_device_csr_dense_blocks(gpu):
    # Fully dense tiles: every aligned run of four columns is one 16-byte store.
    case = cases.uniform_blocks(2048, 3072, 64, 400, seed=9)
    A = sp.csr_matrix(oracle.densify(case.tiles, case.block_rows, case.block_cols, (case.M, case.K)))
    A.sort_indices()
    _same(void_amd.csr_to_void(A, device="cuda"), void_amd.csr_to_void(A))


def test_device_csr_c1_and_explicit_zeros(gpu):
    A, _ = cases.c1_plumbing()
    _same(void_amd.csr_to_void(A, device="cuda"), void_amd.csr_to_void(A))
    # Explicit zeros activate their tiles (format.py:321-327 stores them).
    z = sp.csr_matrix((np.array([0.0, 2.0, 0.0]), (np.array([5, 40, 99]), np.array([7, 70, 1]))), shape=(100, 100))
    dev = void_amd.csr_to_void(z, device="cuda")
    _same(dev, void_amd.csr_to_void(z))
    assert dev.n_blocks == 3


def test_device_csr_empty_and_duplicates(gpu):
    e = sp.csr_matrix((100, 64), dtype=np.float32)
    dev = void_amd.csr_to_void(e, device="cuda")
    assert dev.n_blocks == 0 and dev.values.shape == (0, 32, 32)
    # Duplicate entries (non-canonical CSR) keep the host rule: the last one wins.
    d = sp.csr_matrix((np.array([1.0, 5.0, 3.0]), np.array([4, 4, 9]), np.array([0, 3, 3])), shape=(2, 40))
    assert not d.has_canonical_format
    vt = void_amd.csr_to_void(d, device="cuda")
    assert vt.values.is_cuda and vt.to_dense()[0, 4].item() == 5.0


def test_device_format_feeds_the_spmm(gpu):
    case = cases.c2_int8()
    dense = np.zeros((case.M, case.K), np.float32)
    for t in range(len(case.block_rows)):
        r, c = case.block_rows[t] * 32, case.block_cols[t] * 32
        dense[r:r + 32, c:c + 32] = case.tiles[t]
    A = sp.csr_matrix(dense)
    vt_dev = void_amd.csr_to_void(A, device="cuda")
    q_dev = void_amd.quantize_void_tensor(vt_dev)
    q_host = void_amd.quantize_void_tensor(void_amd.csr_to_void(A))
    assert torch.equal(q_dev.values.cpu(), q_host.values) and torch.equal(q_dev.scales.cpu(), q_host.scales)


@pytest.mark.parametrize("M,K", [(1024, 2048), (1000, 1000)])
def test_device_csr_full_blocks_and_holes(gpu, M, K):
    """Dense blocks, and blocks with one element or one row missing or cut
    by the matrix edge: every element the CSR does not store comes out
    zero, even when the tile memory held NaNs before the conversion."""
    case = cases.uniform_blocks(M, K, 32, 160, seed=17)
    dense = oracle.densify(case.tiles, case.block_rows, case.block_cols, (M, K))
    rng = np.random.default_rng(5)
    nbr, nbc = -(-M // 32), -(-K // 32)
    for t in rng.choice(len(case.block_rows), 40, replace=False):
        r0, c0 = case.block_rows[t] * 32, case.block_cols[t] * 32
        kind = t % 4
        if kind == 0:
            dense[r0 + rng.integers(0, min(32, M - r0)), c0] = 0.0            # first column of a segment
        elif kind == 1:
            dense[r0 + rng.integers(0, min(32, M - r0)), min(c0 + 31, K - 1)] = 0.0  # last column
        elif kind == 2:
            dense[r0 + rng.integers(0, min(32, M - r0)), c0 + rng.integers(1, min(31, K - c0))] = 0.0
        else:
            dense[r0 + rng.integers(0, min(32, M - r0)), c0:c0 + 32] = 0.0   # a whole row of the block
    A = sp.csr_matrix(dense)
    A.sort_indices()
    host = void_amd.csr_to_void(A)
    # Leave NaNs in freed memory of the tile array's size for the caching
    # allocator to hand back to the conversion.
    junk = torch.full((host.n_blocks, 32, 32), float("nan"), device=gpu)
    del junk
    _same(void_amd.csr_to_void(A, device="cuda"), host)
