"""void_spmm_stream_k (stream_k.py:233-301) on the fp32 MFMA kernel, with
the workload's worker ranges run exactly as given.

Bar: a float64 dense product of the same tiles within the recursive fp32
summation bound (n - 1) u sum |a b|, u = 2^-24, n = 32 products per tile of
the longest row; split rows add their partial blocks in worker order, one
more fp32 add per worker.  The reference's own tests
(test_advanced_features.py:757-835) are mirrored with their inputs and
tolerance as well."""

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import cases
import oracle
import void_amd
from void_amd import compute_stream_k_workload, void_spmm_stream_k

pytestmark = pytest.mark.gpu
U = 2.0 ** -24


def _dense_of(vt):
    return oracle.densify(vt.values.float().cpu().numpy(), vt.block_rows.cpu().numpy(), vt.block_cols.cpu().numpy(),
                          vt.shape).astype(np.float64)


def _check(vt, B, out, workers_per_row=1):
    ref = _dense_of(vt) @ B.astype(np.float64)
    n_row = np.bincount(vt.block_rows.cpu().numpy(), minlength=vt.block_grid[0]).max()
    bound = (32 * int(n_row) + workers_per_row) * U * (np.abs(_dense_of(vt)) @ np.abs(B.astype(np.float64)))
    err = np.abs(out.float().cpu().numpy().astype(np.float64) - ref)
    assert np.all(err <= bound + 1e-30), (err / (bound + 1e-30)).max()


def test_reference_stream_k_correctness(gpu):
    """test_advanced_features.py:757-776: 256^2 at density 0.2, N = 64,
    max relative error 1e-3 against the dense product."""
    np.random.seed(42)
    sparse_np = sp.random(256, 256, density=0.2, format="csr", dtype=np.float32)
    vt = void_amd.csr_to_void(sparse_np, tile_size=32).cuda()
    torch.manual_seed(0)
    B = torch.randn(256, 64, device=gpu, dtype=torch.float32)
    C = void_spmm_stream_k(vt, B)
    C_ref = torch.tensor(sparse_np.toarray(), device=gpu) @ B
    assert (C - C_ref).abs().max().item() / C_ref.abs().max().item() < 1e-3
    _check(vt, B.cpu().numpy(), C)


def test_reference_stream_k_precomputed_workload(gpu):
    """test_advanced_features.py:809-835: one workload (n_workers = 64) for
    two B matrices; here also checked for values."""
    np.random.seed(42)
    sparse_np = sp.random(256, 256, density=0.2, format="csr", dtype=np.float32)
    vt = void_amd.csr_to_void(sparse_np, tile_size=32).cuda()
    workload = compute_stream_k_workload(vt, n_workers=64)
    torch.manual_seed(1)
    B1 = torch.randn(256, 64, device=gpu)
    B2 = torch.randn(256, 64, device=gpu)
    C1 = void_spmm_stream_k(vt, B1, workload=workload)
    C2 = void_spmm_stream_k(vt, B2, workload=workload)
    assert C1.shape == (256, 64) and C2.shape == (256, 64)
    _check(vt, B1.cpu().numpy(), C1, workers_per_row=8)
    _check(vt, B2.cpu().numpy(), C2, workers_per_row=8)


@pytest.mark.parametrize("max_work", [4, 16, 100])
def test_zipf_rows_split_workloads(gpu, max_work):
    """Power-law rows (Zipf 1.5, up to 300 tiles) with workloads that cut
    them into chunks of at most max_work tiles (beyond 64 the kernel cuts
    further): split rows everywhere, results deterministic."""
    rng = np.random.default_rng(5)
    nbr = 128
    counts = np.minimum(rng.zipf(1.5, nbr), 300)
    br = np.repeat(np.arange(nbr), counts)
    bc = np.concatenate([rng.choice(320, c, replace=False) for c in counts])
    tiles = rng.standard_normal((len(br), 32, 32)).astype(np.float32)
    case = cases.BlockCase("zipf", nbr * 32, 320 * 32, 96, *cases._sorted(tiles, br, bc),
                           rng.standard_normal((320 * 32, 96)).astype(np.float32))
    vt = cases.make_void_tensor(case, "cpu").to(gpu)
    w = compute_stream_k_workload(vt, max_work_per_worker=max_work)
    assert bool(w.worker_needs_atomic.any())
    B = torch.from_numpy(case.b).to(gpu)
    out = torch.full((case.M, case.N), float("nan"), device=gpu)
    void_spmm_stream_k(vt, B, workload=w, out=out)
    again = void_spmm_stream_k(vt, B, workload=w)
    assert torch.equal(out.view(torch.int32), again.view(torch.int32))
    _check(vt, case.b, out, workers_per_row=-(-300 // min(max_work, 64)))


def test_stream_k_bf16_and_empty_rows(gpu):
    """B in bf16 gives a bf16 C (the reference writes B's dtype); rows with
    no tiles and rows left out of the workload come out zero."""
    case = cases.uniform_blocks(512, 512, 64, 30, seed=8)
    vt = cases.make_void_tensor(case, "cpu").to(gpu)
    w = compute_stream_k_workload(vt, n_workers=16)
    keep = w.worker_rows != int(w.worker_rows[0])
    dropped = int(w.worker_rows[0])
    from void_amd.stream_k import StreamKWorkload
    w2 = StreamKWorkload(w.worker_rows[keep], w.worker_block_start[keep], w.worker_block_end[keep],
                         w.worker_needs_atomic[keep], int(keep.sum()), w.total_work)
    Bb = torch.from_numpy(case.b).to(gpu).to(torch.bfloat16)
    out = void_spmm_stream_k(vt, Bb, workload=w2)
    assert out.dtype == torch.bfloat16
    got = out.float().cpu().numpy()
    assert not np.any(got[dropped * 32:(dropped + 1) * 32])
    ref = _dense_of(vt) @ Bb.float().cpu().numpy().astype(np.float64)
    ref[dropped * 32:(dropped + 1) * 32] = 0
    rows_empty = np.setdiff1d(np.arange(16), case.block_rows)
    for r in rows_empty:
        assert not np.any(got[r * 32:(r + 1) * 32])
    assert np.allclose(got, ref, rtol=2.0 ** -8, atol=1e-3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_stream_k_16bit_tensor(gpu, dtype):
    """A 16-bit VOID tensor with a B of its dtype runs the workload on the
    16-bit kernel (no fp32 copy of the tiles is made); split rows are
    reduced deterministically."""
    rng = np.random.default_rng(9)
    nbr = 64
    counts = np.minimum(rng.zipf(1.5, nbr), 200)
    br = np.repeat(np.arange(nbr), counts)
    bc = np.concatenate([rng.choice(256, c, replace=False) for c in counts])
    tiles = rng.standard_normal((len(br), 32, 32)).astype(np.float32)
    case = cases.BlockCase("zipf16", nbr * 32, 256 * 32, 128, *cases._sorted(tiles, br, bc),
                           rng.standard_normal((256 * 32, 128)).astype(np.float32))
    vt = cases.make_void_tensor(case, "cpu").to_dtype(dtype).to(gpu)
    w = compute_stream_k_workload(vt, max_work_per_worker=16)
    B = torch.from_numpy(case.b).to(dtype).to(gpu)
    out = void_spmm_stream_k(vt, B, workload=w)
    assert out.dtype == dtype
    assert set(vt._device_bsr) == {f"{B.device}/{dtype}"}
    again = void_spmm_stream_k(vt, B, workload=w)
    assert torch.equal(out, again)
    A = _dense_of(vt)
    Bd = B.double().cpu().numpy()
    ref = A @ Bd
    n = 32 * int(counts.max())
    tol = n * 2.0 ** -24 * (np.abs(A) @ np.abs(Bd)) + (2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11) * np.abs(ref) + 2.0 ** -24
    assert np.all(np.abs(out.double().cpu().numpy() - ref) <= tol)
