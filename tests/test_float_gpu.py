"""Float SpMM (void_spmm, void_spmm_gelu on float VOID tiles) against a
float64 dense product of the same tiles.

Bar: recursive fp32 summation of n products errs by at most (n-1) u sum|a b|
(u = 2^-24); n is the number of products per output (32 per tile in the
row) plus the bias add.  An indexing or ordering mistake breaks it by orders
of magnitude.  bf16/f16 outputs add one rounding of the output format."""

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import cases
import oracle
import void_amd

pytestmark = pytest.mark.gpu
U = 2.0 ** -24


@pytest.fixture(params=["ring", "cgd", "cgdk", "f32"])
def fkernel(request, monkeypatch):
    """The float tiles' kernels: the column-group LDS-DMA ring (default for
    row-major 16-byte aligned B, elsewhere the fallback runs anyway) with its
    default ring shape, forced to one ring per workgroup (cgd) or two
    (cgdk), and the fp32 kernel of its own (VOID_AMD_KERNEL=f32)."""
    if request.param == "ring":
        monkeypatch.delenv("VOID_AMD_KERNEL", raising=False)
    else:
        monkeypatch.setenv("VOID_AMD_KERNEL", request.param)
    return request.param


def _dense_of(vt):
    return oracle.densify(vt.values.float().cpu().numpy(), vt.block_rows.cpu().numpy(), vt.block_cols.cpu().numpy(),
                          vt.shape).astype(np.float64)


def _bound(vt, B, extra_terms=0):
    Ad = np.abs(_dense_of(vt))
    n_row = np.bincount(vt.block_rows.cpu().numpy(), minlength=vt.block_grid[0]).max() if vt.n_blocks else 0
    n = 32 * int(n_row) + extra_terms
    return n * U * (Ad @ np.abs(B.astype(np.float64)))


@pytest.mark.parametrize("M,K,N,n_tiles,seed", [(4096, 4096, 512, 1638, 0), (1024, 2048, 256, 900, 3),
                                                (96, 96, 64, 9, 1)])
def test_float_spmm_fp32(gpu, fkernel, M, K, N, n_tiles, seed):
    case = cases.uniform_blocks(M, K, N, n_tiles, seed=seed)
    vt = cases.make_void_tensor(case, "cpu").to(gpu)
    B = case.b.astype(np.float32)
    out = void_amd.void_spmm(vt, torch.from_numpy(B).to(gpu))
    assert out.dtype == torch.float32
    ref = _dense_of(vt) @ B.astype(np.float64)
    err = np.abs(out.cpu().numpy().astype(np.float64) - ref)
    bound = _bound(vt, B)
    assert np.all(err <= bound + 1e-30), (err / (bound + 1e-30)).max()


@pytest.mark.parametrize("M,K,N", [(333, 555, 64), (100, 70, 36), (64, 96, 130), (1000, 70, 257)])
def test_float_spmm_ragged(gpu, fkernel, M, K, N):
    rng = np.random.default_rng(M + K + N)
    dense = np.where(rng.random((M, K)) < 0.1, rng.standard_normal((M, K)), 0).astype(np.float32)
    vt = void_amd.dense_to_void(torch.from_numpy(dense)).to(gpu)
    B = rng.standard_normal((K, N)).astype(np.float32)
    out = void_amd.void_spmm(vt, torch.from_numpy(B).to(gpu))
    ref = dense.astype(np.float64) @ B.astype(np.float64)
    bound = _bound(vt, B)
    assert np.all(np.abs(out.cpu().numpy() - ref) <= bound + 1e-30)


def test_float_spmm_split_rows(gpu, fkernel):
    # Rows of 100 tiles: the 64-tile items split, exercising the fix-up.
    rng = np.random.default_rng(7)
    rows, cols = [], []
    for r in range(8):
        n = 100 if r % 2 == 0 else 5
        cs = rng.choice(128, n, replace=False)
        rows += [r] * n
        cols += list(cs)
    case = cases.BlockCase("long_rows", 256, 4096, 128,
                           rng.standard_normal((len(rows), 32, 32)).astype(np.float32),
                           np.array(rows, np.int32), np.array(cols, np.int32),
                           rng.standard_normal((4096, 128)).astype(np.float32))
    vt = cases.make_void_tensor(case, "cpu").to(gpu)
    assert vt.device_bsr().plan(64).n_split_tiles > 0
    out = void_amd.void_spmm(vt, torch.from_numpy(case.b).to(gpu))
    ref = _dense_of(vt) @ case.b.astype(np.float64)
    assert np.all(np.abs(out.cpu().numpy() - ref) <= _bound(vt, case.b) + 1e-30)
    again = void_amd.void_spmm(vt, torch.from_numpy(case.b).to(gpu))
    assert torch.equal(out, again)  # deterministic fix-up


@pytest.mark.parametrize("act", ["gelu", "relu", "silu"])
def test_float_activation_bias(gpu, fkernel, act):
    case = cases.uniform_blocks(512, 1024, 192, 120, seed=11)
    vt = cases.make_void_tensor(case, "cpu").to(gpu)
    B = case.b.astype(np.float32)
    bias = np.random.default_rng(2).standard_normal(192).astype(np.float32)
    fn = {"gelu": void_amd.void_spmm_gelu, "relu": void_amd.void_spmm_relu, "silu": void_amd.void_spmm_silu}[act]
    out = fn(vt, torch.from_numpy(B).to(gpu), bias=torch.from_numpy(bias).to(gpu))
    pre = _dense_of(vt) @ B.astype(np.float64) + bias[None, :]
    ref = {"gelu": oracle.gelu_tanh, "relu": lambda x: np.maximum(x, 0.0),
           "silu": lambda x: x / (1.0 + np.exp(-x))}[act](pre)
    # activation slopes are below 1.2; the transcendental adds a few ulps of the result
    tol = 1.2 * _bound(vt, B, extra_terms=2) + 8 * U * np.abs(ref) + 1e-6
    assert np.all(np.abs(out.cpu().numpy() - ref) <= tol)


def test_float_bf16_b_and_output(gpu, fkernel):
    case = cases.uniform_blocks(1024, 1024, 256, 300, seed=5)
    vt = cases.make_void_tensor(case, "cpu").to(gpu)
    Bb = torch.from_numpy(case.b).to(torch.bfloat16)
    out = void_amd.void_spmm(vt, Bb.to(gpu))
    assert out.dtype == torch.bfloat16
    B = Bb.float().numpy()
    ref = _dense_of(vt) @ B.astype(np.float64)
    tol = _bound(vt, B) + 2.0 ** -8 * np.abs(ref)
    assert np.all(np.abs(out.float().cpu().numpy() - ref) <= tol + 1e-30)


def test_float_empty_and_reference_defaults(gpu):
    vt = void_amd.dense_to_void(torch.zeros(100, 64)).to(gpu)
    out = void_amd.void_spmm(vt, torch.randn(64, 32, device=gpu))
    assert out.shape == (100, 32) and torch.count_nonzero(out) == 0
    bias = torch.randn(32, device=gpu)
    g = void_amd.void_spmm_gelu(vt, torch.randn(64, 32, device=gpu), bias=bias)
    assert torch.allclose(g, torch.nn.functional.gelu(bias)[None, :].expand(100, 32))
    # csr_to_void on the device feeds the float kernel directly
    A = sp.random(300, 200, density=0.05, format="csr", random_state=1, dtype=np.float32)
    vt2 = void_amd.csr_to_void(A, device="cuda")
    B = np.random.default_rng(0).standard_normal((200, 48)).astype(np.float32)
    out2 = void_amd.void_spmm(vt2, torch.from_numpy(B).to(gpu))
    ref2 = A.toarray().astype(np.float64) @ B.astype(np.float64)
    assert np.all(np.abs(out2.cpu().numpy() - ref2) <= _bound(vt2, B) + 1e-30)
