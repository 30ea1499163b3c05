"""Backward of the float SpMM: the SDDMM kernels (void_sddmm_f32 and the
row-grouped void_sddmm_rows_f32) against
float64 products of the same operands, and the autograd wrappers
(VOIDSpMM, SparseLinear) against float64 dense gradients.  Bound: recursive
fp32 summation, (n-1) 2^-24 sum|x y| with n the reduction length."""

import numpy as np
import pytest
import torch

import cases
import oracle
import void_amd
from void_amd import _runtime

pytestmark = pytest.mark.gpu
U = 2.0 ** -24


@pytest.mark.parametrize("grouped", [None, "tile_rows", "ring", "rows"])
@pytest.mark.parametrize("M,K,N,n,seed", [(1024, 2048, 512, 600, 0), (100, 70, 36, 6, 1), (64, 96, 130, 5, 2),
                                          (256, 4096, 66, 300, 3), (96, 128, 1000, 12, 4), (70, 1000, 20, 40, 5),
                                          (500, 300, 8, 30, 6)])
def test_sddmm_tiles(gpu, M, K, N, n, seed, grouped, monkeypatch):
    # "ring" / "rows": void_sddmm_rows_f32 (tiles of a block-row share their
    # grad_c rows; the fourth shape has rows of up to 128 tiles, i.e. many
    # groups per row), on its LDS-DMA ring where the operands allow (N a
    # multiple of 4: chunks of 32 columns, the last one cut by N in several
    # shapes) or forced onto the register-staged kernel.  None /
    # "tile_rows": void_sddmm_f32 (tiles in the given order, 8 to a
    # workgroup on the per-tile ring with 16-column chunks, or one per
    # workgroup on the register-staged kernel).
    from void_amd.format import build_bsr_layout
    if grouped in ("rows", "tile_rows"):
        monkeypatch.setenv("VOID_AMD_SDDMM", "rows")
    elif grouped == "ring":  # the row-grouped ring even where the per-tile kernel would be chosen
        monkeypatch.setenv("VOID_AMD_SDDMM", "grouped")
    if grouped == "tile_rows":
        grouped = None
    rng = np.random.default_rng(seed)
    nbr, nbc = -(-M // 32), -(-K // 32)
    flat = rng.choice(nbr * nbc, min(n, nbr * nbc), replace=False)
    rows, cols = (flat // nbc).astype(np.int32), (flat % nbc).astype(np.int32)
    G = rng.standard_normal((M, N)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    tr, tc = torch.from_numpy(rows).to(gpu), torch.from_numpy(cols).to(gpu)
    lay = build_bsr_layout(tr, tc, nbr, nbc, gpu) if grouped else None
    got = _runtime.sddmm_tiles(torch.from_numpy(G).to(gpu), torch.from_numpy(B).to(gpu), tr, tc, (M, K),
                               torch.float32, layout=lay)
    Gp = np.zeros((nbr * 32, N)); Gp[:M] = G
    Bp = np.zeros((nbc * 32, N)); Bp[:K] = B
    for t in range(len(rows)):
        x = Gp[rows[t] * 32:(rows[t] + 1) * 32]
        y = Bp[cols[t] * 32:(cols[t] + 1) * 32]
        ref = x @ y.T
        bound = N * U * (np.abs(x) @ np.abs(y).T)
        assert np.all(np.abs(got[t].cpu().numpy() - ref) <= bound + 1e-30), t



# One rounding of the output type on top of the fp32 bound (p significand
# bits: 8 for bf16, 11 for fp16, plus half of fp16's subnormal spacing).
_HALF = {torch.bfloat16: (2.0 ** -8, 0.0), torch.float16: (2.0 ** -11, 2.0 ** -25)}


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("grouped", [None, "tile_rows", "ring", "rows"])
def test_sddmm_tiles_half_outputs(gpu, out_dtype, grouped, monkeypatch):
    """The gradient tiles of a half-precision VOIDTensor come out in its
    dtype (autograd.py passes a_values.dtype): each kernel's bf16 and fp16
    stores."""
    from void_amd.format import build_bsr_layout
    if grouped in ("rows", "tile_rows"):
        monkeypatch.setenv("VOID_AMD_SDDMM", "rows")
    elif grouped == "ring":  # the row-grouped ring even where the per-tile kernel would be chosen
        monkeypatch.setenv("VOID_AMD_SDDMM", "grouped")
    if grouped == "tile_rows":
        grouped = None
    M, K, N = 640, 1024, 200
    rng = np.random.default_rng(7)
    nbr, nbc = M // 32, K // 32
    flat = rng.choice(nbr * nbc, 150, replace=False)
    rows, cols = (flat // nbc).astype(np.int32), (flat % nbc).astype(np.int32)
    G = rng.standard_normal((M, N)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    tr, tc = torch.from_numpy(rows).to(gpu), torch.from_numpy(cols).to(gpu)
    lay = build_bsr_layout(tr, tc, nbr, nbc, gpu) if grouped else None
    got = _runtime.sddmm_tiles(torch.from_numpy(G).to(gpu), torch.from_numpy(B).to(gpu), tr, tc, (M, K),
                               out_dtype, layout=lay)
    assert got.dtype == out_dtype
    rel, ab = _HALF[out_dtype]
    G64, B64 = G.astype(np.float64), B.astype(np.float64)
    for t in range(len(rows)):
        x, y = G64[rows[t] * 32:(rows[t] + 1) * 32], B64[cols[t] * 32:(cols[t] + 1) * 32]
        ref = x @ y.T
        bound = N * U * (np.abs(x) @ np.abs(y).T) * (1 + rel) + rel * np.abs(ref) + ab
        assert np.all(np.abs(got[t].float().cpu().numpy() - ref) <= bound + 1e-30), t

@pytest.mark.parametrize("in_dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("same_out", [True, False], ids=["out16", "out32"])
@pytest.mark.parametrize("M,K,N,n,seed", [(1024, 2048, 512, 600, 0), (100, 70, 40, 6, 1), (64, 96, 136, 5, 2),
                                          (256, 4096, 72, 300, 3), (96, 128, 1000, 12, 4), (500, 300, 8, 30, 6),
                                          (70, 1000, 20, 40, 5)])
def test_sddmm16(gpu, in_dtype, same_out, M, K, N, n, seed):
    """16-bit grad_c and B of one dtype (the backward of a bf16 / fp16 VOID
    tensor): void_sddmm_rows_bf16 / _f16 on the 16-bit MFMA when N % 8 == 0
    (64-column chunks, the last cut by N), the fp32 kernel on widened copies
    otherwise (N = 20).  Same bound on the 16-bit values as the fp32 path,
    plus one rounding of a 16-bit output."""
    from void_amd.format import build_bsr_layout
    rng = np.random.default_rng(100 + seed)
    nbr, nbc = -(-M // 32), -(-K // 32)
    flat = rng.choice(nbr * nbc, min(n, nbr * nbc), replace=False)
    rows, cols = (flat // nbc).astype(np.int32), (flat % nbc).astype(np.int32)
    G = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(in_dtype)
    B = torch.from_numpy(rng.standard_normal((K, N)).astype(np.float32)).to(in_dtype)
    tr, tc = torch.from_numpy(rows).to(gpu), torch.from_numpy(cols).to(gpu)
    lay = build_bsr_layout(tr, tc, nbr, nbc, gpu)
    out_dtype = in_dtype if same_out else torch.float32
    got = _runtime.sddmm_tiles(G.to(gpu), B.to(gpu), tr, tc, (M, K), out_dtype, layout=lay)
    assert got.dtype == out_dtype
    rel, ab = _HALF[out_dtype] if same_out else (0.0, 0.0)
    Gp = np.zeros((nbr * 32, N)); Gp[:M] = G.double().numpy()
    Bp = np.zeros((nbc * 32, N)); Bp[:K] = B.double().numpy()
    for t in range(len(rows)):
        x, y = Gp[rows[t] * 32:(rows[t] + 1) * 32], Bp[cols[t] * 32:(cols[t] + 1) * 32]
        ref = x @ y.T
        bound = N * U * (np.abs(x) @ np.abs(y).T) * (1 + rel) + rel * np.abs(ref) + ab
        assert np.all(np.abs(got[t].float().cpu().numpy() - ref) <= bound + 1e-30), t


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_voidspmm_gradients_16bit(gpu, dtype):
    """A bf16 / fp16 VOID tensor times an input of the same dtype: forward
    and the product for the input's gradient on the 16-bit SpMM, the tiles'
    gradient on the 16-bit SDDMM, each within the fp32 summation bound on the
    16-bit values plus one rounding of the 16-bit result."""
    case = cases.uniform_blocks(512, 1024, 96, 150, seed=5)
    vt = cases.make_void_tensor(case, "cpu").to_dtype(dtype).to(gpu)
    mod = void_amd.VOIDSpMM(vt).to(gpu)
    x = torch.randn(1024, 96, device=gpu).to(dtype).requires_grad_(True)
    w = torch.randn(512, 96, device=gpu).to(dtype)
    y = mod(x)
    assert y.dtype == dtype
    (y * w).sum().backward()
    rel, ab = _HALF[dtype]
    A = oracle.densify(vt.values.float().cpu().numpy(), case.block_rows, case.block_cols, (512, 1024)).astype(np.float64)
    X, W = x.detach().double().cpu().numpy(), w.double().cpu().numpy()
    n_row = np.bincount(case.block_rows, minlength=16).max()
    ref = A @ X
    assert np.all(np.abs(y.detach().double().cpu().numpy() - ref) <=
                  32 * n_row * U * (np.abs(A) @ np.abs(X)) + rel * np.abs(ref) + ab + 1e-30)
    gX = A.T @ W
    n_col = np.bincount(case.block_cols, minlength=32).max()
    assert np.all(np.abs(x.grad.double().cpu().numpy() - gX) <=
                  32 * n_col * U * (np.abs(A).T @ np.abs(W)) + rel * np.abs(gX) + ab + 1e-30)
    gA = W @ X.T
    tiles = mod.values.grad.double().cpu().numpy()
    bound_full = 96 * U * (np.abs(W) @ np.abs(X).T)
    rr, cc = vt.block_rows.cpu().numpy(), vt.block_cols.cpu().numpy()
    for t in range(len(tiles)):
        r, c = rr[t] * 32, cc[t] * 32
        g = gA[r:r + 32, c:c + 32]
        assert np.all(np.abs(tiles[t] - g) <= bound_full[r:r + 32, c:c + 32] + rel * np.abs(g) + ab + 1e-30)


def test_voidspmm_gradients(gpu):
    case = cases.uniform_blocks(512, 1024, 96, 150, seed=5)
    vt = cases.make_void_tensor(case, "cpu").to(gpu)
    mod = void_amd.VOIDSpMM(vt).to(gpu)
    x = torch.randn(1024, 96, device=gpu, requires_grad=True)
    w = torch.randn(512, 96, device=gpu)
    y = mod(x)
    (y * w).sum().backward()
    A = oracle.densify(case.tiles, case.block_rows, case.block_cols, (512, 1024)).astype(np.float64)
    X, W = x.detach().cpu().double().numpy(), w.cpu().double().numpy()
    assert np.all(np.abs(y.detach().cpu().numpy() - A @ X) <= 32 * 10 * U * (np.abs(A) @ np.abs(X)) + 1e-30)
    gX = A.T @ W  # dL/dB = A^T dL/dC
    n_col = np.bincount(case.block_cols, minlength=32).max()
    assert np.all(np.abs(x.grad.cpu().numpy() - gX) <= 32 * n_col * U * (np.abs(A).T @ np.abs(W)) + 1e-30)
    gA = W @ X.T  # dense dL/dA; only the tiles' entries are returned
    tiles = mod.values.grad.cpu().numpy()
    vals_rows, vals_cols = vt.block_rows.cpu().numpy(), vt.block_cols.cpu().numpy()
    bound_full = 96 * U * (np.abs(W) @ np.abs(X).T)
    for t in range(len(tiles)):
        r, c = vals_rows[t] * 32, vals_cols[t] * 32
        assert np.all(np.abs(tiles[t] - gA[r:r + 32, c:c + 32]) <= bound_full[r:r + 32, c:c + 32] + 1e-30)


def test_sparse_linear_training_step(gpu):
    case = cases.uniform_blocks(128, 256, 8, 12, seed=9)
    vt = cases.make_void_tensor(case, "cpu").to(gpu)
    layer = void_amd.SparseLinear(256, 128, vt).to(gpu)
    x = torch.randn(4, 5, 256, device=gpu)
    y = layer(x)
    assert y.shape == (4, 5, 128)
    loss = (y ** 2).mean()
    loss.backward()
    assert layer.sparse_weight.values.grad.shape == vt.values.shape and layer.bias.grad.shape == (128,)
    # an optimiser step changes the values in place; the next forward must see them
    with torch.no_grad():
        layer.sparse_weight.values.mul_(2.0)
        layer.bias.zero_()
    y2 = layer(x)
    W = oracle.densify(vt.values.cpu().numpy() * 2.0, case.block_rows, case.block_cols, (128, 256))
    ref = x.reshape(-1, 256).cpu().double().numpy() @ W.T.astype(np.float64)
    assert np.allclose(y2.detach().reshape(-1, 128).cpu().numpy(), ref, rtol=1e-5, atol=1e-4)



def test_inference_mode(gpu):
    """Tensors made under torch.inference_mode keep no version counter; the
    cached layouts then key on identity alone, and every entry point runs as
    outside that mode."""
    case = cases.uniform_blocks(256, 512, 64, 40, seed=8)
    x_host = torch.randn(512, 64)
    vt_ref = cases.make_void_tensor(case, "cpu").to(gpu)
    y_ref = void_amd.VOIDSpMM(vt_ref).to(gpu)(x_host.to(gpu)).detach()
    q_ref = void_amd.quantize_void_tensor(cases.make_void_tensor(case, "cpu")).to(gpu)
    bq, bs = oracle.quantize_i8_columns(case.b)
    z_ref = void_amd.void_spmm_int8(q_ref, torch.from_numpy(bq).to(gpu), b_scale=torch.from_numpy(bs).to(gpu))
    with torch.inference_mode():
        vt = cases.make_void_tensor(case, "cpu").to(gpu)
        mod = void_amd.VOIDSpMM(vt).to(gpu)
        x = x_host.to(gpu)
        assert torch.equal(mod(x), y_ref)
        assert torch.equal(void_amd.void_spmm(vt, x), y_ref)
        q = void_amd.quantize_void_tensor(cases.make_void_tensor(case, "cpu")).to(gpu)
        z = void_amd.void_spmm_int8(q, torch.from_numpy(bq).to(gpu), b_scale=torch.from_numpy(bs).to(gpu))
        assert torch.equal(z, z_ref)
