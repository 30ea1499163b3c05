"""Float SpMM on 16-bit VOID tensors: bf16 or fp16 tiles times a B of the
same dtype run on the 16-bit MFMA kernel (void_spmm_bf16 / void_spmm_f16),
against a float64 dense product of the same 16-bit values.

Bar: a product of two 16-bit values is exact in fp32, so the only errors
are the fp32 accumulation, at most (n-1) u sum|a b| for n products per
output (u = 2^-24), and one rounding of the output format (bf16 2^-8, fp16
2^-11 relative, fp16 also 2^-25 absolute below its normal range).  A wrong
operand layout (a transposed B read, a swizzle that picks the wrong chunk)
breaks it by orders of magnitude."""

import dataclasses

import numpy as np
import pytest
import torch

import cases
import oracle
import void_amd

pytestmark = pytest.mark.gpu
U = 2.0 ** -24
ROUND = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 0.0}
ABS = {torch.bfloat16: 0.0, torch.float16: 2.0 ** -25, torch.float32: 0.0}


@pytest.fixture(params=["default", "cgd", "cgdk"])
def k16(request, monkeypatch):
    """Ring shapes of the 16-bit kernel: the default choice, one ring per
    workgroup, two rings per 8-wave workgroup."""
    if request.param == "default":
        monkeypatch.delenv("VOID_AMD_KERNEL", raising=False)
    else:
        monkeypatch.setenv("VOID_AMD_KERNEL", request.param)
    return request.param


def _vt16(case, dtype, dev):
    vt = cases.make_void_tensor(case, "cpu")
    vt = dataclasses.replace(vt, values=vt.values.to(dtype), dtype=dtype, _device_bsr={})
    return vt.to(dev)


def _dense(vt):
    return oracle.densify(vt.values.float().cpu().numpy(), vt.block_rows.cpu().numpy(),
                          vt.block_cols.cpu().numpy(), vt.shape).astype(np.float64)


def _check(out, ref, absprod, n, dtype):
    assert out.dtype == dtype
    got = out.float().cpu().numpy().astype(np.float64)
    tol = n * U * absprod + ROUND[dtype] * np.abs(ref) + ABS[dtype] + 1e-30
    err = np.abs(got - ref)
    assert np.all(err <= tol), (err / tol).max()


def _n_row(vt):
    return 32 * int(np.bincount(vt.block_rows.cpu().numpy(), minlength=vt.block_grid[0]).max())


def _used_16bit(vt, dtype):
    return any(k.endswith(str(dtype)) for k in vt._device_bsr)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K,N,n_tiles,seed", [(4096, 4096, 512, 1638, 0), (1024, 2048, 256, 900, 3),
                                                (96, 96, 64, 9, 1), (4096, 4096, 2048, 3277, 4)])
def test_spmm16(gpu, k16, dtype, M, K, N, n_tiles, seed):
    case = cases.uniform_blocks(M, K, N, n_tiles, seed=seed)
    print(f"spmm16 {dtype} M={M} K={K} N={N} tiles={n_tiles}", flush=True)
    vt = _vt16(case, dtype, gpu)
    Bt = torch.from_numpy(case.b).to(dtype)
    out = void_amd.void_spmm(vt, Bt.to(gpu))
    assert _used_16bit(vt, dtype)
    A, B = _dense(vt), Bt.double().numpy()
    _check(out, A @ B, np.abs(A) @ np.abs(B), _n_row(vt), dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_spmm16_f32_output(gpu, dtype):
    # An fp32 out= keeps the fp32 sums (no output rounding).
    case = cases.uniform_blocks(1024, 1024, 384, 500, seed=6)
    vt = _vt16(case, dtype, gpu)
    Bt = torch.from_numpy(case.b).to(dtype)
    out = torch.full((1024, 384), float("nan"), device=gpu)
    void_amd.void_spmm(vt, Bt.to(gpu), out=out)
    A, B = _dense(vt), Bt.double().numpy()
    _check(out, A @ B, np.abs(A) @ np.abs(B), _n_row(vt), torch.float32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K,N", [(333, 555, 64), (100, 70, 40), (64, 96, 136), (1000, 70, 264),
                                   (130, 250, 36), (70, 40, 257)])
def test_spmm16_ragged(gpu, k16, dtype, M, K, N):
    # K not a multiple of 32 (the last slab loads no rows past K); N % 8 != 0
    # takes the fp32 kernel, with the same bound.
    rng = np.random.default_rng(M + K + N)
    dense = np.where(rng.random((M, K)) < 0.1, rng.standard_normal((M, K)), 0).astype(np.float32)
    vt = void_amd.dense_to_void(torch.from_numpy(dense).to(dtype)).to(gpu)
    Bt = torch.from_numpy(rng.standard_normal((K, N)).astype(np.float32)).to(dtype)
    out = void_amd.void_spmm(vt, Bt.to(gpu))
    assert _used_16bit(vt, dtype) == (N % 8 == 0)
    A, B = _dense(vt), Bt.double().numpy()
    _check(out, A @ B, np.abs(A) @ np.abs(B), _n_row(vt), dtype)


def test_spmm16_strided_b_and_out(gpu):
    # B a column slice of a wider matrix (row stride 1024) and out a slice of
    # a wider buffer: both stay in place.
    case = cases.uniform_blocks(512, 1024, 256, 200, seed=9)
    vt = _vt16(case, torch.bfloat16, gpu)
    wide = torch.randn(1024, 1024, dtype=torch.bfloat16, device=gpu)
    wide[:, 128:384] = torch.from_numpy(case.b).to(torch.bfloat16).to(gpu)
    b = wide[:, 128:384]
    big = torch.zeros(512, 512, dtype=torch.bfloat16, device=gpu)
    out = big[:, 64:320]
    void_amd.void_spmm(vt, b, out=out)
    A, B = _dense(vt), b.double().cpu().numpy()
    _check(out, A @ B, np.abs(A) @ np.abs(B), _n_row(vt), torch.bfloat16)
    assert torch.count_nonzero(big[:, :64]) == 0 and torch.count_nonzero(big[:, 320:]) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_spmm16_split_rows(gpu, k16, dtype):
    # Rows of 100 tiles: the 64-tile items split, exercising the fix-up.
    rng = np.random.default_rng(7)
    rows, cols = [], []
    for r in range(8):
        n = 100 if r % 2 == 0 else 5
        rows += [r] * n
        cols += list(rng.choice(128, n, replace=False))
    case = cases.BlockCase("long_rows", 256, 4096, 128,
                           rng.standard_normal((len(rows), 32, 32)).astype(np.float32),
                           np.array(rows, np.int32), np.array(cols, np.int32),
                           rng.standard_normal((4096, 128)).astype(np.float32))
    vt = _vt16(case, dtype, gpu)
    assert vt.device_bsr(dtype).plan(64).n_split_tiles > 0
    Bt = torch.from_numpy(case.b).to(dtype).to(gpu)
    out = void_amd.void_spmm(vt, Bt)
    A, B = _dense(vt), Bt.double().cpu().numpy()
    _check(out, A @ B, np.abs(A) @ np.abs(B), _n_row(vt), dtype)
    assert torch.equal(out, void_amd.void_spmm(vt, Bt))  # deterministic fix-up


@pytest.mark.parametrize("act", ["gelu", "relu", "silu"])
def test_spmm16_activation_bias(gpu, act):
    case = cases.uniform_blocks(512, 1024, 192, 120, seed=11)
    vt = _vt16(case, torch.bfloat16, gpu)
    Bt = torch.from_numpy(case.b).to(torch.bfloat16)
    bias = np.random.default_rng(2).standard_normal(192).astype(np.float32)
    fn = {"gelu": void_amd.void_spmm_gelu, "relu": void_amd.void_spmm_relu, "silu": void_amd.void_spmm_silu}[act]
    out = fn(vt, Bt.to(gpu), bias=torch.from_numpy(bias).to(gpu))
    assert _used_16bit(vt, torch.bfloat16)
    A, B = _dense(vt), Bt.double().numpy()
    pre = A @ B + bias[None, :]
    ref = {"gelu": oracle.gelu_tanh, "relu": lambda x: np.maximum(x, 0.0),
           "silu": lambda x: x / (1.0 + np.exp(-x))}[act](pre)
    # activation slopes are below 1.2; the transcendental adds a few ulps
    absprod = 1.2 * (np.abs(A) @ np.abs(B) + np.abs(bias)[None, :])
    got = out.float().cpu().numpy().astype(np.float64)
    tol = (_n_row(vt) + 2) * U * absprod + (2.0 ** -8 + 8 * U) * np.abs(ref) + 1e-6
    assert np.all(np.abs(got - ref) <= tol)


def test_spmm16_in_place_update(gpu):
    # The 16-bit device copy follows in-place changes of the values.
    case = cases.uniform_blocks(256, 512, 128, 40, seed=12)
    vt = _vt16(case, torch.bfloat16, gpu)
    Bt = torch.from_numpy(case.b).to(torch.bfloat16).to(gpu)
    first = void_amd.void_spmm(vt, Bt)
    vt.values.mul_(2)
    second = void_amd.void_spmm(vt, Bt)
    assert torch.equal(second.float(), (2 * first.float()).to(torch.bfloat16).float())


def test_fused_linear_bf16(gpu):
    # FusedSparseLinear's per-row bias path in bf16: y = W x + b per output row.
    rng = np.random.default_rng(3)
    W = np.where(rng.random((256, 512)) < 0.2, rng.standard_normal((256, 512)), 0).astype(np.float32)
    vt = void_amd.dense_to_void(torch.from_numpy(W).to(torch.bfloat16)).to(gpu)
    X = torch.from_numpy(rng.standard_normal((512, 64)).astype(np.float32)).to(torch.bfloat16).to(gpu)
    bias = torch.from_numpy(rng.standard_normal(256).astype(np.float32)).to(gpu)
    from void_amd.ops import float_spmm
    out = float_spmm(vt, X, bias=bias, bias_per_row=True)
    assert _used_16bit(vt, torch.bfloat16)
    A, B = _dense(vt), X.double().cpu().numpy()
    ref = A @ B + bias.double().cpu().numpy()[:, None]
    absprod = np.abs(A) @ np.abs(B) + np.abs(bias.double().cpu().numpy())[:, None]
    _check(out, ref, absprod, _n_row(vt) + 1, torch.bfloat16)


@pytest.mark.parametrize("seed", range(24))
def test_spmm16_random(gpu, k16, seed):
    """Seeded random ragged shapes and densities (one tile to dense rows,
    N a multiple of 8 so that the 16-bit kernel runs), bf16 and fp16 by
    seed parity, default and forced-small chunks (split rows)."""
    rng = np.random.default_rng(5000 + seed)
    M, K = int(rng.integers(1, 700)), int(rng.integers(1, 2200))
    N = int(rng.choice([8, 16, 40, 64, 128, 136, 256, 384, 520]))
    nbr, nbc = -(-M // 32), -(-K // 32)
    case = cases.uniform_blocks(M, K, N, int(rng.integers(1, nbr * nbc + 1)), seed=seed)
    dtype = torch.bfloat16 if seed % 2 == 0 else torch.float16
    print(f"spmm16 random seed={seed} M={M} K={K} N={N} tiles={len(case.block_rows)} {dtype}", flush=True)
    vt = _vt16(case, dtype, gpu)
    Bt = torch.from_numpy(case.b).to(dtype)
    from void_amd.ops import float_spmm
    plan = vt.device_bsr(dtype).plan(int(rng.choice([8, 24, 64]))) if seed % 3 == 0 else None
    out = float_spmm(vt, Bt.to(gpu), plan=plan)
    assert _used_16bit(vt, dtype)
    A, B = _dense(vt), Bt.double().numpy()
    _check(out, A @ B, np.abs(A) @ np.abs(B), _n_row(vt), dtype)
