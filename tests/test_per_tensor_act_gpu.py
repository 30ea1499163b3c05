"""GPU parity for two paths the other tests leave out: an A quantised with
one per-tensor scale (INT8 PER_TENSOR, FP8 scale_mode="per_tensor"; the
kernels then read scales[0] for every tile), and ReLU / SiLU fused into the
quantised epilogues with bias and 16-bit outputs.  The oracle takes the
per-tensor scale expanded to every tile: int32 accumulators bit-exact,
row-mean bit-exact, per-block within 1e-5 of the product-magnitude bound,
FP8 within 2^-13 of it, 16-bit outputs within one rounding of the
activation of the oracle's value."""

import numpy as np
import pytest
import torch

import cases
import oracle
import void_amd
from void_amd.int_quant import IntFormat, IntQuantConfig, ScaleMode

pytestmark = pytest.mark.gpu

FP8_TOL = 2.0 ** -13


@pytest.fixture(params=["default", "cgd3", "cgdk", "bsr"])
def kernel(request, monkeypatch):
    if request.param == "default":
        monkeypatch.delenv("VOID_AMD_KERNEL", raising=False)
    else:
        monkeypatch.setenv("VOID_AMD_KERNEL", request.param)
    return request.param


def _per_tensor_int8(case, dev):
    vt = cases.make_void_tensor(case, "cpu")
    q = void_amd.quantize_void_tensor(vt, IntQuantConfig(format=IntFormat.INT8, symmetric=True,
                                                         scale_mode=ScaleMode.PER_TENSOR))
    s = float(q.scales.reshape(-1)[0])
    assert torch.all(q.scales == s)
    A = oracle.Bsr(q.values.numpy(), np.full(q.n_blocks, s, np.float32), case.block_rows, case.block_cols,
                   (case.M, case.K))
    return q.to(dev), A


def _abs_bound(A, bq, bs):
    Aabs = oracle.Bsr.__new__(oracle.Bsr)
    Aabs.__dict__.update(A.__dict__)
    Aabs.tiles = np.ascontiguousarray(np.abs(A.tiles.astype(np.int16)).clip(0, 127).astype(np.int8))
    return oracle.i8_per_block(Aabs, np.abs(bq.astype(np.int16)).clip(0, 127).astype(np.int8), np.abs(bs))


@pytest.mark.parametrize("epilogue", ["raw_i32", "row_mean", "per_block"])
def test_int8_per_tensor_a(gpu, kernel, epilogue):
    case = cases.uniform_blocks(1000, 1500, 200, 500, seed=21)
    qd, A = _per_tensor_int8(case, gpu)
    assert qd.device_bsr().per_tensor
    bq, bs = oracle.quantize_i8_columns(case.b)
    if epilogue == "row_mean":
        bs = np.float32(bs.max())  # the reference's row-mean takes a scalar B scale
    out = void_amd.void_spmm_int8(qd, torch.from_numpy(bq).to(gpu),
                                  b_scale=float(bs) if np.ndim(bs) == 0 else torch.from_numpy(bs).to(gpu),
                                  epilogue=epilogue)
    got = out.cpu().numpy()
    if epilogue == "raw_i32":
        assert np.array_equal(got, oracle.i8_acc(A, bq))
    elif epilogue == "row_mean":
        ref = oracle.row_mean(A, oracle.i8_acc(A, bq), bs)
        assert np.array_equal(got.view(np.int32), ref.view(np.int32))
    else:
        ref = oracle.i8_per_block(A, bq, bs)
        assert np.all(np.abs(got - ref) <= 1e-5 * _abs_bound(A, bq, bs) + 1e-30)


def test_fp8_per_tensor_a(gpu, kernel):
    case = cases.uniform_blocks(900, 1100, 256, 400, seed=22)
    vt = cases.make_void_tensor(case, "cpu")
    f8 = void_amd.void_tensor_to_fp8(vt, scale_mode="per_tensor")
    sc = f8.scaling_info.scale.reshape(-1)
    assert sc.numel() == 1 or torch.all(sc == sc[0])
    s = float(sc[0])
    bq, bs = oracle.quantize_fp8_tensor(case.b)
    bt = torch.from_numpy(bq).to(gpu).view(torch.float8_e4m3fn)
    out = void_amd.void_spmm_fp8(f8.to(gpu), bt, output_dtype=torch.float32, b_scale=float(bs))
    A = oracle.Bsr(f8.values_fp8.view(torch.uint8).numpy(), np.full(vt.n_blocks, s, np.float32),
                   case.block_rows, case.block_cols, (case.M, case.K))
    ref = oracle.fp8_spmm(A, bq, bs)
    Aabs = oracle.Bsr.__new__(oracle.Bsr)
    Aabs.__dict__.update(A.__dict__)
    Aabs.tiles = np.ascontiguousarray(A.tiles.view(np.uint8) & 0x7F)
    bound = oracle.fp8_spmm(Aabs, bq & 0x7F, abs(bs))
    assert np.all(np.abs(out.cpu().numpy().astype(np.float64) - ref) <= FP8_TOL * bound + 1e-30)


@pytest.mark.parametrize("act", ["relu", "silu"])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_int8_relu_silu_bias(gpu, kernel, act, out_dtype):
    case = cases.uniform_blocks(700, 1300, 384, 350, seed=23)
    vt = cases.make_void_tensor(case, "cpu")
    q = void_amd.quantize_void_tensor(vt)
    A = oracle.Bsr(q.values.numpy(), q.scales.numpy(), case.block_rows, case.block_cols, (case.M, case.K))
    bq, bs = oracle.quantize_i8_columns(case.b)
    bias = np.random.default_rng(5).standard_normal(case.N).astype(np.float32)
    fn = {"relu": void_amd.void_spmm_relu, "silu": void_amd.void_spmm_silu}[act]
    out = fn(q.to(gpu), torch.from_numpy(bq).to(gpu), bias=torch.from_numpy(bias).to(gpu),
             b_scale=torch.from_numpy(bs).to(gpu), out_dtype=out_dtype)
    assert out.dtype == out_dtype
    pre = oracle.i8_per_block(A, bq, bs) + bias[None, :].astype(np.float64)
    ref = np.maximum(pre, 0.0) if act == "relu" else pre / (1.0 + np.exp(-pre))
    rnd = 2.0 ** -8 if out_dtype == torch.bfloat16 else 2.0 ** -11
    err = np.abs(out.float().cpu().numpy() - ref)
    assert np.all(err <= rnd * np.abs(ref) + 1e-4), err.max()


def test_fp8_gelu_bias_bf16(gpu, kernel):
    case = cases.uniform_blocks(600, 900, 256, 300, seed=24)
    vt = cases.make_void_tensor(case, "cpu")
    f8 = void_amd.void_tensor_to_fp8(vt)
    bq, bs = oracle.quantize_fp8_tensor(case.b)
    bias = np.random.default_rng(6).standard_normal(case.N).astype(np.float32)
    out = void_amd.void_spmm_gelu(f8.to(gpu), torch.from_numpy(bq).to(gpu).view(torch.float8_e4m3fn),
                                  bias=torch.from_numpy(bias).to(gpu), b_scale=float(bs), out_dtype=torch.bfloat16)
    A = oracle.Bsr(f8.values_fp8.view(torch.uint8).numpy(), f8.scaling_info.scale.numpy(), case.block_rows,
                   case.block_cols, (case.M, case.K))
    ref = oracle.gelu_tanh(oracle.fp8_spmm(A, bq, bs) + bias[None, :].astype(np.float64))
    err = np.abs(out.float().cpu().numpy() - ref)
    assert np.all(err <= 2.0 ** -8 * np.abs(ref) + 1e-3), err.max()
