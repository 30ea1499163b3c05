"""INT8 / FP8 quantisation of the host API against the oracle (bit-exact)."""

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import cases
import oracle
import void_amd
from void_amd import FP8Config, IntFormat, IntQuantConfig, ScaleMode


def test_quantize_void_tensor_bit_exact_c1():
    A, _ = cases.c1_plumbing()
    vt = void_amd.csr_to_void(A)
    q = void_amd.quantize_void_tensor(vt)
    oq, os_ = oracle.quantize_i8_blocks(vt.values.numpy())
    assert q.values.dtype == torch.int8
    assert np.array_equal(q.values.numpy(), oq)
    assert np.array_equal(q.scales.numpy().view(np.int32), os_.view(np.int32))
    assert not q.zero_points.any()


def test_quantize_void_tensor_edge_values():
    case = cases.uniform_blocks(128, 128, 8, 10, seed=1)
    case.tiles[0] = 0.0                      # all-zero tile -> scale 1e-8
    case.tiles[1, 0, 0] = 1e-30              # tiny amax
    case.tiles[2, 3, 4] = 1e6                # one huge entry
    vt = cases.make_void_tensor(case)
    q = void_amd.quantize_void_tensor(vt)
    oq, os_ = oracle.quantize_i8_blocks(case.tiles)
    assert np.array_equal(q.values.numpy(), oq) and np.array_equal(q.scales.numpy(), os_)


def test_per_tensor_config_expands_scale():
    vt = cases.make_void_tensor(cases.uniform_blocks(128, 128, 8, 6, seed=2))
    q = void_amd.quantize_void_tensor(vt, IntQuantConfig(scale_mode=ScaleMode.PER_TENSOR))
    assert q.scales.shape == (6,) and torch.all(q.scales == q.scales[0])
    oq, os_ = oracle.quantize_i8_tensor(vt.values.numpy())
    assert np.array_equal(q.values.numpy(), oq) and q.scales[0].item() == float(os_)


def test_quantize_tensor_per_channel_and_asymmetric():
    x = torch.randn(16, 40)
    q, p = void_amd.quantize_tensor(x, IntQuantConfig(scale_mode=ScaleMode.PER_CHANNEL))
    assert p.scale.shape == (16, 1)
    rec = void_amd.dequantize_tensor(q, p)
    # rounding error <= s/2, except +amax which saturates at 127 (error <= s)
    assert torch.all((rec - x).abs() <= p.scale * 1.0001)
    qa, pa = void_amd.quantize_tensor(x, IntQuantConfig(format=IntFormat.UINT8, symmetric=False,
                                                       scale_mode=ScaleMode.PER_TENSOR))
    assert qa.dtype == torch.uint8


def test_quantize_per_column_matches_oracle():
    b = torch.randn(300, 77)
    q, s = void_amd.quantize_per_column(b)
    oq, os_ = oracle.quantize_i8_columns(b.numpy())
    assert np.array_equal(q.numpy(), oq) and np.array_equal(s.numpy(), os_)


def test_dequantize_void_tensor_works():
    # the reference's version raises TypeError (int_quant.py:421-428); this one returns a VOIDTensor
    vt = cases.make_void_tensor(cases.uniform_blocks(96, 64, 8, 4, seed=3))
    q = void_amd.quantize_void_tensor(vt)
    d = void_amd.dequantize_void_tensor(q)
    assert isinstance(d, void_amd.VOIDTensor) and d.n_blocks == 4
    err = (d.values - vt.values).abs().max().item()
    assert err <= q.scales.max().item() * 1.0001  # +amax saturates at 127


def test_quantization_error_report():
    r = void_amd.get_quantization_error(torch.randn(64, 64), IntQuantConfig(scale_mode=ScaleMode.PER_TENSOR))
    assert r["snr_db"] > 30 and r["compression_ratio"] == 4.0


# ---------------------------------------------------------------- FP8

def test_void_tensor_to_fp8_bit_exact():
    case = cases.uniform_blocks(256, 256, 8, 40, seed=4)
    vt = cases.make_void_tensor(case)
    f8 = void_amd.void_tensor_to_fp8(vt)
    codes, scales = oracle.quantize_fp8_blocks(case.tiles)
    assert f8.values_fp8.dtype == torch.float8_e4m3fn
    assert np.array_equal(f8.values_fp8.view(torch.uint8).numpy(), codes)
    assert np.array_equal(f8.scaling_info.scale.numpy(), scales)
    assert f8.n_blocks == vt.n_blocks and f8.memory_bytes < vt.values.numel() * 4 * 0.5


def test_fp8_config_known_answers():
    # test_fp8.py:51-79
    assert FP8Config().max_value == 448.0 and FP8Config().torch_dtype == torch.float8_e4m3fn
    assert FP8Config(format=void_amd.FP8Format.E5M2).max_value == 57344.0
    for mode in ["per_tensor", "per_block", "per_row"]:
        assert FP8Config(scale_mode=mode).scale_mode == mode


def test_compute_amax_known_answers():
    # test_fp8.py:133-150
    t = torch.tensor([[[1.0, 2.0], [3.0, 4.0]], [[5.0, 6.0], [7.0, 8.0]]])
    assert void_amd.compute_amax(t, "per_tensor").item() == 8.0
    assert void_amd.compute_amax(t, "per_block").tolist() == [4.0, 8.0]


def test_fp8_roundtrip_tolerances():
    # test_fp8.py:82-131 (CPU versions of the reference's round-trip checks)
    x = torch.randn(64, 64) * 10
    f, info = void_amd.quantize_to_fp8(x, FP8Config())
    rec = void_amd.dequantize_from_fp8(f, info, output_dtype=torch.float32)
    assert ((x - rec).abs() / (x.abs() + 1e-6)).mean() < 0.2
    t = torch.randn(4, 64, 64)
    t[0] *= 0.01
    t[2] *= 100
    t[3] *= 1000
    f, info = void_amd.quantize_to_fp8(t, FP8Config(scale_mode="per_block"))
    assert info.scale.shape == (4,)
    rec = void_amd.dequantize_from_fp8(f, info, output_dtype=torch.float32)
    assert ((t - rec).abs() / (t.abs() + 1e-6)).mean() < 0.3


def test_fp8_dense_quantizer_matches_oracle():
    b = torch.randn(200, 64)
    q, s = void_amd.fp8.quantize_dense_fp8(b)
    oq, os_ = oracle.quantize_fp8_tensor(b.numpy())
    assert np.array_equal(q.view(torch.uint8).numpy(), oq) and np.float32(s) == os_
