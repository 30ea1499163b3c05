"""The reference's fusion and FP8 tests, on the same inputs and at the same
tolerances (tests/test_fusion.py:22-390, tests/test_fp8.py:209-238), run
through this package.  Where the reference checks only a shape
(FusedSparseLinear) the output is also compared with a float64 dense
restatement of the same layer built from the scipy inputs."""

import numpy as np
import pytest
import scipy.sparse as sparse
import torch

import void_amd
from void_amd import csr_to_void, void_spmm
from void_amd.fusion import (ActivationType, FusedSparseLinear, get_activation_code, void_spmm_gelu, void_spmm_relu,
                             void_spmm_silu)

pytestmark = pytest.mark.gpu


@pytest.fixture
def small():
    np.random.seed(42)
    return sparse.random(256, 256, density=0.1, format="csr", dtype=np.float32)


def _gelu64(x):
    """The tanh-form GELU the fused kernels evaluate (fusion.py:38-43)."""
    return 0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))


_ACT64 = {"gelu": _gelu64, "relu": lambda x: np.maximum(x, 0.0), "silu": lambda x: x / (1.0 + np.exp(-x)),
          "none": lambda x: x}


# tests/test_fusion.py:38-124: each fused activation against void_spmm then torch.
@pytest.mark.parametrize("act,fn,ref,tol", [
    ("gelu", void_spmm_gelu, torch.nn.functional.gelu, 0.05),
    ("relu", void_spmm_relu, torch.relu, 1e-5),
    ("silu", void_spmm_silu, torch.nn.functional.silu, 0.01)])
def test_fused_activation(gpu, small, act, fn, ref, tol):
    vt = csr_to_void(small, device="cuda")
    B = torch.randn(vt.shape[1], 64, device=gpu)
    err = (fn(vt, B) - ref(void_spmm(vt, B))).abs().max().item()
    assert err < tol, f"fused {act} error {err}"


@pytest.mark.parametrize("fn,ref,tol", [(void_spmm_gelu, torch.nn.functional.gelu, 0.01),
                                        (void_spmm_relu, torch.relu, 1e-5)])
def test_fused_bias_activation(gpu, small, fn, ref, tol):
    vt = csr_to_void(small, device="cuda")
    B = torch.randn(vt.shape[1], 64, device=gpu)
    bias = torch.randn(64, device=gpu)
    err = (fn(vt, B, bias=bias) - ref(void_spmm(vt, B) + bias)).abs().max().item()
    assert err < tol


def test_void_spmm_float_against_dense(gpu, small):
    vt = csr_to_void(small, device="cuda")
    B = np.random.default_rng(0).standard_normal((256, 64)).astype(np.float32)
    out = void_spmm(vt, torch.from_numpy(B).to(gpu)).cpu().numpy().astype(np.float64)
    want = small.toarray().astype(np.float64) @ B
    assert np.abs(out - want).max() < 1e-4


# tests/test_fusion.py:273-345 (shapes), plus values.
@pytest.mark.parametrize("act,bias,xshape", [("gelu", True, (32,)), ("relu", False, (4, 8)), ("none", True, (16,))])
def test_fused_sparse_linear(gpu, small, act, bias, xshape):
    vt = csr_to_void(small, device="cuda")
    M, K = vt.shape
    layer = FusedSparseLinear(in_features=K, out_features=M, void_tensor=vt, activation=act, bias=bias).to(gpu)
    if bias:
        with torch.no_grad():
            layer.bias.copy_(torch.randn(M))
    x = torch.randn(*xshape, K, device=gpu)
    y = layer(x)
    assert y.shape == xshape + (M,)
    x64 = x.reshape(-1, K).double().cpu().numpy()
    h = small.toarray().astype(np.float64) @ x64.T
    if bias:
        h += layer.bias.detach().double().cpu().numpy()[:, None]
    want = _ACT64[act](h).T.reshape(xshape + (M,))
    assert np.abs(y.double().cpu().numpy() - want).max() < 1e-4


def test_activation_codes():
    """tests/test_fusion.py:350-362 (no device work)."""
    assert [get_activation_code(a) for a in ("none", "relu", "gelu", "silu", "swish")] == [0, 1, 2, 3, 3]
    assert get_activation_code(ActivationType.RELU) == 1 and get_activation_code(ActivationType.GELU) == 2


# tests/test_fp8.py:209-238.  The reference's statistic (mean of
# |C32 - C8| / (|C32| + 1e-6)) is ruled by the few outputs near zero, so B
# is drawn from a fixed CPU seed, and the product is also held to the
# oracle's restatement of the reference's float-B FP8 SpMM (B stays fp32).
def test_fp8_spmm_against_fp32(gpu, small):
    import oracle
    from void_amd.fp8 import FP8VOIDTensor, void_spmm_fp8
    vt = csr_to_void(small, device="cuda")
    torch.manual_seed(0)
    B = torch.randn(vt.shape[1], 64, dtype=torch.float32)
    c_ref = void_spmm(vt, B.to(gpu))
    f8 = FP8VOIDTensor.from_void_tensor(vt)
    c8 = void_spmm_fp8(f8, B.to(gpu), output_dtype=torch.float32)
    rel = ((c_ref - c8).abs() / (c_ref.abs() + 1e-6)).mean().item()
    assert rel < 0.3, rel

    A = oracle.Bsr(f8.values_fp8.view(torch.uint8).cpu().numpy(), f8.scaling_info.scale.cpu().numpy(),
                   vt.block_rows.cpu().numpy(), vt.block_cols.cpu().numpy(), vt.shape)
    want = oracle.fp8_spmm_float_b(A, B.numpy())
    Aabs = oracle.Bsr.__new__(oracle.Bsr)
    Aabs.__dict__.update(A.__dict__)
    Aabs.tiles = np.ascontiguousarray(A.tiles.view(np.uint8) & 0x7F)
    bound = oracle.fp8_spmm_float_b(Aabs, np.abs(B.numpy()))
    err = np.abs(c8.cpu().numpy().astype(np.float64) - want)
    assert np.all(err <= 2.0 ** -13 * bound + 1e-30), (err / (bound + 1e-30)).max()


def test_to_fp8_keeps_blocks(gpu, small):
    vt = csr_to_void(small, device="cuda")
    assert vt.to_fp8(format="e4m3", scale_mode="per_block").n_blocks == vt.n_blocks
    assert void_amd.FP8VOIDTensor is not None
