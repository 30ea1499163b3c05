"""Device-side tile quantisers (void_quantize_tiles_i8 / _fp8) against the
oracle and the host path, bit for bit, including the rounding edge cases:
ties to even, saturation at +-amax, all-zero tiles, E4M3 subnormals and
midpoints, and the largest finite E4M3 value."""

import numpy as np
import pytest
import torch

import cases
import oracle
import void_amd
from void_amd import _runtime

pytestmark = pytest.mark.gpu


def _edge_tiles(rng):
    n = 48
    t = rng.standard_normal((n, 32, 32)).astype(np.float32)
    t[0] = 0.0                                          # scale floor (1e-8 / 1e-12)
    t[1] *= 1e-30                                       # tiny amax
    t[2, 0, 0] = 1e6                                    # one huge entry
    t[3] = np.abs(t[3])                                 # all positive
    t[4] = -np.abs(t[4])                                # all negative: -amax -> -128
    # INT8 ties: amax 128 -> s = 1 exactly; x = k + 0.5 must round to even.
    t[5] = (np.arange(1024).reshape(32, 32) % 255 - 127).astype(np.float32) + 0.5
    t[5, 0, 0] = 128.0
    # E4M3 with amax 448 -> scale 1 exactly: every code's midpoints and subnormals.
    tab = oracle.e4m3_table()[:127].astype(np.float64)
    mids = ((tab[:-1] + tab[1:]) / 2).astype(np.float32)
    vals = np.concatenate([tab.astype(np.float32), mids, -mids, np.float32([2.0 ** -10, 2.0 ** -9 * 1.5, 447.9])])
    t[6].reshape(-1)[:len(vals)] = vals
    t[6, 31, 31] = 448.0
    t[7] *= 1e-3                                        # many values in the E4M3 subnormal range after scaling
    t[8, :, :16] = 0.0
    return t


def test_device_int8_tiles_bit_exact(gpu):
    tiles = _edge_tiles(np.random.default_rng(0))
    q, s = _runtime.quantize_tiles_i8(torch.from_numpy(tiles).to(gpu))
    oq, os_ = oracle.quantize_i8_blocks(tiles)
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(s.cpu().numpy().view(np.int32), os_.view(np.int32))


def test_device_fp8_tiles_bit_exact(gpu):
    tiles = _edge_tiles(np.random.default_rng(1))
    x = torch.from_numpy(tiles).to(gpu)
    q, s, amax = _runtime.quantize_tiles_fp8(x)
    oq, os_ = oracle.quantize_fp8_blocks(tiles)
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(s.cpu().numpy().view(np.int32), os_.view(np.int32))
    assert np.array_equal(amax.cpu().numpy(), np.abs(tiles).reshape(len(tiles), -1).max(axis=1))
    # and against torch's own cast on the GPU (the reference's quantize_to_fp8 arithmetic)
    inv = 1.0 / s
    ref = torch.clamp(x * inv.view(-1, 1, 1), -448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(q, ref)


def test_public_api_device_matches_host(gpu):
    case = cases.uniform_blocks(1024, 2048, 64, 700, seed=12)
    vt = cases.make_void_tensor(case, "cpu")
    host = void_amd.quantize_void_tensor(vt)
    dev = void_amd.quantize_void_tensor(vt.to(gpu))
    assert dev.values.is_cuda
    assert torch.equal(dev.values.cpu(), host.values) and torch.equal(dev.scales.cpu(), host.scales)
    f_host = void_amd.void_tensor_to_fp8(vt)
    f_dev = void_amd.void_tensor_to_fp8(vt.to(gpu))
    assert torch.equal(f_dev.values_fp8.view(torch.uint8).cpu(), f_host.values_fp8.view(torch.uint8))
    for name in ("scale", "scale_inv", "amax"):
        assert torch.equal(getattr(f_dev.scaling_info, name).cpu(), getattr(f_host.scaling_info, name)), name
    # The device-quantised operands feed the SpMM unchanged.
    bq, bs = oracle.quantize_i8_columns(case.b)
    out = void_amd.void_spmm_int8(dev, torch.from_numpy(bq).to(gpu), b_scale=torch.from_numpy(bs).to(gpu),
                                  epilogue="raw_i32")
    A = oracle.Bsr(host.values.numpy(), host.scales.numpy(), case.block_rows, case.block_cols, (case.M, case.K))
    assert np.array_equal(out.cpu().numpy(), oracle.i8_acc(A, bq))


@pytest.mark.parametrize("shape,kind", [((4096, 512), "normal"), ((1000, 37), "normal"), ((3, 5), "normal"),
                                        ((256, 64), "ties"), ((128, 128), "zeros"), ((77, 1), "negmax"),
                                        ((64, 300), "wide")])
def test_device_b_per_tensor_bit_exact(gpu, shape, kind):
    """void_quantize_b_i8 (a float B's per-tensor INT8 quantisation, on the
    device) gives quantize_tensor's codes and scale bit for bit: scale =
    max|b| / 128 clamped at 1e-8, rint of an IEEE division, clamped to
    [-128, 127]; halfway quotients, an all-zero B, a negative extreme and
    odd element counts (a tail after the 16-byte loads) included."""
    from void_amd.int_quant import _quantize_b_per_tensor, quantize_tensor, IntQuantConfig, IntFormat, ScaleMode
    g = torch.Generator().manual_seed(sum(shape))
    b = torch.randn(shape, generator=g)
    if kind == "ties":
        b = (torch.randint(-300, 300, shape, generator=g).float() + 0.5) * (6.0 / 128)
        b[0, 0] = 6.0  # max |b| = 6: quotients b / (6 / 128) land on halves
    elif kind == "zeros":
        b = torch.zeros(shape)
    elif kind == "negmax":
        b[5, 0] = -40.0
    elif kind == "wide":
        b = b * torch.exp2(torch.randint(-30, 30, shape, generator=g).float())
    cfg = IntQuantConfig(format=IntFormat.INT8, symmetric=True, scale_mode=ScaleMode.PER_TENSOR)
    ref_q, ref_p = quantize_tensor(b, cfg)
    q, scale = _quantize_b_per_tensor(b.to(gpu))
    assert torch.equal(q.cpu(), ref_q)
    assert torch.equal(scale.cpu().view(torch.int32), ref_p.scale.reshape(1).view(torch.int32))


def test_device_b_per_tensor_nan(gpu):
    """A NaN in a float B makes quantize_tensor's scale NaN (torch.clamp keeps
    NaN); the device quantiser keeps it too, so void_spmm_int8 with that B
    gives NaN on every row that has tiles, as the reference's NaN scale does,
    and zeros on empty rows."""
    from void_amd.int_quant import _quantize_b_per_tensor, quantize_tensor, IntQuantConfig, IntFormat, ScaleMode
    b = torch.randn(256, 64, generator=torch.Generator().manual_seed(11))
    b[17, 3] = float("nan")
    cfg = IntQuantConfig(format=IntFormat.INT8, symmetric=True, scale_mode=ScaleMode.PER_TENSOR)
    _, ref_p = quantize_tensor(b, cfg)
    assert torch.isnan(ref_p.scale).all()
    _, scale = _quantize_b_per_tensor(b.to(gpu))
    assert torch.isnan(scale.cpu()).all()
    case = cases.uniform_blocks(128, 256, 64, 12, seed=3)
    q = void_amd.quantize_void_tensor(cases.make_void_tensor(case, "cpu"))
    out = void_amd.void_spmm_int8(q.to(gpu), b.to(gpu)).cpu()
    has = np.zeros(4, bool)
    has[np.unique(case.block_rows)] = True
    rows = torch.from_numpy(np.repeat(has, 32))
    assert torch.isnan(out[rows]).all() and (out[~rows] == 0).all()
