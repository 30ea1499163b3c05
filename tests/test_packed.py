"""Packed BSR blob (void_amd.packed): layout, round trips and corruption
checks on the CPU; GPU loads and FusedSparseLinear on the GPU."""

import struct

import numpy as np
import pytest
import torch

import cases
import oracle
import void_amd
from void_amd import packed
from void_amd.int_quant import IntQuantConfig, ScaleMode


def _vt(seed=0, n=40):
    return cases.make_void_tensor(cases.uniform_blocks(200, 300, 64, n, seed=seed), "cpu")


def test_header_layout_known_answer():
    vt = _vt()
    blob = packed.pack(vt)
    magic, version, kind, M, K, nb, nbr, tile, flags, o_rp, o_ci, o_sc, o_ti, total, nnz = \
        struct.unpack_from("<8sIIqqqqIIQQQQQq", blob, 0)
    assert (magic, version, kind, M, K, nb, nbr, tile, flags) == (b"VOIDBSR\0", 1, 0, 200, 300, 40, 7, 32, 0)
    # sections follow the 256-byte header, each 256-aligned: row_ptr (8 ints), col_idx (40), no scales, tiles
    assert (o_rp, o_ci, o_sc) == (256, 512, 768) and o_ti == 768 and total == 768 + 40 * 4096
    order, rp = oracle.bsr_order(vt.block_rows.numpy(), vt.block_cols.numpy(), 7)
    assert np.array_equal(np.frombuffer(blob[o_rp:o_rp + 32], "<i4"), rp)
    assert np.array_equal(np.frombuffer(blob[o_ci:o_ci + 160], "<i4"), vt.block_cols.numpy()[order])
    tiles = np.frombuffer(blob[o_ti:total], "<f4").reshape(40, 32, 32)
    assert np.array_equal(tiles, vt.values.numpy()[order])


@pytest.mark.parametrize("kind", ["float", "bf16", "f16", "int8", "int8_tensor", "fp8"])
def test_round_trip_cpu(kind):
    vt = _vt(seed=3)
    if kind == "float":
        t = vt
    elif kind in ("bf16", "f16"):
        t = vt.to_dtype(torch.bfloat16 if kind == "bf16" else torch.float16)
    elif kind == "int8":
        t = void_amd.quantize_void_tensor(vt)
    elif kind == "int8_tensor":
        t = void_amd.quantize_void_tensor(vt, IntQuantConfig(scale_mode=ScaleMode.PER_TENSOR))
    else:
        t = void_amd.void_tensor_to_fp8(vt)
    u = packed.unpack(packed.pack(t))
    assert type(u) is type(t) and u.shape == t.shape and u.n_blocks == t.n_blocks
    assert torch.equal(u.block_rows, t.block_rows) and torch.equal(u.block_cols, t.block_cols)
    if kind == "fp8":
        assert torch.equal(u.values_fp8.view(torch.uint8), t.values_fp8.view(torch.uint8))
        assert torch.equal(u.scaling_info.scale, t.scaling_info.scale)
        assert torch.equal(u.morton_codes, t.morton_codes)
    elif kind in ("float", "bf16", "f16"):
        assert u.values.dtype == t.values.dtype and u.dtype == t.values.dtype
        assert torch.equal(u.values, t.values) and torch.equal(u.morton_codes, t.morton_codes)
    else:
        assert torch.equal(u.values, t.values) and torch.equal(u.scales, t.scales)
        assert u.config.scale_mode == t.config.scale_mode


def test_empty_tensor_round_trip(tmp_path):
    vt = void_amd.dense_to_void(torch.zeros(70, 40))
    path = tmp_path / "w.voidbsr"
    packed.save_packed(vt, path)
    u = packed.load_packed(path)
    assert u.n_blocks == 0 and u.shape == (70, 40)


def test_corrupt_blobs_are_rejected():
    blob = bytearray(packed.pack(_vt()))
    with pytest.raises(ValueError):
        packed.unpack(b"NOTVOID!" + bytes(blob[8:]))
    with pytest.raises(ValueError):
        packed.unpack(bytes(blob[:1000]))                      # truncated
    bad = bytearray(blob)
    struct.pack_into("<i", bad, 512, 10 ** 6)                  # block column out of range
    with pytest.raises(ValueError):
        packed.unpack(bytes(bad))
    bad = bytearray(blob)
    struct.pack_into("<i", bad, 256 + 4, 39)                   # row_ptr not ending at n_blocks / decreasing
    struct.pack_into("<i", bad, 256 + 8, 2)
    with pytest.raises(ValueError):
        packed.unpack(bytes(bad))


@pytest.mark.gpu
def test_gpu_load_feeds_kernels(gpu):
    case = cases.uniform_blocks(1024, 2048, 256, 700, seed=21)
    vt = cases.make_void_tensor(case, "cpu")
    q = void_amd.quantize_void_tensor(vt)
    qd = packed.unpack(packed.pack(q), gpu)
    assert qd.values.is_cuda and str(gpu) in qd._device_bsr
    bq, bs = oracle.quantize_i8_columns(case.b)
    out = void_amd.void_spmm_int8(qd, torch.from_numpy(bq).to(gpu), b_scale=torch.from_numpy(bs).to(gpu),
                                  epilogue="raw_i32")
    A = oracle.Bsr(q.values.numpy(), q.scales.numpy(), case.block_rows, case.block_cols, (case.M, case.K))
    assert np.array_equal(out.cpu().numpy(), oracle.i8_acc(A, bq))
    # The unpacked tensor's device copy follows in-place changes of its values
    # (gathered again through the recorded order).
    qd.values.neg_()
    qd.values.clamp_(-127, 127)
    out2 = void_amd.void_spmm_int8(qd, torch.from_numpy(bq).to(gpu), b_scale=torch.from_numpy(bs).to(gpu),
                                   epilogue="raw_i32")
    A2 = oracle.Bsr(qd.values.cpu().numpy(), q.scales.numpy(), case.block_rows, case.block_cols, (case.M, case.K))
    assert np.array_equal(out2.cpu().numpy(), oracle.i8_acc(A2, bq))


@pytest.mark.gpu
@pytest.mark.parametrize("act", ["gelu", "relu"])
def test_fused_sparse_linear(gpu, act):
    case = cases.uniform_blocks(256, 512, 64, 60, seed=4)   # W: 256 out x 512 in
    vt = cases.make_void_tensor(case, "cpu")
    layer = void_amd.FusedSparseLinear.from_packed(packed.pack(vt), device=gpu, activation=act)
    with torch.no_grad():
        layer.bias.copy_(torch.randn(256))
    x = torch.randn(3, 7, 512, device=gpu)
    y = layer(x)
    assert y.shape == (3, 7, 256)
    W = oracle.densify(case.tiles, case.block_rows, case.block_cols, (256, 512)).astype(np.float64)
    pre = x.reshape(-1, 512).cpu().double().numpy() @ W.T + layer.bias.detach().cpu().double().numpy()[None, :]
    ref = oracle.gelu_tanh(pre) if act == "gelu" else np.maximum(pre, 0)
    n = 32 * np.bincount(case.block_rows).max() + 2
    bound = 1.2 * n * 2.0 ** -24 * (np.abs(x.reshape(-1, 512).cpu().double().numpy()) @ np.abs(W).T
                                   + np.abs(layer.bias.detach().cpu().double().numpy())[None, :])
    err = np.abs(y.reshape(-1, 256).detach().cpu().double().numpy() - ref)
    assert np.all(err <= bound + 8 * 2.0 ** -24 * np.abs(ref) + 1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gpu_load_16bit_feeds_kernel(gpu, dtype):
    """A 16-bit blob loads as a 16-bit tensor whose prebuilt device copy the
    16-bit SpMM uses directly, with the same bits as the tensor it came
    from; FusedSparseLinear over it runs in that dtype."""
    case = cases.uniform_blocks(256, 512, 64, 60, seed=4)
    vt = cases.make_void_tensor(case, "cpu").to_dtype(dtype)
    u = packed.unpack(packed.pack(vt), gpu)
    assert u.values.dtype == dtype and set(u._device_bsr) == {f"{gpu}/{dtype}"}
    b = torch.from_numpy(case.b).to(dtype).to(gpu)
    got = void_amd.void_spmm(u, b)
    ref = void_amd.void_spmm(vt.to(gpu), b)
    assert torch.equal(got, ref)
    layer = void_amd.FusedSparseLinear.from_packed(packed.pack(vt), device=gpu, activation="relu").to(dtype)
    x = torch.randn(5, 512, device=gpu).to(dtype)
    y = layer(x)
    assert y.dtype == dtype
    W = vt.values.float()
    Wd = oracle.densify(W.numpy(), case.block_rows, case.block_cols, (256, 512)).astype(np.float64)
    X = x.double().cpu().numpy()
    pre = X @ Wd.T + layer.bias.detach().double().cpu().numpy()[None, :]
    ref = np.maximum(pre, 0)
    n = 32 * np.bincount(case.block_rows).max() + 1
    rel = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    bound = n * 2.0 ** -24 * (np.abs(X) @ np.abs(Wd).T + np.abs(layer.bias.detach().double().cpu().numpy())) \
        + rel * np.abs(ref) + 2.0 ** -24
    assert np.all(np.abs(y.double().cpu().numpy() - ref) <= bound)
