"""Operands beyond 2 GiB: the column-group kernels address with 31-bit buffer
offsets, so a B whose span passes 2^31 bytes runs the general kernel with
64-bit addresses.  B here is 70000 x 32800 int8 (2.29 GB, K % 32 != 0); the
tiles sit at far block columns, the last one ragged.  int32 accumulators are
checked bit-exactly on every output column against an integer product of the
B rows the tiles touch; the per-block output within 1e-5 of its bound."""

import numpy as np
import pytest
import torch

import void_amd

pytestmark = pytest.mark.gpu


def test_b_beyond_2gib(gpu):
    M, K, N = 96, 70000, 32800
    nbc = -(-K // 32)
    rows = np.array([0, 0, 1, 2, 2, 2])
    cols = np.array([0, 1000, 2100, 5, 1999, nbc - 1])
    rng = np.random.default_rng(31)
    dense = np.zeros((M, K), np.float32)
    for r, c in zip(rows, cols):
        w = min(32, K - 32 * c)
        dense[32 * r:32 * r + 32, 32 * c:32 * c + w] = rng.standard_normal((32, w))
    vt = void_amd.dense_to_void(torch.from_numpy(dense))
    q = void_amd.quantize_void_tensor(vt)
    g = torch.Generator(device=gpu).manual_seed(5)
    b = torch.randint(-128, 128, (K, N), dtype=torch.int8, device=gpu, generator=g)
    assert b.numel() > 2 ** 31
    bs = torch.rand(N, device=gpu, generator=g) * 0.01 + 0.001
    qd = q.to(gpu)
    raw = void_amd.void_spmm_int8(qd, b, b_scale=bs, epilogue="raw_i32")
    per = void_amd.void_spmm_int8(qd, b, b_scale=bs, epilogue="per_block")
    torch.cuda.synchronize()
    # Reference on the touched B rows only.
    qv = q.values.numpy().astype(np.int64)
    sc = q.scales.numpy().astype(np.float64)
    br, bc = vt.block_rows.numpy(), vt.block_cols.numpy()
    bsh = bs.double().cpu().numpy()
    acc = np.zeros((M, N), np.int64)
    ref = np.zeros((M, N), np.float64)
    bound = np.zeros((M, N), np.float64)
    for t in range(len(br)):
        k0, k1 = 32 * int(bc[t]), min(32 * int(bc[t]) + 32, K)
        bt = b[k0:k1].cpu().numpy().astype(np.int64)
        part = qv[t][:, :k1 - k0] @ bt
        acc[32 * br[t]:32 * br[t] + 32] += part
        ref[32 * br[t]:32 * br[t] + 32] += sc[t] * part * bsh[None, :]
        bound[32 * br[t]:32 * br[t] + 32] += sc[t] * (np.abs(qv[t][:, :k1 - k0]) @ np.abs(bt)) * bsh[None, :]
    assert np.array_equal(raw.cpu().numpy().astype(np.int64), acc)
    assert np.all(np.abs(per.cpu().numpy() - ref) <= 1e-5 * bound + 1e-30)


def test_fp8_float_b_beyond_2gib(gpu):
    """void_spmm_fp8 with an fp32 B of more than 2^31 bytes (70000 x 7700,
    ragged K, N % 4 == 0 and N % 128 != 0): the wrapper runs column slices
    that fit 31-bit offsets.  Checked against a float64 product of the B rows
    the tiles touch, within 2^-13 of sum |a b| (the fp32-B kernel's products
    are within 2^-16 of exact; its sums are fp32)."""
    M, K, N = 64, 70000, 7700
    nbc = -(-K // 32)
    rows = np.array([0, 0, 1, 1])
    cols = np.array([0, 1500, 7, nbc - 1])
    rng = np.random.default_rng(37)
    dense = np.zeros((M, K), np.float32)
    for r, c in zip(rows, cols):
        w = min(32, K - 32 * c)
        dense[32 * r:32 * r + 32, 32 * c:32 * c + w] = rng.standard_normal((32, w))
    vt = void_amd.dense_to_void(torch.from_numpy(dense))
    f8 = void_amd.void_tensor_to_fp8(vt)
    g = torch.Generator(device=gpu).manual_seed(6)
    b = torch.randn(K, N, device=gpu, generator=g)
    assert b.numel() * 4 > 2 ** 31
    bias = torch.randn(N, device=gpu, generator=g)
    out = void_amd.void_spmm_fp8(f8.to(gpu), b, output_dtype=torch.float32, bias=bias)
    torch.cuda.synchronize()
    codes = f8.values_fp8.float().numpy().astype(np.float64)
    sc = f8.scaling_info.scale.reshape(-1).double().numpy()
    br, bc = vt.block_rows.numpy(), vt.block_cols.numpy()
    ref = np.zeros((M, N), np.float64) + bias.double().cpu().numpy()[None, :]
    bound = np.zeros((M, N), np.float64)
    for t in range(len(br)):
        k0, k1 = 32 * int(bc[t]), min(32 * int(bc[t]) + 32, K)
        bt = b[k0:k1].double().cpu().numpy()
        ref[32 * br[t]:32 * br[t] + 32] += sc[t] * (codes[t][:, :k1 - k0] @ bt)
        bound[32 * br[t]:32 * br[t] + 32] += abs(sc[t]) * (np.abs(codes[t][:, :k1 - k0]) @ np.abs(bt))
    assert np.all(np.abs(out.cpu().numpy() - ref) <= 2.0 ** -13 * bound + 1e-6)
