"""Pinning of the CPU oracle (oracle/) against independent computations.

Each oracle function is checked against something that does not restate
it: the reference's own known answers (test_fp8.py:51-67, 133-150),
hand-computed cases, numpy int64 / float64 dense products, torch's
float8_e4m3fn conversion and torch's tanh GELU.
"""

import math

import numpy as np
import pytest
import torch

import oracle

RNG = np.random.default_rng(1234)


# ---------------------------------------------------------------- Morton

def test_morton_known_values():
    # x bits to even positions, y bits to odd positions (format.py:41-51)
    assert int(oracle.morton_encode(np.array([0]), np.array([0]))[0]) == 0
    assert int(oracle.morton_encode(np.array([1]), np.array([0]))[0]) == 1
    assert int(oracle.morton_encode(np.array([0]), np.array([1]))[0]) == 2
    assert int(oracle.morton_encode(np.array([1]), np.array([1]))[0]) == 3
    # x = 3 (0b011) -> 1 + 4 = 5 ; y = 5 (0b101) -> 2 + 32 = 34
    assert int(oracle.morton_encode(np.array([3]), np.array([5]))[0]) == 39
    assert int(oracle.morton_encode(np.array([0xFFFF]), np.array([0]))[0]) == 0x55555555


def test_morton_is_a_bijection_and_orders_quadrants():
    r, c = np.meshgrid(np.arange(64), np.arange(64), indexing="ij")
    codes = oracle.morton_encode(r.ravel(), c.ravel())
    assert len(np.unique(codes)) == 64 * 64
    assert codes.max() == 64 * 64 - 1
    # Z-order: the 32x32 quadrant (0,0) precedes (row 0..31, col 32..63), then rows 32..63
    q00 = codes[(r.ravel() < 32) & (c.ravel() < 32)]
    q01 = codes[(r.ravel() < 32) & (c.ravel() >= 32)]
    q10 = codes[(r.ravel() >= 32) & (c.ravel() < 32)]
    assert q00.max() < q10.min() and q10.max() < q01.min()


# ---------------------------------------------------------------- format

def test_csr_tiles_roundtrip():
    dense = np.where(RNG.random((100, 77)) < 0.05, RNG.standard_normal((100, 77)), 0).astype(np.float32)
    tiles, br, bc = oracle.csr_tiles(dense)
    assert np.array_equal(oracle.densify(tiles, br, bc, dense.shape), dense)
    # every active tile holds a nonzero, every nonzero lies in an active tile
    assert all(np.any(t != 0) for t in tiles)
    assert len(tiles) == len({(r // 32, c // 32) for r, c in zip(*np.nonzero(dense))})
    codes = oracle.morton_encode(br, bc)
    assert np.all(np.diff(codes.astype(np.int64)) > 0)


def test_bsr_order_rows_then_columns():
    br = np.array([3, 0, 3, 1, 0], np.int32)
    bc = np.array([5, 9, 1, 0, 2], np.int32)
    order, row_ptr = oracle.bsr_order(br, bc, 4)
    assert list(row_ptr) == [0, 2, 3, 3, 5]
    assert list(zip(br[order], bc[order])) == [(0, 2), (0, 9), (1, 0), (3, 1), (3, 5)]


# ---------------------------------------------------------------- INT8 quantisation

def test_quantize_i8_hand_cases():
    blk = np.zeros((1, 32, 32), np.float32)
    blk[0, 0, 0] = 1.0       # amax -> scale = 1/128 exactly
    blk[0, 0, 1] = -1.0
    blk[0, 0, 2] = 0.5
    blk[0, 0, 3] = 2.5 / 128  # tie -> round half to even -> 2
    blk[0, 0, 4] = 3.5 / 128  # tie -> 4
    blk[0, 0, 5] = -2.5 / 128
    q, s = oracle.quantize_i8_blocks(blk)
    assert s[0] == np.float32(1.0 / 128)
    assert list(q[0, 0, :6]) == [127, -128, 64, 2, 4, -2]   # +128 saturates to 127
    zq, zs = oracle.quantize_i8_blocks(np.zeros((1, 32, 32), np.float32))
    assert zs[0] == np.float32(1e-8) and not zq.any()


def test_quantize_i8_tensor_and_columns_hand():
    x = np.array([[1.0, -4.0], [-2.0, 3.0]], np.float32)
    q, s = oracle.quantize_i8_tensor(x)
    assert s == np.float32(4.0 / 128) and q.tolist() == [[32, -128], [-64, 96]]
    qc, sc = oracle.quantize_i8_columns(x)
    assert sc.tolist() == [np.float32(2.0 / 128), np.float32(4.0 / 128)]
    assert qc.tolist() == [[64, -128], [-128, 96]]


# ---------------------------------------------------------------- SpMM (C)

def _random_bsr(M, K, density, seed, amax=1.0):
    rng = np.random.default_rng(seed)
    dense = np.where(rng.random((M, K)) < density, rng.standard_normal((M, K)) * amax, 0).astype(np.float32)
    tiles, br, bc = oracle.csr_tiles(dense)
    q, s = oracle.quantize_i8_blocks(tiles)
    return q, s, br, bc


def _dense_int(q, br, bc, shape):
    return oracle.densify(q.astype(np.int64), br, bc, shape)


@pytest.mark.parametrize("M,K,N", [(64, 96, 40), (100, 70, 33), (256, 256, 64)])
def test_i8_acc_equals_dense_int64(M, K, N):
    q, s, br, bc = _random_bsr(M, K, 0.1, M + K)
    B = RNG.integers(-128, 128, size=(K, N), dtype=np.int8)
    A = oracle.Bsr(q, s, br, bc, (M, K))
    acc = oracle.i8_acc(A, B)
    ref = _dense_int(q, br, bc, (M, K)) @ B.astype(np.int64)
    assert acc.dtype == np.int32 and np.array_equal(acc, ref)


def test_i8_acc_overflow_detected():
    n = 4200  # 4200 * 32 * 127 * 127 = 2.17e9 > 2^31 - 1
    q = np.full((n, 32, 32), 127, np.int8)
    br = np.zeros(n, np.int32)
    bc = np.arange(n, dtype=np.int32)
    A = oracle.Bsr(q, np.ones(n, np.float32), br, bc, (32, n * 32))
    B = np.full((n * 32, 1), 127, np.int8)
    with pytest.raises(OverflowError):
        oracle.i8_acc(A, B)


def test_row_mean_hand_case():
    # one block-row, two tiles with scales 0.5 and 0.25, b_scale 2 -> S = 1 + 0.5, avg = 0.75
    q = np.zeros((2, 32, 32), np.int8)
    q[0, 0, 0] = 3
    q[1, 0, 0] = 5
    A = oracle.Bsr(q, np.array([0.5, 0.25], np.float32), np.array([0, 0]), np.array([0, 1]), (32, 64))
    B = np.zeros((64, 4), np.int8)
    B[0, 0] = 7
    B[32, 0] = 11
    acc = oracle.i8_acc(A, B)
    assert acc[0, 0] == 3 * 7 + 5 * 11
    out = oracle.row_mean(A, acc, np.float32(2.0))
    assert out[0, 0] == np.float32(76 * 0.75)
    assert not out[1:].any() and not out[:, 1:].any()


def test_row_mean_equals_per_block_when_scales_equal():
    q, _, br, bc = _random_bsr(128, 192, 0.2, 7)
    s = np.full(len(br), 0.0123, np.float32)
    B = RNG.integers(-128, 128, size=(192, 24), dtype=np.int8)
    A = oracle.Bsr(q, s, br, bc, (128, 192))
    rm = oracle.row_mean(A, oracle.i8_acc(A, B), np.float32(0.5))
    pb = oracle.i8_per_block(A, B, np.float32(0.5))
    assert np.allclose(rm, pb, rtol=2e-6, atol=0)


def test_per_block_equals_dense_float64():
    q, s, br, bc = _random_bsr(96, 160, 0.15, 11, amax=3.0)
    B = RNG.integers(-128, 128, size=(160, 20), dtype=np.int8)
    sb = RNG.random(20).astype(np.float32) + 0.01
    A = oracle.Bsr(q, s, br, bc, (96, 160))
    got = oracle.i8_per_block(A, B, sb)
    deq = oracle.densify(q.astype(np.float64) * s.astype(np.float64)[:, None, None], br, bc, (96, 160))
    ref = (deq @ B.astype(np.float64)) * sb.astype(np.float64)[None, :]
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- FP8 E4M3FN

def test_e4m3_decode_matches_torch_all_codes():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).to(torch.float64).numpy()
    tab = oracle.e4m3_table()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(tab), nan) and nan.sum() == 2
    assert np.array_equal(tab[~nan], ref[~nan])


def test_fp8_limits_known_answers():
    # test_fp8.py:51-67: E4M3 max 448
    tab = oracle.e4m3_table()
    assert np.nanmax(tab) == 448.0 and np.nanmin(tab) == -448.0
    assert tab[1] == 2.0 ** -9  # smallest subnormal


def test_e4m3_encode_matches_torch():
    tab = oracle.e4m3_table()[:127]
    mids = (tab[1:] + tab[:-1]) / 2  # exact ties between neighbours
    x = np.concatenate([
        RNG.uniform(-448, 448, 20000), RNG.standard_normal(20000) * 1e-2,
        tab, -tab, mids, -mids, [0.0, -0.0, 448.0, -448.0, 1e-9, -1e-9],
    ]).astype(np.float32)
    x = np.clip(x, -448, 448)
    got = oracle.e4m3_encode(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, ref)


def test_compute_amax_known_answers():
    # test_fp8.py:133-150
    t = np.array([[[1.0, 2.0], [3.0, 4.0]], [[5.0, 6.0], [7.0, 8.0]]], np.float32)
    blocks = np.zeros((2, 32, 32), np.float32)
    blocks[:, :2, :2] = t
    _, scales = oracle.quantize_fp8_blocks(blocks)
    assert np.array_equal(scales, (np.array([4.0, 8.0], np.float32) / np.float32(448)).astype(np.float32))


def test_quantize_fp8_tensor_known_answers():
    # Per-tensor amax of the reference's tensor is 8.0 (test_fp8.py:142-143),
    # so the scale is fl(8 / 448) and x * (1 / scale) is 56 x up to an ulp.
    t = np.array([[[1.0, 2.0], [3.0, 4.0]], [[5.0, 6.0], [7.0, 8.0]]], np.float32)
    codes, s = oracle.quantize_fp8_tensor(t)
    assert s == np.float32(np.float32(8.0) / np.float32(448.0))
    # Hand-encoded E4M3FN (bias 7): 56 = 1.75 * 2^5 -> 0 1100 110, 112 -> 0 1101 110,
    # 168 = 1.3125 * 2^7 -> nearest 1.25 * 2^7 = 160 (0 1110 010) or 1.375 * 2^7 = 176
    # (0 1110 011): 168 is the midpoint, ties to the even mantissa 010; 224 -> 0 1110 110,
    # 280 = 1.09375 * 2^8 -> 1.125 * 2^8 = 288 (0 1111 001) is nearest; 336 = 1.3125 * 2^8
    # -> tie between 320 (0 1111 010) and 352 (0 1111 011): even, 0x7A; 392 -> tie between
    # 384 (0 1111 100) and 416 (0 1111 101): 0x7C; 448 -> 0 1111 110.
    expect = np.array([[[0x66, 0x6E], [0x72, 0x76]], [[0x79, 0x7A], [0x7C, 0x7E]]], np.uint8)
    assert np.array_equal(codes, expect), codes
    # Signs, zero and the all-zero tensor (scale clamped at 1e-12).
    codes, s = oracle.quantize_fp8_tensor(np.array([-8.0, 0.0, 8.0], np.float32))
    assert list(codes) == [0xFE, 0x00, 0x7E]
    codes, s = oracle.quantize_fp8_tensor(np.zeros(4, np.float32))
    assert s == np.float32(1e-12) and not codes.any()


def test_fp8_spmm_equals_dense_float64():
    rng = np.random.default_rng(5)
    dense = np.where(rng.random((64, 128)) < 0.2, rng.standard_normal((64, 128)), 0).astype(np.float32)
    tiles, br, bc = oracle.csr_tiles(dense)
    codes, s = oracle.quantize_fp8_blocks(tiles)
    Bc, bs = oracle.quantize_fp8_tensor(rng.standard_normal((128, 48)).astype(np.float32))
    A = oracle.Bsr(codes, s, br, bc, (64, 128))
    got = oracle.fp8_spmm(A, Bc, bs)
    tab = oracle.e4m3_table()
    deq = oracle.densify(tab[codes.astype(np.int64)] * s.astype(np.float64)[:, None, None], br, bc, (64, 128))
    ref = deq @ tab[Bc.astype(np.int64)] * np.float64(bs)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_fp8_spmm_float_b_equals_dense_float64():
    # The reference's FP8 SpMM with a float B (fp8.py:624-671): E4M3 tiles
    # decoded and scaled per tile, B kept in fp32.  Against a numpy float64
    # dense product, on a ragged shape with per-column B scales.
    rng = np.random.default_rng(8)
    M, K, N = 70, 100, 37
    dense = np.where(rng.random((M, K)) < 0.25, rng.standard_normal((M, K)) * 5, 0).astype(np.float32)
    tiles, br, bc = oracle.csr_tiles(dense)
    codes, s = oracle.quantize_fp8_blocks(tiles)
    B = rng.standard_normal((K, N)).astype(np.float32)
    sb = rng.uniform(0.5, 2.0, N).astype(np.float32)
    A = oracle.Bsr(codes, s, br, bc, (M, K))
    got = oracle.fp8_spmm_float_b(A, B, sb)
    tab = oracle.e4m3_table()
    deq = oracle.densify(tab[codes.astype(np.int64)] * s.astype(np.float64)[:, None, None], br, bc, (M, K))
    ref = (deq @ B.astype(np.float64)) * sb.astype(np.float64)[None, :]
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    # With B holding exactly the values of E4M3 codes it is the FP8 x FP8 product.
    Bc, bs = oracle.quantize_fp8_tensor(B)
    assert np.array_equal(oracle.fp8_spmm_float_b(A, tab[Bc.astype(np.int64)].astype(np.float32), 1.0),
                          oracle.fp8_spmm(A, Bc, 1.0))


# ---------------------------------------------------------------- GELU

def test_gelu_tanh_matches_torch():
    x = np.linspace(-12, 12, 20001)
    ref = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    # the reference's constant 0.7978845608 is sqrt(2/pi) to 10 digits
    assert np.allclose(oracle.gelu_tanh(x), ref, rtol=1e-9, atol=1e-12)
    assert abs(0.7978845608 - math.sqrt(2 / math.pi)) < 1e-10


def test_cpu_baseline_matches_dense():
    rng = np.random.default_rng(9)
    dense = np.where(rng.random((128, 96)) < 0.2, rng.standard_normal((128, 96)), 0).astype(np.float32)
    tiles, br, bc = oracle.csr_tiles(dense)
    q, s = oracle.quantize_i8_blocks(tiles)
    B = rng.standard_normal((96, 40)).astype(np.float32)
    bq, bs = oracle.quantize_i8_columns(B)
    bdeq = torch.from_numpy(bq.astype(np.float32) * bs[None, :])
    got = oracle.cpu_baseline_spmm(torch.from_numpy(q.astype(np.float32)), torch.from_numpy(s),
                                   torch.from_numpy(bc.astype(np.int64)), torch.from_numpy(br.astype(np.int64)),
                                   bdeq, 128)
    A = oracle.Bsr(q, s, br, bc, (128, 96))
    ref = oracle.i8_per_block(A, bq, bs)
    assert np.allclose(got.numpy(), ref, rtol=1e-4, atol=1e-5)
