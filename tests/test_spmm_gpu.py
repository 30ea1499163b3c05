"""GPU parity of the gfx950 SpMM kernels against the CPU oracle.

Bars: int32 accumulators bit-exact; the row-mean epilogue bit-exact against
the oracle's fp32 restatement (within 1e-5 of the reference, whose Triton
divide may differ by an ulp); per-block dequantised fp32 within
1e-5 * (sum_t |s_t P_t|) elementwise; FP8 within FP8_TOL of the scale of
the product terms (sum |a b|); bf16 outputs within one bf16 rounding (2^-8
relative) plus the fp32 bound.
"""

import numpy as np
import pytest
import torch

import cases
import oracle
import void_amd
from void_amd import _lib

pytestmark = pytest.mark.gpu

# The fp8 MFMA (v_mfma_f32_32x32x16_fp8_fp8) sums its 16 exact E4M3 products
# with less than fp32 precision: measured deviations from the exact
# (float64) sum reach 2e-5 of sum |a b| on K = 70, against ~1e-7 for fp32
# arithmetic.  Both kernels show the same deviation.  The bound below
# (2^-13, about 1.2e-4) is two orders tighter than the 2e-2 the FP8 path is
# specified to, and far below any indexing or scaling mistake.
FP8_TOL = 2.0 ** -13


@pytest.fixture(params=["cgd", "cgd3", "cgdk", "bsr"])
def kernel(request, monkeypatch):
    """Runs a test on each SpMM kernel: the column-group kernel with its
    LDS-DMA ring of 4 tiles per stage (=cgd; column-major B runs the
    register-staged loop, its only default use), the 3-tile ring that unsplit
    grids beyond 512 workgroups take by default (=cgd3), the two-ring 8-wave
    workgroups that grids of at most 512 workgroups and plans with split rows
    take (=cgdk), and the general kernel (=bsr)."""
    monkeypatch.setenv("VOID_AMD_KERNEL", request.param)
    return request.param


def _int8_setup(case, dev, b_per_column=True):
    vt = cases.make_void_tensor(case, "cpu")
    q = void_amd.quantize_void_tensor(vt)
    qd = q.to(dev)
    if b_per_column:
        bq, bs = oracle.quantize_i8_columns(case.b)
    else:
        bq, bs = oracle.quantize_i8_tensor(case.b)
    A = oracle.Bsr(q.values.numpy(), q.scales.numpy(), case.block_rows, case.block_cols, (case.M, case.K))
    return qd, A, bq, bs


def _abs_bound(A, bq, bs):
    # sum_t s_t |A_t| @ |B| * |s_b| in float64 via the per-block oracle on absolute values.
    tiles = np.abs(A.tiles.astype(np.int16)).clip(0, 127).astype(np.int8)
    Aabs = oracle.Bsr.__new__(oracle.Bsr)
    Aabs.__dict__.update(A.__dict__)
    Aabs.tiles = np.ascontiguousarray(tiles)
    return oracle.i8_per_block(Aabs, np.abs(bq.astype(np.int16)).clip(0, 127).astype(np.int8), np.abs(bs))


def test_c1_plumbing_int8(gpu):
    Acsr, B = cases.c1_plumbing()
    vt = void_amd.csr_to_void(Acsr)
    q = void_amd.quantize_void_tensor(vt)
    qd = q.to(gpu)
    Bt = torch.from_numpy(B).to(gpu)
    # Reference path: float B quantised per tensor inside void_spmm_int8.
    c = void_amd.void_spmm_int8(qd, Bt)
    torch.cuda.synchronize()
    bq, bs = oracle.quantize_i8_tensor(B)
    A = oracle.Bsr(q.values.numpy(), q.scales.numpy(), vt.block_rows.numpy(), vt.block_cols.numpy(), (512, 512))
    acc = oracle.i8_acc(A, bq)
    ref = oracle.row_mean(A, acc, bs)
    got = c.cpu().numpy()
    assert np.array_equal(got.view(np.int32), ref.view(np.int32)), np.abs(got - ref).max()
    raw = void_amd.void_spmm_int8(qd, torch.from_numpy(bq).to(gpu), b_scale=float(bs), epilogue="raw_i32")
    assert np.array_equal(raw.cpu().numpy(), acc)


@pytest.mark.parametrize("epilogue", ["raw_i32", "row_mean", "per_block"])
def test_c2_int8_full(gpu, epilogue, kernel):
    case = cases.c2_int8()
    qd, A, bq, bs = _int8_setup(case, gpu)
    bt = torch.from_numpy(bq).to(gpu)
    st = torch.from_numpy(bs).to(gpu)
    out = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue=epilogue)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    acc = oracle.i8_acc(A, bq)
    if epilogue == "raw_i32":
        assert np.array_equal(got, acc)
    elif epilogue == "row_mean":
        ref = oracle.row_mean(A, acc, bs)
        assert np.array_equal(got.view(np.int32), ref.view(np.int32)), np.abs(got - ref).max()
    else:
        ref = oracle.i8_per_block(A, bq, bs)
        bound = _abs_bound(A, bq, bs)
        err = np.abs(got.astype(np.float64) - ref)
        assert np.all(err <= 1e-5 * bound + 1e-30), (err / (bound + 1e-30)).max()


_C3_CACHE = {}


def _c3_fp8_setup():
    """c3's FP8 A, its E4M3 B and the oracle's product and error scale, computed once."""
    if not _C3_CACHE:
        case = cases.c3_fp8()
        vt = cases.make_void_tensor(case, "cpu")
        f8 = void_amd.void_tensor_to_fp8(vt)
        bq, bs = oracle.quantize_fp8_tensor(case.b)
        A = oracle.Bsr(f8.values_fp8.view(torch.uint8).numpy(), f8.scaling_info.scale.numpy(),
                       case.block_rows, case.block_cols, (case.M, case.K))
        Aabs = oracle.Bsr.__new__(oracle.Bsr)
        Aabs.__dict__.update(A.__dict__)
        Aabs.tiles = np.ascontiguousarray(A.tiles.view(np.uint8) & 0x7F)
        _C3_CACHE.update(case=case, f8=f8, bq=bq, bs=bs, ref=oracle.fp8_spmm(A, bq, bs),
                         bound=oracle.fp8_spmm(Aabs, bq & 0x7F, abs(bs)))
    return _C3_CACHE


# One rounding of the output type on top of the fp32 bound: round to
# nearest even moves a value by at most the unit roundoff 2^-p relative (p
# significand bits: 8 for bf16, 11 for fp16), plus half of fp16's subnormal
# spacing.
_OUT_ROUNDING = {torch.float32: (0.0, 0.0), torch.bfloat16: (2.0 ** -8, 0.0), torch.float16: (2.0 ** -11, 2.0 ** -25)}


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16],
                         ids=["f32", "bf16", "f16"])
def test_c3_fp8_full(gpu, kernel, out_dtype):
    """Config 3 at full size (4096^2 at 80 % block sparsity, E4M3 A and B,
    N = 512) in each output type: bf16 as the config states, fp16 as the
    reference's void_spmm_fp8 defaults to (fp8.py:677), and fp32."""
    d = _c3_fp8_setup()
    bt = torch.from_numpy(d["bq"]).to(gpu).view(torch.float8_e4m3fn)
    out = void_amd.void_spmm_fp8(d["f8"].to(gpu), bt, output_dtype=out_dtype, b_scale=float(d["bs"]))
    torch.cuda.synchronize()
    assert out.dtype == out_dtype
    ref, bound = d["ref"], d["bound"]
    rel, ab = _OUT_ROUNDING[out_dtype]
    err = np.abs(out.float().cpu().numpy().astype(np.float64) - ref)
    lim = FP8_TOL * bound * (1 + rel) + rel * np.abs(ref) + ab + 1e-30
    assert np.all(err <= lim), (err / lim).max()


@pytest.mark.parametrize("chunk", [None, 16])
def test_fp8_rows_beyond_64_tiles(gpu, kernel, chunk):
    """E4M3 block-rows of 65-96 tiles (per-block scales past the 64 a
    workgroup holds one per lane; chunk 16 splits them)."""
    case = cases.uniform_blocks(160, 3072, 256, 430, seed=12)
    f8 = void_amd.void_tensor_to_fp8(cases.make_void_tensor(case, "cpu"))
    bq, bs = oracle.quantize_fp8_tensor(case.b)
    A = oracle.Bsr(f8.values_fp8.view(torch.uint8).numpy(), f8.scaling_info.scale.numpy(),
                   case.block_rows, case.block_cols, (case.M, case.K))
    assert np.diff(A.row_ptr).max() > 64
    Aabs = oracle.Bsr.__new__(oracle.Bsr)
    Aabs.__dict__.update(A.__dict__)
    Aabs.tiles = np.ascontiguousarray(A.tiles.view(np.uint8) & 0x7F)
    ref, bound = oracle.fp8_spmm(A, bq, bs), oracle.fp8_spmm(Aabs, bq & 0x7F, abs(bs))
    bt = torch.from_numpy(bq).to(gpu).view(torch.float8_e4m3fn)
    out = void_amd.void_spmm_fp8(f8.to(gpu), bt, output_dtype=torch.float32, b_scale=float(bs), chunk_tiles=chunk)
    torch.cuda.synchronize()
    err = np.abs(out.cpu().numpy().astype(np.float64) - ref)
    assert np.all(err <= FP8_TOL * bound + 1e-30), (err / (FP8_TOL * bound + 1e-30)).max()


def test_fp8_default_output_is_fp16(gpu):
    """void_spmm_fp8 without output_dtype writes float16, as the reference."""
    case = cases.uniform_blocks(256, 512, 96, 40, seed=4)
    f8 = void_amd.void_tensor_to_fp8(cases.make_void_tensor(case, "cpu")).to(gpu)
    bq, bs = oracle.quantize_fp8_tensor(case.b)
    out = void_amd.void_spmm_fp8(f8, torch.from_numpy(bq).to(gpu).view(torch.float8_e4m3fn), b_scale=float(bs))
    assert out.dtype == torch.float16 and out.shape == (256, 96)


def test_c4_powerlaw_streamk_raw(gpu):
    case = cases.c4_powerlaw()
    qd, A, bq, bs = _int8_setup(case, gpu)
    bt = torch.from_numpy(bq).to(gpu)
    out = void_amd.void_spmm_int8(qd, bt, b_scale=torch.from_numpy(bs).to(gpu), epilogue="raw_i32")
    torch.cuda.synchronize()
    plan = qd.device_bsr().plans
    assert any(p.n_split_tiles > 0 for p in plan.values()), "c4 must exercise split rows"
    assert np.array_equal(out.cpu().numpy(), oracle.i8_acc(A, bq))


def test_c4_powerlaw_per_block_full(gpu, monkeypatch):
    """Config 4 exactly as benched: per-block dequantisation into fp32 with
    per-column B scales, on the default dispatch (rows split at the default
    chunk, two-ring workgroups), checked over the whole 16384 x 256 output
    against the oracle within 1e-5 of sum_t |s_t||A_t||B| |s_b|."""
    monkeypatch.delenv("VOID_AMD_KERNEL", raising=False)
    case = cases.c4_powerlaw()
    qd, A, bq, bs = _int8_setup(case, gpu)
    out = void_amd.void_spmm_int8(qd, torch.from_numpy(bq).to(gpu), b_scale=torch.from_numpy(bs).to(gpu),
                                  epilogue="per_block")
    torch.cuda.synchronize()
    assert any(p.n_split_tiles > 0 for p in qd.device_bsr().plans.values()), "c4 must exercise split rows"
    ref = oracle.i8_per_block(A, bq, bs)
    bound = _abs_bound(A, bq, bs)
    err = np.abs(out.cpu().numpy().astype(np.float64) - ref)
    assert np.all(err <= 1e-5 * bound + 1e-30), (err / (bound + 1e-30)).max()


def test_c5_ffn_full_every_row(gpu, monkeypatch):
    """Config 5 exactly as benched (INT8 per-block, per-token scales, GELU
    into bf16, default dispatch) over every one of its 448 block-rows: the
    int32 accumulators bit-exact against the oracle, the GELU output within
    one bf16 rounding plus 1e-4."""
    monkeypatch.delenv("VOID_AMD_KERNEL", raising=False)
    case = cases.c5_ffn()
    qd, A, bq, bs = _int8_setup(case, gpu)
    bt, st = torch.from_numpy(bq).to(gpu), torch.from_numpy(bs).to(gpu)
    out = void_amd.void_spmm_gelu(qd, bt, b_scale=st, out_dtype=torch.bfloat16, epilogue="per_block")
    raw = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="raw_i32")
    torch.cuda.synchronize()
    assert np.array_equal(raw.cpu().numpy(), oracle.i8_acc(A, bq))
    ref = oracle.gelu_tanh(oracle.i8_per_block(A, bq, bs))
    err = np.abs(out.float().cpu().numpy() - ref)
    assert np.all(err <= 2.0 ** -8 * np.abs(ref) + 1e-4), err.max()


def test_c5_ffn_full_sampled_rows(gpu, monkeypatch):
    """Config 5 at full size (14336 x 4096 W at 75 % block sparsity, 2048
    tokens, GELU in bf16): the default dispatch (a grid of seven resident
    rounds, which takes the 3-tile ring) must give the same bits as the
    4-tile ring, and 24 sampled block-rows -- the longest, the shortest, the
    first, the last and 20 seeded ones -- must match the oracle: int32
    accumulators bit-exact, the GELU output within bf16 rounding."""
    case = cases.c5_ffn()
    qd, A, bq, bs = _int8_setup(case, gpu)
    bt, st = torch.from_numpy(bq).to(gpu), torch.from_numpy(bs).to(gpu)
    monkeypatch.delenv("VOID_AMD_KERNEL", raising=False)
    out = void_amd.void_spmm_gelu(qd, bt, b_scale=st, out_dtype=torch.bfloat16, epilogue="per_block")
    raw = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="raw_i32")
    monkeypatch.setenv("VOID_AMD_KERNEL", "cgd")
    out4 = void_amd.void_spmm_gelu(qd, bt, b_scale=st, out_dtype=torch.bfloat16, epilogue="per_block")
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out4.view(torch.int16))

    lengths = np.diff(A.row_ptr)
    rng = np.random.default_rng(7)
    rows = np.unique(np.concatenate([[np.argmax(lengths), np.argmin(lengths), 0, len(lengths) - 1],
                                     rng.choice(len(lengths), 20, replace=False)]))
    where = np.full(len(lengths), -1)
    where[rows] = np.arange(len(rows))
    keep = where[case.block_rows] >= 0
    q = void_amd.quantize_void_tensor(cases.make_void_tensor(case, "cpu"))
    sub = oracle.Bsr(q.values.numpy()[keep], q.scales.numpy()[keep], where[case.block_rows[keep]],
                     case.block_cols[keep], (len(rows) * 32, case.K))
    sel = (rows[:, None] * 32 + np.arange(32)[None, :]).reshape(-1)
    assert np.array_equal(raw.cpu().numpy()[sel], oracle.i8_acc(sub, bq))
    ref = oracle.gelu_tanh(oracle.i8_per_block(sub, bq, bs))
    got = out.float().cpu().numpy()[sel]
    err = np.abs(got - ref)
    assert np.all(err <= 2.0 ** -8 * np.abs(ref) + 1e-4), err.max()


@pytest.mark.parametrize("per_column", [False, True])
@pytest.mark.parametrize("chunk", [None, 16, 200])
def test_epilogues_rows_beyond_64_tiles(gpu, chunk, per_column, kernel):
    """Block-rows of 65-96 tiles, every epilogue: the row-mean scale sum runs past the 64
    scales a workgroup holds one per lane, and (chunk 16) split rows fold the
    whole row from every chunk."""
    case = cases.uniform_blocks(160, 3072, 256, 430, seed=11)
    qd, A, bq, bs = _int8_setup(case, gpu, b_per_column=per_column)
    assert np.diff(A.row_ptr).max() > 64
    bt = torch.from_numpy(bq).to(gpu)
    st = torch.from_numpy(bs).to(gpu) if per_column else float(bs)
    acc = oracle.i8_acc(A, bq)
    rm = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="row_mean", chunk_tiles=chunk)
    raw = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="raw_i32", chunk_tiles=chunk)
    pb = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="per_block", chunk_tiles=chunk)
    torch.cuda.synchronize()
    ref = oracle.row_mean(A, acc, bs)
    assert np.array_equal(rm.cpu().numpy().view(np.int32), ref.view(np.int32))
    assert np.array_equal(raw.cpu().numpy(), acc)
    refpb = oracle.i8_per_block(A, bq, bs)
    assert np.all(np.abs(pb.cpu().numpy() - refpb) <= 1e-5 * _abs_bound(A, bq, bs) + 1e-30)


@pytest.mark.parametrize("chunk", [1, 3, 8, 100])
def test_forced_split_row_mean_and_per_block(gpu, chunk, kernel):
    case = cases.uniform_blocks(1024, 2048, 256, 900, seed=3)
    qd, A, bq, bs = _int8_setup(case, gpu)
    bt = torch.from_numpy(bq).to(gpu)
    st = torch.from_numpy(bs).to(gpu)
    acc = oracle.i8_acc(A, bq)
    raw = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="raw_i32", chunk_tiles=chunk)
    rm = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="row_mean", chunk_tiles=chunk)
    pb = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="per_block", chunk_tiles=chunk)
    torch.cuda.synchronize()
    assert np.array_equal(raw.cpu().numpy(), acc)
    ref = oracle.row_mean(A, acc, bs)
    assert np.array_equal(rm.cpu().numpy().view(np.int32), ref.view(np.int32))
    refpb = oracle.i8_per_block(A, bq, bs)
    bound = _abs_bound(A, bq, bs)
    assert np.all(np.abs(pb.cpu().numpy() - refpb) <= 1e-5 * bound + 1e-30)


@pytest.mark.parametrize("N", [64, 200, 384, 512, 600])
def test_split_dealing_geometries(gpu, N, kernel):
    """Split rows make the kernels deal the work list among the XCDs that
    share a panel group (8, 4, 2 or 1 of them for 1, 2, 3-4 and 5+ panels),
    with item counts that do not divide evenly: every item must still run
    exactly once."""
    case = cases.uniform_blocks(1056, 1600, N, 700, seed=11)
    qd, A, bq, bs = _int8_setup(case, gpu)
    bt = torch.from_numpy(bq).to(gpu)
    raw = void_amd.void_spmm_int8(qd, bt, b_scale=torch.from_numpy(bs).to(gpu), epilogue="raw_i32", chunk_tiles=3)
    torch.cuda.synchronize()
    assert np.array_equal(raw.cpu().numpy(), oracle.i8_acc(A, bq))


@pytest.mark.parametrize("N", [2048, 4096])
@pytest.mark.parametrize("chunk", [None, 3])
def test_wide_panel_groups(gpu, N, chunk, kernel):
    """N of 2048 and 4096 (16 and 32 panels): each XCD's share of the grid
    covers a group of 2 or 4 panels, in the per-XCD layout both for a
    one-round unsplit grid (second half of each share reversed) and for split
    rows (dealt shares): every (item, panel) must run exactly once."""
    case = cases.uniform_blocks(320 if chunk is None else 640, 1024, N, 150, seed=17)
    qd, A, bq, bs = _int8_setup(case, gpu)
    bt = torch.from_numpy(bq).to(gpu)
    raw = void_amd.void_spmm_int8(qd, bt, b_scale=torch.from_numpy(bs).to(gpu), epilogue="raw_i32", chunk_tiles=chunk)
    torch.cuda.synchronize()
    plans = qd.device_bsr().plans
    if chunk is not None:
        assert any(p.n_split_tiles > 0 for p in plans.values()), "the case must split rows"
    assert np.array_equal(raw.cpu().numpy(), oracle.i8_acc(A, bq))


def test_determinism_split(gpu):
    case = cases.uniform_blocks(512, 4096, 384, 1200, seed=5)
    qd, A, bq, bs = _int8_setup(case, gpu)
    bt = torch.from_numpy(bq).to(gpu)
    st = torch.from_numpy(bs).to(gpu)
    a = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="per_block", chunk_tiles=2)
    b = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="per_block", chunk_tiles=2)
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


@pytest.mark.parametrize("M,K,N", [(333, 555, 64), (100, 100, 36), (64, 96, 130), (32, 32, 1), (1000, 70, 257),
                                   (96, 64, 48), (70, 100, 80), (200, 1000, 16)])
def test_ragged_shapes(gpu, M, K, N, kernel):
    rng = np.random.default_rng(M * 7 + N)
    dense = np.where(rng.random((M, K)) < 0.1, rng.standard_normal((M, K)), 0).astype(np.float32)
    vt = void_amd.dense_to_void(torch.from_numpy(dense))
    q = void_amd.quantize_void_tensor(vt)
    B = rng.standard_normal((K, N)).astype(np.float32)
    bq, bs = oracle.quantize_i8_columns(B)
    A = oracle.Bsr(q.values.numpy(), q.scales.numpy(), vt.block_rows.numpy(), vt.block_cols.numpy(), (M, K))
    acc = oracle.i8_acc(A, bq)
    raw = void_amd.void_spmm_int8(q.to(gpu), torch.from_numpy(bq).to(gpu), b_scale=torch.from_numpy(bs).to(gpu),
                                  epilogue="raw_i32")
    assert np.array_equal(raw.cpu().numpy(), acc)


def test_column_major_b(gpu, kernel):
    case = cases.uniform_blocks(512, 1024, 256, 200, seed=9)
    qd, A, bq, bs = _int8_setup(case, gpu)
    bt_cm = torch.from_numpy(np.ascontiguousarray(bq.T)).to(gpu).t()  # [K, N] view, column-major
    assert bt_cm.stride(0) == 1
    raw = void_amd.void_spmm_int8(qd, bt_cm, b_scale=torch.from_numpy(bs).to(gpu), epilogue="raw_i32")
    assert np.array_equal(raw.cpu().numpy(), oracle.i8_acc(A, bq))


@pytest.mark.parametrize("copy", ["0", "1"])
def test_column_major_b_copy(gpu, copy, monkeypatch):
    """A column-major B is used in place (VOID_AMD_BT=0) or copied to row-major
    for the LDS-DMA ring (1; the default on dense enough grids): the same
    int32 accumulators and row-mean bits either way."""
    monkeypatch.setenv("VOID_AMD_BT", copy)
    case = cases.uniform_blocks(640, 1024, 384, 600, seed=19)
    qd, A, bq, bs = _int8_setup(case, gpu)
    bt_cm = torch.from_numpy(np.ascontiguousarray(bq.T)).to(gpu).t()
    st = torch.from_numpy(bs).to(gpu)
    acc = oracle.i8_acc(A, bq)
    raw = void_amd.void_spmm_int8(qd, bt_cm, b_scale=st, epilogue="raw_i32")
    rm = void_amd.void_spmm_int8(qd, bt_cm, b_scale=st, epilogue="row_mean")
    assert np.array_equal(raw.cpu().numpy(), acc)
    assert np.array_equal(rm.cpu().numpy().view(np.int32), oracle.row_mean(A, acc, bs).view(np.int32))


def test_gelu_bf16_bias(gpu, kernel):
    case = cases.uniform_blocks(256, 512, 192, 60, seed=11)
    qd, A, bq, bs = _int8_setup(case, gpu)
    bias = np.random.default_rng(1).standard_normal(192).astype(np.float32)
    out = void_amd.void_spmm_gelu(qd, torch.from_numpy(bq).to(gpu), bias=torch.from_numpy(bias).to(gpu),
                                  b_scale=torch.from_numpy(bs).to(gpu), out_dtype=torch.bfloat16)
    assert out.dtype == torch.bfloat16
    ref = oracle.gelu_tanh(oracle.i8_per_block(A, bq, bs) + bias[None, :].astype(np.float64))
    got = out.float().cpu().numpy()
    err = np.abs(got - ref)
    assert np.all(err <= 2.0 ** -8 * np.abs(ref) + 1e-4), err.max()


def test_empty_matrix(gpu):
    vt = void_amd.dense_to_void(torch.zeros(100, 100))
    q = void_amd.quantize_void_tensor(vt)
    out = void_amd.void_spmm_int8(q, torch.randn(100, 32, device=gpu))
    assert out.shape == (100, 32) and torch.count_nonzero(out) == 0


def test_empty_rows_written(gpu, kernel):
    # Output buffer prefilled with garbage must be fully overwritten, empty rows included.
    case = cases.uniform_blocks(1024, 1024, 128, 5, seed=2)
    qd, A, bq, bs = _int8_setup(case, gpu)
    out = torch.full((1024, 128), float("nan"), device=gpu)
    void_amd.void_spmm_int8(qd, torch.from_numpy(bq).to(gpu), b_scale=torch.from_numpy(bs).to(gpu),
                            out=out, epilogue="per_block")
    ref = oracle.i8_per_block(A, bq, bs)
    got = out.cpu().numpy()
    assert not np.isnan(got).any()
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("M,K,N", [(100, 70, 64), (64, 200, 48)])
def test_fp8_ragged_k(gpu, M, K, N, kernel):
    # K % 32 != 0: the last B slab crosses K; its rows past K must not meet
    # the A tile's zero padding as NaN codes.
    rng = np.random.default_rng(K + N)
    dense = np.where(rng.random((M, K)) < 0.2, rng.standard_normal((M, K)), 0).astype(np.float32)
    vt = void_amd.dense_to_void(torch.from_numpy(dense))
    f8 = void_amd.void_tensor_to_fp8(vt)
    B = rng.standard_normal((K, N)).astype(np.float32)
    bq, bs = oracle.quantize_fp8_tensor(B)
    # B's storage continues past K with NaN codes (0x7F) to catch any read of them.
    store = np.full((K + 32, N), 0x7F, np.uint8)
    store[:K] = bq
    bt = torch.from_numpy(store).to(gpu).view(torch.float8_e4m3fn)[:K]
    out = void_amd.void_spmm_fp8(f8.to(gpu), bt, output_dtype=torch.float32, b_scale=float(bs))
    A = oracle.Bsr(f8.values_fp8.view(torch.uint8).numpy(), f8.scaling_info.scale.numpy(),
                   vt.block_rows.numpy(), vt.block_cols.numpy(), (M, K))
    ref = oracle.fp8_spmm(A, bq, bs)
    got = out.cpu().numpy()
    assert not np.isnan(got).any()
    Aabs = oracle.Bsr.__new__(oracle.Bsr)
    Aabs.__dict__.update(A.__dict__)
    Aabs.tiles = np.ascontiguousarray(A.tiles.view(np.uint8) & 0x7F)
    bound = oracle.fp8_spmm(Aabs, bq & 0x7F, abs(bs))
    err = np.abs(got.astype(np.float64) - ref)
    bad = np.argwhere(err > FP8_TOL * bound + 1e-30)
    assert len(bad) == 0, [(tuple(i), got[tuple(i)], ref[tuple(i)], bound[tuple(i)]) for i in bad[:8]]


@pytest.mark.parametrize("epilogue", [_lib.EPI_ROW_MEAN, _lib.EPI_PER_BLOCK])
def test_abi_empty_matrix_null_pointers(gpu, epilogue, kernel):
    # Straight through the C ABI: a matrix with no tiles may pass null tile,
    # scale and column pointers; every output element is still written.
    import ctypes
    from void_amd import _runtime
    M, K, N = 96, 64, 128
    row_ptr = np.zeros(M // 32 + 1, np.int32)
    items, n_tiles, n_slots = _runtime.plan_rows(row_ptr, 64, np.zeros(0, np.int32))
    dev_items = torch.from_numpy(items).to(gpu)
    rp = torch.from_numpy(row_ptr).to(gpu)
    b = torch.zeros(K, N, dtype=torch.int8, device=gpu)
    out = torch.full((M, N), float("nan"), device=gpu)
    desc = _lib.BsrDesc(tiles=None, scales=None, row_ptr=rp.data_ptr(), col_idx=None, M=M, K=K, n_blocks=0,
                        n_block_rows=M // 32, per_tensor_a=0, reserved=0)
    dense = _lib.DenseArgs(b=b.data_ptr(), ldb=N, b_col_major=0, N=N, b_scale=1.0, b_scale_vec=None, bias=None,
                           c=out.data_ptr(), ldc=N, out_dtype=_lib.DT_F32, activation=_lib.ACT_NONE)
    plan = _lib.Plan(items=dev_items.data_ptr(), n_items=items.shape[0], n_split_tiles=0, n_slots=0,
                     chunk_tiles=64)
    st = _lib.lib().void_spmm_int8(ctypes.byref(desc), ctypes.byref(dense), epilogue, ctypes.byref(plan),
                                   None, 0, torch.cuda.current_stream().cuda_stream)
    assert st == 0, _lib.lib().void_last_error()
    torch.cuda.synchronize()
    assert torch.count_nonzero(out.nan_to_num(1.0)) == 0


def test_inplace_updates_are_seen(gpu):
    """The reference reads the tiles and scales on every call; the cached
    block-row-major device copy is gathered again after they change in
    place (values or scales of Int8VOIDTensor, values of a float
    VOIDTensor, scales of an FP8VOIDTensor)."""
    case = cases.uniform_blocks(256, 512, 128, 40, seed=21)
    case2 = cases.BlockCase(case.name, case.M, case.K, case.N, (-0.37 * case.tiles[::-1]).copy(),
                            case.block_rows, case.block_cols, case.b)
    qd, A, bq, bs = _int8_setup(case, gpu)
    bt, st = torch.from_numpy(bq).to(gpu), torch.from_numpy(bs).to(gpu)
    first = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="raw_i32")
    q2 = void_amd.quantize_void_tensor(cases.make_void_tensor(case2, "cpu")).to(gpu)
    qd.values.copy_(q2.values)
    qd.scales.copy_(q2.scales)
    for epi in ("raw_i32", "per_block", "row_mean"):
        got = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue=epi)
        ref = void_amd.void_spmm_int8(q2, bt, b_scale=st, epilogue=epi)
        assert torch.equal(got.view(torch.int32), ref.view(torch.int32)), epi
    assert not torch.equal(first, void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="raw_i32"))

    vt = cases.make_void_tensor(case, "cpu").to(gpu)
    b32 = torch.from_numpy(case.b).to(gpu)
    y1 = void_amd.void_spmm(vt, b32)
    vt.values.mul_(0.5)  # a power of two: every product and sum scales exactly
    assert torch.equal(void_amd.void_spmm(vt, b32), 0.5 * y1)

    f8 = void_amd.void_tensor_to_fp8(cases.make_void_tensor(case, "cpu")).to(gpu)
    b8q, b8s = oracle.quantize_fp8_tensor(case.b)
    b8 = torch.from_numpy(b8q).to(gpu).view(torch.float8_e4m3fn)
    z1 = void_amd.void_spmm_fp8(f8, b8, output_dtype=torch.float32, b_scale=float(b8s))
    f8.scaling_info.scale.mul_(2.0)
    assert torch.equal(void_amd.void_spmm_fp8(f8, b8, output_dtype=torch.float32, b_scale=float(b8s)), 2.0 * z1)


@pytest.mark.parametrize("rows,cols,pad", [(16, 16, 0), (384, 1024, 0), (2048, 4096, 0), (48, 272, 32), (1040, 80, 16)])
def test_transpose_b8(gpu, rows, cols, pad):
    """void_transpose_b8 (a column-major 8-bit B made row-major): every byte
    lands at its transposed place, tile edges and padded rows included."""
    from void_amd import _lib
    g = torch.Generator().manual_seed(rows + cols)
    src = torch.randint(-128, 128, (rows, cols + pad), dtype=torch.int8, generator=g).to(gpu)
    dst = torch.full((cols, rows + 16), 7, dtype=torch.int8, device=gpu)
    st = _lib.lib().void_transpose_b8(src.data_ptr(), cols + pad, rows, cols, dst.data_ptr(), rows + 16,
                                      torch.cuda.current_stream(gpu).cuda_stream)
    _lib.check(st, "void_transpose_b8")
    assert torch.equal(dst[:, :rows], src[:, :cols].t())
    assert torch.all(dst[:, rows:] == 7)
