"""Seeded random sweep of the SpMM entry points on every kernel: random
ragged shapes, block densities from a single tile to dense rows, row
lengths that cross the ring's stage and two-ring boundaries, per-tensor and
per-column B scales, all three INT8 epilogues, FP8, and split rows.  int32
accumulators and the row-mean epilogue are held bit-exact to the oracle, the
per-block and FP8 outputs to the error bounds the other tests state."""

import numpy as np
import pytest
import torch

import oracle
import void_amd
import cases

pytestmark = pytest.mark.gpu

FP8_TOL = 2.0 ** -13


@pytest.fixture(params=["default", "cgd", "cgd3", "cgdk", "bsr"])
def kernel(request, monkeypatch):
    if request.param == "default":
        monkeypatch.delenv("VOID_AMD_KERNEL", raising=False)
    else:
        monkeypatch.setenv("VOID_AMD_KERNEL", request.param)
    return request.param


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    M = int(rng.integers(1, 700))
    K = int(rng.integers(1, 2200))
    N = int(rng.choice([1, 7, 16, 64, 100, 128, 200, 256, 384, 520]))
    nbr, nbc = -(-M // 32), -(-K // 32)
    n_active = int(rng.integers(1, nbr * nbc + 1))
    return cases.uniform_blocks(M, K, N, n_active, seed=seed), rng


def _abs_bound(A, bq, bs):
    Aabs = oracle.Bsr.__new__(oracle.Bsr)
    Aabs.__dict__.update(A.__dict__)
    Aabs.tiles = np.ascontiguousarray(np.abs(A.tiles.astype(np.int16)).clip(0, 127).astype(np.int8))
    return oracle.i8_per_block(Aabs, np.abs(bq.astype(np.int16)).clip(0, 127).astype(np.int8), np.abs(bs))


@pytest.mark.parametrize("seed", range(64))
def test_random_int8(gpu, kernel, seed):
    case, rng = _case(seed)
    vt = cases.make_void_tensor(case, "cpu")
    q = void_amd.quantize_void_tensor(vt)
    qd = q.to(gpu)
    if seed % 3 == 0:
        bq, bs = oracle.quantize_i8_tensor(case.b)
        st = float(bs)
    else:
        bq, bs = oracle.quantize_i8_columns(case.b)
        st = torch.from_numpy(bs).to(gpu)
    A = oracle.Bsr(q.values.numpy(), q.scales.numpy(), case.block_rows, case.block_cols, (case.M, case.K))
    bt = torch.from_numpy(bq).to(gpu)
    chunk = int(rng.choice([None, 2, 5, 9, 33], p=[0.6, 0.1, 0.1, 0.1, 0.1]) or 0) or None
    acc = oracle.i8_acc(A, bq)
    raw = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="raw_i32", chunk_tiles=chunk)
    pb = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="per_block", chunk_tiles=chunk)
    torch.cuda.synchronize()
    assert np.array_equal(raw.cpu().numpy(), acc), (case.M, case.K, case.N, chunk)
    ref = oracle.i8_per_block(A, bq, bs)
    bound = _abs_bound(A, bq, bs)
    assert np.all(np.abs(pb.cpu().numpy() - ref) <= 1e-5 * bound + 1e-30), (case.M, case.K, case.N, chunk)
    if seed % 3 == 0:  # the reference's own epilogue, scalar B scale
        rm = void_amd.void_spmm_int8(qd, bt, b_scale=st, epilogue="row_mean", chunk_tiles=chunk)
        torch.cuda.synchronize()
        want = oracle.row_mean(A, acc, bs)
        assert np.array_equal(rm.cpu().numpy().view(np.int32), want.view(np.int32)), (case.M, case.K, case.N)


@pytest.mark.parametrize("seed", list(range(24, 32)) + list(range(64, 72)))
def test_random_fp8(gpu, kernel, seed):
    case, rng = _case(seed)
    vt = cases.make_void_tensor(case, "cpu")
    f8 = void_amd.void_tensor_to_fp8(vt)
    bq, bs = oracle.quantize_fp8_tensor(case.b)
    bt = torch.from_numpy(bq).to(gpu).view(torch.float8_e4m3fn)
    out = void_amd.void_spmm_fp8(f8.to(gpu), bt, output_dtype=torch.float32, b_scale=float(bs))
    torch.cuda.synchronize()
    A = oracle.Bsr(f8.values_fp8.view(torch.uint8).numpy(), f8.scaling_info.scale.numpy(),
                   case.block_rows, case.block_cols, (case.M, case.K))
    ref = oracle.fp8_spmm(A, bq, bs)
    Aabs = oracle.Bsr.__new__(oracle.Bsr)
    Aabs.__dict__.update(A.__dict__)
    Aabs.tiles = np.ascontiguousarray(A.tiles.view(np.uint8) & 0x7F)
    bound = oracle.fp8_spmm(Aabs, bq & 0x7F, abs(bs))
    err = np.abs(out.cpu().numpy().astype(np.float64) - ref)
    assert np.all(err <= FP8_TOL * bound + 1e-30), (case.M, case.K, case.N)


@pytest.mark.parametrize("seed", range(24))
def test_random_fp8_float_b(gpu, seed, monkeypatch):
    """E4M3 tiles times a float B kept as given (fp32, bf16 or fp16 by seed),
    on random ragged shapes, each ring shape in turn; the float64 oracle of
    the reference's upcast semantics (fp8.py:624-671) is the bar."""
    ring = (None, "cgd", "cgdk")[seed % 3]
    if ring:
        monkeypatch.setenv("VOID_AMD_KERNEL", ring)
    else:
        monkeypatch.delenv("VOID_AMD_KERNEL", raising=False)
    case, rng = _case(seed)
    dtype = (torch.float32, torch.bfloat16, torch.float16)[seed % 3 if seed % 2 else (seed // 2) % 3]
    print(f"fp8 float-B seed={seed} M={case.M} K={case.K} N={case.N} {dtype}", flush=True)
    f8 = void_amd.void_tensor_to_fp8(cases.make_void_tensor(case, "cpu"))
    b = torch.from_numpy(case.b).to(dtype)
    out = void_amd.void_spmm_fp8(f8.to(gpu), b.to(gpu), output_dtype=torch.float32)
    A = oracle.Bsr(f8.values_fp8.view(torch.uint8).numpy(), f8.scaling_info.scale.numpy(),
                   case.block_rows, case.block_cols, (case.M, case.K))
    bf = b.float().numpy()
    ref = oracle.fp8_spmm_float_b(A, bf)
    Aabs = oracle.Bsr.__new__(oracle.Bsr)
    Aabs.__dict__.update(A.__dict__)
    Aabs.tiles = np.ascontiguousarray(A.tiles.view(np.uint8) & 0x7F)
    bound = oracle.fp8_spmm_float_b(Aabs, np.abs(bf))
    err = np.abs(out.cpu().numpy().astype(np.float64) - ref)
    assert np.all(err <= FP8_TOL * bound + 1e-30), (case.M, case.K, case.N)
