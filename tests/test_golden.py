"""Golden fixtures (tests/golden/, written by make_golden.py): the oracle must
reproduce them on the CPU, the gfx950 kernel on the GPU."""

import hashlib
import os

import numpy as np
import pytest
import torch

import cases
import oracle
import void_amd

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _c1_inputs():
    A, B = cases.c1_plumbing()
    vt = void_amd.csr_to_void(A)
    q = void_amd.quantize_void_tensor(vt)
    bq, bs = oracle.quantize_i8_tensor(B)
    return vt, q, bq, bs


def test_hand_case_known_values():
    d = np.load(os.path.join(GOLDEN, "hand_case.npz"))
    assert d["acc"][0, 0] == 3 * 7 + 5 * 11 and d["acc"][5, 3] == -128 * 127
    assert d["row_mean"][0, 0] == np.float32(76 * 0.75)  # S = 0.5*2 + 0.25*2, n = 2
    A = oracle.Bsr(d["tiles"], d["scales"], d["block_rows"], d["block_cols"], (32, 64))
    assert np.array_equal(oracle.i8_acc(A, d["b"]), d["acc"])


def test_c1_fixture_oracle_cpu():
    d = np.load(os.path.join(GOLDEN, "c1_int8.npz"))
    vt, q, bq, bs = _c1_inputs()
    order = np.argsort(oracle.morton_encode(vt.block_rows.numpy(), vt.block_cols.numpy()))
    assert _sha(q.values.numpy()[order]) == str(d["tiles_sha256"]), "input generator drifted"
    assert _sha(bq) == str(d["b_sha256"]) and np.float32(bs) == d["b_scale"]
    A = oracle.Bsr(q.values.numpy(), q.scales.numpy(), vt.block_rows.numpy(), vt.block_cols.numpy(), (512, 512))
    acc = oracle.i8_acc(A, bq)
    assert np.array_equal(acc, d["acc"])
    out = oracle.row_mean(A, acc, bs)
    assert _sha(out) == str(d["out_sha256"])


@pytest.mark.gpu
def test_c1_fixture_kernel(gpu):
    d = np.load(os.path.join(GOLDEN, "c1_int8.npz"))
    vt, q, bq, bs = _c1_inputs()
    qd = q.to(gpu)
    bt = torch.from_numpy(bq).to(gpu)
    acc = void_amd.void_spmm_int8(qd, bt, b_scale=float(bs), epilogue="raw_i32")
    out = void_amd.void_spmm_int8(qd, bt, b_scale=float(bs))
    torch.cuda.synchronize()
    assert np.array_equal(acc.cpu().numpy(), d["acc"])
    o = out.cpu().numpy()
    assert np.array_equal(o.reshape(-1)[d["out_sample_idx"]], d["out_sample"])
    assert _sha(o) == str(d["out_sha256"])


@pytest.mark.gpu
def test_hand_case_kernel(gpu):
    d = np.load(os.path.join(GOLDEN, "hand_case.npz"))
    from void_amd.format import VOIDTensor
    from void_amd.int_quant import Int8VOIDTensor, IntQuantConfig
    q = Int8VOIDTensor(values=torch.from_numpy(d["tiles"]), scales=torch.from_numpy(d["scales"]),
                       zero_points=torch.zeros(2, dtype=torch.int8),
                       block_rows=torch.from_numpy(d["block_rows"]), block_cols=torch.from_numpy(d["block_cols"]),
                       shape=(32, 64), tile_size=(32, 32), n_blocks=2, config=IntQuantConfig()).to(gpu)
    b = torch.from_numpy(d["b"]).to(gpu)
    acc = void_amd.void_spmm_int8(q, b, b_scale=2.0, epilogue="raw_i32")
    rm = void_amd.void_spmm_int8(q, b, b_scale=2.0)
    assert np.array_equal(acc.cpu().numpy(), d["acc"])
    assert np.array_equal(rm.cpu().numpy(), d["row_mean"])
