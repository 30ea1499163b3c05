"""void_spmm_int8_noalloc through the C ABI: the allocation-free entry point
gives the same bits as void_spmm_int8 with a caller's workspace, on plans
that split rows (so its static scratch is used) and on plans that do not,
on two calls in a row with the second smaller, and replayed from a HIP
graph that captured only the library call; it rejects plans beyond its
scratch with VOID_ERR_WORKSPACE."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import cases
import oracle
import void_amd
from void_amd import _lib, tuning

pytestmark = pytest.mark.gpu


def _setup(case, dev):
    vt = cases.make_void_tensor(case, "cpu")
    q = void_amd.quantize_void_tensor(vt)
    qd = q.to(dev)
    bq, bs = oracle.quantize_i8_columns(case.b)
    return qd, torch.from_numpy(bq).to(dev), torch.from_numpy(bs).to(dev)


def _noalloc(qd, b, bs, epilogue, chunk, out_dtype, out=None):
    """One call of void_spmm_int8_noalloc on the current stream (into out
    when given, else into a new NaN-filled tensor)."""
    dbsr = qd.device_bsr()
    plan = dbsr.plan(chunk)
    M, N = qd.shape[0], b.shape[1]
    if out is None:
        out = torch.full((M, N), float("nan"), device=b.device).to(out_dtype)
    cplan = _lib.Plan(items=plan.items.data_ptr(), n_items=plan.n_items, n_split_tiles=plan.n_split_tiles,
                      n_slots=plan.n_slots, chunk_tiles=plan.chunk)
    dense = _lib.DenseArgs(b=b.data_ptr(), ldb=b.stride(0), b_col_major=0, N=N, b_scale=1.0,
                           b_scale_vec=bs.data_ptr(), bias=None, c=out.data_ptr(), ldc=out.stride(0),
                           out_dtype={torch.float32: _lib.DT_F32, torch.int32: _lib.DT_I32}[out_dtype],
                           activation=_lib.ACT_NONE)
    desc = dbsr.desc()
    st = _lib.lib().void_spmm_int8_noalloc(ctypes.byref(desc), ctypes.byref(dense), epilogue, ctypes.byref(cplan),
                                           torch.cuda.current_stream(b.device).cuda_stream)
    _lib.check(st, "void_spmm_int8_noalloc")
    return out, plan


def _with_workspace(qd, b, bs, epilogue, chunk):
    name = {_lib.EPI_PER_BLOCK: "per_block", _lib.EPI_RAW_I32: "raw_i32", _lib.EPI_ROW_MEAN: "row_mean"}[epilogue]
    return void_amd.void_spmm_int8(qd, b, b_scale=bs, epilogue=name, chunk_tiles=chunk)


@pytest.mark.parametrize("epilogue", [_lib.EPI_PER_BLOCK, _lib.EPI_RAW_I32, _lib.EPI_ROW_MEAN])
def test_noalloc_matches_workspace_twice(gpu, epilogue):
    out_dtype = torch.int32 if epilogue == _lib.EPI_RAW_I32 else torch.float32
    big = cases.uniform_blocks(2048, 4096, 384, 2400, seed=11)    # ~19 tiles per block-row
    small = cases.uniform_blocks(640, 2048, 200, 300, seed=12)     # ~15 tiles per block-row, ragged N
    for case, chunk in ((big, 6), (small, 4)):                     # both plans split rows
        print(f"noalloc case {case.name} M={case.M} K={case.K} N={case.N} chunk={chunk} epi={epilogue}", flush=True)
        qd, b, bs = _setup(case, gpu)
        got, plan = _noalloc(qd, b, bs, epilogue, chunk, out_dtype)
        assert plan.n_split_tiles > 0
        ref = _with_workspace(qd, b, bs, epilogue, chunk)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), ref.view(torch.int32))


def test_noalloc_unsplit_and_c4(gpu):
    # An unsplit plan (no scratch) and the full power-law config with its
    # default chunk (8 MB of partials in the scratch), then a smaller call.
    for case in (cases.c4_powerlaw(), cases.uniform_blocks(1024, 1024, 128, 200, seed=13)):
        print(f"noalloc case {case.name}", flush=True)
        qd, b, bs = _setup(case, gpu)
        chunk = tuning.select_chunk("int8", qd.n_blocks, case.N, qd.device_bsr().max_row)
        got, _ = _noalloc(qd, b, bs, _lib.EPI_PER_BLOCK, chunk, torch.float32)
        ref = _with_workspace(qd, b, bs, _lib.EPI_PER_BLOCK, chunk)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), ref.view(torch.int32))


def test_noalloc_graph_replays(gpu):
    """Captured alone in a HIP graph (plan, output and scratch set up
    eagerly beforehand), the call replays to the same bits as
    void_spmm_int8 with a workspace, with the output cleared, other eager
    work and a synchronisation between replays."""
    case = cases.uniform_blocks(1024, 2048, 256, 900, seed=3)
    other = cases.uniform_blocks(512, 1024, 128, 120, seed=99)
    qd, b, bs = _setup(case, gpu)
    qo, bo, so = _setup(other, gpu)
    chunk = 3
    ref = _with_workspace(qd, b, bs, _lib.EPI_PER_BLOCK, chunk)
    out = torch.empty(case.M, case.N, device=gpu)
    _noalloc(qd, b, bs, _lib.EPI_PER_BLOCK, chunk, torch.float32, out=out)  # eager: plan and scratch ready
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), ref.view(torch.int32))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _noalloc(qd, b, bs, _lib.EPI_PER_BLOCK, chunk, torch.float32, out=out)
    for rep in range(4):
        print(f"noalloc graph replay {rep}", flush=True)
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        _noalloc(qo, bo, so, _lib.EPI_PER_BLOCK, 2, torch.float32)  # eager use of the same scratch, ordered after
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32))
    del g


def test_noalloc_rejects_oversize_plan(gpu):
    # A plan whose partials exceed the scratch fails before any launch.
    items = torch.zeros(32, dtype=torch.int32, device=gpu)
    rp = torch.zeros(2, dtype=torch.int32, device=gpu)
    b = torch.zeros(32, 128, dtype=torch.int8, device=gpu)
    out = torch.zeros(32, 128, device=gpu)
    desc = _lib.BsrDesc(tiles=None, scales=None, row_ptr=rp.data_ptr(), col_idx=None, M=32, K=32, n_blocks=0,
                        n_block_rows=1, per_tensor_a=0, reserved=0)
    dense = _lib.DenseArgs(b=b.data_ptr(), ldb=128, b_col_major=0, N=128, b_scale=1.0, b_scale_vec=None, bias=None,
                           c=out.data_ptr(), ldc=128, out_dtype=_lib.DT_F32, activation=_lib.ACT_NONE)
    n_slots = (_lib.NOALLOC_PARTIAL_BYTES // (32 * 128 * 4)) + 1
    plan = _lib.Plan(items=items.data_ptr(), n_items=1, n_split_tiles=1, n_slots=n_slots, chunk_tiles=64)
    st = _lib.lib().void_spmm_int8_noalloc(ctypes.byref(desc), ctypes.byref(dense), _lib.EPI_PER_BLOCK,
                                           ctypes.byref(plan), torch.cuda.current_stream(gpu).cuda_stream)
    assert st == -4  # VOID_ERR_WORKSPACE
    assert b"allocation-free" in _lib.lib().void_last_error()
