"""HIP graph capture of the SpMM entry points.

A serving loop records its launches in a HIP graph and replays them.  The
library launches kernels only (no memset nodes), and once a plan, its
row-major view and its split-row workspace exist, a call allocates nothing
but its output.  So a replay must reproduce the eager result bit for bit.

Each case warms up eagerly (which builds and caches the plan and view),
captures one call on torch's capture stream (which gets its own split-row
workspace, zeroed by a captured fill kernel), then replays the graph several
times.  Between replays it clears the captured output, runs other eager SpMM
work on the default stream and synchronises, and it checks every replay.  A
final eager call checks that capturing left the cached state intact.
"""

import numpy as np
import pytest
import torch

import cases
import oracle
import void_amd

pytestmark = pytest.mark.gpu

REPLAYS = 4


def _bits(t):
    if t.dtype in (torch.float32, torch.int32):
        return t.view(torch.int32)
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16)
    return t


def _capture_and_check(fn, other):
    ref = fn()
    torch.cuda.synchronize()
    ref = ref.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    for _ in range(REPLAYS):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        other()
        torch.cuda.synchronize()
        assert torch.equal(_bits(out), _bits(ref))
    again = fn()
    torch.cuda.synchronize()
    assert torch.equal(_bits(again), _bits(ref))
    del g


def _int8(case, dev):
    q = void_amd.quantize_void_tensor(cases.make_void_tensor(case, "cpu")).to(dev)
    bq, bs = oracle.quantize_i8_columns(case.b)
    return q, torch.from_numpy(bq).to(dev), torch.from_numpy(bs).to(dev)


def _other(dev):
    """Eager SpMM work of its own, run between replays on the default stream."""
    case = cases.uniform_blocks(512, 1024, 128, 120, seed=99)
    q, bt, st = _int8(case, dev)
    return lambda: void_amd.void_spmm_int8(q, bt, b_scale=st, epilogue="per_block", chunk_tiles=2)


@pytest.mark.parametrize("epilogue", ["raw_i32", "row_mean", "per_block"])
def test_graph_int8_one_round(gpu, epilogue):
    """At most 512 workgroups and no split rows (the two-ring kernel)."""
    case = cases.uniform_blocks(1024, 2048, 256, 300, seed=21)
    q, bt, st = _int8(case, gpu)
    _capture_and_check(lambda: void_amd.void_spmm_int8(q, bt, b_scale=st, epilogue=epilogue), _other(gpu))


@pytest.mark.parametrize("epilogue", ["raw_i32", "row_mean", "per_block"])
def test_graph_int8_split_rows(gpu, epilogue):
    """Split rows: the fix-up's arrival counters must be back at zero after
    every replay, or the next replay's reduction would go wrong."""
    case = cases.uniform_blocks(1024, 2048, 256, 900, seed=3)
    q, bt, st = _int8(case, gpu)
    _capture_and_check(lambda: void_amd.void_spmm_int8(q, bt, b_scale=st, epilogue=epilogue, chunk_tiles=3),
                       _other(gpu))


def test_graph_int8_deep_grid(gpu):
    """More than 512 workgroups without splits (the 3-tile ring)."""
    case = cases.uniform_blocks(4096, 1024, 1024, 1500, seed=8)
    q, bt, st = _int8(case, gpu)
    _capture_and_check(lambda: void_amd.void_spmm_int8(q, bt, b_scale=st, epilogue="per_block"), _other(gpu))


def test_graph_gelu_bf16_bias(gpu):
    case = cases.uniform_blocks(512, 1024, 384, 200, seed=12)
    q, bt, st = _int8(case, gpu)
    bias = torch.from_numpy(np.random.default_rng(2).standard_normal(384).astype(np.float32)).to(gpu)
    _capture_and_check(
        lambda: void_amd.void_spmm_gelu(q, bt, bias=bias, b_scale=st, out_dtype=torch.bfloat16), _other(gpu))


def test_graph_fp8(gpu):
    case = cases.uniform_blocks(512, 1024, 256, 250, seed=13)
    f8 = void_amd.void_tensor_to_fp8(cases.make_void_tensor(case, "cpu")).to(gpu)
    bq, bs = oracle.quantize_fp8_tensor(case.b)
    bt = torch.from_numpy(bq).to(gpu).view(torch.float8_e4m3fn)
    _capture_and_check(
        lambda: void_amd.void_spmm_fp8(f8, bt, output_dtype=torch.bfloat16, b_scale=float(bs)), _other(gpu))


def test_graph_float(gpu):
    case = cases.uniform_blocks(512, 1024, 256, 150, seed=14)
    vt = cases.make_void_tensor(case, "cpu").to(gpu)
    b = torch.from_numpy(case.b).to(gpu)
    _capture_and_check(lambda: void_amd.void_spmm(vt, b), _other(gpu))


def test_graph_bf16(gpu):
    """16-bit float tiles and B (void_spmm_bf16), split rows included."""
    case = cases.uniform_blocks(512, 4096, 256, 900, seed=15)
    vt = cases.make_void_tensor(case, "cpu").to_dtype(torch.bfloat16).to(gpu)
    b = torch.from_numpy(case.b).to(torch.bfloat16).to(gpu)
    from void_amd.ops import float_spmm
    plan = vt.device_bsr(torch.bfloat16).plan(12)
    assert plan.n_split_tiles > 0
    _capture_and_check(lambda: float_spmm(vt, b, plan=plan), _other(gpu))


def test_graph_fp8_bf16_b(gpu):
    """E4M3 tiles times a bf16 B (void_spmm_fp8_b16), fp16 output."""
    case = cases.uniform_blocks(512, 1024, 256, 250, seed=16)
    f8 = void_amd.void_tensor_to_fp8(cases.make_void_tensor(case, "cpu")).to(gpu)
    bt = torch.from_numpy(case.b).to(torch.bfloat16).to(gpu)
    _capture_and_check(lambda: void_amd.void_spmm_fp8(f8, bt, output_dtype=torch.float16), _other(gpu))


def test_graph_int8_float_b(gpu):
    """A float B is quantised per tensor on the device with its scale kept
    there (no host read-back), so the whole call, quantisation included,
    captures and replays."""
    case = cases.uniform_blocks(512, 1024, 256, 200, seed=17)
    q = void_amd.quantize_void_tensor(cases.make_void_tensor(case, "cpu")).to(gpu)
    bf = torch.from_numpy(case.b).to(gpu)
    _capture_and_check(lambda: void_amd.void_spmm_int8(q, bf), _other(gpu))


def test_graph_two_captures_of_one_split_plan(gpu):
    """Two graphs captured from one split plan, the second replayed first and
    then the two alternately: each capture owns a workspace (the first the
    plan's spare, zeroed before the capture; the second one zeroed inside its
    own graph), so no replay depends on another graph's zeroing or shares its
    arrival counters."""
    case = cases.uniform_blocks(1024, 2048, 256, 900, seed=5)
    q, bt, st = _int8(case, gpu)
    fn = lambda: void_amd.void_spmm_int8(q, bt, b_scale=st, epilogue="per_block", chunk_tiles=3)
    ref = fn()
    torch.cuda.synchronize()
    ref = ref.clone()
    assert any(p.n_split_tiles > 0 for p in q.device_bsr().plans.values())
    graphs, outs = [], []
    for _ in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(fn())
        graphs.append(g)
    torch.cuda.synchronize()
    plan = next(p for p in q.device_bsr().plans.values() if p.n_split_tiles > 0)
    ws = plan.capture_workspaces[-2:]
    assert len(ws) == 2 and ws[0].data_ptr() != ws[1].data_ptr() and not plan.capture_spares
    other = _other(gpu)
    for k in (1, 0, 1, 0, 0, 1):
        outs[k].zero_()
        torch.cuda.synchronize()
        graphs[k].replay()
        other()
        torch.cuda.synchronize()
        assert torch.equal(_bits(outs[k]), _bits(ref)), k
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for k, s in ((0, s1), (1, s2)):
        outs[k].zero_()
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        graphs[0].replay()
    with torch.cuda.stream(s2):
        graphs[1].replay()
    torch.cuda.synchronize()
    assert torch.equal(_bits(outs[0]), _bits(ref)) and torch.equal(_bits(outs[1]), _bits(ref))


def test_graph_split_plan_captured_first(gpu):
    """A split plan whose very first call is captured (no eager call before
    it, so no spare workspace): the captured fill clears the counters, and
    every replay, and an eager call after them, give the eager result."""
    case = cases.uniform_blocks(1024, 2048, 256, 900, seed=6)
    q, bt, st = _int8(case, gpu)
    fn = lambda: void_amd.void_spmm_int8(q, bt, b_scale=st, epilogue="per_block", chunk_tiles=4)
    q.device_bsr().plan(4)  # the plan exists, no workspace yet
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    other = _other(gpu)
    results = []
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        other()
        torch.cuda.synchronize()
        results.append(out.clone())
    ref = fn()
    torch.cuda.synchronize()
    for r in results:
        assert torch.equal(_bits(r), _bits(ref))


def test_graph_calls_of_one_capture_share_a_workspace(gpu):
    """Several calls of one split plan in one capture, on one stream, with
    different B operands: they run in order and share one workspace (each
    launch leaves the counters at zero for the next), and every replay
    gives each call's eager result."""
    case = cases.uniform_blocks(1024, 2048, 256, 900, seed=7)
    q, bt, st = _int8(case, gpu)
    bt2 = torch.flip(bt, dims=[0]).contiguous()
    f1 = lambda: void_amd.void_spmm_int8(q, bt, b_scale=st, epilogue="per_block", chunk_tiles=5)
    f2 = lambda: void_amd.void_spmm_int8(q, bt2, b_scale=st, epilogue="per_block", chunk_tiles=5)
    r1, r2 = f1().clone(), f2().clone()
    torch.cuda.synchronize()
    plan = q.device_bsr().plans[5]
    assert plan.n_split_tiles > 0
    n_before = len(plan.capture_workspaces)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        o1, o2, o3 = f1(), f2(), f1()
    assert len(plan.capture_workspaces) == n_before + 1
    other = _other(gpu)
    for _ in range(3):
        for o in (o1, o2, o3):
            o.zero_()
        torch.cuda.synchronize()
        g.replay()
        other()
        torch.cuda.synchronize()
        assert torch.equal(_bits(o1), _bits(r1)) and torch.equal(_bits(o2), _bits(r2)) and torch.equal(_bits(o3), _bits(r1))
