"""The C ABI of libvoid_amd.so on the CPU: exported symbols, the host-side
Stream-K planner, argument validation, and loud failure of the SpMM entry
points without a GPU.  No kernel is launched here."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import cases
import void_amd
from void_amd import _lib, _runtime, tuning

HEADER = Path(__file__).resolve().parents[1] / "include" / "void_amd.h"


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(void_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_function():
    names = header_functions()
    assert {"void_spmm_int8", "void_spmm_fp8", "void_streamk_plan", "void_workspace_bytes",
            "void_last_error", "void_abi_version", "void_panel_width"} <= set(names)
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for n in names:
        assert hasattr(lib, n), f"{n} declared in void_amd.h but not exported"
    assert set(names) == set(_lib.SIGNATURES)


def test_abi_version_and_panel():
    assert _lib.lib().void_abi_version() == _lib.ABI_VERSION
    assert _lib.panel_width() == tuning.PANEL_COLUMNS
    assert ctypes.sizeof(_lib.WorkItem) == 4 * _lib.ITEM_INTS == 128


def _check_plan(row_ptr, col_idx, chunk):
    items, n_tiles, n_slots = _runtime.plan_rows(row_ptr, chunk, col_idx)
    covered = np.zeros(row_ptr[-1], dtype=np.int32)
    lengths = items[:, 2] - items[:, 1]
    # longest first (the kernels deal the list among XCDs themselves)
    expect = np.sort(lengths)[::-1]
    assert np.array_equal(lengths, expect), "items must be longest first"
    tiles, slots = set(), set()
    for it in items:
        row, b, e, tile, nch, ch, slot = it[:7]
        assert row_ptr[row] <= b <= e <= row_ptr[row + 1]
        covered[b:e] += 1
        if tile < 0:
            assert (b, e) == (row_ptr[row], row_ptr[row + 1]) and e - b <= chunk
        else:
            assert 0 <= ch < nch and e - b <= chunk and e - b >= 1
            tiles.add(tile)
            slots.add(slot + ch)
        inline = it[8:]
        for i in range(min(e - b, len(inline))):
            assert inline[i] == col_idx[b + i]
        assert np.all(inline[max(e - b, 0):] == -1)
    assert np.all(covered == 1), "every tile is covered exactly once"
    assert len(tiles) == n_tiles and slots == set(range(n_slots))
    rows_present = set(items[:, 0].tolist())
    assert rows_present == set(range(len(row_ptr) - 1)), "every block-row (also empty) has an item"
    return items


@pytest.mark.parametrize("chunk", [1, 3, 16, 64, 10 ** 6])
def test_planner_invariants_powerlaw(chunk):
    rng = np.random.default_rng(0)
    counts = np.minimum(rng.zipf(1.5, size=200), 300)
    counts[::17] = 0
    row_ptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    col_idx = rng.integers(0, 1000, size=row_ptr[-1]).astype(np.int32)
    items = _check_plan(row_ptr, col_idx, chunk)
    # chunks of a split row differ in length by at most one tile
    for row in np.unique(items[:, 0]):
        ln = (items[items[:, 0] == row][:, 2] - items[items[:, 0] == row][:, 1])
        if len(ln) > 1:
            assert ln.max() - ln.min() <= 1


def test_planner_errors():
    lib = _lib.lib()
    n = ctypes.c_int32()
    rp = np.array([0, 5, 3], np.int32)  # decreasing
    st = lib.void_streamk_plan(rp.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), None, 2, 4, None, 0,
                               ctypes.byref(n), ctypes.byref(ctypes.c_int32()), ctypes.byref(ctypes.c_int32()))
    assert st == -1 and b"decreases" in lib.void_last_error()
    rp = np.array([0, 5, 9], np.int32)
    st = lib.void_streamk_plan(rp.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), None, 2, 4, None, 0,
                               ctypes.byref(n), ctypes.byref(ctypes.c_int32()), ctypes.byref(ctypes.c_int32()))
    assert st == -5 and n.value == 3  # rows of 5 and 4 tiles in chunks of 4: 2 + 1 items needed


def test_workspace_bytes():
    lib = _lib.lib()
    assert lib.void_workspace_bytes(0, 0, 512) == 0
    # counters (3 tiles x 4 panels, rounded to 256 B) + 7 slots x 4 panels x 32 x 128 x 4 B
    assert lib.void_workspace_bytes(3, 7, 512) == 256 + 7 * 4 * 32 * 128 * 4


def _descs(M=64, K=64, N=32, n_blocks=1):
    a = _lib.BsrDesc(tiles=0x1000, scales=0x1000, row_ptr=0x1000, col_idx=0x1000, M=M, K=K,
                     n_blocks=n_blocks, n_block_rows=(M + 31) // 32, per_tensor_a=0, reserved=0)
    d = _lib.DenseArgs(b=0x1000, ldb=N, b_col_major=0, N=N, b_scale=1.0, b_scale_vec=None, bias=None,
                       c=0x1000, ldc=N, out_dtype=_lib.DT_F32, activation=0)
    p = _lib.Plan(items=0x1000, n_items=2, n_split_tiles=0, n_slots=0, chunk_tiles=64)
    return a, d, p


def _call_int8(a, d, p, epi=_lib.EPI_ROW_MEAN, ws=None, ws_bytes=0):
    return _lib.lib().void_spmm_int8(ctypes.byref(a), ctypes.byref(d), epi, ctypes.byref(p), ws, ws_bytes, None)


def test_argument_validation_without_launch():
    lib = _lib.lib()
    assert lib.void_spmm_int8(None, None, 0, None, None, 0, None) == -1
    a, d, p = _descs()
    a.n_block_rows = 5
    assert _call_int8(a, d, p) == -1 and b"n_block_rows" in lib.void_last_error()
    a, d, p = _descs()
    assert _call_int8(a, d, p, epi=_lib.EPI_RAW_I32) == -2          # RAW needs an int32 output
    d.out_dtype = _lib.DT_I32
    assert _call_int8(a, d, p, epi=_lib.EPI_PER_BLOCK) == -2        # int32 output needs RAW
    a, d, p = _descs()
    d.ldc = 8
    assert _call_int8(a, d, p) == -1
    a, d, p = _descs()
    d.activation = 9
    assert _call_int8(a, d, p) == -1
    a, d, p = _descs()
    p.n_split_tiles = 2
    p.n_slots = 4
    assert _call_int8(a, d, p) == -4                                # split plan without workspace
    assert _call_int8(a, d, p, ws=0x1000, ws_bytes=100) == -4
    a, d, p = _descs()
    assert lib.void_spmm_fp8(ctypes.byref(a), ctypes.byref(d), None, None, 0, None) == -1
    a, d, p = _descs()
    a.M = 0
    a.n_block_rows = 0
    assert _call_int8(a, d, p) == 0                                 # empty problem: nothing to do


def test_spmm_fails_loudly_on_cpu_tensors():
    vt = cases.make_void_tensor(cases.uniform_blocks(64, 64, 8, 2, seed=0))
    q = void_amd.quantize_void_tensor(vt)
    with pytest.raises(RuntimeError, match="GPU"):
        void_amd.void_spmm_int8(q, torch.randn(64, 16))
    f8 = void_amd.void_tensor_to_fp8(vt)
    with pytest.raises(RuntimeError, match="GPU"):
        void_amd.void_spmm_fp8(f8, torch.randn(64, 16))
    with pytest.raises(RuntimeError, match="GPU"):
        void_amd.void_spmm(vt, torch.randn(64, 16))
    with pytest.raises(RuntimeError, match="GPU"):
        void_amd.void_spmm_gelu(vt, torch.randn(64, 16))


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libvoid_amd.so")
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.lib()


def test_shape_checks():
    vt = cases.make_void_tensor(cases.uniform_blocks(64, 64, 8, 2, seed=0))
    q = void_amd.quantize_void_tensor(vt)
    with pytest.raises(ValueError):
        void_amd.void_spmm_int8(q, torch.zeros(65, 8, dtype=torch.int8))



def test_bad_bias_rejected_before_launch():
    # A bias that is not [N] would let the epilogue read past its end on the
    # device; both quantised wrappers reject it before touching the GPU.
    vt = cases.make_void_tensor(cases.uniform_blocks(64, 64, 8, 2, seed=0))
    q = void_amd.quantize_void_tensor(vt)
    f8 = void_amd.void_tensor_to_fp8(vt)
    b8 = torch.zeros(64, 16, dtype=torch.int8)
    bf8 = torch.zeros(64, 16, dtype=torch.float8_e4m3fn)
    for bias in (torch.zeros(8), torch.zeros(17), torch.zeros(16, 1)):
        with pytest.raises(ValueError, match="bias"):
            void_amd.void_spmm_int8(q, b8, bias=bias)
        with pytest.raises(ValueError, match="bias"):
            void_amd.void_spmm_fp8(f8, bf8, bias=bias)
        with pytest.raises(ValueError, match="bias"):
            void_amd.void_spmm_gelu(f8, bf8, bias=bias)

# ---------------------------------------------------------------- Stream-K host API

def test_compute_stream_k_workload_balanced():
    # test_advanced_features.py:688-701
    np.random.seed(42)
    vt = void_amd.csr_to_void(sp.random(256, 256, density=0.2, format="csr", dtype=np.float32))
    w = void_amd.compute_stream_k_workload(vt, n_workers=64)
    assert w.n_workers > 0 and w.total_work == vt.n_blocks and len(w.worker_rows) == w.n_workers
    assert int((w.worker_block_end - w.worker_block_start).sum()) == vt.n_blocks


def test_compute_stream_k_workload_imbalanced():
    # test_advanced_features.py:703-735: the heavy row is split
    rows, cols = [0] * 1000, [i % 512 for i in range(1000)]
    for i in range(1, 256):
        rows += [i] * 5
        cols += [j * 10 for j in range(5)]
    m = sp.csr_matrix((np.ones(len(rows), np.float32), (rows, cols)), shape=(256, 512))
    vt = void_amd.csr_to_void(m)
    w = void_amd.compute_stream_k_workload(vt, max_work_per_worker=4)
    assert int((w.worker_rows == 0).sum()) > 1
    assert bool(w.worker_needs_atomic[w.worker_rows == 0].all())


def test_analyze_workload_balance():
    np.random.seed(42)
    vt = void_amd.csr_to_void(sp.random(256, 256, density=0.1, format="csr", dtype=np.float32))
    a = void_amd.analyze_workload_balance(vt)
    assert not a["empty"] and a["imbalance_ratio"] >= 1.0


def test_chunk_table():
    assert tuning.select_chunk("int8", 1638, 512) == 64                       # c2: no split
    assert tuning.select_chunk("int8", 17960, 256) == 64                      # rows of <= 64 tiles: no split
    assert tuning.select_chunk("int8", 17960, 256, max_row=512) == 64         # c4: 1.3 x per-slot average (91), clamped
    assert tuning.select_chunk("int8", 100, 128, max_row=200) == 32           # clamped to [32, 64]
    assert tuning.select_chunk("int8", 16000, 128, max_row=200) == 41         # 1.3 x 16000 / 512 slots
    assert tuning.n_panels(512) == 4 and tuning.n_panels(130) == 2


def test_quantiser_argument_checks():
    lib = _lib.lib()
    assert lib.void_quantize_tiles_i8(None, 0, None, None, None) == 0          # nothing to do
    assert lib.void_quantize_tiles_i8(None, -1, None, None, None) == -1
    assert lib.void_quantize_tiles_i8(None, 3, None, None, None) == -1
    assert b"null" in lib.void_last_error()
    assert lib.void_quantize_tiles_fp8(0x1008, 3, 0x1000, 0x1000, None, None) == -1  # misaligned tiles
    assert b"aligned" in lib.void_last_error()


def test_csr_conversion_argument_checks():
    lib = _lib.lib()
    assert lib.void_csr_workspace_bytes(100, 100) > 0
    assert lib.void_csr_workspace_bytes(2 ** 30, 2 ** 30) == 0          # block grid beyond the device limit
    assert lib.void_csr_count_blocks(None, None, 10, 10, None, 0, None, None) == -1
    assert lib.void_csr_to_tiles(None, None, None, 10, 10, None, 0, 0, None, None, None, None, None) == 0
    assert lib.void_csr_to_tiles(None, None, None, 10, 10, None, 0, 1, None, None, None, None, None) == -1


def test_plan_from_workload_covers_every_tile_once():
    # void_spmm_stream_k runs a workload's worker ranges as work items: every
    # tile of every row exactly once, split rows numbered densely, rows
    # without workers still present (empty items), items of at most 64 tiles.
    from void_amd import _runtime
    from void_amd.stream_k import StreamKWorkload
    rng = np.random.default_rng(3)
    counts = np.minimum(rng.zipf(1.5, 200), 300)
    counts[5] = 0
    rp = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    ci = rng.integers(0, 512, rp[-1]).astype(np.int32)
    vt = None
    rows, begins, ends = [], [], []
    for r in range(200):
        if r == 7:
            continue  # a row the workload leaves out
        b, e = rp[r], rp[r + 1]
        step = 16
        for s in range(b, e, step):
            rows.append(r), begins.append(s), ends.append(min(e, s + step))
    items, n_split, n_slots, longest = _runtime.plan_from_ranges(rp, ci, np.array(rows), np.array(begins),
                                                                  np.array(ends), 64)
    assert longest <= 64
    seen = np.zeros(rp[-1], np.int32)
    for it in items:
        seen[it[1]:it[2]] += 1
        m = min(it[2] - it[1], 24)
        assert np.array_equal(it[8:8 + m], ci[it[1]:it[1] + m])
    expect = np.ones(rp[-1], np.int32)
    expect[rp[7]:rp[8]] = 0
    assert np.array_equal(seen, expect)
    assert set(items[:, 0]) == set(range(200))
    split = items[items[:, 3] >= 0]
    assert sorted(set(split[:, 3])) == list(range(n_split))
    assert n_slots == len(split)
    for t in range(n_split):
        ch = split[split[:, 3] == t]
        assert sorted(ch[:, 5]) == list(range(len(ch))) and np.all(ch[:, 4] == len(ch))
        assert len(set(ch[:, 6])) == 1
    with pytest.raises(ValueError):
        _runtime.plan_from_ranges(rp, ci, np.array([0]), np.array([rp[0]]), np.array([rp[2]]), 64)


def test_b_scale_args_keep_scales_on_the_device():
    """A per-tensor B scale given as a tensor is never read back to the host:
    it becomes N device copies with the per-tensor defaults kept."""
    from void_amd.int_quant import _b_scale_args
    s, v, per_col = _b_scale_args(torch.tensor([0.5]), 4, torch.device("cpu"))
    assert s == 1.0 and per_col is False and torch.equal(v, torch.full((4,), 0.5))
    s, v, per_col = _b_scale_args(torch.tensor([1.0, 2.0, 3.0]), 3, torch.device("cpu"))
    assert per_col is True and torch.equal(v, torch.tensor([1.0, 2.0, 3.0]))
    assert _b_scale_args(2.0, 7, torch.device("cpu")) == (2.0, None, False)
    assert _b_scale_args(None, 7, torch.device("cpu")) == (1.0, None, False)
    with pytest.raises(ValueError):
        _b_scale_args(torch.ones(5), 4, torch.device("cpu"))


def test_col_major_copy_rule(monkeypatch):
    monkeypatch.delenv("VOID_AMD_BT", raising=False)
    assert tuning.copy_col_major_b(14336, 4096)       # FFN config: tiles gather 112x B
    assert not tuning.copy_col_major_b(1638, 4096)    # c2: 13x B, read in place
    monkeypatch.setenv("VOID_AMD_BT", "0")
    assert not tuning.copy_col_major_b(14336, 4096)
    monkeypatch.setenv("VOID_AMD_BT", "1")
    assert tuning.copy_col_major_b(1, 4096)
