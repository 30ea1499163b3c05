"""Benchmark of the quantised block-sparse SpMM on one MI355X.

Default workload: A 4096x4096 in 32x32 tiles at
90 % block sparsity (1638 uniformly chosen tiles, N(0,1) entries, INT8
per-tile), B 4096x512 N(0,1) INT8 per-column, fp32 output, per-block
dequantising epilogue.  One "step" is one SpMM launch over that batch with
all inputs resident in HBM.

Timing: the K steps are captured in a HIP graph, each step preceded by an
overwrite of a 1 GiB buffer so that L2 and the 256 MB Infinity Cache hold
none of the inputs (cold cache); the graph replay is bracketed by HIP events
on the launch stream, and the replay time of a graph of the overwrites
alone is subtracted.  A hot-cache figure (a graph of back-to-back launches)
is reported alongside.

value = effective TOPS = 2 * n_tiles * 32 * 32 * N / kernel time (nonzero
tiles only).  roofline: HBM-bound; achieved = algorithmic bytes (A tiles +
A scales + column indices + row pointer + B + B scales + C, each once) /
kernel time, against 8 TB/s.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0   # dense MFMA int8, MI355X
FP8_PEAK_TFLOPS = 5000.0  # dense MFMA fp8, MI355X
BF16_PEAK_TFLOPS = 2500.0  # dense MFMA bf16, MI355X

# Per-launch memory traffic of the SpMM kernels, measured with rocprofv3 PMC
# passes over `bench.py --counters` and summarised by `bench.py
# --traffic-summary` into this file (with the commit and the kernel source's
# hash it was measured on).  A summary of other kernel source reports null.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.json")
KERNEL_SOURCES = ("void_amd/csrc/void_spmm.hip", "void_amd/csrc/lds_dma.h")


def kernel_source_sha() -> str:
    import hashlib
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(ROOT, rel), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def measured_traffic(cfg: str):
    """(bytes per launch, provenance) of a config from the traffic summary, or
    (None, reason) when there is none for the current kernel source."""
    try:
        with open(TRAFFIC_FILE) as fh:
            summ = json.load(fh)
    except (OSError, ValueError):
        return None, "no traffic summary"
    ent = summ.get("configs", {}).get(cfg)
    if ent is None:
        return None, f"{cfg} not in the traffic summary"
    src = {"file": os.path.relpath(TRAFFIC_FILE, ROOT), "commit": summ.get("commit"),
           "kernel_source_sha": summ.get("kernel_source_sha"), "counters": summ.get("counters")}
    if summ.get("kernel_source_sha") != kernel_source_sha():
        return None, dict(src, stale="kernel source changed since the measurement")
    return ent["traffic_bytes"], src


def gather_bytes(prob) -> int:
    """Bytes the column-group kernel moves from L2 into LDS per launch: every
    (nonzero tile, 128-column panel) pair stages its A tile (1024 elements)
    and its 32-row B slab (32 x 128 elements)."""
    n_panels = -(-prob["N"] // 128)
    return prob["nb"] * n_panels * (1024 * prob["a_esz"] + 32 * 128 * prob["b_esz"])


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default=None, choices=["c1", "c2", "c3", "c3f", "c3h", "c4", "c5"],
                    help="workload (default c2, the headline; c3f / c3h are config 3 with B kept in fp32 / bf16)")
    ap.add_argument("--no-per-config", dest="per_config", action="store_false",
                    help="the default run skips the other configs' extra.per_config entries")
    ap.add_argument("--op", default="spmm",
                    choices=["spmm", "quantize", "format", "float", "sddmm", "floor", "clock", "phases"],
                    help="spmm (default): the SpMM; quantize: device per-tile INT8 quantisation of the config's "
                         "A tiles; format: device CSR -> VOID tiles of the config's A; float: the float "
                         "SpMM (void_spmm) on the config's fp32 tiles and fp32 B; sddmm: the backward of A "
                         "(gradient on the config's nonzero tiles); floor: a tiny kernel and plain copies "
                         "of c2's byte count in the same cold harness; clock: the engine clock of the SpMM's "
                         "workgroups in the hot and cold graphs (instrumented library, built with "
                         "`python -m void_amd.build --clock-probe`); phases: per-workgroup phase timeline of "
                         "the SpMM in the cold and hot graphs (instrumented library, built with "
                         "`python -m void_amd.build --phase-probe`)")
    ap.add_argument("--epilogue", default=None, help="int8 epilogue (default per_block)")
    ap.add_argument("--dtype", default="f32", choices=["f32", "bf16", "f16"],
                    help="--op float / sddmm: operand dtype (bf16 / f16 run the 16-bit MFMA kernels, output in "
                         "the same dtype)")
    ap.add_argument("--chunk", type=int, default=None, help="override the Stream-K chunk")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline budget (0 = skip)")
    ap.add_argument("--profile", action="store_true", help="no CPU leg, no flush: for rocprofv3 runs")
    ap.add_argument("--traffic-summary", default=None, metavar="PMC_DIR",
                    help="summarise the rocprofv3 counter passes under PMC_DIR into profiles/hbm_traffic.json")
    ap.add_argument("--counters", action="store_true",
                    help="eager launches for rocprofv3 --pmc: each step overwrites 1 GiB, copies a "
                         "64 MiB calibration buffer, then runs the SpMM; prints no JSON line")
    return ap.parse_args()


def build_problem(cfg: str, dev, epilogue):
    """Inputs of one config on the device, quantised with the product's own
    quantisers (on the host, outside every timed region), and the SpMM call.

    cfg: c1..c5 as BASELINE.json lists them; c3f is config 3's A with B kept
    in fp32, the reference's default FP8 call (float B, fp16 output); c3h the
    same call with B in bf16."""
    import torch

    import cases
    import oracle
    import void_amd
    from void_amd.fp8 import quantize_dense_fp8

    if cfg == "c1":
        A, B = cases.c1_plumbing()
        vt = void_amd.csr_to_void(A)
        case = cases.BlockCase("c1_plumbing_512_n128", 512, 512, 128, vt.values.numpy(),
                               vt.block_rows.numpy(), vt.block_cols.numpy(), B)
    else:
        gen = {"c2": cases.c2_int8, "c3": cases.c3_fp8, "c3f": cases.c3_fp8, "c3h": cases.c3_fp8, "c4": cases.c4_powerlaw,
               "c5": cases.c5_ffn}[cfg]
        case = gen()
        vt = cases.make_void_tensor(case, "cpu")
    M, K, N = case.M, case.K, case.N
    nb = len(case.block_rows)
    nbr = -(-M // 32)
    prob = {"case": case, "M": M, "K": K, "N": N, "nb": nb, "b_bytes": K * N}
    if cfg == "c3f":
        f8 = void_amd.void_tensor_to_fp8(vt).to(dev)
        bt = torch.from_numpy(case.b).to(dev)
        out = torch.empty(M, N, dtype=torch.float16, device=dev)

        def run():
            return void_amd.void_spmm_fp8(f8, bt, output_dtype=torch.float16, out=out)

        # Rated against the bf16 MFMA peak the kernel runs on (each product
        # takes two bf16 MFMA products, B's hi and lo halves: that is the
        # design's cost, not the roofline's), or HBM, whichever bounds it.
        prob.update(kind="fp8", dtype="fp8e4m3 x f32 (bf16 hi/lo)", out_bytes=2, b_scale_bytes=0, run=run,
                    peak_ops=BF16_PEAK_TFLOPS, epilogue="per_block", b_bytes=4 * K * N, b_esz=4,
                    workload=case.name.replace("c3_fp8", "c3f_fp8_float_b"))
        a_scales = f8.scaling_info.scale.cpu().numpy()
        tiles_f = f8.values_fp8.float().cpu()
        b_deq = torch.from_numpy(case.b)
    elif cfg == "c3h":
        f8 = void_amd.void_tensor_to_fp8(vt).to(dev)
        bt = torch.from_numpy(case.b).to(torch.bfloat16).to(dev)
        out = torch.empty(M, N, dtype=torch.float16, device=dev)

        def run():
            return void_amd.void_spmm_fp8(f8, bt, output_dtype=torch.float16, out=out)

        prob.update(kind="fp8", dtype="fp8e4m3 x bf16", out_bytes=2, b_scale_bytes=0, run=run,
                    peak_ops=BF16_PEAK_TFLOPS, epilogue="per_block", b_bytes=2 * K * N, b_esz=2,
                    workload=case.name.replace("c3_fp8", "c3h_fp8_bf16_b"))
        a_scales = f8.scaling_info.scale.cpu().numpy()
        tiles_f = f8.values_fp8.float().cpu()
        b_deq = bt.float().cpu()
    elif cfg == "c3":
        f8 = void_amd.void_tensor_to_fp8(vt).to(dev)
        bq, bs = quantize_dense_fp8(torch.from_numpy(case.b))
        bt = bq.to(dev)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)

        def run():
            return void_amd.void_spmm_fp8(f8, bt, output_dtype=torch.bfloat16, b_scale=bs, out=out)

        prob.update(kind="fp8", dtype="fp8e4m3", out_bytes=2, b_scale_bytes=0, run=run,
                    peak_ops=FP8_PEAK_TFLOPS, epilogue="per_block")
        a_scales = f8.scaling_info.scale.cpu().numpy()
        tiles_f = f8.values_fp8.float().cpu()
        b_deq = torch.from_numpy(oracle.e4m3_table()[bq.view(torch.uint8).numpy().astype(np.int64)]
                                 .astype(np.float32) * np.float32(bs))
    else:
        q = void_amd.quantize_void_tensor(vt)
        qd = q.to(dev)
        if cfg == "c1":
            bq_t, params = void_amd.quantize_tensor(torch.from_numpy(case.b), void_amd.IntQuantConfig(
                scale_mode=void_amd.ScaleMode.PER_TENSOR))
            bs = float(params.scale.reshape(-1)[0])
            st = bs
            bsv = np.full(N, bs, np.float32)
        else:
            bq_t, bsv_t = void_amd.quantize_per_column(torch.from_numpy(case.b))
            bsv = bsv_t.numpy()
            st = bsv_t.to(dev)
        bq = bq_t.numpy()
        bt = bq_t.to(dev)
        gelu = cfg == "c5"
        ep = epilogue or ("row_mean" if cfg == "c1" else "per_block")
        out_dtype = torch.int32 if ep == "raw_i32" else torch.bfloat16 if gelu else torch.float32
        out = torch.empty(M, N, dtype=out_dtype, device=dev)

        def run():
            if gelu and ep != "raw_i32":
                return void_amd.void_spmm_gelu(qd, bt, b_scale=st, out=out, out_dtype=torch.bfloat16,
                                               epilogue=ep)
            return void_amd.void_spmm_int8(qd, bt, b_scale=st, out=out, epilogue=ep, chunk_tiles=prob.get("chunk"))

        prob.update(kind="int8", dtype="int8", out_bytes=2 if gelu else 4,
                    b_scale_bytes=0 if cfg == "c1" else 4 * N, run=run, peak_ops=INT8_PEAK_TOPS,
                    epilogue=ep, qd=qd)
        a_scales = q.scales.cpu().numpy()
        tiles_f = q.values.float()
        b_deq = torch.from_numpy(bq.astype(np.float32) * bsv[None, :])
    prob.setdefault("workload", case.name)
    prob.setdefault("a_esz", 1)
    prob.setdefault("b_esz", 1)
    prob["ops"] = 2.0 * nb * 32 * 32 * N
    prob["bytes"] = (nb * 1024 + 4 * nb + 4 * nb + 4 * (nbr + 1) + prob["b_bytes"]
                     + prob["b_scale_bytes"] + M * N * prob["out_bytes"])
    prob["cpu"] = dict(tiles=tiles_f, scales=torch.from_numpy(np.asarray(a_scales, np.float32).reshape(-1)),
                       col_idx=torch.from_numpy(case.block_cols.astype(np.int64)),
                       row=torch.from_numpy(case.block_rows.astype(np.int64)), b=b_deq)
    return prob


def device_peaks():
    """The peaks re-derived from this device's reported properties, next to
    the published figures the roofline fractions divide by: int8 MFMA at
    4 SIMDs x 2048 ops per clock per CU (v_mfma_i32_32x32x32_i8: 65536 ops
    in 32 cycles), HBM at the memory clock x bus width x 4 (HBM3E moves 8
    Gb/s per pin, four transfers per cycle of the 2 GHz clock the device
    reports).  The reported clocks are the peak ones, so these are ceilings."""
    from ctypes import byref, c_int32
    from void_amd import _lib
    v = [c_int32() for _ in range(4)]
    if _lib.lib().void_device_info(*(byref(x) for x in v)) != 0:
        return None
    cus, sclk, mclk, bus = (x.value for x in v)
    return {"compute_units": cus, "sclk_mhz": round(sclk / 1e3), "mclk_mhz": round(mclk / 1e3), "bus_bits": bus,
            "derived_int8_tops": round(cus * 4 * 2048 * sclk * 1e3 / 1e12, 1),
            "derived_hbm_gbs": round(mclk * 1e3 * bus / 8 * 4 / 1e9, 1),
            "published_int8_tops": INT8_PEAK_TOPS, "published_hbm_gbs": HBM_PEAK_GBS}


def time_gpu(prob, steps: int, warmup: int, flush: bool):
    """Kernel time from HIP-graph replays, so host launch overhead is excluded.

    cold: a graph of `steps` x (overwrite a 1 GiB buffer, SpMM) minus a graph of
    `steps` x (overwrite), median over 11 alternating pairs of replays -- the
    SpMM then always starts with L2 and the Infinity Cache holding none of its
    inputs; hot: a graph of `steps` x SpMM.
    Both graphs are bracketed by events on the capture-replay stream with a
    device synchronisation on either side.
    """
    import torch
    run = prob["run"]
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    scratch = torch.empty(1 << 28, dtype=torch.float32, device="cuda")

    def capture(body):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(steps):
                body(i)
        return g

    def replay_ms(g, reps=3):
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    def cold_body(i):
        scratch.fill_(float(i))
        run()

    t0 = time.perf_counter()
    g_hot = capture(lambda i: run())
    hot = replay_ms(g_hot) / steps
    cold = None
    if flush:
        g_cold = capture(cold_body)
        g_flush = capture(lambda i: scratch.fill_(float(i)))
        for _ in range(3):  # settle clocks and caches on a fresh box
            g_cold.replay()
            g_flush.replay()
        torch.cuda.synchronize()
        # Replays of the two graphs alternate and the median of the pairwise
        # differences is kept: the overwrites take ~15x the SpMM, so drift in
        # their speed between two separate averages would swamp the result.
        diffs = []
        for _ in range(11):
            diffs.append(replay_ms(g_cold, reps=1) - replay_ms(g_flush, reps=1))
        cold = sorted(diffs)[len(diffs) // 2] / steps
    wall = time.perf_counter() - t0
    return cold, hot, wall


def run_for_counters(prob, steps: int):
    """Eager sequence for HBM-traffic counters (no graph: per-dispatch counters
    need one dispatch per kernel).  Per step: a 1 GiB overwrite (cold L2 and
    Infinity Cache), a plain 64 MiB device-to-device copy whose FETCH_SIZE and
    WRITE_SIZE calibrate the counters against a known byte count, and the SpMM."""
    import torch
    scratch = torch.empty(1 << 28, dtype=torch.float32, device="cuda")
    src = torch.ones(1 << 24, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for i in range(steps):
        scratch.fill_(float(i))
        dst.copy_(src)
        prob["run"]()
    torch.cuda.synchronize()


FP32_PEAK_TFLOPS = 157.3  # dense MFMA fp32, MI355X


def bench_float(args, dev):
    """void_spmm on the float tiles and B of a config (the reference's float
    path): fp32 (fp32 MFMA) or, with --dtype bf16 / f16, both operands and the
    output in that dtype (16-bit MFMA); CPU baseline: the torch-CPU tile path
    in fp32."""
    import torch

    import cases
    import oracle
    import void_amd
    case = {"c2": cases.c2_int8, "c3": cases.c3_fp8, "c4": cases.c4_powerlaw, "c5": cases.c5_ffn}[args.config]()
    vt = cases.make_void_tensor(case, "cpu").to(dev)
    B = torch.from_numpy(case.b).to(dev)
    dt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[args.dtype]
    esz = 4 if dt == torch.float32 else 2
    if dt != torch.float32:
        vt, B = vt.to_dtype(dt), B.to(dt)
    nb = vt.n_blocks
    ops = 2.0 * nb * 1024 * case.N
    if args.op == "sddmm":
        from void_amd import _runtime
        from void_amd.format import build_bsr_layout
        G = torch.randn(case.M, case.N, device=dev).to(dt)
        rows, cols = vt.block_rows.to(torch.int32), vt.block_cols.to(torch.int32)
        # The backward's own path: tiles grouped by block-row (void_sddmm_rows_f32).
        lay = build_bsr_layout(rows, cols, vt.block_grid[0], vt.block_grid[1], dev)
        lay.row_groups()
        run = lambda: _runtime.sddmm_tiles(G, B, rows, cols, (case.M, case.K), dt, layout=lay)
        nbytes = nb * (1024 * esz + 8) + esz * case.M * case.N + esz * case.K * case.N
    else:
        out = torch.empty(case.M, case.N, device=dev, dtype=dt)
        run = lambda: void_amd.void_spmm(vt, B, out=out)
        nbytes = nb * (1024 * esz + 4) + 4 * (vt.block_grid[0] + 1) + esz * case.K * case.N + esz * case.M * case.N
    cold, hot, wall = time_gpu({"run": run}, args.steps, args.warmup, flush=True)
    peak = FP32_PEAK_TFLOPS if esz == 4 else BF16_PEAK_TFLOPS
    t_mem, t_ops = nbytes / (HBM_PEAK_GBS * 1e9), ops / (peak * 1e12)
    tflops = ops / (cold * 1e-3) / 1e12
    if t_ops >= t_mem:
        roof = {"bound": "mfma", "achieved": round(tflops, 2), "peak": peak, "unit": "TFLOP/s",
                "frac": round(tflops / peak, 4)}
    else:
        gbs = nbytes / (cold * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4)}
    roof.update(traffic=None, algorithmic_bytes=nbytes)
    cpu = None
    if args.cpu_seconds > 0 and args.op == "sddmm":
        Gh, Bh = G.cpu(), case.b
        rh, ch = case.block_rows.astype(np.int64), case.block_cols.astype(np.int64)
        Bt = torch.from_numpy(Bh)
        torch.set_num_threads(len(os.sched_getaffinity(0)))

        def host():  # torch CPU: gather the row and column blocks, batched matmul
            Gb = Gh.view(-1, 32, case.N)[torch.from_numpy(rh)]
            Bb = Bt.view(-1, 32, case.N)[torch.from_numpy(ch)]
            return torch.bmm(Gb, Bb.transpose(1, 2))
        times, t_end = [], time.perf_counter() + args.cpu_seconds
        while True:
            t = time.perf_counter()
            host()
            times.append(time.perf_counter() - t)
            if time.perf_counter() > t_end and len(times) >= 3:
                break
        med = statistics.median(times[1:]) if len(times) > 1 else times[0]
        cpu = {"value": round(ops / med / 1e12, 4), "unit": "TFLOP/s", "cores": len(os.sched_getaffinity(0)),
               "kind": "port", "ms": round(med * 1e3, 3),
               "sample": f"full {args.config} tile set, torch CPU gather + bmm, median of {len(times) - 1} reps"}
    elif args.cpu_seconds > 0:
        tiles = torch.from_numpy(case.tiles)
        rows = torch.from_numpy(case.block_rows.astype(np.int64))
        cols = torch.from_numpy(case.block_cols.astype(np.int64))
        ones = torch.ones(nb)
        bh = torch.from_numpy(case.b)
        torch.set_num_threads(len(os.sched_getaffinity(0)))
        times, t_end = [], time.perf_counter() + args.cpu_seconds
        while True:
            t = time.perf_counter()
            oracle.cpu_baseline_spmm(tiles, ones, cols, rows, bh, case.M)
            times.append(time.perf_counter() - t)
            if time.perf_counter() > t_end and len(times) >= 3:
                break
        med = statistics.median(times[1:]) if len(times) > 1 else times[0]
        cpu = {"value": round(ops / med / 1e12, 4), "unit": "TFLOP/s", "cores": len(os.sched_getaffinity(0)),
               "kind": "port", "ms": round(med * 1e3, 3),
               "sample": f"full {args.config} problem in fp32, torch CPU tile bmm + index_add, median of {len(times) - 1} reps"}
    what = "SDDMM backward of A (autograd's kernel choice)" if args.op == "sddmm" else "BSpMM (void_spmm)"
    dname = args.dtype
    line = {"metric": f"{dname.upper()} {what} effective TFLOP/s, {case.name} in {dname}", "value": round(tflops, 3),
            "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(cold, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": dname, "data": "synthetic (seeded generators of BASELINE.json configs)",
            "config": {"workload": case.name, "op": args.op, "M": case.M, "K": case.K, "N": case.N, "n_tiles": nb,
                       "cache": "cold (1 GiB overwrite between steps)"},
            "roofline": roof, "cpu_baseline": cpu,
            "extra": {"hot_ms": round(hot, 5), "wall_s": round(wall, 3)}}
    print(json.dumps(line), flush=True)


def bench_input_side(args, dev):
    """The device quantiser or the device CSR -> tiles conversion on the A
    operand of a config, timed like the SpMM (cold: after a 1 GiB overwrite),
    with the host path on the same input as the CPU baseline."""
    import scipy.sparse as sp
    import torch

    import cases
    import void_amd
    from void_amd import _lib, _runtime
    case = {"c1": None, "c2": cases.c2_int8, "c3": cases.c3_fp8, "c4": cases.c4_powerlaw, "c5": cases.c5_ffn}[args.config]
    if case is None:
        A, _ = cases.c1_plumbing()
        vt_host = void_amd.csr_to_void(A)
        name = "c1_plumbing_512_n128"
    else:
        case = case()
        vt_host = cases.make_void_tensor(case, "cpu")
        name = case.name
    nb = vt_host.n_blocks
    M, K = vt_host.shape
    if args.op == "quantize":
        x = vt_host.values.to(dev)
        run = lambda: _runtime.quantize_tiles_i8(x)
        nbytes = nb * (4096 + 1024 + 4)
        host = lambda: void_amd.quantize_void_tensor(vt_host)
        metric = f"INT8 per-tile quantisation GB/s, A tiles of {name}"
        sample = f"quantize_void_tensor on the host (batched torch CPU), all {nb} tiles"
    else:
        dense = vt_host.to_dense().numpy()
        A = sp.csr_matrix(dense)
        nnz = A.nnz
        lib = _lib.lib()
        ws_bytes = lib.void_csr_workspace_bytes(M, K)
        d_indptr = torch.from_numpy(A.indptr.astype(np.int32)).to(dev)
        d_indices = torch.from_numpy(A.indices.astype(np.int32)).to(dev)
        d_data = torch.from_numpy(A.data.astype(np.float32)).to(dev)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        cnt = torch.empty(1, dtype=torch.int64, device=dev)
        values = torch.empty((nb, 32, 32), dtype=torch.float32, device=dev)
        rows = torch.empty(nb, dtype=torch.int32, device=dev)
        cols = torch.empty(nb, dtype=torch.int32, device=dev)
        mort = torch.empty(nb, dtype=torch.int64, device=dev)

        def run():
            st = torch.cuda.current_stream().cuda_stream
            _lib.check(lib.void_csr_count_blocks(d_indptr.data_ptr(), d_indices.data_ptr(), M, K, ws.data_ptr(),
                                                 ws_bytes, cnt.data_ptr(), st), "count")
            _lib.check(lib.void_csr_to_tiles(d_indptr.data_ptr(), d_indices.data_ptr(), d_data.data_ptr(), M, K,
                                             ws.data_ptr(), ws_bytes, nb, values.data_ptr(), rows.data_ptr(),
                                             cols.data_ptr(), mort.data_ptr(), st), "to_tiles")
        run()
        torch.cuda.synchronize()
        assert int(cnt.item()) == nb and torch.equal(values.cpu(), vt_host.values)
        nbytes = 4 * (M + 1) + 8 * nnz + nb * (4096 + 16)
        host = lambda: void_amd.csr_to_void(A)
        metric = f"CSR -> VOID tiles GB/s (device csr_to_void), A of {name}"
        sample = f"csr_to_void on the host (vectorised numpy scatter), nnz {nnz}"
    cold, hot, wall = time_gpu({"run": run}, args.steps, args.warmup, flush=True)
    gbs = nbytes / (cold * 1e-3) / 1e9
    cpu = None
    if args.cpu_seconds > 0:
        t_end = time.perf_counter() + args.cpu_seconds
        times = []
        while True:
            t = time.perf_counter()
            host()
            times.append(time.perf_counter() - t)
            if time.perf_counter() > t_end and len(times) >= 3:
                break
        med = statistics.median(times[1:]) if len(times) > 1 else times[0]
        cpu = {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": len(os.sched_getaffinity(0)),
               "kind": "port", "ms": round(med * 1e3, 3), "sample": sample + f", median of {len(times) - 1} reps"}
    line = {"metric": metric, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(cold, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32->int8" if args.op == "quantize" else "f32",
            "data": "synthetic (seeded generators of BASELINE.json configs)",
            "config": {"workload": name, "op": args.op, "n_tiles": nb, "M": M, "K": K,
                       "cache": "cold (1 GiB overwrite between steps)"},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "algorithmic_bytes": nbytes},
            "cpu_baseline": cpu,
            "extra": {"hot_ms": round(hot, 5), "hot_gbs": round(nbytes / (hot * 1e-3) / 1e9, 1),
                      "wall_s": round(wall, 3)}}
    print(json.dumps(line), flush=True)


def time_cpu(prob, budget_s: float):
    import torch

    import oracle
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    c = prob["cpu"]
    times = []
    t_end = time.perf_counter() + budget_s
    while True:
        t = time.perf_counter()
        oracle.cpu_baseline_spmm(c["tiles"], c["scales"], c["col_idx"], c["row"], c["b"], prob["M"])
        times.append(time.perf_counter() - t)
        if time.perf_counter() > t_end and len(times) >= 3:
            break
    med = statistics.median(times[1:]) if len(times) > 1 else times[0]
    return med, threads, len(times)


def roofline_of(prob, t_ms: float, cfg: str) -> dict:
    """The applicable roofline of one timed SpMM: HBM (algorithmic bytes) or
    MFMA (effective ops), whichever bounds the config."""
    tops = prob["ops"] / (t_ms * 1e-3) / 1e12
    gbs = prob["bytes"] / (t_ms * 1e-3) / 1e9
    t_roof_mem = prob["bytes"] / (HBM_PEAK_GBS * 1e9)
    t_roof_ops = prob["ops"] / (prob["peak_ops"] * 1e12)
    if t_roof_mem >= t_roof_ops:
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4)}
    else:
        roof = {"bound": "mfma", "achieved": round(tops, 2), "peak": prob["peak_ops"], "unit": "TFLOP/s",
                "frac": round(tops / prob["peak_ops"], 4)}
    roof["traffic"], roof["traffic_source"] = measured_traffic(cfg)
    roof["algorithmic_bytes"] = prob["bytes"]
    roof["roofline_ms"] = round(max(t_roof_mem, t_roof_ops) * 1e3, 5)
    return roof


def cpu_leg(prob, budget_s: float, cfg: str) -> dict:
    med, threads, reps = time_cpu(prob, budget_s)
    return {"value": round(prob["ops"] / med / 1e12, 4), "unit": "TOPS", "cores": threads, "kind": "port",
            "ms": round(med * 1e3, 3),
            "sample": f"full {cfg} problem, torch CPU dequantise + tile bmm + index_add, "
                      f"median of {reps - 1} reps after 1 warm-up"}


# Configs reported next to the headline (BASELINE.json asks for every one):
# c1, c3 as configured (E4M3 B, bf16 out), c3f (the reference's default FP8
# call: float B, fp16 out), c3h (the same with a bf16 B), c4 and c5.
PER_CONFIG = ("c1", "c3", "c3f", "c3h", "c4", "c5")


def per_config_line(cfg: str, dev, args) -> dict:
    """Cold kernel time, TOPS, roofline fraction, traffic ratio and CPU
    baseline of one more config, for the headline line's extra.per_config."""
    import torch
    prob = build_problem(cfg, dev, None)
    cold, hot, _ = time_gpu(prob, min(args.steps, 20), args.warmup, flush=True)
    roof = roofline_of(prob, cold, cfg)
    res = {"workload": prob["workload"], "kind": prob["kind"], "dtype": prob["dtype"], "ms": round(cold, 5),
           "hot_ms": round(hot, 5), "tops": round(prob["ops"] / (cold * 1e-3) / 1e12, 3),
           "bound": roof["bound"], "frac": roof["frac"], "peak": roof["peak"], "roofline_ms": roof["roofline_ms"],
           "traffic_ratio": (round(roof["traffic"] / prob["bytes"], 3) if roof["traffic"] else None),
           "gather_bytes": gather_bytes(prob), "gather_tbs": round(gather_bytes(prob) / (cold * 1e-3) / 1e12, 2)}
    if args.cpu_seconds > 0:
        c = cpu_leg(prob, min(args.cpu_seconds, 3.0), cfg)
        res.update(cpu_ms=c["ms"], cpu_tops=c["value"], cpu_cores=c["cores"])
    del prob
    torch.cuda.empty_cache()
    return res


def floor_measure(dev, steps: int, warmup: int) -> dict:
    """Practical floor for c2 in the same graph-and-flush harness: a launch of
    a tiny kernel (the fixed cost of one dispatch after the 1 GiB overwrite)
    and plain device copies moving c2's algorithmic bytes: all of them
    (read + write = 12.18 MB) and the SpMM's own split (3.8 MB read and
    8.4 MB written are bounded by the larger, so a fill of the output size
    shows the write side alone)."""
    import torch
    n_alg = 12178740  # c2's algorithmic bytes per launch
    half = torch.empty(n_alg // 2 // 4, dtype=torch.float32, device=dev)
    half_dst = torch.empty_like(half)
    c_out = torch.empty(4096 * 512, dtype=torch.float32, device=dev)
    tiny = torch.empty(64, dtype=torch.float32, device=dev)
    res = {}
    for name, fn, nbytes in (("tiny_kernel", lambda: tiny.fill_(1.0), 256),
                             ("copy_c2_bytes", lambda: half_dst.copy_(half), 2 * half.numel() * 4),
                             ("write_c2_output", lambda: c_out.fill_(2.0), c_out.numel() * 4)):
        cold, hot, _ = time_gpu({"run": fn}, steps, warmup, flush=True)
        res[name] = {"ms": round(cold, 5), "hot_ms": round(hot, 5), "bytes": nbytes,
                     "gbs": round(nbytes / (cold * 1e-3) / 1e9, 1)}
    return res


def bench_floor(args, dev):
    res = floor_measure(dev, args.steps, args.warmup)
    line = {"metric": "practical floor for c2 (cold graph-and-flush harness)", "value": res["copy_c2_bytes"]["ms"],
            "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": res["copy_c2_bytes"]["ms"], "higher_is_better": False, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "floor_c2", "cache": "cold (1 GiB overwrite between steps)"},
            "roofline": {"bound": "hbm", "achieved": res["copy_c2_bytes"]["gbs"], "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(res["copy_c2_bytes"]["gbs"] / HBM_PEAK_GBS, 4),
                         "traffic": None},
            "cpu_baseline": None, "extra": res}
    print(json.dumps(line), flush=True)


# Counter passes the traffic summary reads, one rocprofv3 run per pass (the
# two DRAM counters share one pass; FETCH_SIZE and WRITE_SIZE take one each):
#   rocprofv3 --pmc <counters> -d <pmc_dir>/pmc_<cfg>_<pass> -o run --output-format csv -- \
#       python bench.py --config <cfg> --counters --steps 5
TRAFFIC_COUNTERS = ("TCC_EA0_RDREQ_DRAM_32B_sum", "TCC_EA0_WRREQ_WRITE_DRAM_32B_sum", "FETCH_SIZE", "WRITE_SIZE")
TRAFFIC_CONFIGS = ("c2", "c3", "c4", "c5")


def traffic_summary(pmc_dir: str) -> None:
    """Summarise the counter passes under pmc_dir into profiles/hbm_traffic.json.

    Each pass's CSV holds, per step, the 64 MiB calibration copy and the SpMM.
    A counter's value per dispatch is the mean over the steps after the first;
    it is scaled by the copy's reading against the copy's known byte count
    (64 MiB read, 64 MiB written).  DRAM_32B counters count 32-byte units of
    L2 requests to device memory, which the Infinity Cache may serve; FETCH_SIZE
    and WRITE_SIZE are in KiB."""
    import csv
    import glob
    import subprocess
    copy_bytes = 64 << 20
    unit = {"TCC_EA0_RDREQ_DRAM_32B_sum": 32.0, "TCC_EA0_WRREQ_WRITE_DRAM_32B_sum": 32.0,
            "FETCH_SIZE": 1024.0, "WRITE_SIZE": 1024.0}
    out = {"counters": list(TRAFFIC_COUNTERS), "kernel_source_sha": kernel_source_sha(), "configs": {}}
    try:
        out["commit"] = subprocess.run(["git", "-C", ROOT, "rev-parse", "--short", "HEAD"], capture_output=True,
                                       text=True).stdout.strip() or None
    except OSError:
        out["commit"] = None
    for cfg in TRAFFIC_CONFIGS:
        ent = {}
        for ctr in TRAFFIC_COUNTERS:
            files = glob.glob(os.path.join(pmc_dir, f"pmc_{cfg}_*", "**", "*counter_collection.csv"), recursive=True)
            rows = [r for fn in files for r in csv.DictReader(open(fn)) if r["Counter_Name"] == ctr]
            # Per step, the SpMM dispatch and the copy dispatched just before it
            # (setup copies earlier in the run are not steps).
            disp = {}
            for r in rows:
                name = r["Kernel_Name"]
                kind = "spmm" if "spmm" in name else "copy" if "copy" in name.lower() else None
                if kind is not None:
                    d = disp.setdefault(int(r["Dispatch_Id"]), [kind, 0.0])
                    d[1] += float(r["Counter_Value"])
            vals = {"spmm": [], "copy": []}
            last_copy = None
            for _, (kind, v) in sorted(disp.items()):
                if kind == "copy":
                    last_copy = v
                elif last_copy is not None:
                    vals["spmm"].append(v)
                    vals["copy"].append(last_copy)
                    last_copy = None
            vals = {k: v[1:] for k, v in vals.items()}
            if not vals["spmm"]:
                continue
            spmm = sum(vals["spmm"]) / len(vals["spmm"]) * unit[ctr]
            copy = sum(vals["copy"]) / len(vals["copy"]) * unit[ctr]
            scale = copy_bytes / copy if copy else None
            ent[ctr] = {"raw_bytes": round(spmm), "copy_raw_bytes": round(copy),
                        "scale": None if scale is None else round(scale, 4),
                        "bytes": None if scale is None else round(spmm * scale)}
        rd, wr = ent.get(TRAFFIC_COUNTERS[0]), ent.get(TRAFFIC_COUNTERS[1])
        if rd and wr and rd["bytes"] is not None and wr["bytes"] is not None:
            ent["traffic_bytes"] = rd["bytes"] + wr["bytes"]
            out["configs"][cfg] = ent
    with open(TRAFFIC_FILE, "w") as fh:
        json.dump(out, fh, indent=1)
    print(json.dumps(out), flush=True)


def bench_clock(args, dev):
    """Engine clock of the SpMM's workgroups, hot against cold.  The
    instrumented library makes every workgroup record s_memrealtime (100 MHz)
    and s_memtime (shader clock) at its start and end; the clock of a
    workgroup is the ratio of the two intervals.  Hot: a graph of K
    back-to-back launches; cold: K x (1 GiB overwrite, launch).  The stamps
    are those of each graph's last launch; three replays of each graph,
    alternating."""
    import ctypes
    import torch
    from void_amd import _lib, build as vbuild
    if not vbuild.CLOCK_LIB_PATH.exists():
        raise SystemExit(f"{vbuild.CLOCK_LIB_PATH} is missing: build it with `python -m void_amd.build --clock-probe`")
    _lib.LIB_PATH = vbuild.CLOCK_LIB_PATH
    prob = build_problem(args.config, dev, args.epilogue)
    L = _lib.lib()
    L.void_debug_set_trace.argtypes = [ctypes.c_void_p]
    buf = torch.zeros(8 * (1 << 16), dtype=torch.int64, device=dev)
    scratch = torch.empty(1 << 28, dtype=torch.float32, device=dev)
    L.void_debug_set_trace(ctypes.c_void_p(buf.data_ptr()))
    for _ in range(args.warmup):
        prob["run"]()
    torch.cuda.synchronize()

    def capture(body):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(args.steps):
                body(i)
        return g

    def cold(i):
        scratch.fill_(float(i))
        prob["run"]()
    graphs = {"hot": capture(lambda i: prob["run"]()), "cold": capture(cold)}
    res = {"hot": [], "cold": []}
    for _ in range(3):
        for name, g in graphs.items():
            buf.zero_()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            g.replay()
            e1.record()
            torch.cuda.synchronize()
            t = buf.view(-1, 8).cpu().numpy().astype(np.int64)
            t = t[t[:, 0] != 0]
            mhz = (t[:, 2] - t[:, 1]) / ((t[:, 4] - t[:, 0]) * 10e-9) / 1e6
            res[name].append({"graph_us_per_step": round(e0.elapsed_time(e1) / args.steps * 1e3, 2),
                              "workgroups": int(len(t)), "clock_mhz_median": round(float(np.median(mhz))),
                              "clock_mhz_p10": round(float(np.percentile(mhz, 10))),
                              "clock_mhz_p90": round(float(np.percentile(mhz, 90)))})
    line = {"metric": f"engine clock of the SpMM workgroups, {prob['workload']}", "unit": "MHz",
            "value": res["hot"][-1]["clock_mhz_median"], "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "config": {"workload": prob["workload"]}, "extra": res}
    print(json.dumps(line), flush=True)


def bench_phases(args, dev):
    """Per-workgroup phase timeline of the SpMM (the column-group kernel's LDS-DMA
    ring).  The instrumented library makes workgroup thread 0 record
    s_memrealtime (100 MHz) at: 0 the work item read, 1 the first stage
    issued, 5 the first stage landed, 6 the tile loop done, 2 the two rings'
    hand-off done (split rows: the fix-up too), 3 the epilogue staged, 4 the
    stores issued.  Cold: K x (1 GiB overwrite, launch); hot: K back-to-back
    launches; the stamps are those of each graph's last launch, three replays
    of each, alternating.  Phases are medians (and 10th / 90th percentiles)
    over workgroups, in microseconds."""
    import ctypes
    import torch
    from void_amd import _lib, build as vbuild
    if not vbuild.PHASE_LIB_PATH.exists():
        raise SystemExit(f"{vbuild.PHASE_LIB_PATH} is missing: build it with `python -m void_amd.build --phase-probe`")
    _lib.LIB_PATH = vbuild.PHASE_LIB_PATH
    prob = build_problem(args.config, dev, args.epilogue)
    L = _lib.lib()
    L.void_debug_set_trace.argtypes = [ctypes.c_void_p]
    buf = torch.zeros(8 * (1 << 16), dtype=torch.int64, device=dev)
    scratch = torch.empty(1 << 28, dtype=torch.float32, device=dev)
    L.void_debug_set_trace(ctypes.c_void_p(buf.data_ptr()))
    for _ in range(args.warmup):
        prob["run"]()
    torch.cuda.synchronize()

    def capture(body):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(args.steps):
                body(i)
        return g

    def cold(i):
        scratch.fill_(float(i))
        prob["run"]()
    graphs = {"hot": capture(lambda i: prob["run"]()), "cold": capture(cold)}
    names = [("issue", 0, 1), ("first_stage_landed", 0, 5), ("loop", 5, 6), ("hand_off", 6, 2),
             ("epilogue_math_staging", 2, 3), ("store_issue", 3, 4), ("life", 0, 4)]
    res = {"hot": [], "cold": []}
    for _ in range(3):
        for name, g in graphs.items():
            buf.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            t = buf.view(-1, 8).cpu().numpy().astype(np.int64)
            t = t[t[:, 0] != 0]
            full = t[t[:, 4] != 0]  # workgroups that ran the staged epilogue (not split chunks)
            q = lambda x: [round(float(np.percentile(x, p)) / 100, 2) for p in (10, 50, 90)]
            t0 = t[:, 0].min()
            ends = np.max(t[:, [2, 4, 6]], axis=1)
            rec = {"workgroups": int(len(t)), "start_spread_us": q(t[:, 0] - t0),
                   "span_us": round(float(ends.max() - t0) / 100, 2)}
            for nm, a, b in names:
                rec[nm + "_us"] = q(full[:, b] - full[:, a])
            res[name].append(rec)
    line = {"metric": f"SpMM phase timeline, {prob['workload']}", "unit": "us", "value": res["cold"][-1]["span_us"],
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": False,
            "config": {"workload": prob["workload"]}, "extra": res}
    print(json.dumps(line), flush=True)


def main():
    args = parse()
    if args.traffic_summary:
        traffic_summary(args.traffic_summary)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); every GPU box here has one "
              "GPU and the SpMM path is built and measured on a single MI355X.", file=sys.stderr)
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    explicit = args.config is not None
    args.config = args.config or "c2"
    if args.op in ("float", "sddmm"):
        bench_float(args, dev)
        return
    if args.op == "floor":
        bench_floor(args, dev)
        return
    if args.op == "clock":
        bench_clock(args, dev)
        return
    if args.op == "phases":
        bench_phases(args, dev)
        return
    if args.op != "spmm":
        bench_input_side(args, dev)
        return
    cfg = args.config
    prob = build_problem(cfg, dev, args.epilogue)
    if args.chunk:
        prob["chunk"] = args.chunk
    if args.counters:
        run_for_counters(prob, args.steps)
        return
    cold, hot, wall = time_gpu(prob, args.steps, args.warmup, flush=not args.profile)
    t_ms = cold if cold is not None else hot
    tops = prob["ops"] / (t_ms * 1e-3) / 1e12
    roof = roofline_of(prob, t_ms, cfg)
    roofline_ms = roof.pop("roofline_ms")
    cpu = None
    if args.cpu_seconds > 0 and not args.profile:
        cpu = cpu_leg(prob, args.cpu_seconds, cfg)
    line = {
        "metric": "INT8 BSpMM effective TOPS + % roofline, 4096x4096 90% sparse, N=512",
        "value": round(tops, 3),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": prob["dtype"],
        "data": "synthetic (seeded generators of BASELINE.json configs)",
        "config": {"workload": prob["workload"], "M": prob["M"], "K": prob["K"], "N": prob["N"],
                   "n_tiles": prob["nb"], "epilogue": prob["epilogue"], "kind": prob["kind"],
                   "cache": "cold (1 GiB overwrite between steps)" if not args.profile else "hot"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": {"hot_ms": round(hot, 5),
                  "hot_tops": round(prob["ops"] / (hot * 1e-3) / 1e12, 3),
                  "hot_gbs": round(prob["bytes"] / (hot * 1e-3) / 1e9, 1),
                  "roofline_ms": roofline_ms,
                  "gather_bytes": gather_bytes(prob),
                  "gather_tbs": round(gather_bytes(prob) / (t_ms * 1e-3) / 1e12, 2),
                  "dense_equiv_tops": round(2.0 * prob["M"] * prob["K"] * prob["N"] / (t_ms * 1e-3) / 1e12, 2),
                  "wall_s": round(wall, 3),
                  "device": device_peaks()},
    }
    if cfg != "c2":
        line["metric"] = f"{prob['kind'].upper()} BSpMM effective TOPS + % roofline, {prob['workload']}"
    elif not explicit and not args.profile and args.per_config:
        # The default run also reports every other config (cold ms, TOPS,
        # roofline fraction, traffic ratio, CPU baseline); the headline
        # fields above stay c2's.
        del prob
        torch.cuda.empty_cache()
        line["extra"]["per_config"] = {c: per_config_line(c, dev, args) for c in PER_CONFIG}
        # The harness floor measured in the same run: c2's time over a plain
        # copy of its algorithmic bytes.
        fl = floor_measure(dev, min(args.steps, 20), args.warmup)
        line["extra"]["floor"] = fl
        line["extra"]["c2_over_copy"] = round(t_ms / fl["copy_c2_bytes"]["ms"], 3)
        line["extra"]["c2_over_tiny_kernel"] = round(t_ms / fl["tiny_kernel"]["ms"], 3)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
