"""Benchmark of the gtx16_fp16 GEMM hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--report FILE]

Prints ONE JSON line for the BASELINE metric "TFLOPS (% MFMA peak) at 4096^3; GB/s (% HBM peak)
for M=1 4096x4096 mm_t":

* ``value`` -- TFLOPS of ``gtx16_fp16.mm_t`` on the 4096^3 configuration with fp32 activations
  (1% of rows pushed to |max| in [2e3, 2e5], so the power-of-two row rescale is exercised) and
  fp16 weights, fp32 out: one step = one mm_t call (rowscale cast + MFMA GEMM), inputs resident in
  HBM, ``steps`` calls timed between two ``torch.cuda.synchronize()``. Before the ``warmup``
  steps, untimed mm_t calls run for ``--settle-ms`` (default 200 ms) so the timed steps see the
  part's working clock; the line reports that phase (``clock_settle``) and the shader clock the
  last timed step's GEMM held (``clock_mhz_last_timed_gemm``, from the kernel's own clock stamps).
* ``roofline`` -- the GEMM kernel alone (the dominant kernel): 2*M*N*K flop per launch divided by
  its average duration in the timed steps (``kernel_ms``: the steps' HIP-event time per step minus
  the rowscale kernel's own time, on the stream the kernels run on), against the fp16 dense MFMA
  peak; next to it an event pair around the GEMM of each of ``steps`` (rowscale, GEMM) sequences
  (``kernel_ms_event_pairs``) and the same kernel launched back to back
  (``kernel_ms_back_to_back``, at a lower clock: the part is power-limited), each with the shader
  clock its last GEMM held.
* ``skinny_m1`` -- the second half of the metric: GB/s of the M=1 K=N=4096 skinny path, kernel
  time from HIP events around a captured HIP graph of launches that rotate over 16 distinct 32 MiB
  weight copies (512 MiB, twice the 256 MB Infinity Cache, so bytes come from HBM), against the
  8 TB/s HBM peak; plus the per-call mm_t time and its own ``cpu_baseline``, and the same
  product on FastLinear's decode layout (``fastlinear_decode_layout``, timed the same way; not the
  metric, which is mm_t on w_t as given).
* ``cpu_baseline`` -- the reference's CPU path (torch fp32 matmul, the fallback of ops.py:119)
  on a 4096^3 sample on the host cores of the same run (the skinny half: fp32 addmm at M=1).

Inputs are synthetic and seeded on the CPU (x = seed 0, w = 1, bias = 2, outlier rows = 3).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (str(REPO), str(REPO / "gtx16-fp16_amd"), str(REPO / "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

MFMA_F16_PEAK_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 flop/clk/CU (dense fp16)
TRAFFIC_FILE = REPO / "profiles" / "traffic.json"  # FETCH_SIZE/WRITE_SIZE runs (calibrated), per launch
HBM_PEAK_GBS = 8000.0
METRIC = "TFLOPS (% MFMA peak) at 4096^3; GB/s (% HBM peak) for M=1 4096x4096 mm_t"


def parse(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # ~30 ms of MFMA load brings the part to its working clock: with 5 warm-up steps the first timed
    # steps still run slow (measured 869 vs 1001 TFLOPS for 5 vs 200 warm-up steps with the earlier
    # 32x32x16 GEMM).
    ap.add_argument("--warmup", type=int, default=200)
    # Independently of --warmup, untimed mm_t calls run for this long before the warm-up steps: the
    # part needs ~35 ms of load to reach its working clock (measured: the first steps take 139-148 us,
    # ~126 us after 35 ms, flat for the next 3 s). The line reports the phase as `clock_settle`.
    ap.add_argument("--settle-ms", type=float, default=200.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--report", type=str, default=None, help="also write per-kernel details to this JSON file")
    ap.add_argument("--all", action="store_true",
                    help="also time every BASELINE configuration through the public API and write the per-config "
                         "table to --report (default bench_configs.json in the working directory); the JSON line is unchanged")
    ap.add_argument("--only", choices=["gemm", "rowscale", "skinny", "copy", "c1", "c3"], default=None,
                    help="launch just this kernel --steps times on the headline shapes (for rocprofv3 counter "
                         "runs) and print its average time; copy = a plain 256 MiB device copy, the "
                         "calibration for FETCH_SIZE / WRITE_SIZE; c1 / c3 = the C1 matmul 1024^3 and the "
                         "C3 split-K 64x4096x1024 mm_t through the public API")
    ap.add_argument("--bert", action="store_true",
                    help="time only the BERT-base configuration (fp32 vs patch()) and print its JSON line")
    ap.add_argument("--peak", action="store_true",
                    help="measure this part's fp32/fp16 VALU, MFMA and HBM read peaks and print them")
    ap.add_argument("--overhead", action="store_true",
                    help="time only the per-call cost of FastLinear vs nn.Linear at one token and print it")
    return ap.parse_args(argv)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def event_time_ms(fn, reps: int, torch) -> float:
    """Average ms per call of ``fn`` from HIP events on torch's current stream."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / reps


def gemm_clock_mhz(torch, lib, dev) -> float:
    """Shader clock the latest GEMM launch on the current stream held: its workgroup 0's main-loop
    shader cycles over 100 MHz reference ticks (g16_gemm_clock)."""
    buf = torch.zeros(2, dtype=torch.int64, device=dev)
    _clib_ok(lib.g16_gemm_clock(buf.data_ptr(), torch.cuda.current_stream(dev).cuda_stream))
    cyc, ticks = buf.tolist()
    return 100.0 * cyc / ticks if ticks else 0.0


def bench_c4(torch, g, lib, steps: int, warmup: int, dev, settle_ms: float = 0.0) -> dict:
    from _inputs import outlier_rows, randn

    M = K = N = 4096
    x = outlier_rows(randn((M, K), seed=0), 0.01, 2e3, 2e5, seed=3).to(dev)
    w = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).to(dev)
    flop = 2.0 * M * N * K

    # clock settle: untimed mm_t calls for settle_ms of wall time, then the warm-up steps
    settle_calls = 0
    t_settle = time.perf_counter()
    while (time.perf_counter() - t_settle) * 1e3 < settle_ms:
        for _ in range(8):
            g.mm_t(x, w, None, torch.float32)
        settle_calls += 8
        torch.cuda.synchronize()
    settle_wall_ms = (time.perf_counter() - t_settle) * 1e3
    for _ in range(warmup):
        g.mm_t(x, w, None, torch.float32)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        g.mm_t(x, w, None, torch.float32)
    ev1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    step_ms_events = ev0.elapsed_time(ev1) / steps  # the same steps on the GPU's clock
    clock_after = gemm_clock_mhz(torch, lib, dev)  # the last timed step's GEMM

    # Kernel-level timing on the stream the kernels are launched on (torch's current stream).
    stream = torch.cuda.current_stream(dev).cuda_stream
    # mm_t's route for this shape: the cast writes the tile-packed fp16 copy, the 256x256 GEMM reads it
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    assert lib.g16_hgemm_use_packed(M, N, K, cus) == 1
    xp = torch.empty(lib.g16_packed_a_bytes(M, K) // 2, dtype=torch.float16, device=dev)
    rs = torch.empty(M, dtype=torch.float32, device=dev)
    out = torch.empty(M, N, dtype=torch.float32, device=dev)

    def rowscale():
        lib.g16_rowscale_pack_f32(x.data_ptr(), xp.data_ptr(), rs.data_ptr(), M, K, 1024.0, stream)

    def gemm():
        lib.g16_hgemm_packed_f32out(xp.data_ptr(), w.data_ptr(), out.data_ptr(), None, rs.data_ptr(), M, N, K, stream)

    # The GEMM's time in the timed steps themselves: each step's HIP-event time minus the rowscale
    # kernel's own time (measured below, back to back). Two other views are reported next to it:
    # an event pair around the GEMM of each of `steps` (rowscale, GEMM) sequences, which adds the
    # events' own packets to every GEMM (and read 1-7 % above the kernel trace's average on some
    # boxes), and the GEMM launched back to back. The part is power-limited, and its clock follows
    # the average power of the last milliseconds: the rowscale pass (HBM-bound, little MFMA power)
    # between GEMMs lets it hold a higher clock for the GEMM than back-to-back GEMM launches get.
    # Each figure comes with the clock the last GEMM of its batch held (the kernel's own s_memtime /
    # s_memrealtime stamps).
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    for b, c in evs:
        rowscale()
        b.record()
        gemm()
        c.record()
    torch.cuda.synchronize()
    gemm_ms = statistics.fmean(b.elapsed_time(c) for b, c in evs)
    clock_in_steps = gemm_clock_mhz(torch, lib, dev)
    # back to back: `steps` launches between one event pair, the median of 3 such batches
    gemm_b2b_ms = statistics.median(event_time_ms(gemm, steps, torch) for _ in range(3))
    clock_b2b = gemm_clock_mhz(torch, lib, dev)
    rowscale_ms = statistics.median(event_time_ms(rowscale, steps, torch) for _ in range(3))
    gemm_in_steps_ms = step_ms_events - rowscale_ms
    tflops = flop / (wall_ms * 1e-3) / 1e12
    gemm_tflops = flop / (gemm_in_steps_ms * 1e-3) / 1e12
    # rowscale: reads 64 MiB fp32, writes 32 MiB fp16 + 16 KiB of scales
    rs_bytes = M * K * 4 + M * K * 2 + M * 4
    return {
        "wall_ms_per_step": wall_ms,
        "tflops": tflops,
        "step_ms_events": step_ms_events,
        "gemm_kernel_ms": gemm_in_steps_ms,
        "gemm_kernel_tflops": gemm_tflops,
        "gemm_event_pair_ms": gemm_ms,
        "gemm_event_pair_clock_mhz": clock_in_steps,
        "gemm_b2b_ms": gemm_b2b_ms,
        "gemm_b2b_clock_mhz": clock_b2b,
        "rowscale_kernel_ms": rowscale_ms,
        "rowscale_kernel_gbs": rs_bytes / (rowscale_ms * 1e-3) / 1e9,
        "flop_per_step": flop,
        "outlier_rows": int(round(0.01 * M)),
        "settle_ms": settle_wall_ms,
        "settle_calls": settle_calls,
        "clock_mhz_after_timed": clock_after,
    }


def bench_skinny(torch, lib, g, steps: int, warmup: int, dev, copies: int = 16) -> dict:
    from _inputs import randn

    M, K, N = 1, 4096, 4096
    x = randn((M, K), seed=0).to(dev)
    b = randn((N,), seed=2, scale=0.02).to(dev)
    w0 = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).to(dev)
    # distinct allocations of the weight, so consecutive launches never find it in a cache
    ws = [w0.clone() for _ in range(copies)]
    nbytes = M * K * 4 + K * N * 2 + N * 4 + M * N * 4
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    ksplit = lib.g16_skinny_plan(M, N, K, cus)
    work = torch.empty(max(lib.g16_skinny_workspace_bytes(M, N, K, ksplit), 256), dtype=torch.uint8, device=dev)
    cnt = torch.zeros(max(lib.g16_skinny_counter_bytes(M, N, K, ksplit), 256), dtype=torch.uint8, device=dev)
    out = torch.empty(M, N, dtype=torch.float32, device=dev)

    # per-call wall time of the Python API, rotating the weight copies
    for i in range(warmup):
        g.mm_t(x, ws[i % copies], b, torch.float32)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    calls = max(steps, copies)
    for i in range(calls):
        g.mm_t(x, ws[i % copies], b, torch.float32)
    torch.cuda.synchronize()
    call_us = (time.perf_counter() - t0) * 1e6 / calls

    # kernel time: a HIP graph of `copies` launches, replayed between events
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        st = side.cuda_stream
        for wi in ws:  # warm the exact launches once before capture
            assert lib.g16_skinny_f32in(x.data_ptr(), wi.data_ptr(), out.data_ptr(), b.data_ptr(), M, N, K, ksplit,
                                        work.data_ptr(), work.numel(), cnt.data_ptr(), cnt.numel(), st) == 0
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            cap = torch.cuda.current_stream(dev).cuda_stream
            for wi in ws:
                lib.g16_skinny_f32in(x.data_ptr(), wi.data_ptr(), out.data_ptr(), b.data_ptr(), M, N, K, ksplit,
                                     work.data_ptr(), work.numel(), cnt.data_ptr(), cnt.numel(), cap)
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    # 20 replays of the 16-launch graph per timing (each replay adds the graph's own launch cost once)
    reps = 20
    per_launch = []
    for _ in range(3):
        ms = event_time_ms(graph.replay, reps, torch)
        per_launch.append(ms / copies)
    kern_ms = min(per_launch)

    # FastLinear's decode layout of the same weights (not mm_t's path: mm_t takes w_t as given),
    # timed the same way
    wds = []
    for wi in ws:
        wd = torch.empty(K * N, dtype=torch.float16, device=dev)
        _clib_ok(lib.g16_pack_decode_weight(wi.data_ptr(), wd.data_ptr(), K, N, torch.cuda.current_stream(dev).cuda_stream))
        wds.append(wd)
    out2 = torch.empty(M, N, dtype=torch.float32, device=dev)
    graph2 = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        side.wait_stream(torch.cuda.current_stream(dev))
        for wd in wds:
            _clib_ok(lib.g16_skinny_strips_f32in(x.data_ptr(), wd.data_ptr(), out2.data_ptr(), b.data_ptr(), M, N, K,
                                                 side.cuda_stream))
        side.synchronize()
        with torch.cuda.graph(graph2, stream=side):
            cap = torch.cuda.current_stream(dev).cuda_stream
            for wd in wds:
                lib.g16_skinny_strips_f32in(x.data_ptr(), wd.data_ptr(), out2.data_ptr(), b.data_ptr(), M, N, K, cap)
    torch.cuda.synchronize()
    for _ in range(3):
        graph2.replay()
    torch.cuda.synchronize()
    strips_ms = min(event_time_ms(graph2.replay, reps, torch) / copies for _ in range(3))
    del graph2, wds
    return {
        "M": M, "K": K, "N": N,
        "ksplit": ksplit,
        "bytes_per_launch": nbytes,
        "kernel_us": kern_ms * 1e3,
        "kernel_gbs": nbytes / (kern_ms * 1e-3) / 1e9,
        "fastlinear_decode_layout_kernel_us": strips_ms * 1e3,
        "fastlinear_decode_layout_kernel_gbs": nbytes / (strips_ms * 1e-3) / 1e9,
        "call_us": call_us,
        "call_gbs": nbytes / (call_us * 1e-6) / 1e9,
        "weight_copies": copies,
        "weight_bytes_rotated": copies * K * N * 2,
    }


def _time_call(torch, fn, steps: int, warmup: int = 20) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    return min(event_time_ms(fn, steps, torch) for _ in range(3))


def _cpu_ms(fn, budget_s: float = 4.0) -> tuple[float, int]:
    """Host time of ``fn`` in ms: 2 warm-ups and the median of 5 reps (fewer when one call is long,
    so a row stays within ~budget_s). Returns (median ms, reps)."""
    t0 = time.perf_counter()
    fn()
    one = time.perf_counter() - t0
    if one < budget_s / 7:
        fn()
    reps = max(1, min(5, int(budget_s / max(one, 1e-6)) - 1))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times) * 1e3, reps


def bench_all(torch, g, steps: int, dev) -> list:
    """Every BASELINE configuration through the public API (algorithmic units: flops = 2MNK,
    bytes = M*K*sizeof(x) + 2*K*N + 4*N*[bias] + M*N*sizeof(out)), each row with its roofline
    (the bound its arithmetic intensity puts it under, and the fraction of that peak reached) and
    the reference's CPU path on the same inputs (torch fp32 on the host cores, the fallback of
    ops.py:119 / linear.py:69-70); then the reference's own GEMM sweep (bench/bench_gemm.py:24-35)."""
    from _inputs import outlier_rows, randn

    rows = []
    ridge = MFMA_F16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)  # flop per byte where the two roofs meet
    threads = torch.get_num_threads()

    def add(name, M, K, N, xbytes, obytes, bias, ms, cpu_fn=None, extra=None):
        flop = 2.0 * M * N * K
        nbytes = M * K * xbytes + 2 * K * N + (4 * N if bias else 0) + M * N * obytes
        tflops = flop / (ms * 1e-3) / 1e12
        gbs = nbytes / (ms * 1e-3) / 1e9
        bound = "mfma" if flop / nbytes > ridge else "hbm"
        r = {"config": name, "M": M, "K": K, "N": N, "us": round(ms * 1e3, 2),
             "TFLOPS": round(tflops, 2), "GB/s": round(gbs, 1),
             "pct_mfma_peak": round(100 * tflops / MFMA_F16_PEAK_TFLOPS, 2),
             "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
             "roofline": {"bound": bound, "arith_intensity": round(flop / nbytes, 1),
                          "frac": round(tflops / MFMA_F16_PEAK_TFLOPS if bound == "mfma" else gbs / HBM_PEAK_GBS, 4)}}
        if cpu_fn is not None:
            cms, reps = _cpu_ms(cpu_fn)
            r["cpu_baseline"] = {"us": round(cms * 1e3, 1), "TFLOPS": round(flop / (cms * 1e-3) / 1e12, 4),
                                 "GB/s": round(nbytes / (cms * 1e-3) / 1e9, 2), "cores": threads,
                                 "reps": reps, "what": "torch fp32 on the host (the reference's CPU path)"}
            r["speedup_vs_cpu"] = round(cms / ms, 1)
        if extra:
            r.update(extra)
        rows.append(r)
        print(json.dumps(r), flush=True)

    # C1: matmul 1024^3, fp16 in/out
    a = randn((1024, 1024), seed=0, dtype=torch.float16)
    b = randn((1024, 1024), seed=1, dtype=torch.float16)
    af, bf = a.float(), b.float()
    ad, bd = a.to(dev), b.to(dev)
    add("C1 matmul fp16 1024^3", 1024, 1024, 1024, 2, 2, False, _time_call(torch, lambda: g.matmul(ad, bd), steps),
        cpu_fn=lambda: af @ bf)
    # C2: skinny decode (fp32 x, fp16 w_t, fp32 bias, fp32 out), weights rotated over 16 copies
    for (M, K, N) in ((1, 4096, 4096), (4, 4096, 4096), (1, 1024, 3072)):
        x = randn((M, K), seed=0)
        w0 = randn((K, N), seed=1, scale=0.02, dtype=torch.float16)
        bias = randn((N,), seed=2, scale=0.02)
        wf = w0.float()
        xd, bdv = x.to(dev), bias.to(dev)
        copies = max(16, (512 << 20) // (K * N * 2))
        ws = [w0.to(dev) for _ in range(copies)]
        idx = iter(range(1 << 30))
        ms = _time_call(torch, lambda: g.mm_t(xd, ws[next(idx) % copies], bdv, torch.float32), max(steps, copies))
        add(f"C2 skinny {M}x{K}x{N}", M, K, N, 4, 4, True, ms, cpu_fn=lambda: torch.addmm(bias, x, wf),
            extra={"weight_copies": copies, "timing": "per mm_t call"})
        del ws
        # the same product through FastLinear's token-by-token path (its decode layout where the
        # library's rule takes it), one layer per weight copy
        layers = []
        for _ in range(copies):
            fl = g.FastLinear(K, N, bias=True, device=dev)
            fl.prepack_decode = True  # opt-in: the decode-layout copy of the weight
            with torch.no_grad():
                fl.weight_t.copy_(w0.to(dev))
                fl.bias.copy_(bdv)
            layers.append(fl)
        lib = _clib_lib()
        route = "decode layout" if lib.g16_skinny_strips_route(M, N, K, 1) else "split kernel on weight_t"
        idx = iter(range(1 << 30))
        with torch.no_grad():
            ms = _time_call(torch, lambda: layers[next(idx) % copies](xd), max(steps, copies))
        add(f"C2 FastLinear decode {M}x{K}x{N}", M, K, N, 4, 4, True, ms,
            extra={"weight_copies": copies, "timing": "per FastLinear call", "route": route})
        del layers
    # M = 8 through mm_t, where the skinny kernel multiplies on the matrix cores (32..128 K rows per
    # wavefront on 256-column strips; an fp16 hi/lo split of the activations)
    lib = _clib_lib()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    for (M, K, N) in ((8, 4096, 4096), (8, 11008, 4096)):
        x = randn((M, K), seed=0)
        w0 = randn((K, N), seed=1, scale=0.02, dtype=torch.float16)
        bias = randn((N,), seed=2, scale=0.02)
        wf = w0.float()
        xd, bdv = x.to(dev), bias.to(dev)
        copies = max(16, (512 << 20) // (K * N * 2))
        ws = [w0.to(dev) for _ in range(copies)]
        ks = lib.g16_skinny_plan(M, N, K, cus)
        rpw = -(-(-(-K // ks)) // 8)
        form = ("matrix cores" if lib.g16_skinny_strip_cols(M, N) == 256 and 32 <= rpw <= 128
                else "fp32 FMA loop")
        idx = iter(range(1 << 30))
        ms = _time_call(torch, lambda: g.mm_t(xd, ws[next(idx) % copies], bdv, torch.float32), max(steps, copies))
        add(f"skinny {M}x{K}x{N}", M, K, N, 4, 4, True, ms, cpu_fn=lambda: torch.addmm(bias, x, wf),
            extra={"weight_copies": copies, "timing": "per mm_t call", "form": form, "ksplit": ks,
                   "rows_per_wavefront": rpw})
        del ws
    # C3: split-K (fp16 A, fp32 out + bias); repeat runs must be bitwise equal
    for (M, K, N) in ((64, 1024, 1024), (64, 4096, 1024)):
        x = randn((M, K), seed=0, dtype=torch.float16)
        w = randn((K, N), seed=1, scale=0.02, dtype=torch.float16)
        bias = randn((N,), seed=2, scale=0.02)
        xf, wf = x.float(), w.float()
        xd, wd, bdv = x.to(dev), w.to(dev), bias.to(dev)
        outs = [g.mm_t(xd, wd, bdv, torch.float32) for _ in range(10)]
        same = all(torch.equal(o, outs[0]) for o in outs[1:])
        ms = _time_call(torch, lambda: g.mm_t(xd, wd, bdv, torch.float32), steps)
        add(f"C3 split-K {M}x{K}x{N}", M, K, N, 2, 4, True, ms, cpu_fn=lambda: torch.addmm(bias, xf, wf),
            extra={"repeat_bitwise_equal": same})
    # C4: 4096^3 fp32 activations with outlier rows, fp32 out
    x = outlier_rows(randn((4096, 4096), seed=0), 0.01, 2e3, 2e5, seed=3)
    w = randn((4096, 4096), seed=1, scale=0.02, dtype=torch.float16)
    wf = w.float()
    xd, wd = x.to(dev), w.to(dev)
    t_settle = time.perf_counter()  # the same 200 ms clock settle as the headline line
    while time.perf_counter() - t_settle < 0.2:
        for _ in range(8):
            g.mm_t(xd, wd, None, torch.float32)
        torch.cuda.synchronize()
    add("C4 mm_t 4096^3 fp32 x", 4096, 4096, 4096, 4, 4, False,
        _time_call(torch, lambda: g.mm_t(xd, wd, None, torch.float32), steps), cpu_fn=lambda: x @ wf,
        extra={"clock_settle_ms": 200})
    del x, xd, wd
    rows.append(bench_bert(torch, g, dev, cpu_reps=1))
    print(json.dumps(rows[-1]), flush=True)
    rows.extend(bench_reference_sweep(torch, g, steps, dev))
    rows.extend(bench_overhead(torch, g, dev))
    return rows


def bench_reference_sweep(torch, g, steps: int, dev) -> list:
    """The reference's GEMM sweep (bench/bench_gemm.py:22-35): its nine shapes, fp16 x and w drawn
    as 0.5 * N(0,1) (seeded on the CPU here), and three columns -- torch fp32 matmul, torch fp16
    matmul (both hipBLASLt on this GPU, the vendor library the reference's cuBLAS columns stand
    for) and gtx16_fp16.mm_t(x, w, None, fp32) -- with each one's relative error against the fp32
    product. Times from HIP events over back-to-back calls after 20 warm-ups."""
    from _inputs import randn

    shapes = [(1, 4096, 4096), (4, 4096, 4096), (1, 1024, 3072), (64, 1024, 1024), (512, 1024, 4096),
              (1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096), (8192, 2048, 2048)]
    rows = []
    for M, K, N in shapes:
        x = randn((M, K), seed=0, scale=0.5, dtype=torch.float16).to(dev)
        w = randn((K, N), seed=1, scale=0.5, dtype=torch.float16).to(dev)
        xf, wf = x.float(), w.float()
        ref = xf @ wf
        fl = 2.0 * M * K * N
        t32 = _time_call(torch, lambda: xf @ wf, steps)
        t16 = _time_call(torch, lambda: x @ w, steps)
        ours = _time_call(torch, lambda: g.mm_t(x, w, None, torch.float32), steps)
        e16 = ((x @ w).float() - ref).norm() / ref.norm()
        eo = (g.mm_t(x, w, None, torch.float32) - ref).norm() / ref.norm()
        r = {"config": f"reference sweep {M}x{K}x{N}", "M": M, "K": K, "N": N,
             "torch_fp32_TFLOPS": round(fl / (t32 * 1e-3) / 1e12, 2),
             "torch_fp16_TFLOPS": round(fl / (t16 * 1e-3) / 1e12, 2),
             "gtx16_fp16_TFLOPS": round(fl / (ours * 1e-3) / 1e12, 2), "gtx16_fp16_us": round(ours * 1e3, 2),
             "vs_fp32": round(t32 / ours, 2), "vs_fp16": round(t16 / ours, 2),
             "rel_err_fp16": float(f"{e16.item():.2e}"), "rel_err_ours": float(f"{eo.item():.2e}")}
        rows.append(r)
        print(json.dumps(r), flush=True)
        del x, w, xf, wf, ref
    return rows


def bench_overhead(torch, g, dev, n: int = 1000) -> list:
    """Per-call host cost and wall time of FastLinear vs nn.Linear at one token (the decode path),
    as bench/overhead.py:9-29 of the reference measures it: `cpu` is the time to enqueue n calls,
    `wall` the time until they have also finished on the GPU. `fast_linear_graph_us` is the same
    FastLinear call replayed from a HIP graph of 32 captured calls (per call: replay time / 32),
    which removes the host cost the reference's README (README.md:77) leaves to CUDA graphs."""
    import torch.nn as nn

    def graph_cost(fl, x, calls: int = 32, reps: int = 50):
        with torch.no_grad():
            for _ in range(3):  # eager first: split buffers exist before capture (no fills recorded)
                ref = fl(x)
            torch.cuda.synchronize()
            s = torch.cuda.Stream(dev)
            s.wait_stream(torch.cuda.current_stream(dev))
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.stream(s):
                fl(x)
                torch.cuda.synchronize()
                with torch.cuda.graph(graph, stream=s):
                    outs = [fl(x) for _ in range(calls)]
            torch.cuda.current_stream(dev).wait_stream(s)
            graph.replay()
            torch.cuda.synchronize()
            if not all(torch.equal(o, ref) for o in outs):
                raise RuntimeError("graph replay differs from the eager FastLinear call")
            for _ in range(5):
                graph.replay()
            torch.cuda.synchronize()
            t = time.perf_counter()
            for _ in range(reps):
                graph.replay()
            torch.cuda.synchronize()
            return round((time.perf_counter() - t) / (reps * calls) * 1e6, 2)

    def cost(fn):
        with torch.no_grad():
            for _ in range(50):
                fn()
            torch.cuda.synchronize()
            t = time.perf_counter()
            for _ in range(n):
                fn()
            cpu = (time.perf_counter() - t) / n
            torch.cuda.synchronize()
            wall = (time.perf_counter() - t) / n
        return round(cpu * 1e6, 2), round(wall * 1e6, 2)

    rows = []
    for K, N in ((1024, 1024), (1024, 3072), (3072, 1024), (4096, 4096)):
        torch.manual_seed(0)
        lin = nn.Linear(K, N).to(dev)
        fl = g.FastLinear.from_linear(lin)
        fl.prepack_decode = True  # opt-in: the decode-layout copy of the weight
        x = torch.randn(1, 1, K, device=dev)
        a, b = cost(lambda: lin(x)), cost(lambda: fl(x))
        rows.append({"config": f"decode overhead 1x{K}x{N}", "nn_linear_cpu_us": a[0], "nn_linear_wall_us": a[1],
                     "fast_linear_cpu_us": b[0], "fast_linear_wall_us": b[1],
                     "fast_linear_graph_us": graph_cost(fl, x)})
        print(json.dumps(rows[-1]), flush=True)
    return rows


def bench_peak(torch, lib, dev) -> list:
    """Instruction and HBM peaks of this part (the analogue of the reference's bench/peak.py):
    fp32 FMA, packed fp16 FMA and the two fp16 MFMA shapes from register-only loops (the MFMA ones
    on near-constant and on random operand bits), the LDS read bandwidth for 16-byte and
    transposing reads, and a streaming read of a 4 GiB buffer. Each is
    the best of 3 timed launches after a warm-up; the instruction peaks also report the shader
    clock their loop ran at (s_memtime cycles over 100 MHz reference ticks)."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = torch.cuda.current_stream(dev).cuda_stream
    rows = []
    clocks = torch.zeros(2, dtype=torch.int64, device=dev)
    for kind, name, waves_per_simd, iters in (
            (0, "fp32 FMA (VALU)", 8, 20000), (1, "packed fp16 FMA (VALU)", 8, 20000),
            (2, "MFMA f16 32x32x16", 2, 20000), (3, "MFMA f16 16x16x32", 2, 20000),
            (4, "MFMA f16 32x32x16, random operands", 2, 20000), (5, "MFMA f16 16x16x32, random operands", 2, 20000),
            (8, "MFMA f16 16x16x32 in the 256x256 tile's order, C4-distributed operands", 2, 10000)):
        blocks = cus * waves_per_simd  # 256-lane workgroups: 4 wavefronts each, one per SIMD
        tflops, mhz = time_mfma_probe(torch, lib, dev, kind, blocks, iters)
        rows.append({"peak": name, "TFLOP/s": round(tflops, 1), "clock_MHz": round(mhz)})
        print(json.dumps(rows[-1]), flush=True)
    for kind, name in ((6, "LDS read, ds_read_b128"), (7, "LDS transposing read, ds_read_b64_tr_b16")):
        for per_cu in (1, 2, 4):  # 32 KB of LDS per workgroup: at most 5 per CU
            blocks, iters = cus * per_cu, 20000
            out = torch.empty(blocks * 256, device=dev)
            _clib_ok(lib.g16_peak_run(kind, blocks, 100, out.data_ptr(), stream))
            torch.cuda.synchronize()
            best, mhz = float("inf"), 0.0
            for _ in range(3):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                _clib_ok(lib.g16_peak_run_clocked(kind, blocks, iters, out.data_ptr(), clocks.data_ptr(), stream))
                e1.record()
                e1.synchronize()
                t = e0.elapsed_time(e1) * 1e-3
                if t < best:
                    cyc, ticks = clocks.tolist()
                    best, mhz = t, (100.0 * cyc / ticks if ticks else 0.0)
            nb = lib.g16_peak_flops_per_lane_iter(kind) * blocks * 256 * iters
            rows.append({"peak": f"{name} ({per_cu} workgroups/CU)", "GB/s": round(nb / best / 1e9, 1),
                         "bytes_per_clk_per_CU": round(nb / best / (mhz * 1e6) / cus, 1) if mhz else None,
                         "ms": round(best * 1e3, 3), "clock_MHz": round(mhz)})
            print(json.dumps(rows[-1]), flush=True)
    rot = stream_read_rotated(torch, lib, dev)
    rows.append({"peak": "HBM read stream, one launch per 32 MiB buffer rotated over 16 buffers "
                         f"({rot['workgroups_per_cu']} workgroups/CU, the best of 2-16)", "GB/s": round(rot["gbs"], 1)})
    print(json.dumps(rows[-1]), flush=True)
    nbytes = 4 << 30
    buf = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    for per_cu in (4, 8, 16):  # workgroups of 256 lanes per CU, 8 loads in flight per lane
        blocks = cus * per_cu
        out = torch.empty(blocks * 256, device=dev)
        _clib_ok(lib.g16_stream_read(buf.data_ptr(), nbytes, blocks, out.data_ptr(), stream))
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            _clib_ok(lib.g16_stream_read(buf.data_ptr(), nbytes, blocks, out.data_ptr(), stream))
            e1.record()
            e1.synchronize()
            best = min(best, e0.elapsed_time(e1) * 1e-3)
        rows.append({"peak": f"HBM read stream (4 GiB, 16-byte loads, {per_cu} workgroups/CU)",
                     "GB/s": round(nbytes / best / 1e9, 1), "ms": round(best * 1e3, 3)})
        print(json.dumps(rows[-1]), flush=True)
    del buf
    return rows


def c4_mfma_operands(torch, dev, groups: int, seed: int = 0):
    """Operands of the GEMM-order MFMA probe (g16_peak_mfma_data) for `groups` workgroups: per
    lane, two sets of 8 A fragments of fp16(N(0,1)) and 4 B fragments of fp16(N(0, 0.02^2)), the
    distributions of C4's activations (outlier rows aside) and weights, as int16 bit patterns."""
    gen = torch.Generator(dev).manual_seed(seed)
    v = torch.randn(groups, 256, 2, 12, 8, device=dev, generator=gen)
    v[..., 8:, :] *= 0.02
    return v.half().view(torch.int16).contiguous()


def time_mfma_probe(torch, lib, dev, kind: int, blocks: int, iters: int) -> tuple[float, float]:
    """(TFLOP/s, MHz) of an MFMA probe (kinds 0-7 through g16_peak_run_clocked; kind 8 is the
    GEMM-order probe on C4-distributed operands, every workgroup its own): best of 3 launches
    after a warm-up, with the shader clock workgroup 0's loop held."""
    stream = torch.cuda.current_stream(dev).cuda_stream
    clocks = torch.zeros(2, dtype=torch.int64, device=dev)
    if kind == 8:
        ops = c4_mfma_operands(torch, dev, blocks)
        out = torch.empty(blocks * 256 * 128, device=dev)

        def run(n, clk):
            return lib.g16_peak_mfma_data(blocks, n, ops.data_ptr(), blocks, out.data_ptr(), clk, stream)
    else:
        out = torch.empty(blocks * 256, device=dev)

        def run(n, clk):
            return lib.g16_peak_run_clocked(kind, blocks, n, out.data_ptr(), clk, stream)
    _clib_ok(run(100, None))
    best, mhz = float("inf"), 0.0
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        _clib_ok(run(iters, clocks.data_ptr()))
        e1.record()
        e1.synchronize()
        t = e0.elapsed_time(e1) * 1e-3
        if t < best:
            cyc, ticks = clocks.tolist()
            best, mhz = t, (100.0 * cyc / ticks if ticks else 0.0)
    return lib.g16_peak_flops_per_lane_iter(kind) * blocks * 256 * iters / best / 1e12, mhz


def measured_peaks(torch, lib, dev) -> dict:
    """The part's own ceilings for the two rooflines, next to the published peaks: the GEMM's MFMA
    stream without its memory traffic (g16_peak_mfma_data: the 256x256 tile's per-wavefront MFMA
    order on C4-distributed operands that change every instruction, two wavefronts per SIMD), with
    the clock it held; the register-only 16x16x32 loop on fixed uniform random bits (--peak kind 5)
    beside it; and the 4 GiB read stream at 16 workgroups per CU."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = torch.cuda.current_stream(dev).cuda_stream
    mfma, mhz = time_mfma_probe(torch, lib, dev, 8, cus * 2, 10000)
    mfma5, mhz5 = time_mfma_probe(torch, lib, dev, 5, cus * 2, 20000)
    nbytes = 4 << 30
    buf = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    sblocks = cus * 16
    sout = torch.empty(sblocks * 256, device=dev)
    _clib_ok(lib.g16_stream_read(buf.data_ptr(), nbytes, sblocks, sout.data_ptr(), stream))
    sbest = float("inf")
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        _clib_ok(lib.g16_stream_read(buf.data_ptr(), nbytes, sblocks, sout.data_ptr(), stream))
        e1.record()
        e1.synchronize()
        sbest = min(sbest, e0.elapsed_time(e1) * 1e-3)
    del buf
    return {"mfma_tflops": mfma, "mfma_clock_mhz": mhz, "mfma_uniform_bits_tflops": mfma5,
            "mfma_uniform_bits_clock_mhz": mhz5, "stream_gbs": nbytes / sbest / 1e9}


def stream_read_rotated(torch, lib, dev, nbytes: int = 32 << 20, copies: int = 16) -> dict:
    """Read-stream ceiling at the skinny kernel's own size: one g16_stream_read launch per 32 MiB
    buffer, rotating over `copies` buffers (512 MiB, twice the Infinity Cache) like the skinny
    benchmark rotates its weight copies, timed the same way (a HIP graph of `copies` launches
    replayed between events). Best over 2-16 workgroups per CU."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    bufs = [torch.ones(nbytes, dtype=torch.uint8, device=dev) for _ in range(copies)]
    best = (0.0, 0)
    for per_cu in (2, 4, 8, 16):
        blocks = cus * per_cu
        out = torch.empty(blocks * 256, device=dev)
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            for bf in bufs:
                _clib_ok(lib.g16_stream_read(bf.data_ptr(), nbytes, blocks, out.data_ptr(), side.cuda_stream))
            side.synchronize()
            with torch.cuda.graph(graph, stream=side):
                cap = torch.cuda.current_stream(dev).cuda_stream
                for bf in bufs:
                    lib.g16_stream_read(bf.data_ptr(), nbytes, blocks, out.data_ptr(), cap)
        torch.cuda.synchronize()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        ms = min(event_time_ms(graph.replay, 8, torch) for _ in range(3)) / copies
        gbs = nbytes / (ms * 1e-3) / 1e9
        if gbs > best[0]:
            best = (gbs, per_cu)
        del graph
    del bufs
    return {"gbs": best[0], "workgroups_per_cu": best[1], "bytes": nbytes, "copies": copies}


def _clib_lib():
    from gtx16_fp16 import _clib

    return _clib.load()


def _clib_ok(status: int) -> None:
    if status != 0:
        raise RuntimeError(f"peak kernel launch failed with status {status}")


def bench_bert(torch, g, dev, reps: int = 3, cpu_reps: int = 0) -> dict:
    """C5: random-init BERT-base, 256 x 256 token ids, fp32 forward, then patch() and again; tokens/s
    of each and the cosine of the mean-pooled (and CLS) embeddings. With cpu_reps > 0, also the
    fp32 forward of the same model and ids on the host cores (the reference's CPU path), that many
    timed reps after one warm-up."""
    import torch.nn.functional as F
    from _models import BERT_LINEARS, bert_base, embeddings, token_ids

    torch.backends.cuda.matmul.allow_tf32 = False
    model = bert_base(seed=0).to(dev)
    ids = token_ids(256, 256, seed=0).to(dev)

    def timed():
        emb = embeddings(model, ids)  # warm-up
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(reps):
            emb = embeddings(model, ids)
        torch.cuda.synchronize()
        return emb, (time.perf_counter() - t) / reps

    ref, t32 = timed()
    cpu = None
    if cpu_reps > 0:
        cmodel = bert_base(seed=0)
        cids = ids.cpu()
        cms, creps = _cpu_ms(lambda: embeddings(cmodel, cids), budget_s=0.0)
        cpu = {"tokens_per_s": round(ids.numel() / (cms * 1e-3), 1), "ms_per_forward": round(cms, 1),
               "cores": torch.get_num_threads(), "reps": creps,
               "what": "the same fp32 model and ids on the host (the reference's CPU path), 1 warm-up"}
        del cmodel
    n = g.patch(model)
    torch.cuda.empty_cache()
    out, t16 = timed()
    # the same with the opt-in shared activation cast (Q, K and V of a layer share one rowscale cast)
    fls = [m for m in model.modules() if isinstance(m, g.FastLinear)]
    for m in fls:
        m.share_cast = True
    out_sc, t16_sc = timed()
    for m in fls:
        m.share_cast = False
    same_sc = all(torch.equal(a, b) for a, b in zip(out, out_sc))
    del out_sc
    # activation ranges the patched linears see (reference bench/diag_ranges.py), on 16 sequences
    from gtx16_fp16.diag import range_hooks, risky

    stats, handles = range_hooks(model)
    embeddings(model, ids[:16])
    for h in handles:
        h.remove()
    ranges = {"layers": len(stats), "layers_needing_care": len(risky(stats)),
              "rows_rescaled": sum(v["rows_rescaled"] for v in stats.values()),
              "rows_seen": sum(v["rows"] for v in stats.values()),
              "max_exponent": max((v["max_exponent"] for v in stats.values()), default=0),
              "x_amax": round(max((v["x_amax"] for v in stats.values()), default=0.0), 2)}
    cos = [F.cosine_similarity(o.double(), r.double(), dim=1) for o, r in zip(out, ref)]
    tokens = ids.numel()
    # Linear work per forward: 12 layers x (4 x 768^2 + 2 x 768 x 3072) MACs per token, plus the pooler.
    lin_flop = 2.0 * tokens * 12 * (4 * 768 * 768 + 2 * 768 * 3072) + 2.0 * 256 * 768 * 768
    del model
    torch.cuda.empty_cache()
    return {"config": "C5 BERT-base patch, 256x256 tokens, fp32 activations", "linears_patched": n,
            "linears_expected": BERT_LINEARS, "tokens_per_s": round(tokens / t16, 1),
            "fp32_tokens_per_s": round(tokens / t32, 1), "speedup_vs_fp32": round(t32 / t16, 3),
            "ms_per_forward": round(t16 * 1e3, 2), "fp32_ms_per_forward": round(t32 * 1e3, 2),
            "share_cast": {"tokens_per_s": round(tokens / t16_sc, 1), "ms_per_forward": round(t16_sc * 1e3, 2),
                           "bitwise_equal_to_default": same_sc,
                           "what": "FastLinear.share_cast = True (opt-in): consecutive layers on the same input "
                                   "share its rowscale cast"},
            "linear_TFLOPS_equiv": round(lin_flop / t16 / 1e12, 1),
            "cosine_mean_pooled_min": round(cos[0].min().item(), 8),
            "cosine_cls_min": round(cos[1].min().item(), 8), "activation_ranges": ranges,
            **({"cpu_baseline": cpu} if cpu else {})}


def cpu_baseline(torch) -> dict:
    """The reference's CPU path: torch fp32 matmul (ops.py:119 fallback) at 4096^3 on the host."""
    from _inputs import outlier_rows, randn

    M = K = N = 4096
    x = outlier_rows(randn((M, K), seed=0), 0.01, 2e3, 2e5, seed=3)
    w = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).float()
    torch.matmul(x, w)  # warm-up
    times = []
    t_end = time.perf_counter() + 10.0
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 30):
        t0 = time.perf_counter()
        torch.matmul(x, w)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": 2.0 * M * N * K / med / 1e12,
        "unit": "TFLOPS",
        "cores": torch.get_num_threads(),
        "kind": "reference",
        "sample": (f"torch fp32 x@w at M=K=N=4096 on the host (the reference's CPU path: ops.py:119 "
                   f"fallback), 1 warm-up + median of {len(times)} reps; cpu '{cpu_model()}', "
                   f"os.cpu_count()={os.cpu_count()}"),
    }


def cpu_baseline_skinny(torch) -> dict:
    """The reference's CPU path for the skinny half: torch fp32 x @ w + b (the ops.py:119 /
    linear.py:69-70 fallback) at M=1, K=N=4096 on the host, in the metric's unit (algorithmic GB/s:
    x, w as fp16, bias and out; w is held as fp32 on the host, since that is what the fallback
    multiplies)."""
    from _inputs import randn

    M, K, N = 1, 4096, 4096
    x = randn((M, K), seed=0)
    w = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).float()
    b = randn((N,), seed=2, scale=0.02)
    torch.addmm(b, x, w)  # warm-up
    times = []
    t_end = time.perf_counter() + 3.0
    while len(times) < 20 or (time.perf_counter() < t_end and len(times) < 2000):
        t0 = time.perf_counter()
        torch.addmm(b, x, w)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    nbytes = M * K * 4 + K * N * 2 + N * 4 + M * N * 4
    return {
        "value": nbytes / med / 1e9,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "reference",
        "sample": (f"torch fp32 addmm(b, x, w) at M=1 K=N=4096 on the host (the reference's CPU path), "
                   f"{med * 1e6:.1f} us per call, 1 warm-up + median of {len(times)} reps; cpu '{cpu_model()}', "
                   f"os.cpu_count()={os.cpu_count()}"),
    }


def run_only(torch, lib, what: str, steps: int, dev) -> dict:
    """Back-to-back launches of one kernel, for profiling runs."""
    from _inputs import outlier_rows, randn

    stream = torch.cuda.current_stream(dev).cuda_stream
    if what == "copy":
        n = 256 << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        fn = lambda: dst.copy_(src)  # noqa: E731
        bytes_moved = 2 * n
    elif what == "skinny":
        M, K, N = 1, 4096, 4096
        x = randn((M, K), seed=0).to(dev)
        b = randn((N,), seed=2, scale=0.02).to(dev)
        ws = [randn((K, N), seed=1, scale=0.02, dtype=torch.float16).to(dev) for _ in range(16)]
        out = torch.empty(M, N, device=dev)
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        ks = lib.g16_skinny_plan(M, N, K, cus)
        part = torch.empty(max(lib.g16_skinny_workspace_bytes(M, N, K, ks), 256), dtype=torch.uint8, device=dev)
        cnt = torch.zeros(max(lib.g16_skinny_counter_bytes(M, N, K, ks), 256), dtype=torch.uint8, device=dev)
        it = iter(range(1 << 30))

        def fn():
            w = ws[next(it) % 16]
            lib.g16_skinny_f32in(x.data_ptr(), w.data_ptr(), out.data_ptr(), b.data_ptr(), M, N, K, ks,
                                 part.data_ptr(), part.numel(), cnt.data_ptr(), cnt.numel(), stream)
        bytes_moved = M * K * 4 + K * N * 2 + N * 4 + M * N * 4
    elif what in ("c1", "c3"):
        import gtx16_fp16 as g

        if what == "c1":
            M = K = N = 1024
            a = randn((M, K), seed=0, dtype=torch.float16).to(dev)
            w = randn((K, N), seed=1, dtype=torch.float16).to(dev)
            fn = lambda: g.matmul(a, w)  # noqa: E731
        else:
            M, K, N = 64, 4096, 1024
            a = randn((M, K), seed=0, dtype=torch.float16).to(dev)
            w = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).to(dev)
            b = randn((N,), seed=2, scale=0.02).to(dev)
            fn = lambda: g.mm_t(a, w, b)  # noqa: E731
        bytes_moved = None
    else:
        M = K = N = 4096
        x = outlier_rows(randn((M, K), seed=0), 0.01, 2e3, 2e5, seed=3).to(dev)
        xp = torch.empty(lib.g16_packed_a_bytes(M, K) // 2, dtype=torch.float16, device=dev)
        rs = torch.empty(M, device=dev)
        lib.g16_rowscale_pack_f32(x.data_ptr(), xp.data_ptr(), rs.data_ptr(), M, K, 1024.0, stream)
        if what == "rowscale":
            fn = lambda: lib.g16_rowscale_pack_f32(x.data_ptr(), xp.data_ptr(), rs.data_ptr(), M, K,  # noqa: E731
                                                   1024.0, stream)
            bytes_moved = M * K * 6 + M * 4
        else:
            w = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).to(dev)
            out = torch.empty(M, N, device=dev)
            fn = lambda: lib.g16_hgemm_packed_f32out(xp.data_ptr(), w.data_ptr(), out.data_ptr(), None,  # noqa: E731
                                                     rs.data_ptr(), M, N, K, stream)
            bytes_moved = None
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    ms = event_time_ms(fn, steps, torch)
    res = {"only": what, "steps": steps, "avg_ms": round(ms, 5)}
    if bytes_moved:
        res["GB/s"] = round(bytes_moved / (ms * 1e-3) / 1e9, 1)
    else:
        res["TFLOP/s"] = round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1)
    return res


def traffic_bytes(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE runs
    (scaled by a plain copy's readings), or None when they are not there."""
    try:
        return int(json.loads(TRAFFIC_FILE.read_text())[kernel]["traffic_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def main(argv=None) -> int:
    args = parse(argv)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); the GEMM path "
              "has no multi-GPU component to time. Run with --gpus 1.", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    import gtx16_fp16 as g
    from gtx16_fp16 import _clib

    lib = _clib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.only:
        print(json.dumps(run_only(torch, lib, args.only, args.steps, dev)), flush=True)
        return 0
    if args.bert:
        print(json.dumps(bench_bert(torch, g, dev)), flush=True)
        return 0
    if args.overhead:
        bench_overhead(torch, g, dev)
        return 0
    if args.peak:
        bench_peak(torch, lib, dev)
        return 0
    configs = bench_all(torch, g, args.steps, dev) if args.all else None
    c4 = bench_c4(torch, g, lib, args.steps, args.warmup, dev, args.settle_ms)
    sk = bench_skinny(torch, lib, g, args.steps, args.warmup, dev)
    cpu = None if args.no_cpu_baseline else cpu_baseline(torch)
    cpu_sk = None if args.no_cpu_baseline else cpu_baseline_skinny(torch)
    mp = measured_peaks(torch, lib, dev)
    rot = stream_read_rotated(torch, lib, dev)

    gemm_tflops = c4["gemm_kernel_tflops"]
    line = {
        "metric": METRIC,
        "value": round(c4["tflops"], 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c4["wall_ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 (fp32 accumulate)",
        "data": "synthetic (seeded CPU randn: x fp32 with 1% outlier rows, w fp16 ~N(0,0.02^2))",
        "config": {"workload": "mm_t C4: M=K=N=4096, fp32 activations + pow2 rowscale, fp16 weights, fp32 out",
                   "M": 4096, "K": 4096, "N": 4096, "outlier_rows": c4["outlier_rows"]},
        "pct_of_peak": round(100.0 * c4["tflops"] / MFMA_F16_PEAK_TFLOPS, 2),
        "clock_settle": {"ms": round(c4["settle_ms"], 1), "mm_t_calls": c4["settle_calls"],
                         "what": "untimed mm_t calls before the warm-up steps (working clock after ~35 ms of load)"},
        "clock_mhz_last_timed_gemm": round(c4["clock_mhz_after_timed"]),
        "roofline": {
            "bound": "mfma",
            "kernel": "hgemm_kernel<256x256, packed A> (g16_hgemm_packed_f32out)",
            "achieved": round(gemm_tflops, 2),
            "peak": MFMA_F16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "traffic": traffic_bytes("gemm"),
            "kernel_ms": round(c4["gemm_kernel_ms"], 5),
            "timing": "the timed steps' HIP-event time per step minus the rowscale kernel's own time: the GEMM's share of each step",
            "clock_mhz": round(c4["clock_mhz_after_timed"]),
            "step_ms_events": round(c4["step_ms_events"], 5),
            "kernel_ms_event_pairs": round(c4["gemm_event_pair_ms"], 5),
            "clock_mhz_event_pairs": round(c4["gemm_event_pair_clock_mhz"]),
            "kernel_ms_back_to_back": round(c4["gemm_b2b_ms"], 5),
            "clock_mhz_back_to_back": round(c4["gemm_b2b_clock_mhz"]),
            "measured_peak_random_operands": round(mp["mfma_tflops"], 1),
            "measured_peak_clock_mhz": round(mp["mfma_clock_mhz"]),
            "measured_peak_what": "the GEMM tile's MFMA stream (order, operand reuse) on C4-distributed fp16 "
                                  "operands that change every instruction, registers only (g16_peak_mfma_data)",
            "measured_peak_uniform_random_bits": round(mp["mfma_uniform_bits_tflops"], 1),
            "measured_peak_uniform_random_bits_clock_mhz": round(mp["mfma_uniform_bits_clock_mhz"]),
            "frac_of_measured_peak": round(gemm_tflops / mp["mfma_tflops"], 4),
        },
        "rowscale_kernel": {"kernel": "rowscale_kernel<float, packed> (g16_rowscale_pack_f32)", "ms": round(c4["rowscale_kernel_ms"], 5), "GB/s": round(c4["rowscale_kernel_gbs"], 1),
                            "frac_hbm": round(c4["rowscale_kernel_gbs"] / HBM_PEAK_GBS, 4),
                            "traffic": traffic_bytes("rowscale")},
        "skinny_m1": {
            "workload": "mm_t M=1 K=N=4096, fp32 x, fp16 w_t, fp32 bias, fp32 out (16 rotated weight copies)",
            "value": round(sk["kernel_gbs"], 1),
            "unit": "GB/s",
            "pct_of_peak": round(100.0 * sk["kernel_gbs"] / HBM_PEAK_GBS, 2),
            "roofline": {
                "bound": "hbm",
                "kernel": "skinny_kernel<float,1> (g16_skinny_f32in)",
                "achieved": round(sk["kernel_gbs"], 1),
                "peak": HBM_PEAK_GBS,
                "unit": "GB/s",
                "frac": round(sk["kernel_gbs"] / HBM_PEAK_GBS, 4),
                "traffic": traffic_bytes("skinny"),
                "kernel_us": round(sk["kernel_us"], 3),
                "measured_peak_read_stream": round(mp["stream_gbs"], 1),
                "frac_of_measured_peak": round(sk["kernel_gbs"] / mp["stream_gbs"], 4),
                # the same read stream at the kernel's own size: one launch per 32 MiB buffer,
                # rotated over 16 buffers and timed like the skinny launches
                "measured_peak_read_stream_32mib": round(rot["gbs"], 1),
                "frac_of_measured_peak_32mib": round(sk["kernel_gbs"] / rot["gbs"], 4),
            },
            # FastLinear's token-by-token path on its decode layout (same product and bytes; not the
            # metric, which is mm_t on w_t as given)
            "fastlinear_decode_layout": {
                "kernel": "strips_kernel<float,1> (g16_skinny_strips_f32in)",
                "kernel_us": round(sk["fastlinear_decode_layout_kernel_us"], 3),
                "GB/s": round(sk["fastlinear_decode_layout_kernel_gbs"], 1),
                "frac": round(sk["fastlinear_decode_layout_kernel_gbs"] / HBM_PEAK_GBS, 4),
            },
            "bytes_per_launch": sk["bytes_per_launch"],
            "ksplit": sk["ksplit"],
            "mm_t_call_us": round(sk["call_us"], 2),
            "cpu_baseline": cpu_sk,
        },
        "cpu_baseline": cpu,
    }
    report = args.report or ("bench_configs.json" if args.all else None)
    if report:
        Path(report).parent.mkdir(parents=True, exist_ok=True)
        Path(report).write_text(json.dumps({"c4": c4, "skinny_m1": sk, "cpu": cpu, "configs": configs}, indent=2))
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
