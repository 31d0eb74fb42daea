#!/usr/bin/env python3
"""Benchmark of the W4A8 quantized linear on one MI355X.

Workload: one W4A8 linear, rotate (Hadamard 256) + int8 per-token
quantize + uint4-asymmetric group-64 GEMM + scale/zero/bias epilogue to bf16, at M=4096, K=3072,
N=12288, on seeded synthetic DiT-shaped data with every input resident in HBM. A step is one
call of kitchen_amd.w4a8_int8_linear (two kernel launches on the current stream).

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--settle-ms 200]

Before the W warmup steps the step runs untimed for settle_ms of wall time (and each kernel timed
alone for half of that before its own measurement): the GPU clock ramps for tens of milliseconds
after idle or after different work, and the figures are for the loaded steady state.

Prints one JSON line: whole-linear int8 TOPS (2*M*N*K / step time), the GEMM kernel's roofline
(average launch duration from HIP events on the launch stream, against the 5.0 POPS dense int8
MFMA peak; HBM traffic per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE counters, calibrated
on a device-to-device copy of known size), the rotate+quantize kernel's HBM roofline at the
video-token shape (M=32760), and the reference's CPU torch path timed on a bounded sample of the
same workload.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import platform
import shutil
import subprocess
import sys
import tempfile

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "comfy-quant-bench_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "int8-MFMA TOPS & % peak for W4A8/W4A4 linear (rot+quant+GEMM), M=4096"
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA, 5.0 POPS
HBM_PEAK_GBPS = 8000.0       # MI355X HBM3E, 8 TB/s
# Measured on MI355X by a standalone gfx950 probe: v_mfma_i32_16x16x64_i8 on random int8 register
# operands, 8 waves per SIMD, each MFMA followed by the four fp32 fmas of a per-group scale step, no
# memory traffic (2109 TOPS; 4042 without the fmas). Reported beside the spec peak, not instead of it.
GROUP_SCALE_CEILING_TOPS = 2109.0
RQ_M = 32760                 # video-token shape of the rotate+quantize roofline (302 MB, above the MALL)
COPY_BYTES = 256 << 20       # calibration copy for the traffic counters
GEMM_KERNEL = "gemm_wide_kernel"
RQ_KERNEL = "rotquant_kernel"
GEMV_KERNEL = "gemv_kernel<(mq::WKind)0"
GEMV_I8_KERNEL = "gemv_kernel<(mq::WKind)2"
GEMV_N = 18432               # config 1's adaLN linear at M = 1: K = 3072 -> N = 18432
GEMV_COPIES = 10             # weight copies cycled over the calls: 305 MB, above the 256 MB MALL
GEMV_I8_COPIES = 6           # int8 weight copies for the W8A8 GEMV: 340 MB, above the MALL
COPY_KERNEL = "copyBuffer"


def cpu_info() -> dict:
    """The host CPU as lscpu reports it (model name, sockets, cores per socket, threads per core,
    logical CPUs) plus /proc/cpuinfo's model name where lscpu's is shorter."""
    info: dict = {}
    keys = {"Model name": "model", "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
            "Thread(s) per core": "threads_per_core", "CPU(s)": "logical_cpus", "Vendor ID": "vendor"}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            if key.strip() in keys and keys[key.strip()] not in info:
                info[keys[key.strip()]] = val.strip()
    except OSError:
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    full = line.split(":", 1)[1].strip()
                    if len(full) > len(info.get("model", "")):
                        info["model"] = full
                    break
    except OSError:
        pass
    info.setdefault("model", platform.processor() or "unknown")
    try:
        info["physical_cores"] = int(info["sockets"]) * int(info["cores_per_socket"])
    except (KeyError, ValueError):
        pass
    return info


def settle(fn, ms: float) -> None:
    """Run fn untimed for `ms` milliseconds of wall time, so the GPU clock reaches its loaded
    steady state for this work (it ramps over tens of milliseconds after idle or after other work)."""
    import time

    import torch

    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def time_launches(fn, iters: int, rounds: int = 5, warm: int = 3, settle_ms: float = 0.0) -> float:
    """Median over `rounds` of the average milliseconds per call of fn (HIP events recorded on
    torch's current stream, which is the stream the library launches on), after `settle_ms` of
    untimed calls and `warm` more."""
    import torch

    settle(fn, settle_ms)
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    per = []
    for _ in range(rounds):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) / iters)
    per.sort()
    return per[len(per) // 2]


def make_inputs(m: int, k: int, n: int):
    import numpy as np
    import torch

    import kitchen_amd as ck
    from kitchen_amd import synth

    dev = torch.device("cuda:0")
    xb = synth.activations(m, k, seed=0)
    w = synth.weight(n, k, seed=1)
    rng = np.random.default_rng(2)
    bias_f = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(rng.standard_normal(n).astype(np.float32) * 0.1))
    qd, s16, zp = ck.quantize_w4a8_asym_weight(torch.from_numpy(w).to(dev), 64, 256)
    x = synth.to_bf16_tensor(xb, dev)
    bias = torch.from_numpy(bias_f).to(dev, torch.bfloat16)
    torch.cuda.synchronize()
    return xb, bias_f, x, qd, s16, zp, bias


def gemv_inputs(x, k: int):
    """The M = 1 GEMM's operands: the quantized first activation row and GEMV_COPIES random-code
    uint4-asymmetric g64 weight sets [GEMV_N, k] (packed codes, fp16 scales, packed zero-points)."""
    import torch

    import kitchen_amd as ck

    dev = x.device
    gen = torch.Generator(device=dev).manual_seed(5)
    qa, sa = ck.quantize_int8_rowwise_convrot(x[:1], 256)
    g = k // 64
    copies = [(torch.randint(0, 256, (GEMV_N, k // 2), generator=gen, device=dev, dtype=torch.uint8),
               (torch.rand(GEMV_N, g, generator=gen, device=dev) * 0.004 + 0.004).to(torch.float16),
               torch.randint(0, 256, (GEMV_N, (g + 1) // 2), generator=gen, device=dev, dtype=torch.uint8))
              for _ in range(GEMV_COPIES)]
    bias = torch.zeros(GEMV_N, dtype=torch.bfloat16, device=dev)
    return qa, sa, copies, bias


def gemv_bytes(k: int) -> int:
    """Algorithmic bytes of one M = 1 call: packed weights, fp16 scales, packed zero-points, the
    int8 activation row and its scale, bias and bf16 output."""
    g = k // 64
    return GEMV_N * k // 2 + GEMV_N * g * 2 + GEMV_N * ((g + 1) // 2) + k + 4 + 2 * GEMV_N + 2 * GEMV_N


def measure_gemv(x, settle_ms: float, launches: int = 40) -> dict:
    """The M = 1 W4A8 GEMM (the few-row GEMV kernel) at config 1's adaLN shape, HBM-bound on the
    packed weights. Consecutive calls read different weight copies (GEMV_COPIES of them, more than
    the MALL holds), so each call's weights come from HBM. `launches` calls are captured in one HIP
    graph and replayed, so the host's launch cost (longer than the kernel) stays out of the timing;
    the time per launch still includes the graph's gap between consecutive kernels."""
    import torch

    import kitchen_amd as ck

    k = x.shape[1]
    qa, sa, copies, bias = gemv_inputs(x, k)

    def calls():
        for i in range(launches):
            qd, s16, zp = copies[i % GEMV_COPIES]
            ck.gemm_w4_group(qa, sa, qd, s16, zp, bias, GEMV_N)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        calls()                                      # warm the allocator on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        calls()
    ms = time_launches(graph.replay, 5, settle_ms=settle_ms) / launches
    nbytes = gemv_bytes(k)
    gbps = nbytes / (ms * 1e-3) / 1e9
    del graph

    # the whole one-row linear on the same weights (bf16 row in; the GEMV rotates and quantizes it
    # in its own prologue, one launch), timed the same way
    xrow = x[:1]

    def linear_calls():
        for i in range(launches):
            qd, s16, zp = copies[i % GEMV_COPIES]
            ck.w4a8_int8_linear(xrow, qd, s16, None, None, zp, bias)

    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        linear_calls()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        linear_calls()
    ms_lin = time_launches(graph.replay, 5, settle_ms=settle_ms) / launches
    lin_bytes = nbytes - k - 4 + 2 * k                # the bf16 row in place of its codes and scale
    del graph, copies
    torch.cuda.empty_cache()
    return {"bound": "hbm", "kernel": "gemv_kernel<U4Asym,GroupScale,0,1>", "M": 1, "K": k, "N": GEMV_N,
            "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "bytes_per_launch": nbytes, "avg_launch_ms": round(ms, 5), "weight_copies": GEMV_COPIES,
            "timing": f"HIP graph of {launches} launches over {GEMV_COPIES} weight copies, per launch",
            "whole_linear": {"kernel": "gemv_kernel<U4Asym,GroupScale,0,1,FQ=1> (the row rotated and quantized "
                                       "in the GEMV's prologue)",
                             "avg_launch_ms": round(ms_lin, 5), "bytes_per_launch": lin_bytes,
                             "achieved": round(lin_bytes / (ms_lin * 1e-3) / 1e9, 1),
                             "frac": round(lin_bytes / (ms_lin * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}}


def gemv_i8_inputs(x, k: int):
    """The M = 1 W8A8 GEMM's operands (config 4's adaLN linear on W8A8): the quantized first
    activation row and GEMV_I8_COPIES random int8 weight sets [GEMV_N, k] in the 16-row tiles the
    stack holds them in, with fp32 per-row scales."""
    import torch

    import kitchen_amd as ck

    dev = x.device
    gen = torch.Generator(device=dev).manual_seed(7)
    qa, sa = ck.quantize_int8_rowwise_convrot(x[:1], 256)
    copies = [(ck.tile_int8_weight(torch.randint(-127, 128, (GEMV_N, k), generator=gen, device=dev, dtype=torch.int8)),
               torch.rand(GEMV_N, generator=gen, device=dev) * 2e-4 + 3e-4)
              for _ in range(GEMV_I8_COPIES)]
    bias = torch.zeros(GEMV_N, dtype=torch.bfloat16, device=dev)
    return qa, sa, copies, bias


def gemv_i8_bytes(k: int) -> int:
    """Algorithmic bytes of one M = 1 W8A8 call: int8 weights, fp32 row scales, the int8 activation
    row and its scale, bias and bf16 output."""
    return GEMV_N * k + 4 * GEMV_N + k + 4 + 2 * GEMV_N + 2 * GEMV_N


def measure_gemv_i8(x, settle_ms: float, launches: int = 36) -> dict:
    """The M = 1 W8A8 GEMM (the int8 row-scale GEMV) at the adaLN shape, timed as measure_gemv:
    weight copies cycled past the MALL, the calls replayed from one HIP graph."""
    import torch

    import kitchen_amd as ck

    k = x.shape[1]
    qa, sa, copies, bias = gemv_i8_inputs(x, k)

    def calls():
        for i in range(launches):
            q8, ws = copies[i % GEMV_I8_COPIES]
            ck.gemm_rowscale(qa, sa, q8, ws, bias, GEMV_N, 8)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        calls()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        calls()
    ms = time_launches(graph.replay, 5, settle_ms=settle_ms) / launches
    nbytes = gemv_i8_bytes(k)
    gbps = nbytes / (ms * 1e-3) / 1e9
    del graph, copies
    torch.cuda.empty_cache()
    return {"bound": "hbm", "kernel": "gemv_kernel<I8,RowScale,0,1> (weights in 16-row tiles)", "M": 1, "K": k,
            "N": GEMV_N, "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "bytes_per_launch": nbytes, "avg_launch_ms": round(ms, 5),
            "weight_copies": GEMV_I8_COPIES,
            "timing": f"HIP graph of {launches} launches over {GEMV_I8_COPIES} weight copies, per launch"}


def _aux(fn) -> dict:
    """An auxiliary measurement of the bench line: its result, or {"error": ...} if it raised, so
    that the headline figures are still printed (the error names what to look at)."""
    try:
        return fn()
    except Exception as e:  # noqa: BLE001 - reported in the JSON line instead of ending the run
        return {"error": f"{type(e).__name__}: {e}"[:300]}


def kernels_child(args) -> int:
    """Launch each measured kernel a few times and exit (run under rocprofv3 by measure_traffic)."""
    import torch

    import kitchen_amd as ck
    from kitchen_amd import synth

    m, k, n = args.m, args.k, args.n
    _, _, x, qd, s16, zp, bias = make_inputs(m, k, n)
    qa, sa = ck.quantize_int8_rowwise_convrot(x, 256)
    xw = ck.expand_w4_weight(qd.view(torch.uint8), zp.view(torch.uint8), 0, s16)   # the linear's GEMM operand
    for _ in range(3):
        ck.gemm_w4_group(qa, sa, xw, s16, None, bias, n)
    if args.with_rowscale:
        # the W8A8 linear of the same shape (random int8 weights in 16-row tiles, per-row scales),
        # for profiles and counter runs that compare the two epilogues: its GEMM reads activation
        # codes and weights in 16-row tiles, as in the config-4 stack; the traffic runs leave it out
        gen = torch.Generator(device=x.device).manual_seed(6)
        q8 = ck.tile_int8_weight(torch.randint(-127, 128, (n, k), generator=gen, device=x.device, dtype=torch.int8))
        ws = torch.rand(n, generator=gen, device=x.device) * 1e-3
        for _ in range(args.rowscale_calls):
            ck.int8_linear(x, q8, ws, bias, torch.bfloat16, True, 256)
        del q8
    x3 = synth.to_bf16_tensor(synth.activations(RQ_M, k, seed=3), x.device)
    for _ in range(3):
        ck.quantize_int8_rowwise_convrot(x3, 256)
    del x3
    gqa, gsa, copies, gbias = gemv_inputs(x, k)
    for qdc, s16c, zpc in copies[:3]:
        ck.gemm_w4_group(gqa, gsa, qdc, s16c, zpc, gbias, GEMV_N)
    del copies
    gqa, gsa, copies, gbias = gemv_i8_inputs(x, k)
    for q8c, wsc in copies[:3]:
        ck.gemm_rowscale(gqa, gsa, q8c, wsc, gbias, GEMV_N, 8)
    del copies
    src = torch.empty(COPY_BYTES // 4, dtype=torch.int32, device=x.device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    return 0


def _counter_means(csv_path: str, counter: str) -> dict:
    """Per kernel, the counter's mean over the dispatches of the largest grid: the measured shape
    (the child also quantizes the M=4096 GEMM input, a smaller rotquant grid); for the copy kernel
    the maximum (the calibration copies are identical, other copies are smaller)."""
    sums: dict = {}
    for row in csv.DictReader(open(csv_path)):
        if row.get("Counter_Name") != counter:
            continue
        name = row["Kernel_Name"]
        for key in (GEMM_KERNEL, RQ_KERNEL, GEMV_KERNEL, GEMV_I8_KERNEL, COPY_KERNEL):
            if key in name:
                sums.setdefault(key, []).append((int(row.get("Grid_Size") or 0), float(row["Counter_Value"])))
    out = {}
    for key, v in sums.items():
        if key == COPY_KERNEL:
            out[key] = max(val for _, val in v)
        else:
            grid = max(g for g, _ in v)
            vals = [val for g, val in v if g == grid]
            out[key] = sum(vals) / len(vals)
    return out


def measure_traffic(args) -> dict:
    """HBM bytes per launch of the GEMM and rotate+quantize kernels from two rocprofv3 --pmc runs
    (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by bytes / counter of a
    device-to-device copy of COPY_BYTES in the same run."""
    prof = shutil.which("rocprofv3")
    if prof is None:
        return {"error": "rocprofv3 not found"}
    out: dict = {}
    with tempfile.TemporaryDirectory(prefix="mq_bench_pmc_") as tmp:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            d = os.path.join(tmp, counter)
            cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "pmc", "--",
                   sys.executable, os.path.abspath(__file__), "--kernels-child",
                   "--m", str(args.m), "--k", str(args.k), "--n", str(args.n)]
            try:
                res = subprocess.run(cmd, capture_output=True, text=True, timeout=180, env=dict(os.environ, TMPDIR=tmp))
            except subprocess.TimeoutExpired:
                return {"error": f"rocprofv3 {counter} run timed out"}
            files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
            if res.returncode != 0 and not files:
                return {"error": f"rocprofv3 {counter} run failed ({res.returncode})"}
            if not files:
                return {"error": f"no counter file for {counter}"}
            means = _counter_means(files[0], counter)
            if COPY_KERNEL not in means or GEMM_KERNEL not in means:
                return {"error": f"{counter}: kernels not found in the counter file"}
            out[counter] = means
    f_fetch = COPY_BYTES / (out["FETCH_SIZE"][COPY_KERNEL] * 1024.0)
    f_write = COPY_BYTES / (out["WRITE_SIZE"][COPY_KERNEL] * 1024.0)
    res = {"fetch_scale": round(f_fetch, 4), "write_scale": round(f_write, 4)}
    for key in (GEMM_KERNEL, RQ_KERNEL, GEMV_KERNEL, GEMV_I8_KERNEL):
        if key in out["FETCH_SIZE"] and key in out["WRITE_SIZE"]:
            fetch = out["FETCH_SIZE"][key] * 1024.0 * f_fetch
            write = out["WRITE_SIZE"][key] * 1024.0 * f_write
            res[key] = {"fetch_bytes": int(fetch), "write_bytes": int(write), "bytes": int(fetch + write)}
    return res


def measure_stack(steps: int = 3) -> dict:
    """ms per pass over the config-4 linear stack (every linear: rotate + quantize + GEMM +
    epilogue, inputs resident, random-init quantized weights): eager (one Python call per linear,
    as a loader runs it), replayed from one captured HIP graph (the 840 linears' kernels,
    workspaces and outputs from the graph's memory pool), and replayed from a graph of the
    dual-stream pass (synth.stack_pass with a side stream); 1 untimed pass each, then `steps`."""
    import torch

    from kitchen_amd import synth

    dev = torch.device("cuda:0")
    layers = synth.mmdit_linear_stack(blocks=60, device=dev)
    acts = synth.stack_activations(dev)

    def one_pass():
        for layer in layers:
            synth.stack_layer(layer, acts[(layer["M"], layer["K"])])

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    ms_eager = timed(one_pass)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        one_pass()                                   # warm the allocator on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        one_pass()
    ms_graph = timed(graph.replay)
    # the same pass with each block's text and image linears on two streams (joined at the
    # block's attention and end), captured in one graph
    graph2 = torch.cuda.CUDAGraph()
    side2 = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        synth.stack_pass(layers, acts, side=side2)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph2):
        synth.stack_pass(layers, acts, side=side2)
    ms_dual = timed(graph2.replay)
    ops = synth.stack_ops(layers)
    w4 = sum(l["fmt"] == "w4a4" for l in layers)
    out = {"workload": "config 4: 60 dual-stream MMDiT blocks x 14 linears (q k v out mlp_up mlp_down mod), "
                       "image M=4096, text M=256, mod M=1; seeded 35% W4A4 (H64, int4 acts, int4 g64 fp16 "
                       "weights), rest W8A8 (H256, int8 per-token acts, int8 per-row weights)",
           "ms_per_step": round(ms_graph, 3), "tops": round(ops / (ms_graph * 1e-3) / 1e12, 1),
           "ms_per_step_eager": round(ms_eager, 3), "timing": "HIP graph replay of one pass (eager alongside)",
           "ms_per_step_dual_stream": round(ms_dual, 3), "tops_dual_stream": round(ops / (ms_dual * 1e-3) / 1e12, 1),
           "dual_stream": "each block's text linears on a second stream, joined after q/k/v and at the block end",
           "ops_per_step": ops, "linears": len(layers), "w4a4_linears": w4, "steps": steps}
    del graph, graph2, layers, acts
    torch.cuda.empty_cache()
    return out


def graph_ms(fn, calls: int) -> float:
    """GPU time per call of fn without the host: `calls` calls captured in one HIP graph (their
    kernels, outputs and workspaces from the graph's pool) and replayed; median of 3 rounds of 5
    replays after 50 ms of untimed replays."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()                                         # warm the allocator on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    ms = time_launches(graph.replay, 5, rounds=3, settle_ms=50.0) / calls
    del graph
    return ms


def sweep() -> dict:
    """Every BASELINE configuration's linear shapes, timed end to end (rotate + quantize + GEMM +
    epilogue through the drop-in ops; median of 3 rounds of 10 calls after 50 ms of untimed calls,
    inputs resident; `gpu_ms` the same calls replayed from a HIP graph, i.e. without the host) on
    random-code quantized weights of each shape, plus the rotate+quantize kernel at config 3's
    two activation widths. Returns {"linears": [...], "rotquant": [...]}."""
    import torch

    import kitchen_amd as ck

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(7)

    def w4a8_weights(n, k):
        qd = torch.randint(0, 256, (n, k // 2), generator=gen, device=dev, dtype=torch.uint8)
        s16 = (torch.rand(n, k // 64, generator=gen, device=dev) * 0.004 + 0.004).to(torch.float16)
        zp = torch.randint(0, 256, (n, (k // 64 + 1) // 2), generator=gen, device=dev, dtype=torch.uint8)
        return qd, s16, zp

    def w4a4_weights(n, k):
        qw = torch.randint(-128, 128, (n, k // 2), generator=gen, device=dev, dtype=torch.int8)
        s16 = (torch.rand(n, k // 64, generator=gen, device=dev) * 0.004 + 0.004).to(torch.float16)
        return qw, s16

    shapes = [("C0", "w4a8", 1024, 3072, 3072, 256)]
    c1_kn = [(3072, 3072), (3072, 9216), (3072, 12288), (12288, 3072)]
    shapes += [("C1", "w4a8", m, k, n, 256) for m in (4352, 8192) for k, n in c1_kn]
    shapes += [("C1", "w4a8", 1, 3072, 18432, 256)]
    shapes += [("C2", "w4a4", m, k, n, hb) for hb in (16, 64, 256) for m in (4352, 8192) for k, n in c1_kn]
    shapes += [("C2", "w4a4", 1, 3072, 18432, hb) for hb in (16, 64, 256)]
    shapes += [("C3", "w4a8", 32760, k, n, 256) for k, n in ((3072, 9216), (3072, 14336), (14336, 3072))]
    # config 4's W8A8 linears (image and text tokens), int8 weights held in 16-row tiles
    shapes += [("C4", "w8a8", m, k, n, 256) for m in (4096, 256) for k, n in c1_kn]
    out = {"linears": [], "rotquant": []}
    acts: dict = {}
    for cfg, fmt, m, k, n, hb in shapes:
        if (m, k) not in acts:
            acts[(m, k)] = torch.randn(m, k, generator=gen, device=dev).to(torch.bfloat16)
        x = acts[(m, k)]
        bias = (torch.randn(n, generator=gen, device=dev) * 0.1).to(torch.bfloat16)
        if fmt == "w8a8":
            q8 = ck.tile_int8_weight(torch.randint(-127, 128, (n, k), generator=gen, device=dev, dtype=torch.int8))
            rs = torch.rand(n, generator=gen, device=dev) * 2e-4 + 3e-4
            fn = lambda: ck.int8_linear(x, q8, rs, bias, torch.bfloat16, True, hb)  # noqa: E731
        elif fmt == "w4a8":
            qd, s16, zp = w4a8_weights(n, k)
            fn = lambda: ck.w4a8_int8_linear(x, qd, s16, None, None, zp, bias, 64, hb, torch.bfloat16)  # noqa: E731
        else:
            qw, s16 = w4a4_weights(n, k)
            fn = lambda: ck.convrot_w4a4_linear(x, qw, s16, bias, convrot_groupsize=hb, quant_group_size=64,  # noqa: E731
                                                linear_dtype="int4")
        ms = time_launches(fn, 10, rounds=3, settle_ms=50.0)
        gpu_ms = graph_ms(fn, 10)
        tops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        out["linears"].append({"config": cfg, "format": fmt, "M": m, "K": k, "N": n, "hadamard_block": hb,
                               "ms": round(ms, 5), "tops": round(tops, 1), "frac": round(tops / INT8_PEAK_TOPS, 4),
                               "gpu_ms": round(gpu_ms, 5)})
        print(json.dumps(out["linears"][-1]), file=sys.stderr, flush=True)
        del fn
    acts.clear()
    for k in (3072, 14336):
        x = torch.randn(RQ_M, k, generator=gen, device=dev).to(torch.bfloat16)
        ms = time_launches(lambda: ck.quantize_int8_rowwise_convrot(x, 256), 10, rounds=3, settle_ms=50.0)
        nbytes = RQ_M * k * 3 + 4 * RQ_M
        out["rotquant"].append({"config": "C3", "M": RQ_M, "K": k, "ms": round(ms, 5),
                                "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)})
        print(json.dumps(out["rotquant"][-1]), file=sys.stderr, flush=True)
        del x
    torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--settle-ms", type=float, default=200.0,
                    help="untimed steps for this long before the warmup steps (clock steady state)")
    ap.add_argument("--m", type=int, default=4096)
    ap.add_argument("--k", type=int, default=3072)
    ap.add_argument("--n", type=int, default=12288)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 traffic counters")
    ap.add_argument("--no-stack", action="store_true", help="skip the config-4 linear stack")
    ap.add_argument("--sweep", action="store_true",
                    help="time every configuration's linear shapes instead (one JSON object, not the bench line)")
    ap.add_argument("--kernels-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--with-rowscale", action="store_true",
                    help="with --kernels-child: also run the W8A8 linear of the same shape (profiles, counter runs)")
    ap.add_argument("--rowscale-calls", type=int, default=3, help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the W4A8 linear would shard over tokens or output channels with no exchange between GPUs.",
              file=sys.stderr)
        return 2
    if args.kernels_child:
        return kernels_child(args)
    if args.sweep:
        print(json.dumps(sweep()))
        return 0

    import torch

    import kitchen_amd as ck
    from kitchen_amd import synth

    m, k, n = args.m, args.k, args.n
    xb, bias_f, x, qd, s16, zp, bias = make_inputs(m, k, n)

    def step():
        return ck.w4a8_int8_linear(x, qd, s16, None, None, zp, bias, 64, 256, torch.bfloat16)

    # ---- whole linear: untimed steps for settle_ms, W untimed warmup steps, then exactly K timed steps
    settle(step, args.settle_ms)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps
    ops = 2.0 * m * n * k
    tops = ops / (ms_step * 1e-3) / 1e12

    # ---- dominant kernel (GEMM) alone, same stream, inputs resident: on the int8 expansion of the
    # packed weights the linear made at its first call (the same bits as on the packed weights), and
    # for comparison on the packed weights themselves
    qa, sa = ck.quantize_int8_rowwise_convrot(x, 256)
    qdu, zpu = qd.view(torch.uint8), zp.view(torch.uint8)
    xw = ck.expand_w4_weight(qdu, zpu, 0, s16)
    ms_gemm = time_launches(lambda: ck.gemm_w4_group(qa, sa, xw, s16, None, bias, n), 20, settle_ms=args.settle_ms / 2)
    ms_gemm_packed = time_launches(lambda: ck.gemm_w4_group(qa, sa, qdu, s16, zpu, bias, n), 20,
                                   settle_ms=args.settle_ms / 4)
    gemm_tops = ops / (ms_gemm * 1e-3) / 1e12
    ms_rq_ns = time_launches(lambda: ck.quantize_int8_rowwise_convrot(x, 256), 20)

    # ---- rotate+quantize kernel at the HBM-bound video-token shape (C3: 32760 x 3072, 302 MB)
    x3 = synth.to_bf16_tensor(synth.activations(RQ_M, k, seed=3), x.device)
    ms_rq = time_launches(lambda: ck.quantize_int8_rowwise_convrot(x3, 256), 20, settle_ms=args.settle_ms / 2)
    rq_bytes = RQ_M * k * 2 + RQ_M * k + 4 * RQ_M
    rq_gbps = rq_bytes / (ms_rq * 1e-3) / 1e9
    del x3

    # ---- M = 1 GEMV (config 1's adaLN shape), weights cycled past the MALL
    gemv = _aux(lambda: measure_gemv(x, args.settle_ms / 2))
    gemv_i8 = _aux(lambda: measure_gemv_i8(x, args.settle_ms / 2))

    # ---- the mixed W4A4 / W8A8 MMDiT linear stack (60 blocks x 14 linears)
    stack = None if args.no_stack else _aux(measure_stack)

    traffic = None if args.no_traffic else measure_traffic(args)
    gemm_traffic = traffic.get(GEMM_KERNEL, {}).get("bytes") if traffic else None
    rq_traffic = traffic.get(RQ_KERNEL, {}).get("bytes") if traffic else None
    if "error" not in gemv:
        gemv["traffic"] = traffic.get(GEMV_KERNEL, {}).get("bytes") if traffic else None
    if "error" not in gemv_i8:
        gemv_i8["traffic"] = traffic.get(GEMV_I8_KERNEL, {}).get("bytes") if traffic else None

    result = {
        "metric": METRIC,
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: seeded N(0,1) bf16 activations with 1% x20 outlier channels, N(0,0.02) weights",
        "config": {"workload": "w4a8_linear (rotate H256 + int8 per-token quant + uint4-asym g64 GEMM + epilogue)",
                   "M": m, "K": k, "N": n, "hadamard_block": 256, "group": 64, "out": "bf16"},
        "roofline": {"bound": "mfma", "kernel": "gemm_wide_kernel<256,256,U4Asym,GroupScale,0,expanded>",
                     "achieved": round(gemm_tops, 2), "peak": INT8_PEAK_TOPS, "unit": "TOPS",
                     "frac": round(gemm_tops / INT8_PEAK_TOPS, 4), "traffic": gemm_traffic,
                     "ops_per_launch": ops, "avg_launch_ms": round(ms_gemm, 5),
                     "weights": "the uint4 codes and zero-points as stored, expanded once per weight to int8 "
                                "(q - z, negated in odd K groups) in 16-row tiles, which the GEMM reads; "
                                "the same bits as the packed weights' GEMM",
                     "packed_weights_avg_launch_ms": round(ms_gemm_packed, 5),
                     "measured_ceiling": {"tops": GROUP_SCALE_CEILING_TOPS,
                                          "frac": round(gemm_tops / GROUP_SCALE_CEILING_TOPS, 4),
                                          "what": "int8 MFMA + 4 fp32 group-scale fmas per MFMA, random int8 "
                                                  "operands, no memory traffic (gfx950 probe)"}},
        "rotquant_roofline": {"bound": "hbm", "kernel": "rotquant_kernel<256,int8,3>", "M": RQ_M, "K": k,
                              "achieved": round(rq_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                              "frac": round(rq_gbps / HBM_PEAK_GBPS, 4), "bytes_per_launch": rq_bytes,
                              "traffic": rq_traffic, "avg_launch_ms": round(ms_rq, 5),
                              "north_star_M_launch_ms": round(ms_rq_ns, 5)},
        "gemv_roofline": gemv,
        "gemv_i8_roofline": gemv_i8,
    }
    if stack is not None:
        result["c4_linear_stack"] = stack
    if traffic is not None:
        result["traffic_counters"] = {k2: v for k2, v in traffic.items() if k2 in ("fetch_scale", "write_scale", "error")}

    if not args.no_cpu_baseline:
        from oracle import quant
        from oracle.torch_path import W4A8CpuLinear, time_cpu

        ms = m   # the whole workload's rows: the sample is one full step, repeated for ~10 s
        q_codes = quant.unpack_u4(qd.cpu().numpy())
        z_codes = quant.unpack_u4(zp.cpu().numpy())[:, : k // 64]
        lin = W4A8CpuLinear(q_codes, s16.cpu().numpy(), z_codes, bias_f, 256, 64)
        xs = torch.from_numpy(synth.bf16_bits_to_f32(xb[:ms]))
        # every CPU this process may use, capped by the host's CPU share for this job
        # (OMP_NUM_THREADS, which torch's default thread count already follows)
        usable = len(os.sched_getaffinity(0))
        share = int(os.environ.get("OMP_NUM_THREADS", usable) or usable)
        threads = max(1, min(usable, share))
        torch.set_num_threads(threads)
        t, calls = time_cpu(lin, xs, runs=5, min_seconds=10.0)
        cpu = cpu_info()
        result["cpu_baseline"] = {
            "value": round(2.0 * ms * n * k / t / 1e12, 4), "unit": "TOPS", "cores": threads,
            "threads": threads, "kind": "port", "cpu": cpu.get("model"), "lscpu": cpu,
            "threads_rule": "threads = CPUs in this process's affinity mask, capped by OMP_NUM_THREADS "
                            "(the job's CPU share on the GPU host); cores = those threads",
            "sample": f"the whole step, M={ms} rows of the same linear (K={k}, N={n}): torch fp32 "
                      f"rotate-by-matmul, int8 per-token quant, dequantized-weight matmul, bias; median of "
                      f"{calls} calls (at least 5, and at least 10 s of timed work) after 1 warm-up",
            "seconds_per_sample": round(t, 4), "calls": calls}
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
