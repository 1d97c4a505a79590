"""Benchmark of the quantized-inference hot path on one MI355X.

Headline line (value): W8A8 prefill GEMM, M=2048 K=4096 N=14336, int8 x int8 ->
int32 -> fp32 per-channel/per-row dequant epilogue, inputs resident in HBM, in
TOPS (2*M*N*K int ops per step). The same JSON line carries the roofline of that
kernel (with the HBM traffic and MFMA-busy / clock counters of its committed
rocprofv3 passes), the CPU baseline (the oracle's AVX-512 VNNI igemm path over
the whole workload) and the other configurations as `components`, each with its
own CPU baseline where the reference has a CPU path: decode GEMV (GB/s, weight
buffers rotated past the 256 MB MALL, beside a same-bytes read-only floor timed
the same way), the 784-256-128-10 int8 MLP (end-to-end us), ternary GEMM (TOPS),
the RotorQuant K+V round trip (GB/s), attention over the RotorQuant KV cache,
the QuantizedLinear GEMV, igemm at the reference's published 512^3 shape, the f32
BlasBackend GEMM and the copy ceiling.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "rust-neural-network_amd"), os.path.join(ROOT, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "W8A8 GEMM TOPS (% int8 MFMA peak); GEMV & RotorQuant GB/s (% HBM peak)"
PEAK_INT8_TOPS = 5033.0   # MI355X dense int8 MFMA (datasheet, no sparsity)
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E
PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix
PEAK_BF16_MFMA_TFLOPS = 2500.0  # MI355X dense bf16 matrix
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
COUNTERS_FILE = os.path.join(ROOT, "profiles", "counters.json")
PROBE_LIB = os.path.join(ROOT, "rust-neural-network_amd", "librnn_probe.so")
# From idle the GPU needs ~10 ms of load to raise its clocks; every timed
# figure below is taken after this long of untimed launches of its own kernel.
SETTLE_S = 0.25


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def settle(fn, seconds=SETTLE_S):
    """Untimed launches of fn() for `seconds`, so the clocks have settled for
    this kernel before it is timed."""
    import torch
    t_end = time.time() + seconds
    while time.time() < t_end:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def timed(fn, steps, warmup):
    """Average ms per call of fn() over `steps` calls after `warmup` calls,
    measured with events on the current stream (the stream the C ABI launches
    on), bracketed by device synchronisation."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        fn()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def gen_f32(shape, seed, dev, scale=1.0):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
    return x * scale if scale != 1.0 else x


def _profile_entry(path, name):
    try:
        with open(path) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


def traffic_for(name):
    t = _profile_entry(TRAFFIC_FILE, name)
    return None if t is None else t.get("bytes_per_launch")


def counters_for(name):
    """MFMA-busy fraction and effective clock of a kernel from its committed
    rocprofv3 counter pass (profiles/counters.json), or None."""
    c = _profile_entry(COUNTERS_FILE, name)
    if c is None:
        return None
    return {k: c[k] for k in ("mfma_busy", "clock_ghz", "duration_us_under_counters",
                              "lds_bank_conflict_cycles", "source") if k in c}


# ---------------------------------------------------------------- CPU side
def cpu_threads():
    """Worker threads for the reference's rayon-parallel igemm: one per logical
    core this process may run on, capped by OMP_NUM_THREADS where the host sets
    it (the GPU box's CPU share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, n)


def cpu_info():
    model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = None
    return {"model": model, "nproc": os.cpu_count(), "affinity": aff,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def cpu_time(fn, max_repeats=5, budget_s=4.0):
    """Median wall time of fn() over up to `max_repeats` runs (at least one),
    stopping once `budget_s` seconds are spent."""
    times = []
    start = time.perf_counter()
    while len(times) < max_repeats and (not times or time.perf_counter() - start < budget_s):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_w8a8(O, aq, sa, wq, sw, threads, bias=None, relu=False):
    """The reference CPU path of one W8A8 layer: igemm (src/int8.rs:285-314:
    AVX-512 VNNI when the host has it, B repacked on every call, 4-row blocks
    over threads) on a_u8 = a_s8 + 128 and B = W^T, then the zero-point
    correction and the per-row/per-channel dequant epilogue."""
    import numpy as np
    m, k = aq.shape
    n = wq.shape[0]
    b_kn = np.ascontiguousarray(wq.T)
    colsum128 = 128 * b_kn.astype(np.int64).sum(axis=0).astype(np.int32)

    def run():
        a_u8 = aq.view(np.uint8) ^ np.uint8(0x80)
        c, vnni = O.igemm(a_u8, b_kn, m, k, n, threads)
        acc = (c - colsum128).astype(np.int32)
        y = (acc.astype(np.float32) * sa[:, None]) * sw[None, :]
        if bias is not None:
            y = y + bias[None, :]
        if relu:
            y = np.maximum(y, np.float32(0.0))
        return y, vnni
    return run


# ---------------------------------------------------------------- prefill
def bench_prefill(H, W, dev, steps, warmup):
    import torch
    c = W.PREFILL
    m, k, n = c["m"], c["k"], c["n"]
    w = gen_f32((n, k), 1, dev, 0.02)
    wq, sw = H.quant_rows_i8(w)
    del w
    x = gen_f32((m, k), 2, dev)
    aq, sa = H.quant_rows_i8(x)
    y = torch.empty((m, n), dtype=torch.float32, device=dev)
    fn = lambda: H.w8a8_linear(aq, sa, wq, sw, y=y)  # noqa: E731
    settle(fn)
    ms = timed(fn, steps, warmup)
    ops = 2.0 * m * n * k
    tops = ops / (ms * 1e-3) / 1e12
    # The whole W8A8 layer as a caller runs it: the fp32 activations quantized
    # per row (rnn_quant_rows_i8) and then the GEMM with its epilogue.
    layer = lambda: H.w8a8_linear(*H.quant_rows_i8(x, aq, sa), wq, sw, y=y)  # noqa: E731
    settle(layer, 0.1)
    ms_layer = timed(layer, steps, warmup)
    quant = lambda: H.quant_rows_i8(x, aq, sa)  # noqa: E731
    ms_quant = graph_timed(lambda i: quant(), 50)
    state = dict(aq=aq, sa=sa, wq=wq, sw=sw, m=m, k=k, n=n,
                 layer={"us": round(ms_layer * 1e3, 2), "quant_us": round(ms_quant * 1e3, 2),
                        "TOPS": round(ops / (ms_layer * 1e-3) / 1e12, 1)})
    return ms, tops, state


def prefill_ksweep(H, W, dev, steps, warmup, ks=(1024, 2048, 3072, 4096)):
    """The prefill GEMM at the same M and N for several K, and the least-squares
    line T(K) = fixed + slope * K through them: `fixed_us` is what a launch
    costs whatever its K (launch ramp, prologue, the fp32 epilogue of M x N
    outputs, the tail), `loop_us` = slope * K the K loop of the configured K.
    Each K is settled and timed as the headline launch. The shorter launches
    draw less power, so their clock can be higher: the split is a model, its
    residuals are reported with it."""
    import torch
    c = W.PREFILL
    m, n = c["m"], c["n"]
    us = []
    for k in ks:
        wq, sw = H.quant_rows_i8(gen_f32((n, k), 1, dev, 0.02))
        aq, sa = H.quant_rows_i8(gen_f32((m, k), 2, dev))
        y = torch.empty((m, n), dtype=torch.float32, device=dev)
        fn = lambda: H.w8a8_linear(aq, sa, wq, sw, y=y)  # noqa: E731
        settle(fn)
        us.append(timed(fn, steps, warmup) * 1e3)
        del wq, sw, aq, sa, y
        torch.cuda.empty_cache()
    mk, mu = sum(ks) / len(ks), sum(us) / len(us)
    slope = (sum((k - mk) * (u - mu) for k, u in zip(ks, us)) /
             sum((k - mk) ** 2 for k in ks))
    fixed = mu - slope * mk
    return {"k": list(ks), "us": [round(u, 2) for u in us], "fixed_us": round(fixed, 2),
            "loop_us": round(slope * c["k"], 2),
            "residual_us": [round(u - fixed - slope * k, 2) for k, u in zip(ks, us)],
            "note": f"T(K) = fixed + slope*K at M={m}, N={n}; loop_us = slope*{c['k']}"}


def cpu_baseline(state, budget_s=20.0):
    """The reference CPU path for the whole prefill workload (all 2048 rows),
    see cpu_w8a8."""
    import numpy as np

    import oracle as O
    m, k, n = state["m"], state["k"], state["n"]
    aq, sa = state["aq"].cpu().numpy(), state["sa"].cpu().numpy()
    wq, sw = state["wq"].cpu().numpy(), state["sw"].cpu().numpy()
    threads = cpu_threads()
    run = cpu_w8a8(O, aq, sa, wq, sw, threads)
    y, vnni = run()
    t, reps = cpu_time(run, 5, budget_s)
    ops = 2.0 * m * n * k
    return {"value": round(ops / t / 1e12, 4), "unit": "TOPS", "cores": threads,
            "kind": "port",
            "sample": f"the full W8A8 prefill workload {m}x{k}x{n} (no subsampling): oracle igemm "
                      f"({'AVX-512 VNNI' if vnni else 'scalar'}, B repacked per call as "
                      f"src/int8.rs:296 does, 4-row blocks over {threads} threads) + zero-point + "
                      f"dequant epilogue, median of {reps} runs, {t:.3f} s per run",
            "cpu": cpu_info(), "y_checksum": float(np.float64(y).sum())}


# ---------------------------------------------------------------- graph timing
def graph_timed(launch, n_launch, replays=5, settle_s=0.1):
    """ms per launch of `launch(i)` for i in range(n_launch), captured once
    into a HIP graph and replayed (events on the replay stream), so the
    per-call host overhead of the Python binding is not part of the figure.
    Untimed replays for `settle_s` seconds come first, so the clocks have
    settled for this kernel before the timed replays. Each replay is timed on
    its own and the median replay is reported, so that one slow replay (a
    replay of a short kernel lasts about a millisecond) does not move the
    figure."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(min(n_launch, 8)):      # warm up outside the capture
            launch(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n_launch):
            launch(i)
    g.replay()
    torch.cuda.synchronize()
    t_end = time.time() + settle_s
    while time.time() < t_end:
        g.replay()
        torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]
    ev[0].record(st)
    for r in range(replays):
        g.replay()
        ev[r + 1].record(st)
    torch.cuda.synchronize()
    del g
    per = [ev[r].elapsed_time(ev[r + 1]) for r in range(replays)]
    return statistics.median(per) / n_launch


class ReadFloor:
    """The same-bytes read-only floor: librnn_probe.so's streaming read of a
    buffer (16-byte non-temporal loads, 4 to 32 in flight per lane; the fastest
    of those four variants is the floor), launched and timed exactly as the
    kernel it is set beside."""

    def __init__(self, dev):
        import torch
        self.lib = ctypes.CDLL(PROBE_LIB)
        self.lib.rnn_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint32,
                                            ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        self.sink = torch.zeros(1, dtype=torch.int32, device=dev)

    def read(self, t, nbytes, per_lane):
        import torch
        nbytes = nbytes // 16 * 16
        rc = self.lib.rnn_probe_read(ctypes.c_void_p(t.data_ptr()), nbytes, 0x9E3779B9,
                                     ctypes.c_void_p(self.sink.data_ptr()), per_lane,
                                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError("rnn_probe_read failed")


def _floor(floor, bufs, nbytes, n_launch):
    if floor is None:
        return None
    copies = len(bufs)
    return min(graph_timed(lambda i: floor.read(bufs[i % copies], nbytes, per), n_launch,
                           replays=3, settle_s=0.03)
               for per in (4, 8, 16, 32))


# ---------------------------------------------------------------- GEMV
def bench_gemv(H, W, dev, steps, floor, with_cpu):
    import numpy as np
    import torch

    import oracle as O
    out = {}
    threads = cpu_threads()
    for (m, k, n) in W.GEMV_SHAPES:
        wbytes = k * n
        copies = max(2, -(-640 * 2**20 // wbytes))  # > 2.5x the 256 MB MALL
        ws, sws = [], []
        for i in range(copies):
            wq, sw = H.quant_rows_i8(gen_f32((n, k), 100 + i, dev, 0.02))
            ws.append(wq)
            sws.append(sw)
        x = gen_f32((m, k), 7, dev)
        mask = torch.rand((m, k), generator=torch.Generator(device=dev).manual_seed(8),
                          device=dev) < 0.01
        x = torch.where(mask, x * 20.0, x)
        aq, sa = H.quant_rows_i8(x)
        y = torch.empty((m, n), dtype=torch.float32, device=dev)
        n_launch = copies * max(1, -(-max(steps, 100) // copies))
        ms = graph_timed(lambda i: H.w8a8_linear(aq, sa, ws[i % copies], sws[i % copies], y=y),
                         n_launch)
        nbytes = k * n + 4 * n + m * k + 4 * m + 4 * m * n
        gbs = nbytes / (ms * 1e-3) / 1e9
        ent = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
               "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": nbytes,
               "weight_copies": copies, "launches_timed": 5 * n_launch,
               "timing": "HIP graph replay: events around each replay, median replay / launches per replay"}
        fl = _floor(floor, ws, k * n, n_launch)
        if fl is not None:
            ent["read_floor_us"] = round(fl * 1e3, 3)
            ent["frac_of_read_floor"] = round(fl / ms, 4)
        if with_cpu:
            run = cpu_w8a8(O, aq.cpu().numpy(), sa.cpu().numpy(), ws[0].cpu().numpy(),
                           sws[0].cpu().numpy(), threads)
            t, reps = cpu_time(run, 3, 2.0)
            ent["cpu_baseline"] = {
                "us": round(t * 1e6, 1), "GB/s": round(nbytes / t / 1e9, 2),
                "cores": min(threads, -(-m // 4)), "kind": "port",
                "sample": f"oracle igemm (src/int8.rs:285-314, B repacked per call, {-(-m // 4)} "
                          f"4-row block(s) over {threads} threads) + epilogue, full shape, median "
                          f"of {reps}"}
        out[f"m{m}_k{k}_n{n}"] = ent
        del ws, sws
        torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------- QuantizedLinear GEMV
QT_SHAPES = [(1, 4096, 11008), (4, 4096, 11008), (8, 4096, 11008), (16, 4096, 11008),
             (1, 4096, 4096)]
QT_FORMATS = [("INT4_g128", 3, 128), ("GGUF_Q4_0", 6, 32), ("GGUF_Q8_0", 8, 32), ("BF16", 1, 0),
              ("NF4_g64", 4, 64)]


def qt_bf16_path(fmt, m, k, n, g, cus):
    """Whether AUTO takes the bf16 MFMA GEMV (the conditions of
    rnn_qt_linear_forward for INT4 / GGUF Q4 / INT8 / GGUF Q8_0 / BF16 --
    groups of whole 4-piece chunks, whole rows or 32 elements: m >= 5, or
    4- and 8-bit codes at m = 3, 4 with at least two 16-row tiles of W per
    CU)."""
    kinds = {3: 32, 6: 32, 7: 32, 2: 16, 8: 16, 1: 8}   # format -> elements per 16 bytes
    if fmt not in kinds or m < 3:
        return False
    ep = kinds[fmt]
    fits = k % (32 * ep) == 0 and (fmt == 1 or (g % (4 * ep) == 0 and k % g == 0) or g % k == 0
                                   or g == 32)
    if not fits:
        return False
    if m >= 5:
        return True
    if ep == 8:
        return False
    r = max(min(-(-n // 16), cus), -(-n // 64))     # ranges of the m <= 8 plan (S = 1)
    return -(-(-(-n // r)) // 16) >= 2


def bench_qt_gemv(H, dev, steps, floor):
    """QuantizedLinear::forward (src/quantize.rs:744-754) at decode shapes:
    the fused GEMV that decodes INT4/GGUF/BF16/NF4 weights in registers (the
    VALU GEMV for small m, the bf16- or f32-MFMA GEMV for more rows, as AUTO
    picks). Bytes per
    launch = weight codes + f32 scales + x (4 m k) + y (4 m n); weights
    rotate over copies past the MALL as for the W8A8 GEMV. For the MFMA GEMVs
    the MFMA rate they run at (flops with rows padded to 16; three bf16
    products per MAC for the bf16 kernel) is given beside the HBM fraction."""
    import torch
    out = {}
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    for name, fmt, gs in QT_FORMATS:
        for (m, k, n) in QT_SHAPES:
            if (name in ("BF16", "NF4_g64") and (m, n) != (1, 11008)) or \
                    (name == "GGUF_Q4_0" and m in (8, 16)):
                continue
            nb, ns, g = H.qt_layout(fmt, n * k, gs)
            wbytes = nb + 4 * ns
            copies = max(2, -(-640 * 2**20 // wbytes))
            ds, ss = [], []
            for i in range(copies):
                d, s_, _ = H.qt_quantize(fmt, gen_f32((n, k), 300 + i, dev, 0.02), gs)
                ds.append(d)
                ss.append(s_ if s_.numel() else torch.zeros(1, device=dev))
            x = gen_f32((m, k), 9, dev)
            y = torch.empty((m, n), dtype=torch.float32, device=dev)
            n_launch = copies * max(1, -(-max(steps, 100) // copies))
            ws = torch.zeros(H.qt_linear_workspace_size(k, n), dtype=torch.uint8, device=dev)
            ms = graph_timed(lambda i: H.qt_linear_forward(fmt, x, ds[i % copies], ss[i % copies],
                                                           g, n, y=y, workspace=ws), n_launch)
            nbytes = wbytes + 4 * m * k + 4 * m * n
            gbs = nbytes / (ms * 1e-3) / 1e9
            ent = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                   "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": nbytes,
                   "weight_copies": copies, "launches_timed": 5 * n_launch,
                   "timing": "HIP graph replay: events around each replay, median replay / launches per replay"}
            if qt_bf16_path(fmt, m, k, n, g, cus):
                # three bf16 MFMAs per product (x split in three parts)
                tf = 3 * 2.0 * 16 * k * n / (ms * 1e-3) / 1e12
                ent["kernel"] = "bf16 MFMA GEMV (split x, caller workspace)"
                ent["TFLOP/s_bf16_mfma"] = round(tf, 2)
                ent["frac_bf16_mfma_peak"] = round(tf / PEAK_BF16_MFMA_TFLOPS, 4)
            elif m >= 5:
                tf = 2.0 * 16 * k * n / (ms * 1e-3) / 1e12
                ent["kernel"] = "f32 MFMA GEMV"
                ent["TFLOP/s_f32_mfma"] = round(tf, 2)
                ent["frac_fp32_mfma_peak"] = round(tf / PEAK_FP32_MFMA_TFLOPS, 4)
            fl = _floor(floor, ds, nb, n_launch)
            if fl is not None:
                ent["read_floor_us"] = round(fl * 1e3, 3)
                ent["frac_of_read_floor"] = round(fl / ms, 4)
            out[f"{name}_m{m}_k{k}_n{n}"] = ent
            del ds, ss
            torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------- MLP
def bench_mlp(H, W, dev, steps, with_cpu):
    """the 784-256-128-10 int8 MLP, batch 32, W8A8 per layer
    (activations quantized per row, int32 accumulate, fp32 dequant + bias, ReLU
    fused between layers): six launches end to end. Timed by HIP-graph replay
    of the whole forward (device latency) and as plain calls from Python (with
    the binding's per-call host cost)."""
    import numpy as np
    import torch

    import layers as L
    import oracle as O
    params = []
    for i, (fi, fo) in enumerate(zip(W.MLP_LAYERS[:-1], W.MLP_LAYERS[1:])):
        params += [W.weights(fo, fi, seed=10 + i), W.weights(1, fo, seed=20 + i)[0]]
    model = L.Int8Model.from_model([torch.from_numpy(p).to(dev) for p in params])
    x_np = W.activations(W.MLP_BATCH, W.MLP_LAYERS[0], seed=1)
    x = torch.from_numpy(x_np).to(dev)
    ms_graph = graph_timed(lambda i: model.forward(x), max(steps, 100))
    settle(lambda: model.forward(x), 0.05)
    ms_eager = timed(lambda: model.forward(x), max(steps, 100), 20)
    ms_layers = graph_timed(lambda i: model.forward_per_layer(x), max(steps, 100))
    y = model.forward(x).cpu().numpy()
    same = bool(np.array_equal(y, model.forward_per_layer(x).cpu().numpy()))
    ops = 2.0 * W.MLP_BATCH * sum(a * b for a, b in zip(W.MLP_LAYERS[:-1], W.MLP_LAYERS[1:]))
    ent = {"us_graph": round(ms_graph * 1e3, 2), "us_eager": round(ms_eager * 1e3, 2),
           "us_graph_per_layer_launches": round(ms_layers * 1e3, 2),
           "per_layer_bit_identical": same,
           "ops": ops, "launches": 1, "batch": W.MLP_BATCH, "layers": list(W.MLP_LAYERS),
           "weight_bytes": sum(a * b + 4 * b + 4 * b for a, b in zip(W.MLP_LAYERS[:-1], W.MLP_LAYERS[1:])),
           "traffic": traffic_for("int8_mlp_784_256_128_10"),
           "kernel": "w8a8_mlp_kernel (rnn_w8a8_mlp: the whole chain in one launch, "
                     "activations in LDS between layers)",
           "timing": "us_graph: HIP graph replay of the whole forward; us_eager: Python calls, "
                     "events over back-to-back forwards; us_graph_per_layer_launches: the same "
                     "chain as 6 launches (quantize + GEMM per layer)"}
    if with_cpu:
        threads = cpu_threads()
        qw = [O.quant_rows_i8(params[2 * i]) for i in range(3)]

        def run():
            h = x_np
            for i in range(3):
                aq, sa = O.quant_rows_i8(h)
                h, _ = cpu_w8a8(O, aq, sa, qw[i][0], qw[i][1], threads, params[2 * i + 1],
                                i < 2)()
            return h
        h = run()
        ent["max_abs_diff_vs_cpu"] = float(np.abs(h - y).max())
        t, reps = cpu_time(run, 20, 1.0)
        ent["cpu_baseline"] = {"us": round(t * 1e6, 1), "cores": threads, "kind": "port",
                               "sample": f"the whole forward on the oracle: per layer per-row "
                                         f"quantization + igemm (src/int8.rs:285-314) + "
                                         f"epilogue, median of {reps}"}
    return ent


# ---------------------------------------------------------------- ternary
def bench_ternary(H, W, dev, steps, with_cpu):
    import numpy as np
    import torch

    import oracle as O
    c = W.TERNARY
    m, k, n = c["m"], c["k"], c["n"]
    packed, scales = H.ternary_quantize(gen_f32((n, k), 3, dev), H.TERNARY_ABSMEAN)
    aq, sa = H.quant_rows_i8(gen_f32((m, k), 4, dev))
    y = torch.empty((m, n), dtype=torch.float32, device=dev)
    # a launch (~13 us) is shorter than the Python binding's per-call host
    # cost, so launches are replayed from a HIP graph as for the GEMV
    # the codes in the GEMM's own 2-bit layout (a one-time weight preparation)
    packed_mfma = H.ternary_prepack(packed, n, k)
    n_launch = max(steps, 100)
    ms = graph_timed(lambda i: H.ternary_gemm(aq, sa, packed_mfma, scales, n, y=y,
                                              mfma_layout=True), n_launch)
    ms_ref_layout = graph_timed(lambda i: H.ternary_gemm(aq, sa, packed, scales, n, y=y), n_launch)
    ops = 2.0 * m * n * k
    tops = ops / (ms * 1e-3) / 1e12
    nbytes = n * k // 4 + 4 * n + m * k + 4 * m + 4 * m * n
    ent = {"us": round(ms * 1e3, 3), "TOPS": round(tops, 1),
           "frac_int8_peak": round(tops / PEAK_INT8_TOPS, 4), "ops": ops, "bytes": nbytes,
           "launches_timed": 5 * n_launch, "timing": "HIP graph replay: events around each replay, median replay / launches per replay",
           "weights": "2-bit codes in the MFMA layout of rnn_ternary_prepack (decoded by byte "
                      "permutes); us_reference_layout: the same GEMM on TernaryTensor::packed "
                      "as the reference lays it out (decoded through an LDS table)",
           "us_reference_layout": round(ms_ref_layout * 1e3, 3),
           "traffic": traffic_for("ternary_gemm"), "counters": counters_for("ternary_gemm")}
    if with_cpu:
        rows = 8
        x = gen_f32((rows, k), 5, dev).cpu().numpy()
        p_np = packed.cpu().numpy().view(np.uint32)
        s_np = scales.cpu().numpy()
        t, reps = cpu_time(lambda: O.ternary_linear_f32(x, p_np, s_np, n), 3, 4.0)
        full = t * m / rows
        ent["cpu_baseline"] = {
            "us": round(full * 1e6, 1), "TOPS": round(ops / full / 1e12, 5), "cores": 1,
            "kind": "port",
            "sample": f"TernaryLinear::forward (src/ternary.rs:239-279, serial f32 shift-and-add as "
                      f"the reference runs it) on {rows} of the {m} rows, scaled x{m // rows}; "
                      f"{t:.3f} s per sample, median of {reps}"}
    return ent


# ---------------------------------------------------------------- RotorQuant
def bench_rotorquant(H, W, dev, steps, with_cpu):
    """RotorQuant K+V [8,32,4096,128] f32, 4-bit, fused quantize + dequantize:
    one launch per tensor, timed by HIP-graph replay after the same clock
    settle as the other HBM-bound components. Bytes = one f32 read + one f32
    write per element."""
    import torch

    import oracle as O
    c = W.ROTORQUANT
    shape = (c["batch"], c["heads"], c["seq"], c["head_dim"])
    dim, bits = c["head_dim"], c["bits"]
    ng = (dim + 2) // 3
    kv, outs, rots = [], [], []
    for which, seed in (("K", 11), ("V", 12)):
        x = gen_f32(shape, seed, dev)
        ch = torch.as_tensor(W.kv_outlier_channels(dim, seed), device=dev)
        x[..., ch] *= 10.0
        kv.append(x)
        outs.append(torch.empty_like(x))
        rots.append(torch.from_numpy(W.rotors(ng, seed)).to(dev))
    n_launch = 2 * max(10, steps // 2)
    ms = graph_timed(lambda i: H.rotorquant_quantize(kv[i % 2], rots[i % 2], bits, y=outs[i % 2]),
                     n_launch, replays=3, settle_s=0.2)
    nbytes = sum(2 * x.numel() * 4 for x in kv)
    us_step = 2 * ms * 1e3
    gbs = nbytes / (us_step * 1e-6) / 1e9
    ent = {"us_per_step": round(us_step, 2), "GB/s": round(gbs, 1),
           "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes_per_step": nbytes,
           "launches_per_step": 2, "launches_timed": 3 * n_launch,
           "timing": "HIP graph replay after a 0.2 s settle, events / launches",
           "traffic": traffic_for("rotorquant_kv")}
    if with_cpu:
        rows = 16384
        xs = [kv[i].reshape(-1, dim)[:rows].cpu().numpy() for i in range(2)]
        rs = [r.cpu().numpy() for r in rots]
        t, reps = cpu_time(lambda: [O.rotorquant_quantize(xs[i], rs[i], bits) for i in range(2)],
                           3, 3.0)
        total_rows = 2 * kv[0].numel() // dim
        full = t * total_rows / (2 * rows)
        ent["cpu_baseline"] = {
            "us_per_step": round(full * 1e6, 1), "GB/s": round(nbytes / full / 1e9, 3), "cores": 1,
            "kind": "port",
            "sample": f"RotorQuant::quantize (src/quant.rs:212-239, serial as the reference runs "
                      f"it) on {rows} rows of K and of V, scaled x{total_rows // (2 * rows)}; "
                      f"{t:.3f} s per sample, median of {reps}"}
    return ent


def bench_rq_attention(H, W, dev, steps):
    """Decode attention over the RotorQuant KV cache (the RotorQuant config's
    K and V, [8, 32, 4096, 128], 4-bit, as pages): one query per (batch,
    head). Algorithmic bytes per position = 6 per group (a 4-bit code triple in
    a u16 and an f32 scale) for K and for V; the K page pads codes to 8 groups
    and scales to 4, so the bytes it reads are given beside. Timed by graph
    replay, and again at batch 1 (the sequence split). Beside it, torch's f32
    scaled_dot_product_attention over the reconstructed K and V (what a cache
    without the codes would read), timed by events around back-to-back calls
    (each takes far longer than its host call), for context."""
    import torch
    c = W.ROTORQUANT
    b, h, seq, dim, bits = c["batch"], c["heads"], c["seq"], c["head_dim"], c["bits"]
    bh, ng = b * h, (dim + 2) // 3
    pages, rots, recon = [], [], []
    for seed, kind in ((11, H.RQ_PAGE_K), (12, H.RQ_PAGE_V)):
        x = gen_f32((bh * seq, dim), seed, dev)
        ch = torch.as_tensor(W.kv_outlier_channels(dim, seed), device=dev)
        x[:, ch] *= 10.0
        r = torch.from_numpy(W.rotors(ng, seed)).to(dev)
        _, codes, scales = H.rotorquant_quantize(x, r, bits, want_y=False, want_codes=True)
        pages.append(H.rotorquant_kv_pack(codes, scales, bh, seq, dim, bits, kind))
        recon.append(H.rotorquant_dequantize(codes, scales, dim, r).view(b, h, seq, dim))
        rots.append(r)
        del x, codes, scales
    q = gen_f32((bh, 1, dim), 13, dev)
    out = torch.empty_like(q)
    scale = 1.0 / dim ** 0.5
    ws = torch.zeros(max(1, H.rotorquant_kv_attention_workspace_size(bh, 1, seq, dim)),
                     dtype=torch.uint8, device=dev)
    ms = graph_timed(lambda i: H.rotorquant_kv_attention(q, pages[0], pages[1], rots[0], rots[1],
                                                         seq, scale, out=out, workspace=ws), 20)
    # batch 1 (the first h sequences of the same pages): too few queries to
    # fill the device, so each sequence is split over several workgroups
    b1 = h
    nc1, ns1 = H.rotorquant_kv_page_elems(b1, seq, dim)
    p1 = [(pg[0][:nc1], pg[1][:ns1]) for pg in pages]
    q1, out1 = q[:b1], out[:b1]
    ws1 = torch.zeros(max(1, H.rotorquant_kv_attention_workspace_size(b1, 1, seq, dim)),
                      dtype=torch.uint8, device=dev)
    ms1 = graph_timed(lambda i: H.rotorquant_kv_attention(q1, p1[0], p1[1], rots[0], rots[1], seq,
                                                          scale, out=out1, workspace=ws1), 20)
    nbytes1 = 2 * b1 * seq * 6 * ng + 2 * q1.numel() * 4
    npos = bh * seq
    nbytes = 2 * npos * 6 * ng + 2 * q.numel() * 4
    npos_t = bh * -(-seq // 64) * 64
    read = npos_t * (2 * 8 * -(-ng // 8) + 4 * 4 * -(-ng // 4)) + npos_t * 6 * ng + 2 * q.numel() * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    qf = q.view(b, h, 1, dim)
    sdpa = lambda: torch.nn.functional.scaled_dot_product_attention(  # noqa: E731
        qf, recon[0], recon[1], scale=scale)
    settle(sdpa, 0.1)
    ms_f32 = timed(sdpa, max(steps // 2, 20), 10)
    del recon
    torch.cuda.empty_cache()
    return {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
            "bytes": nbytes, "bytes_read_with_padding": read,
            "traffic": traffic_for("rotorquant_kv_attention"),
            "kernel": "rq_kv_attn_kernel (scores and V in the rotated domain)",
            "batch1": {"us": round(ms1 * 1e3, 2), "bytes": nbytes1,
                       "frac_hbm": round(nbytes1 / (ms1 * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                       "traffic": traffic_for("rotorquant_kv_attention_batch1"),
                       "note": "32 queries: sequence split over workgroups, merged by the last split"},
            "f32_kv_sdpa_us": round(ms_f32 * 1e3, 2),
            "f32_kv_bytes": 2 * bh * seq * dim * 4,
            "shape": {"batch": b, "heads": h, "seq": seq, "head_dim": dim, "bits": bits, "nq": 1}}


# ---------------------------------------------------------------- igemm 512^3
def bench_igemm_512(H, dev, steps, with_cpu):
    """The reference's only published hot-path number: igemm (u8 x i8 [K,N] ->
    i32) at 512x512x512 in 1.96 ms on an AVX-512 VNNI CPU (README.md:657-659,
    harness benches/core_ops.rs:123-160, inputs (i%251) as u8 and (i%255) as
    i8). rnn_igemm on the same inputs (a caller workspace passed, which a
    problem this small does not use: one launch stages a as signed bytes and b
    transposed in LDS, with b's column sums from an all-ones MFMA); timed by
    graph replay."""
    import numpy as np
    import torch

    import oracle as O
    m = k = n = 512
    a_np = (np.arange(m * k) % 251).astype(np.uint8).reshape(m, k)
    b_np = (np.arange(k * n) % 255).astype(np.int8).reshape(k, n)   # (i % 255) as i8 wraps
    a, b = torch.from_numpy(a_np).to(dev), torch.from_numpy(b_np).to(dev)
    ws = torch.empty(H.igemm_workspace_size(m, k, n), dtype=torch.uint8, device=dev)
    c = torch.empty((m, n), dtype=torch.int32, device=dev)
    ms = graph_timed(lambda i: H.igemm(a, b, m, k, n, workspace=ws, c=c), max(steps, 100))
    ops = 2.0 * m * n * k
    ent = {"us": round(ms * 1e3, 3), "TOPS": round(ops / (ms * 1e-3) / 1e12, 2),
           "reference_published_ms": 1.96, "speedup_vs_published": round(1.96 / ms, 1),
           "launches": 1, "kernel": "igemm_small_kernel (one launch for m n k <= 2^28)",
           "timing": "HIP graph replay, events / calls"}
    if with_cpu:
        threads = cpu_threads()
        ref = O.igemm_scalar(a_np, b_np, m, k, n)
        ent["bit_exact_vs_scalar"] = bool(np.array_equal(c.cpu().numpy(), ref))
        t, reps = cpu_time(lambda: O.igemm(a_np, b_np, m, k, n, threads), 5, 2.0)
        ent["cpu_baseline"] = {"us": round(t * 1e6, 1), "cores": threads, "kind": "port",
                               "sample": f"oracle igemm (AVX-512 VNNI restatement of "
                                         f"src/int8.rs:285-314) on the same inputs, median of "
                                         f"{reps}"}
    return ent


# ---------------------------------------------------------------- f32 GEMM
SGEMM_MNK = (4096, 4096, 4096)
SGEMM_DECODE_MNK = (16, 11008, 4096)


def bench_sgemm(H, dev, steps):
    """rnn_sgemm (the BlasBackend::sgemm plugin point) on a 4096^3 f32
    product, beside torch.matmul (the ROCm library GEMM, TF32 off) on the same
    operands, for the two calls the reference makes: C = A*B with both
    operands as stored (Tensor::matmul, src/tensor.rs:403-412) and
    C = A*B^T with B stored [n, k] (Linear::forward, x * W^T,
    src/tensor.rs:765-775)."""
    import torch
    m, n, k = SGEMM_MNK
    a = gen_f32((m, k), 21, dev)
    b = gen_f32((k, n), 22, dev)
    bt = gen_f32((n, k), 23, dev)
    c = torch.empty((m, n), dtype=torch.float32, device=dev)
    n_iter = max(steps // 4, 20)
    flops = 2.0 * m * n * k

    def run(fn, fn_lib):
        settle(fn, 0.1)
        ms = timed(fn, n_iter, 10)
        tf32 = torch.backends.cuda.matmul.allow_tf32
        torch.backends.cuda.matmul.allow_tf32 = False
        try:
            ms_lib = timed(fn_lib, n_iter, 10)
        finally:
            torch.backends.cuda.matmul.allow_tf32 = tf32
        return flops / (ms * 1e-3) / 1e12, flops / (ms_lib * 1e-3) / 1e12, ms
    tflops, tflops_lib, ms = run(
        lambda: H.sgemm(H.NO_TRANS, H.NO_TRANS, m, n, k, 1.0, a, k, b, n, 0.0, c, n),
        lambda: torch.matmul(a, b, out=c))
    nt, nt_lib, ms_nt = run(
        lambda: H.sgemm(H.NO_TRANS, H.TRANS, m, n, k, 1.0, a, k, bt, k, 0.0, c, n),
        lambda: torch.matmul(a, bt.t(), out=c))
    del a, b, bt, c
    # Linear::forward at decode (x [16, 4096] * W^T, W [11008, 4096] f32):
    # bound by reading W once; W rotates over copies past the MALL
    dm, dn, dk = SGEMM_DECODE_MNK
    wbytes = 4 * dn * dk
    copies = max(2, -(-640 * 2**20 // wbytes))
    ws = [gen_f32((dn, dk), 30 + i, dev) for i in range(copies)]
    x = gen_f32((dm, dk), 29, dev)
    y = torch.empty((dm, dn), dtype=torch.float32, device=dev)
    nl = copies * 10
    ms_d = graph_timed(lambda i: H.sgemm(H.NO_TRANS, H.TRANS, dm, dn, dk, 1.0, x, dk, ws[i % copies], dk,
                                         0.0, y, dn), nl)
    tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        ms_dt = graph_timed(lambda i: torch.matmul(x, ws[i % copies].t(), out=y), nl)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = tf32
    dbytes = wbytes + 4 * dm * dk + 4 * dm * dn
    del ws
    torch.cuda.empty_cache()
    return {"m": m, "n": n, "k": k, "trans": "nn", "us": round(ms * 1e3, 1), "TFLOP/s": round(tflops, 1),
            "frac_fp32_mfma_peak": round(tflops / PEAK_FP32_MFMA_TFLOPS, 4),
            "torch_matmul_TFLOP/s": round(tflops_lib, 1), "traffic": traffic_for("f32_sgemm"),
            "kernel": "sgemm_transpose_kernel (B [k, n] -> [n, k] in scratch) + sgemm_mfma2_kernel<false,true> "
                      "(v_mfma_f32_16x16x4f32, 128x128 tiles, both operands as 4-k quads in LDS)",
            "nt": {"us": round(ms_nt * 1e3, 1), "TFLOP/s": round(nt, 1),
                   "frac_fp32_mfma_peak": round(nt / PEAK_FP32_MFMA_TFLOPS, 4),
                   "torch_matmul_TFLOP/s": round(nt_lib, 1),
                   "kernel": "sgemm_mfma2_kernel<false,true> (B stored [n, k]: both operands K-contiguous)"},
            "decode": {"m": dm, "n": dn, "k": dk, "trans": "nt", "us": round(ms_d * 1e3, 2),
                       "GB/s": round(dbytes / (ms_d * 1e-3) / 1e9, 1),
                       "frac_hbm": round(dbytes / (ms_d * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                       "torch_matmul_us": round(ms_dt * 1e3, 2),
                       "kernel": "sgemm_skinny_nt_kernel<1,64,4> (m <= 16, B in whole lines regrouped "
                                 "through LDS, v_mfma_f32_16x16x4f32)",
                       "timing": "HIP-graph replay, median replay / launches, W rotated over copies"}}


# ---------------------------------------------------------------- copy ceiling
COPY_BYTES = 512 * 2**20


def bench_copy(dev, steps):
    """The measured HBM ceiling: a plain device-to-device copy of COPY_BYTES
    (read + write = 2 * COPY_BYTES of traffic per launch). The same launch is
    the known-size reference that FETCH_SIZE / WRITE_SIZE counters are scaled
    by when HBM traffic per kernel is derived from rocprofv3 --pmc runs."""
    import torch
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    fn = lambda: dst.copy_(src)  # noqa: E731
    settle(fn, 0.1)
    ms = timed(fn, max(steps, 20), 5)
    gbs = 2 * COPY_BYTES / (ms * 1e-3) / 1e9
    return {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
            "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes_per_launch": 2 * COPY_BYTES}


# ---------------------------------------------------------------- load window
def bench_read_window(dev, floor):
    """Streaming reads of the decode GEMV's weight bytes (4096 x 11008 and
    4096 x 4096) in the launch shape of the balanced-row GEMV -- one workgroup
    per CU streaming its contiguous share -- at several depths of loads in
    flight per CU (waves x loads per lane x 1 KiB), beside the read floor
    (small streaming workgroups). The same buffer rotation and graph timing as
    the GEMV. It measures how the in-flight depth of one-workgroup-per-CU
    streams sets their rate, which fixes the GEMV's load window."""
    import torch
    lib = floor.lib
    lib.rnn_probe_range_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_uint32,
                                         ctypes.c_void_p, ctypes.c_void_p]
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    out = {}
    for nbytes in (4096 * 11008, 4096 * 4096):
        copies = max(2, -(-640 * 2**20 // nbytes))
        bufs = [torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=dev)
                for _ in range(copies)]
        n_launch = 15 * copies if nbytes > 2**25 else 40 * copies
        ent = {"floor_us": round(_floor(floor, bufs, nbytes, n_launch) * 1e3, 3)}
        for waves, per in ((4, 2), (4, 4), (4, 8), (4, 24), (8, 2), (8, 4), (8, 8), (8, 24)):
            def launch(i, waves=waves, per=per):
                rc = lib.rnn_probe_range_read(
                    ctypes.c_void_p(bufs[i % copies].data_ptr()), nbytes, cus, waves, per,
                    0x9E3779B9, ctypes.c_void_p(floor.sink.data_ptr()),
                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
                if rc != 0:
                    raise RuntimeError("rnn_probe_range_read failed")
            ms = graph_timed(launch, n_launch)
            ent[f"w{waves}_p{per}_{waves * per}KiB_us"] = round(ms * 1e3, 3)
        out[f"{nbytes}_bytes"] = ent
        del bufs
    return out


def bench_l2_rate(dev, steps):
    """The rate at which a CU takes in L2-resident data (librnn_probe.so's
    l2_rate_kernel): one block of 8 waves per CU, each wave reading its own
    64 KiB window of a 4 MiB buffer (resident in every XCD's L2 after the
    first launch) 1 MiB over, with 4 or 8 loads of 1 KiB in flight, into VGPRs
    or into LDS (the GEMM kernels' DMA). It prices the operand bytes a GEMM
    block pulls through its CU."""
    import torch
    lib = ctypes.CDLL(PROBE_LIB)
    lib.rnn_probe_l2_rate.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_uint32, ctypes.c_void_p,
                                      ctypes.c_void_p]
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    nbytes = 4 << 20
    buf = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    per_wave = 1 << 20
    out = {"buffer_bytes": nbytes, "blocks": cus, "bytes_per_wave": per_wave}
    for to_lds in (0, 1):
        for per in (4, 8):
            def launch(i, to_lds=to_lds, per=per):
                rc = lib.rnn_probe_l2_rate(ctypes.c_void_p(buf.data_ptr()), nbytes, cus, to_lds, per,
                                           per_wave // 1024 // per, 0x9E3779B9,
                                           ctypes.c_void_p(sink.data_ptr()),
                                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
                if rc != 0:
                    raise RuntimeError("rnn_probe_l2_rate failed")
            ms = graph_timed(launch, max(steps, 20))
            key = f"{'lds' if to_lds else 'vgpr'}_p{per}"
            out[key + "_us"] = round(ms * 1e3, 2)
            out[key + "_GBps_per_cu"] = round(8 * per_wave / (ms * 1e-3) / 1e9, 1)
    out["method"] = ("HIP graph replay: events around each replay, median replay / launches per "
                     "replay; GB/s per CU = 8 waves x 1 MiB / launch time")
    return out


# ---------------------------------------------------------------- clock probe
def bench_clock_probe(dev):
    """The shader clock under a plain int8 MFMA load: librnn_probe.so's
    mfma_clock_kernel (constant operands, one wave per SIMD on every CU) reads
    the shader-clock and 100 MHz real-time counters at the start and end of
    each block. It pins what "clock" means for the counter-derived figures
    (SQ_BUSY_CYCLES per shader engine over the launch) of the GEMM profiles,
    and gives the int8 MFMA rate the chip reaches with no memory traffic."""
    import torch
    lib = ctypes.CDLL(PROBE_LIB)
    lib.rnn_probe_mfma_clock.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                         ctypes.c_void_p, ctypes.c_void_p]
    blocks = torch.cuda.get_device_properties(dev).multi_processor_count
    iters = 20000
    out = torch.zeros(4 * blocks, dtype=torch.int64, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run():
        if lib.rnn_probe_mfma_clock(blocks, iters, ctypes.c_void_p(out.data_ptr()),
                                    ctypes.c_void_p(sink.data_ptr()), st) != 0:
            raise RuntimeError("rnn_probe_mfma_clock failed")
    settle(run, 0.2)
    ms = timed(run, 5, 1)
    o = out.cpu().numpy().reshape(blocks, 4).astype("float64")
    ghz = sorted(((o[:, 1] - o[:, 0]) / (o[:, 3] - o[:, 2]) * 0.1).tolist())
    ops = 2.0 * 16 * 16 * 64 * 8 * iters * 4 * blocks
    return {"ghz_median": round(ghz[len(ghz) // 2], 3), "ghz_min": round(ghz[0], 3),
            "ghz_max": round(ghz[-1], 3), "int8_TOPS": round(ops / (ms * 1e-3) / 1e12, 1),
            "us": round(ms * 1e3, 1), "blocks": blocks,
            "method": "s_memtime / s_memrealtime deltas per block (100 MHz real-time clock)"}


COMPONENTS = ["gemv", "mlp", "ternary", "rotorquant", "rq_attention", "qt_gemv", "igemm512",
              "sgemm", "copy", "clock", "window", "l2rate"]

# QuantizedLinear entries carried on the printed line (all of them go to --full-json)
QT_LINE = ("INT4_g128_m1_k4096_n11008", "INT4_g128_m16_k4096_n11008", "GGUF_Q8_0_m16_k4096_n11008")


def _pick(d, *keys):
    return {k: d[k] for k in keys if k in d}


def compact(result):
    """The printed line: the headline fields, then the secondary rows, then
    BASELINE configs 1, 2, 4 and 5 last (so that a reader keeping only the
    tail of stdout still has every configuration). The full record, with the
    per-entry method strings, is what --full-json writes."""
    comp = result.get("components", {})
    line = {k: result[k] for k in result if k != "components"}
    if "prefill_ksweep" in line:
        line["prefill_ksweep"] = _pick(line["prefill_ksweep"], "k", "us", "fixed_us", "loop_us")
    if "cpu_baseline" in line:
        cb = line["cpu_baseline"]
        line["cpu_baseline"] = dict(_pick(cb, "value", "unit", "cores", "kind", "sample"),
                                    cpu=cb.get("cpu", {}).get("model"))
    other = {}
    if "rotorquant_kv_attention" in comp:
        a = comp["rotorquant_kv_attention"]
        other["rq_kv_attention"] = {"us": a["us"], "frac_hbm": a["frac_hbm"],
                                    "b1_us": a["batch1"]["us"],
                                    "b1_frac_hbm": a["batch1"]["frac_hbm"],
                                    "f32_sdpa_us": a["f32_kv_sdpa_us"]}
    if "quantized_linear_gemv" in comp:
        q = comp["quantized_linear_gemv"]
        other["qt_gemv"] = {k: _pick(q[k], "us", "frac_hbm", "frac_of_read_floor")
                            for k in QT_LINE if k in q}
    if "igemm_512" in comp:
        g = comp["igemm_512"]
        other["igemm_512"] = _pick(g, "us", "speedup_vs_published", "bit_exact_vs_scalar")
        if "cpu_baseline" in g:
            other["igemm_512"]["cpu_us"] = g["cpu_baseline"]["us"]
    if "f32_sgemm" in comp:
        other["f32_sgemm"] = _pick(comp["f32_sgemm"], "TFLOP/s", "frac_fp32_mfma_peak",
                                   "torch_matmul_TFLOP/s")
        if "nt" in comp["f32_sgemm"]:
            other["f32_sgemm"]["nt_TFLOP/s"] = comp["f32_sgemm"]["nt"]["TFLOP/s"]
            other["f32_sgemm"]["nt_frac"] = comp["f32_sgemm"]["nt"]["frac_fp32_mfma_peak"]
        if "decode" in comp["f32_sgemm"]:
            other["f32_sgemm"]["decode_m16_n11008_us"] = comp["f32_sgemm"]["decode"]["us"]
            other["f32_sgemm"]["decode_frac_hbm"] = comp["f32_sgemm"]["decode"]["frac_hbm"]
            other["f32_sgemm"]["decode_torch_us"] = comp["f32_sgemm"]["decode"]["torch_matmul_us"]
    if "copy_ceiling" in comp:
        other["copy_ceiling_GBs"] = comp["copy_ceiling"]["GB/s"]
    if "mfma_clock_probe" in comp:
        c = comp["mfma_clock_probe"]
        other["mfma_clock_probe"] = {"ghz": c["ghz_median"], "TOPS": c["int8_TOPS"]}
    if other:
        line["other"] = other
    if "int8_mlp_784_256_128_10" in comp:
        e = comp["int8_mlp_784_256_128_10"]
        c1 = _pick(e, "us_graph", "us_eager", "us_graph_per_layer_launches", "ops",
                   "max_abs_diff_vs_cpu")
        if "cpu_baseline" in e:
            c1["cpu_us"] = e["cpu_baseline"]["us"]
            c1["cpu_cores"] = e["cpu_baseline"]["cores"]
        line["C1_mlp_784_256_128_10_b32"] = c1
    if "w8a8_decode_gemv" in comp:
        c2 = {}
        for name, e in comp["w8a8_decode_gemv"].items():
            s = {"us": e["us"], "GB/s": e["GB/s"], "frac_hbm": e["frac_hbm"]}
            if "read_floor_us" in e:
                s["floor_us"] = e["read_floor_us"]
                s["of_floor"] = e["frac_of_read_floor"]
            if "cpu_baseline" in e:
                s["cpu_us"] = e["cpu_baseline"]["us"]
                s["cpu_cores"] = e["cpu_baseline"]["cores"]
            c2[name] = s
        c2["note"] = ("floor = same-bytes one-launch read (probe), timed as the GEMV; "
                      "cpu = oracle igemm + epilogue, 4-row blocks over threads")
        line["C2_decode_gemv"] = c2
    if "ternary_gemm" in comp:
        e = comp["ternary_gemm"]
        c4 = _pick(e, "us", "TOPS", "frac_int8_peak", "us_reference_layout", "traffic")
        if e.get("counters"):
            c4["mfma_busy"] = e["counters"].get("mfma_busy")
            c4["clock_ghz"] = e["counters"].get("clock_ghz")
            c4["counter_run_us"] = e["counters"].get("duration_us_under_counters")
        if "cpu_baseline" in e:
            c4["cpu_us"] = e["cpu_baseline"]["us"]
            c4["cpu_cores"] = 1
        line["C4_ternary_512x4096x4096"] = c4
    if "rotorquant_kv" in comp:
        e = comp["rotorquant_kv"]
        c5 = _pick(e, "us_per_step", "GB/s", "frac_hbm", "traffic")
        if "cpu_baseline" in e:
            c5["cpu_us_per_step"] = e["cpu_baseline"]["us_per_step"]
            c5["cpu_cores"] = 1
        line["C5_rotorquant_kv_8x32x4096x128"] = c5
    return line


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # Every timed figure follows a SETTLE_S clock settle of its own kernel;
    # --warmup launches come after it and are untimed too.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", default="all", choices=["all", "prefill"] + COMPONENTS)
    ap.add_argument("--no-cpu", action="store_true")
    # (a separate run: its launches share the headline kernel's name, so they
    # would enter that kernel's rocprofv3 --stats average)
    ap.add_argument("--ksweep", action="store_true",
                    help="also time the prefill GEMM at K = 1024..4096 (fixed vs K-loop cost)")
    ap.add_argument("--full-json", default=None,
                    help="also write the full record (every entry with its method) to this file")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(the quantized-inference path runs on one GPU; every kernel shards by output "
              "columns or KV heads, with no collective on the hot path)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import rnn_hip as H
    import workloads as W
    H.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    with_cpu = not args.no_cpu
    floor = ReadFloor(dev) if os.path.exists(PROBE_LIB) else None

    result = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
              "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
              "data": "synthetic (seeded N(0,0.02) weights, N(0,1) activations)"}
    components = {}
    if args.only in ("all", "prefill"):
        log("prefill: W8A8 2048x4096x14336")
        ms, tops, state = bench_prefill(H, W, dev, args.steps, args.warmup)
        ops = 2.0 * state["m"] * state["n"] * state["k"]
        result.update({
            "value": round(tops, 2), "unit": "TOPS", "ms_per_step": round(ms, 5),
            "config": {"workload": "w8a8_prefill_gemm", "m": state["m"], "k": state["k"],
                       "n": state["n"], "out": "fp32", "epilogue": "(acc*sa[m])*sw[n]",
                       "baseline_config_index": 2},
            "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": PEAK_INT8_TOPS,
                         "unit": "TFLOP/s", "frac": round(tops / PEAK_INT8_TOPS, 4),
                         "traffic": traffic_for("w8a8_prefill_gemm"),
                         "counters": counters_for("w8a8_prefill_gemm"),
                         "op_kind": "int8 MFMA ops, 2 per multiply-accumulate (T int-op/s)",
                         "ops_per_launch": ops,
                         "kernel": "gemm_pp_kernel<L128Cfg<256,224,4,2,0,1>> (ping-pong, v_mfma_i32_16x16x64_i8, 128-byte LDS rows)",
                         "timing": f"HIP events on the launch stream, average over the timed "
                                   f"launches; {SETTLE_S} s clock settle and {args.warmup} "
                                   f"warmup launches before them"},
        })
        result["prefill_layer"] = dict(state["layer"], note="rnn_quant_rows_i8 of the fp32 "
                                       "activations + the GEMM, events over back-to-back calls")
        if with_cpu:
            log("cpu baseline: oracle igemm over the whole workload")
            result["cpu_baseline"] = cpu_baseline(state)
        del state
        torch.cuda.empty_cache()
        if args.ksweep:
            log("prefill: the same M and N at K = 1024..4096")
            result["prefill_ksweep"] = prefill_ksweep(H, W, dev, args.steps, args.warmup)
    if args.only in ("all", "gemv"):
        log("decode GEMV: 6 shapes")
        components["w8a8_decode_gemv"] = bench_gemv(H, W, dev, args.steps, floor, with_cpu)
    if args.only in ("all", "mlp"):
        log("int8 MLP 784-256-128-10, batch 32")
        components["int8_mlp_784_256_128_10"] = bench_mlp(H, W, dev, args.steps, with_cpu)
    if args.only in ("all", "ternary"):
        log("ternary GEMM 512x4096x4096")
        components["ternary_gemm"] = bench_ternary(H, W, dev, args.steps, with_cpu)
    if args.only in ("all", "rotorquant"):
        log("RotorQuant K+V [8,32,4096,128] 4-bit round trip")
        components["rotorquant_kv"] = bench_rotorquant(H, W, dev, args.steps, with_cpu)
    if args.only in ("all", "rq_attention"):
        log("attention over the RotorQuant KV cache [8,32,4096,128], 4-bit, one query per head")
        components["rotorquant_kv_attention"] = bench_rq_attention(H, W, dev, args.steps)
    if args.only in ("all", "qt_gemv"):
        log("QuantizedLinear GEMV: INT4/GGUF/BF16 weights, decode shapes")
        components["quantized_linear_gemv"] = bench_qt_gemv(H, dev, args.steps, floor)
    if args.only in ("all", "igemm512"):
        log("igemm 512x512x512 (the reference's published shape)")
        components["igemm_512"] = bench_igemm_512(H, dev, args.steps, with_cpu)
    if args.only in ("all", "sgemm"):
        log("f32 GEMM 4096x4096x4096 (BlasBackend::sgemm)")
        components["f32_sgemm"] = bench_sgemm(H, dev, args.steps)
    if args.only in ("all", "copy"):
        log("streaming copy ceiling: 512 MiB device-to-device")
        components["copy_ceiling"] = bench_copy(dev, args.steps)
    if args.only in ("all", "clock") and os.path.exists(PROBE_LIB):
        log("MFMA clock probe")
        components["mfma_clock_probe"] = bench_clock_probe(dev)
    # (not part of "all": studies of the GEMV's load window and of the
    # per-CU load rate, run on their own)
    if args.only == "window" and floor is not None:
        log("one-workgroup-per-CU streaming reads at several load depths")
        components["read_window"] = bench_read_window(dev, floor)
    if args.only == "l2rate" and os.path.exists(PROBE_LIB):
        log("per-CU rate of L2-resident loads into VGPRs and into LDS")
        components["l2_load_rate"] = bench_l2_rate(dev, args.steps)
    if components:
        result["components"] = components
    if "value" not in result:  # a single non-headline component was requested
        result.update({"value": None, "unit": None, "ms_per_step": None,
                       "config": {"workload": args.only}})
    if args.full_json:
        with open(args.full_json, "w") as f:
            json.dump(result, f, indent=1)
    print(json.dumps(compact(result)), flush=True)


if __name__ == "__main__":
    main()
