"""Benchmark of the quantized-inference hot path on one MI355X.

Headline line (value): W8A8 prefill GEMM, M=2048 K=4096 N=14336, int8 x int8 ->
int32 -> fp32 per-channel/per-row dequant epilogue, inputs resident in HBM, in
TOPS (2*M*N*K int ops per step). The same JSON line carries the roofline of that
kernel, the CPU baseline (the oracle's AVX-512 VNNI igemm path over the whole
workload) and the other configurations as `components`: decode GEMV (GB/s, weight
buffers rotated past the 256 MB MALL), ternary GEMM (TOPS; both timed by HIP-graph
replay), the RotorQuant K+V round trip (GB/s) and the f32 BlasBackend GEMM
(TFLOP/s, beside torch.matmul's library GEMM on the same operands).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
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
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


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


def traffic_for(name):
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f).get(name)
        return None if t is None else t.get("bytes_per_launch")
    except (OSError, ValueError):
        return None


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
    ms = timed(fn, steps, warmup)
    ops = 2.0 * m * n * k
    tops = ops / (ms * 1e-3) / 1e12
    state = dict(aq=aq, sa=sa, wq=wq, sw=sw, m=m, k=k, n=n)
    return ms, tops, state


# ---------------------------------------------------------------- GEMV
def graph_timed(launch, n_launch, replays=5, settle_s=0.1):
    """Average ms per launch of `launch(i)` for i in range(n_launch), captured
    once into a HIP graph and replayed (events on the replay stream), so the
    per-call host overhead of the Python binding is not part of the figure.
    Untimed replays for `settle_s` seconds come first, so the clocks have
    settled for this kernel before the timed replays."""
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
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(replays):
        g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) / (replays * n_launch)


def bench_gemv(H, W, dev, steps):
    import torch
    out = {}
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
        out[f"m{m}_k{k}_n{n}"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                                  "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": nbytes,
                                  "weight_copies": copies, "launches_timed": n_launch,
                                  "timing": "HIP graph replay, events / launches"}
        del ws, sws
        torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------- QuantizedLinear GEMV
QT_SHAPES = [(1, 4096, 11008), (4, 4096, 11008), (8, 4096, 11008), (16, 4096, 11008),
             (1, 4096, 4096)]
QT_FORMATS = [("INT4_g128", 3, 128), ("GGUF_Q4_0", 6, 32), ("GGUF_Q8_0", 8, 32), ("BF16", 1, 0),
              ("NF4_g64", 4, 64)]


def bench_qt_gemv(H, dev, steps):
    """QuantizedLinear::forward (src/quantize.rs:744-754) at decode shapes:
    the fused GEMV that decodes INT4/GGUF/BF16/NF4 weights in registers (the
    VALU GEMV for m <= 4, the f32-MFMA GEMV for m >= 5, as AUTO picks). Bytes per
    launch = weight codes + f32 scales + x (4 m k) + y (4 m n); weights
    rotate over copies past the MALL as for the W8A8 GEMV."""
    import torch
    out = {}
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
            ms = graph_timed(lambda i: H.qt_linear_forward(fmt, x, ds[i % copies], ss[i % copies],
                                                           g, n, y=y), n_launch)
            nbytes = wbytes + 4 * m * k + 4 * m * n
            gbs = nbytes / (ms * 1e-3) / 1e9
            out[f"{name}_m{m}_k{k}_n{n}"] = {
                "us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": nbytes,
                "weight_copies": copies, "launches_timed": n_launch,
                "timing": "HIP graph replay, events / launches"}
            del ds, ss
            torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------- ternary
def bench_ternary(H, W, dev, steps):
    import torch
    c = W.TERNARY
    m, k, n = c["m"], c["k"], c["n"]
    packed, scales = H.ternary_quantize(gen_f32((n, k), 3, dev), H.TERNARY_ABSMEAN)
    aq, sa = H.quant_rows_i8(gen_f32((m, k), 4, dev))
    y = torch.empty((m, n), dtype=torch.float32, device=dev)
    # a launch (~13 us) is shorter than the Python binding's per-call host
    # cost, so launches are replayed from a HIP graph as for the GEMV
    n_launch = max(steps, 100)
    ms = graph_timed(lambda i: H.ternary_gemm(aq, sa, packed, scales, n, y=y), n_launch)
    ops = 2.0 * m * n * k
    tops = ops / (ms * 1e-3) / 1e12
    nbytes = n * k // 4 + 4 * n + m * k + 4 * m + 4 * m * n
    return {"us": round(ms * 1e3, 3), "TOPS": round(tops, 1),
            "frac_int8_peak": round(tops / PEAK_INT8_TOPS, 4), "ops": ops, "bytes": nbytes,
            "launches_timed": 5 * n_launch, "timing": "HIP graph replay, events / launches"}


# ---------------------------------------------------------------- RotorQuant
def bench_rotorquant(H, W, dev, steps):
    import torch
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

    def step():
        for x, y, r in zip(kv, outs, rots):
            H.rotorquant_quantize(x, r, bits, y=y)

    ms = timed(step, max(steps // 2, 10), 3)
    nbytes = sum(2 * x.numel() * 4 for x in kv)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"us_per_step": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
            "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes_per_step": nbytes,
            "launches_per_step": 2}


def bench_rq_attention(H, W, dev, steps):
    """Decode attention over the RotorQuant KV cache (the RotorQuant config's
    K and V, [8, 32, 4096, 128], 4-bit, as pages): one query per (batch,
    head). Bytes per launch = both pages (6 bytes per position and group) +
    q + out. Beside it, torch's f32 scaled_dot_product_attention over the
    reconstructed K and V (what a cache without the codes would read), timed
    the same way, for context."""
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

    def step():
        H.rotorquant_kv_attention(q, pages[0], pages[1], rots[0], rots[1], seq, scale, out=out)

    ms = timed(step, max(steps // 2, 20), 10)
    # bytes the kernel reads: K pages pad each position to 8 groups of codes
    # and 4 of scales, V pages hold exactly ng of each
    npos = bh * -(-seq // 64) * 64
    nbytes = npos * (2 * 8 * -(-ng // 8) + 4 * 4 * -(-ng // 4)) + npos * 6 * ng + 2 * q.numel() * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    qf = q.view(b, h, 1, dim)
    ms_f32 = timed(lambda: torch.nn.functional.scaled_dot_product_attention(
        qf, recon[0], recon[1], scale=scale), max(steps // 2, 20), 10)
    del recon
    torch.cuda.empty_cache()
    return {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
            "bytes": nbytes, "kernel": "rq_kv_attn_kernel (scores and V in the rotated domain)",
            "f32_kv_sdpa_us": round(ms_f32 * 1e3, 2),
            "f32_kv_bytes": 2 * bh * seq * dim * 4,
            "shape": {"batch": b, "heads": h, "seq": seq, "head_dim": dim, "bits": bits, "nq": 1}}


# ---------------------------------------------------------------- f32 GEMM
SGEMM_MNK = (4096, 4096, 4096)


def bench_sgemm(H, dev, steps):
    """rnn_sgemm (the BlasBackend::sgemm plugin point) on a 4096^3 f32
    product, C = A*B with both operands as stored (no transpose), beside
    torch.matmul (the ROCm library GEMM, TF32 off) on the same operands."""
    import torch
    m, n, k = SGEMM_MNK
    a = gen_f32((m, k), 21, dev)
    b = gen_f32((k, n), 22, dev)
    c = torch.empty((m, n), dtype=torch.float32, device=dev)
    n_iter = max(steps // 4, 20)
    ms = timed(lambda: H.sgemm(H.NO_TRANS, H.NO_TRANS, m, n, k, 1.0, a, k, b, n, 0.0, c, n), n_iter, 10)
    tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        ms_lib = timed(lambda: torch.matmul(a, b, out=c), n_iter, 10)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = tf32
    flops = 2.0 * m * n * k
    tflops, tflops_lib = flops / (ms * 1e-3) / 1e12, flops / (ms_lib * 1e-3) / 1e12
    return {"m": m, "n": n, "k": k, "trans": "nn", "us": round(ms * 1e3, 1), "TFLOP/s": round(tflops, 1),
            "frac_fp32_mfma_peak": round(tflops / PEAK_FP32_MFMA_TFLOPS, 4),
            "torch_matmul_TFLOP/s": round(tflops_lib, 1), "traffic": traffic_for("f32_sgemm"),
            "kernel": "sgemm_mfma_kernel<false,false> (v_mfma_f32_16x16x4f32, 128x128 tiles)"}


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
    ms = timed(lambda: dst.copy_(src), max(steps, 20), 5)
    gbs = 2 * COPY_BYTES / (ms * 1e-3) / 1e9
    return {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
            "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes_per_launch": 2 * COPY_BYTES}


# ---------------------------------------------------------------- CPU baseline
def cpu_baseline(state, max_repeats=5, budget_s=20.0):
    """The reference CPU path for the whole prefill workload (all 2048 rows):
    igemm (src/int8.rs:285-314: AVX-512 VNNI when the host has it, B repacked
    on every call, 4-row blocks over threads) on a_u8 = a_s8 + 128 and
    B = W^T, then the zero-point correction and the per-row/per-channel
    dequant epilogue. Median of up to `max_repeats` runs, stopping once
    `budget_s` seconds of wall time are spent."""
    import numpy as np

    import oracle as O
    m, k, n = state["m"], state["k"], state["n"]
    aq = state["aq"].cpu().numpy()
    sa = state["sa"].cpu().numpy()
    wq = state["wq"].cpu().numpy()
    sw = state["sw"].cpu().numpy()
    b_kn = np.ascontiguousarray(wq.T)                   # weight layout prep, not timed
    colsum128 = 128 * b_kn.astype(np.int64).sum(axis=0).astype(np.int32)
    threads = max(1, min(16, os.cpu_count() or 1))
    times = []
    used_vnni = False
    start = time.perf_counter()
    while len(times) < max_repeats and (not times or time.perf_counter() - start < budget_s):
        t0 = time.perf_counter()
        a_u8 = (aq.view(np.uint8) ^ np.uint8(0x80))
        c, used_vnni = O.igemm(a_u8, b_kn, m, k, n, threads)
        acc = (c - colsum128).astype(np.int32)
        y = (acc.astype(np.float32) * sa[:, None]) * sw[None, :]
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    ops = 2.0 * m * n * k
    return {"value": round(ops / t / 1e12, 4), "unit": "TOPS", "cores": threads,
            "kind": "port",
            "sample": f"the full W8A8 prefill workload {m}x{k}x{n} (no subsampling): oracle igemm "
                      f"({'AVX-512 VNNI' if used_vnni else 'scalar'}, B repacked per call as "
                      f"src/int8.rs:296 does) + zero-point + dequant epilogue, {threads} threads, "
                      f"median of {len(times)} runs, {t:.3f} s per run",
            "y_checksum": float(np.float64(y).sum())}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # The warmup covers the clock ramp: from idle the first ~100 prefill
    # launches run up to 25% slower while the GPU raises its clocks.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--only", default="all",
                    choices=["all", "prefill", "gemv", "qt_gemv", "ternary", "rotorquant", "rq_attention",
                             "sgemm", "copy"])
    ap.add_argument("--no-cpu", action="store_true")
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
                         "op_kind": "int8 MFMA ops, 2 per multiply-accumulate (T int-op/s)",
                         "ops_per_launch": ops,
                         "kernel": "gemm_pp_kernel<L128Cfg<256,224,4,2,0,1>> (ping-pong, v_mfma_i32_16x16x64_i8, 128-byte LDS rows)",
                         "timing": "HIP events on the launch stream, average over the timed "
                                   "launches"},
        })
        if not args.no_cpu:
            log("cpu baseline: oracle igemm over the whole workload")
            result["cpu_baseline"] = cpu_baseline(state)
        del state
        torch.cuda.empty_cache()
    if args.only in ("all", "gemv"):
        log("decode GEMV: 6 shapes")
        components["w8a8_decode_gemv"] = bench_gemv(H, W, dev, args.steps)
    if args.only in ("all", "qt_gemv"):
        log("QuantizedLinear GEMV: INT4/GGUF/BF16 weights, decode shapes")
        components["quantized_linear_gemv"] = bench_qt_gemv(H, dev, args.steps)
    if args.only in ("all", "ternary"):
        log("ternary GEMM 512x4096x4096")
        components["ternary_gemm"] = bench_ternary(H, W, dev, args.steps)
    if args.only in ("all", "rotorquant"):
        log("RotorQuant K+V [8,32,4096,128] 4-bit round trip")
        components["rotorquant_kv"] = bench_rotorquant(H, W, dev, args.steps)
    if args.only in ("all", "rq_attention"):
        log("attention over the RotorQuant KV cache [8,32,4096,128], 4-bit, one query per head")
        components["rotorquant_kv_attention"] = bench_rq_attention(H, W, dev, args.steps)
    if args.only in ("all", "sgemm"):
        log("f32 GEMM 4096x4096x4096 (BlasBackend::sgemm)")
        components["f32_sgemm"] = bench_sgemm(H, dev, args.steps)
    if args.only in ("all", "copy"):
        log("streaming copy ceiling: 512 MiB device-to-device")
        components["copy_ceiling"] = bench_copy(dev, args.steps)
    if components:
        result["components"] = components
    if "value" not in result:  # a single non-headline component was requested
        result.update({"value": None, "unit": None, "ms_per_step": None,
                       "config": {"workload": args.only}})
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
