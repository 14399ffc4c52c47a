#!/usr/bin/env python3
"""Benchmark of the MI355X Q4_K weight path.

Default workload: the 3B-class decode set at M=1,
36 layers with distinct seeded Q4_K weights, each layer
  QKV    gemv_quant_triple  [2048 | 256 | 256] x 2048
  O      gemv_quant_add     [2048 x 2048]   (+ fp16 residual)
  gate+up gemv_quant_pair   [11008 | 11008] x 2048
  down   gemv_quant_add     [2048 x 11008]  (+ fp16 residual)
issued through the reflex::infer C++ API (weights_device set, as a runtime
with resolved weight aliases does) on one stream and replayed as a HIP graph.
A step is one pass over all 36 layers (144 launches); `value` is algorithmic
bytes per step / seconds per step.  Inputs are resident in HBM; the 1.56 GB
of weights exceed the 256 MB Infinity Cache, so every step streams from HBM.

Also reported, each as n launches captured in a HIP graph on the bench
stream and timed with HIP events recorded on that stream around replays:
  roofline     the dominant kernel (gate+up pair GEMV), per-launch duration;
               `traffic` comes from the committed rocprofv3 PMC summary
               (FETCH_SIZE + WRITE_SIZE scaled by a copy of known size)
  per_kernel   every decode projection, the LM head [151936 x 2048] fp32
               GEMV, the 4096-id Zipf(1.1) embedding gather, and the prefill
               GEMM at m=512 (TFLOP/s, BASELINE metric's second half) and
               m=2048
  attn_*       decode attention over 4096 and 16384 positions and causal
               prefill of 512 tokens (32 query / 8 KV heads, head_dim 128,
               fp16 KV)
  q6k_*, q5k_* Q6_K (ggml type 14) LM head, embedding gather, down, the
               mixed Q4_K/Q4_K/Q6_K QKV triple (the Q4_K_M file layout), and
               the Q6_K / Q5_K prefill GEMM at m=512
  small_batch_decode  m in {1,2,4,8,16} tokens on gate+up and down
               (where weight reuse ends the purely
               bandwidth-bound regime)
  floors       what the box gives any kernel: an empty kernel per graph
               launch, the sustained read ceiling (a persistent grid-stride
               read of 2 GiB, the best of a sweep of grid sizes and the
               nontemporal bit), the fill and nontemporal write rates; each
               decode projection carries floor_us = empty + bytes / ceiling,
               its fraction of it, and whether the launch or HBM bounds it
  cpu_baseline the oracle's restatement of the reference CPU GEMV
               (gemv_quant_cpu) over the full 36-layer set, single thread
               (median of 5); cpu_baseline_per_config times BASELINE
               configs 1, 3, 4 (16-token subset, extrapolated), 5a and 5b the
               same way, with the host CPU model and core count.
Every extra whose working set could sit in the 256 MB Infinity Cache
rotates distinct copies totalling more than 512 MB.

Profiling entry points (no timing, for rocprofv3 counter passes):
  --leg NAME        one kernel's workload, 20 eager launches on distinct weight
                    copies (gate_up, down, lm_head, embed, the m=512 GEMM
                    shapes, small batch gate_up_m8 / gate_up_m16 / down_m16,
                    attn_prefill)
  --leg NAME --graph  the same workload as 72 launches in a HIP graph,
                    replayed 20 times untimed and 10 times timed; prints the
                    per-launch time from HIP events (the figure the kernel
                    trace is compared with)
  --calibrate-copy  a 256 MiB device copy, to scale FETCH_SIZE / WRITE_SIZE
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "reflex-infer_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
HIDDEN, FFN, N_LAYERS = 2048, 11008, 36
QKV = (2048, 256, 256)
VOCAB = 151936
METRIC = "Q4_K GEMV HBM GB/s (% of peak) at M=1; Q4 GEMM TFLOP/s at M=512"


def qbytes(rows: int, K: int) -> int:
    return rows * (K // 256) * 144


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_gate_up_pair_decode36.txt")


def measured_traffic():
    """HBM bytes per gate+up launch from the committed rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE, each scaled by what it reads for a plain
    copy of known size); (None, None) when the summary is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].split()[0]), os.path.relpath(TRAFFIC_FILE, ROOT)
    except OSError:
        pass
    return None, None


def host_cpu() -> dict:
    """The host CPU model and the cores this process may run on."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count()
    return {"model": model, "nproc": nproc, "os_cpu_count": os.cpu_count()}


# Single-kernel workloads for counter collection (bench.py --leg NAME):
# (ggml type, rows, K, tokens, kind); weights are distinct copies so that
# every launch streams from HBM.
LEGS = {
    "gate_up": (12, 2 * FFN, HIDDEN, 1, "pair"),
    "qkv": (12, sum(QKV), HIDDEN, 1, "triple"),
    "o": (12, HIDDEN, HIDDEN, 1, "add"),
    "down": (12, HIDDEN, FFN, 1, "add"),
    "lm_head": (12, VOCAB, HIDDEN, 1, "f32"),
    "embed": (12, VOCAB, HIDDEN, 4096, "embed"),
    "gemm512_11008x2048": (12, FFN, HIDDEN, 512, "gemm"),
    "gemm512_2048x11008": (12, HIDDEN, FFN, 512, "gemm"),
    "gemm2048_11008x2048": (12, FFN, HIDDEN, 2048, "gemm"),
    "gate_up_m8": (12, 2 * FFN, HIDDEN, 8, "tokens"),
    "gate_up_m16": (12, 2 * FFN, HIDDEN, 16, "tokens"),
    "down_m16": (12, HIDDEN, FFN, 16, "tokens"),
    "attn_prefill": (0, 0, 0, 512, "attn_prefill"),
    "q6k_lm_head": (14, VOCAB, HIDDEN, 1, "f32"),
    "q6k_gemm512_2048x11008": (14, HIDDEN, FFN, 512, "gemm"),
}


def run_leg(name: str, graph: bool = False) -> int:
    import numpy as np
    import torch

    import rxq4
    from rxq4 import capi

    rxq4.load()
    dev = torch.device("cuda:0")
    t, M, K, m, kind = LEGS[name]

    def gen(seed, shape, sigma):
        g = torch.Generator(device=dev).manual_seed(seed)
        return torch.randn(shape, generator=g, device=dev) * sigma

    launches = 20
    if kind == "attn_prefill":
        # causal prefill of m tokens from position 0, 32 query / 8 KV heads,
        # head_dim 128, fp16 (the bench's attn_prefill_fp16_512 workload)
        AH, AKV, AD = 32, 8, 128
        n_copies = 8
        caches = [(gen(70_000 + i, (m, AKV, AD), 1.0).half(), gen(71_000 + i, (m, AKV, AD), 1.0).half())
                  for i in range(n_copies)]
        qp = gen(73_000, (m, AH * AD), 1.0).half()
        op = torch.empty_like(qp)
        run = lambda i: capi.attention_prefill_f16(  # noqa: E731
            op, qp, caches[i % n_copies][0], caches[i % n_copies][1], AH, AKV, AD, m, 0, AD ** -0.5)
    else:
        n_copies = 3 if M == VOCAB else max(2, -(-(600 << 20) // qbytes(M, K)))
        ws = [capi.quantize_ggml(gen(80_000 + i, (M, K), 0.02), t) for i in range(n_copies)]
    if kind == "attn_prefill":
        pass
    elif kind == "embed":
        rng = np.random.default_rng(5)
        ranks = np.arange(1, VOCAB + 1, dtype=np.float64)
        cdf = np.cumsum(ranks ** -1.1)
        cdf /= cdf[-1]
        ids = torch.from_numpy(rng.permutation(VOCAB)[np.minimum(
            np.searchsorted(cdf, rng.random(m)), VOCAB - 1)].astype(np.int32)).to(dev)
        out = torch.empty((m, K), dtype=torch.float16, device=dev)
        run = lambda i: capi.embed_rows_f16(out, ws[i % n_copies], VOCAB, ids, K, ggml_type=t)  # noqa: E731
    elif kind == "gemm":
        xb = gen(1, (m, K), 1.0).to(torch.bfloat16)
        yb = torch.empty((m, M), dtype=torch.bfloat16, device=dev)
        run = lambda i: capi.gemm(yb, ws[i % n_copies], xb, M, m, K, ggml_type=t)  # noqa: E731
    elif kind == "tokens":
        xt = gen(4, (m, K), 1.0).half()
        yt = torch.empty((m, M), dtype=torch.float16, device=dev)
        run = lambda i: capi.gemm_f16(yt, ws[i % n_copies], xt, M, m, K, ggml_type=t)  # noqa: E731
    else:
        x = gen(2, (K,), 1.0).half()
        if kind == "f32":
            y = torch.empty(M, dtype=torch.float32, device=dev)
            run = lambda i: capi.gemv_f32(y, ws[i % n_copies], x, M, K, ggml_type=t)  # noqa: E731
        elif kind == "add":
            y = torch.empty(M, dtype=torch.float16, device=dev)
            res = gen(3, (M,), 1.0).half()
            run = lambda i: capi.gemv_add_f16(y, ws[i % n_copies], x, res, M, K, ggml_type=t)  # noqa: E731
        elif kind == "triple":
            y = torch.empty(M, dtype=torch.float16, device=dev)
            a, b = QKV[0], QKV[0] + QKV[1]
            run = lambda i: capi.gemv_multi_f16(  # noqa: E731
                [(y[:a], ws[i % n_copies][:a], a, t), (y[a:b], ws[i % n_copies][a:b], b - a, t),
                 (y[b:], ws[i % n_copies][b:], M - b, t)], x, K)
        else:
            y = torch.empty(M, dtype=torch.float16, device=dev)
            h = M // 2
            run = lambda i: capi.gemv_multi_f16(  # noqa: E731
                [(y[:h], ws[i % n_copies][:h], h, t), (y[h:], ws[i % n_copies][h:], h, t)], x, K)
    torch.cuda.synchronize()
    if not graph:
        for i in range(launches):
            run(i)
        torch.cuda.synchronize()
        print(json.dumps({"leg": name, "launches": launches, "weight_copies": n_copies}), flush=True)
        return 0
    # --graph: 72 launches (distinct copies in rotation) captured in a HIP
    # graph on a side stream, replayed 20 times untimed (the clock ramps up
    # over the first replays) and 10 times between HIP events on that
    # stream, as the bench's per-kernel figures are taken after the decode
    # step; the kernel trace of this same command is what profiles/ compares
    # them with.
    n_graph, reps, warm = 72, 10, 20
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for i in range(3):
            run(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream, capture_error_mode="relaxed"):
        for i in range(n_graph):
            run(i)
    with torch.cuda.stream(stream):
        for _ in range(warm):
            g.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            g.replay()
            e1.record(stream)
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) * 1e3 / n_graph)
    print(json.dumps({"leg": name, "graph_launches": n_graph, "replays": reps + warm, "timed_replays": reps,
                      "weight_copies": n_copies, "us_per_launch_median": round(float(np.median(per)), 3),
                      "us_per_launch_mean": round(float(np.mean(per)), 3),
                      "us_per_launch_all": [round(v, 3) for v in per]}), flush=True)
    return 0


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip LM head / embedding / GEMM")
    ap.add_argument("--eager", action="store_true", help="time eager launches, not a graph")
    ap.add_argument("--graph", action="store_true",
                    help="with --leg: replay the leg's launches as a HIP graph and print the "
                         "per-launch time from HIP events")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 256 MiB device copy (PMC byte-counter calibration)")
    ap.add_argument("--leg", choices=sorted(LEGS),
                    help="only run one kernel's workload, eagerly, 20 launches on distinct "
                         "weights (for rocprofv3 counter passes); prints one JSON line")
    return ap.parse_args()


def main() -> int:
    args = parse()
    if args.leg:
        return run_leg(args.leg, args.graph)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the Q4_K kernels run on one MI355X; sharding is design-only). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import rxq4
    from rxq4 import api, capi

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate_copy:
        # A plain copy of known size: what FETCH_SIZE / WRITE_SIZE read for
        # it calibrates the byte counters of the kernels profiled beside it.
        a = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)  # 256 MiB
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "device copy", "bytes_read": a.numel() * 4,
                          "bytes_written": b.numel() * 4, "copies": 3}), flush=True)
        return 0
    rxq4.load()
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream

    def gen(seed: int, shape, sigma: float) -> torch.Tensor:
        g = torch.Generator(device=dev).manual_seed(seed)
        return torch.randn(shape, generator=g, device=dev) * sigma

    def qweights(seed: int, rows: int, K: int, ggml_type: int = 12) -> torch.Tensor:
        # ggml's reference quantiser (what llama.cpp writes into GGUF files)
        src = gen(seed, (rows, K), 0.02)
        w = capi.quantize_ggml(src, ggml_type)
        del src
        return w

    # ------------------------------------------------------------- inputs
    log("quantising 36 layers of Q4_K weights on the GPU (ggml's reference quantiser)")
    layers = []
    for l in range(N_LAYERS):
        layers.append({
            "qkv": qweights(10_000 + 10 * l + 0, sum(QKV), HIDDEN),
            "o": qweights(10_000 + 10 * l + 1, HIDDEN, HIDDEN),
            "gu": qweights(10_000 + 10 * l + 2, 2 * FFN, HIDDEN),
            "down": qweights(10_000 + 10 * l + 3, HIDDEN, FFN),
        })
    x_h = gen(1, (HIDDEN,), 1.0).half()
    x_a = gen(2, (HIDDEN,), 1.0).half()
    x_f = gen(3, (FFN,), 1.0).half()
    res = gen(4, (HIDDEN,), 1.0).half()
    y_qkv = torch.empty(sum(QKV), dtype=torch.float16, device=dev)
    y_o = torch.empty(HIDDEN, dtype=torch.float16, device=dev)
    y_gu = torch.empty(2 * FFN, dtype=torch.float16, device=dev)
    y_d = torch.empty(HIDDEN, dtype=torch.float16, device=dev)
    torch.cuda.synchronize()

    rb = qbytes(1, HIDDEN)
    calls = []  # (api name, args struct) in issue order
    for L in layers:
        q = L["qkv"].data_ptr()
        calls.append(("gemv_quant_triple", api.GemvQuantTripleArgs(
            y0=y_qkv.data_ptr(), weights0=q, weights0_device=q, ggml_type0=12, M0=QKV[0],
            y1=y_qkv.data_ptr() + 2 * QKV[0], weights1=q + QKV[0] * rb,
            weights1_device=q + QKV[0] * rb, ggml_type1=12, M1=QKV[1],
            y2=y_qkv.data_ptr() + 2 * (QKV[0] + QKV[1]),
            weights2=q + (QKV[0] + QKV[1]) * rb, weights2_device=q + (QKV[0] + QKV[1]) * rb,
            ggml_type2=12, M2=QKV[2], x=x_h.data_ptr(), K=HIDDEN, stream=sp)))
        calls.append(("gemv_quant_add", api.GemvQuantAddArgs(
            y=y_o.data_ptr(), weights=L["o"].data_ptr(), weights_device=L["o"].data_ptr(),
            ggml_type=12, x=x_a.data_ptr(), residual=res.data_ptr(), M=HIDDEN, K=HIDDEN,
            stream=sp)))
        g = L["gu"].data_ptr()
        calls.append(("gemv_quant_pair", api.GemvQuantPairArgs(
            y0=y_gu.data_ptr(), weights0=g, weights0_device=g, ggml_type0=12, M0=FFN,
            y1=y_gu.data_ptr() + 2 * FFN, weights1=g + FFN * rb, weights1_device=g + FFN * rb,
            ggml_type1=12, M1=FFN, x=x_h.data_ptr(), K=HIDDEN, stream=sp)))
        calls.append(("gemv_quant_add", api.GemvQuantAddArgs(
            y=y_d.data_ptr(), weights=L["down"].data_ptr(),
            weights_device=L["down"].data_ptr(), ggml_type=12, x=x_f.data_ptr(),
            residual=res.data_ptr(), M=HIDDEN, K=FFN, stream=sp)))
    fns = {name: api._fn(name) for name in {c[0] for c in calls}}
    import ctypes
    bound = [(fns[n], ctypes.byref(a)) for n, a in calls]

    def step():
        for f, a in bound:
            s = f(a)
            if s != 0:
                raise RuntimeError(f"API call failed with status {s}: {capi.last_error()}")

    # algorithmic bytes of one step
    step_bytes = 0
    step_bytes += N_LAYERS * (qbytes(sum(QKV), HIDDEN) + 2 * HIDDEN + 2 * sum(QKV))
    step_bytes += N_LAYERS * (qbytes(HIDDEN, HIDDEN) + 2 * HIDDEN + 2 * HIDDEN + 2 * HIDDEN)
    step_bytes += N_LAYERS * (qbytes(2 * FFN, HIDDEN) + 2 * HIDDEN + 2 * 2 * FFN)
    step_bytes += N_LAYERS * (qbytes(HIDDEN, FFN) + 2 * FFN + 2 * HIDDEN + 2 * HIDDEN)

    with torch.cuda.stream(stream):
        step()  # eager warm-up (also caches device properties)
    torch.cuda.synchronize()

    graph = None
    if not args.eager:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream, capture_error_mode="relaxed"):
            step()
        torch.cuda.synchronize()

    def run_once():
        if graph is not None:
            graph.replay()
        else:
            step()

    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            run_once()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        ev0.record(stream)
        for _ in range(args.steps):
            run_once()
        ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = wall * 1e3 / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"decode36: {ms_per_step:.3f} ms/step (events {gpu_ms / args.steps:.3f}), "
        f"{value:.1f} GB/s = {100 * value / HBM_PEAK_GBS:.1f}% of 8 TB/s")

    # eager time for reference
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        for _ in range(3):
            step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / 3

    # ------------------------------------------------ per-kernel durations
    def per_launch(launch, n, reps=5):
        """Duration of one `launch(i)` as the decode graph issues it: n
        launches (distinct weights) captured in a HIP graph on `stream`,
        replayed 10 times untimed (the clock ramps over the first replays)
        and `reps` times between events recorded on `stream`; returns the
        median and mean over the timed replays of elapsed / n, in us."""
        with torch.cuda.stream(stream):
            for i in range(3):
                launch(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream, capture_error_mode="relaxed"):
            for i in range(n):
                launch(i)
        with torch.cuda.stream(stream):
            for _ in range(10):
                g.replay()
        torch.cuda.synchronize()
        d = []
        for _ in range(reps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(stream):
                e0.record(stream)
                g.replay()
                e1.record(stream)
            torch.cuda.synchronize()
            d.append(e0.elapsed_time(e1) * 1e3 / n)
        del g
        return float(np.median(d)), float(np.mean(d))

    kernels = {}
    R = 72
    rows_multi = lambda ws: [(w[0], w[1], w[2]) for w in ws]  # noqa: E731

    def gu_launch(i):
        L = layers[i % N_LAYERS]
        g = L["gu"]
        capi.gemv_multi_f16([(y_gu[:FFN], g[:FFN], FFN), (y_gu[FFN:], g[FFN:], FFN)], x_h,
                            HIDDEN, stream=sp)

    med, mean = per_launch(gu_launch, R)
    gu_bytes = qbytes(2 * FFN, HIDDEN) + 2 * HIDDEN + 2 * 2 * FFN
    kernels["gate_up_pair_22016x2048"] = {"us": round(med, 3), "GBps": round(gu_bytes / med / 1e3, 1)}
    traffic, traffic_src = measured_traffic()
    roofline = {"bound": "hbm", "achieved": round(gu_bytes / med / 1e3, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(gu_bytes / med / 1e3 / HBM_PEAK_GBS, 4),
                "traffic": traffic, "traffic_source": traffic_src,
                "kernel": "gemv_stream_kernel<32,F16,1,4,1,prefetch> (gate+up pair)",
                "bytes_per_launch": gu_bytes, "us_per_launch": round(med, 3),
                "us_mean": round(mean, 3),
                "timing": "72 launches on distinct layers in a HIP graph, replayed 5 times between "
                          "HIP events on the launch stream; median of elapsed/72 (the kernel trace "
                          "of `bench.py --leg gate_up --graph` averages the same kernel within 1%)"}

    # O and QKV: 36 layers are 85 / 106 MB, which the Infinity Cache could
    # hold across replays; extra copies take each rotation past 512 MB
    o_ws = [L["o"] for L in layers] + [qweights(90_000 + i, HIDDEN, HIDDEN) for i in range(184)]
    qkv_ws = [L["qkv"] for L in layers] + [qweights(91_000 + i, sum(QKV), HIDDEN)
                                           for i in range(144)]

    def qkv_launch(i):
        q = qkv_ws[i % len(qkv_ws)]
        capi.gemv_multi_f16([(y_qkv[:2048], q[:2048], 2048), (y_qkv[2048:2304], q[2048:2304], 256),
                             (y_qkv[2304:], q[2304:], 256)], x_h, HIDDEN, stream=sp)
    med, _ = per_launch(qkv_launch, len(qkv_ws))
    b = qbytes(2560, HIDDEN) + 2 * HIDDEN + 2 * 2560
    kernels["qkv_triple_2560x2048"] = {"us": round(med, 3), "GBps": round(b / med / 1e3, 1)}

    def o_launch(i):
        capi.gemv_add_f16(y_o, o_ws[i % len(o_ws)], x_a, res, HIDDEN, HIDDEN, stream=sp)
    med, _ = per_launch(o_launch, len(o_ws))
    b = qbytes(HIDDEN, HIDDEN) + 6 * HIDDEN
    kernels["o_add_2048x2048"] = {"us": round(med, 3), "GBps": round(b / med / 1e3, 1)}

    def d_launch(i):
        capi.gemv_add_f16(y_d, layers[i % N_LAYERS]["down"], x_f, res, HIDDEN, FFN, stream=sp)
    med, _ = per_launch(d_launch, R)  # 36 layers: 457 MB, and replays cycle 72 launches
    b = qbytes(HIDDEN, FFN) + 2 * FFN + 4 * HIDDEN
    kernels["down_add_2048x11008"] = {"us": round(med, 3), "GBps": round(b / med / 1e3, 1)}

    # ------------------------------------------------ launch / read floors
    # What the box gives any kernel: an empty kernel per graph launch, the
    # sustained read ceiling (a persistent grid-stride read of one 2 GiB
    # buffer, the best of a small sweep of grid sizes, with and without the
    # nontemporal bit), and the fill / nontemporal write rates.  A decode
    # projection of B bytes cannot take less than empty + B / ceiling.
    import ctypes
    flib = ctypes.CDLL(os.path.join(ROOT, "reflex-infer_amd", "lib", "librxq4_floors.so"))
    flib.rxq4_floor_empty.argtypes = [ctypes.c_void_p]
    flib.rxq4_floor_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    flib.rxq4_floor_write.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_void_p]
    floors = {}
    med, _ = per_launch(lambda i: flib.rxq4_floor_empty(sp), R)
    floors["empty_kernel_us"] = round(med, 3)
    big = torch.empty(2 << 30, dtype=torch.uint8, device=dev)
    big.fill_(1)
    sink = torch.empty(1 << 16, dtype=torch.int32, device=dev)
    sweep = {}
    for nt in (0, 1):
        for blocks in (256, 512, 1024):
            med, _ = per_launch(lambda i: flib.rxq4_floor_stream(big.data_ptr(), 2 << 30, sink.data_ptr(),
                                                                 blocks, 4, nt, sp), 3)
            sweep[f"nt{nt}_b{blocks}"] = round((2 << 30) / med / 1e3, 1)
    best = max(sweep, key=sweep.get)
    ceiling = sweep[best]
    floors["stream_read_2GiB"] = {"bytes": 2 << 30, "GBps": ceiling,
                                  "pct_of_peak": round(100 * ceiling / HBM_PEAK_GBS, 1),
                                  "kernel": f"persistent grid-stride read, {best}", "sweep_GBps": sweep}
    med, _ = per_launch(lambda i: big.fill_(i & 7), 3)
    floors["fill_2GiB_GBps"] = round((2 << 30) / med / 1e3, 1)
    med, _ = per_launch(lambda i: flib.rxq4_floor_write(big.data_ptr(), 2 << 30, 256, 1, sp), 3)
    floors["write_nt_2GiB_GBps"] = round((2 << 30) / med / 1e3, 1)
    del big, sink
    # every decode projection against empty + bytes / ceiling; "launch" where
    # the launch alone costs more than streaming the bytes at the ceiling
    for name, nbytes in (("qkv_triple_2560x2048", qbytes(sum(QKV), HIDDEN)),
                         ("o_add_2048x2048", qbytes(HIDDEN, HIDDEN)),
                         ("gate_up_pair_22016x2048", qbytes(2 * FFN, HIDDEN)),
                         ("down_add_2048x11008", qbytes(HIDDEN, FFN))):
        stream_us = nbytes / ceiling / 1e3
        k = kernels[name]
        k["floor_us"] = round(floors["empty_kernel_us"] + stream_us, 3)
        k["of_floor"] = round(k["floor_us"] / k["us"], 3)
        k["bound"] = "launch" if floors["empty_kernel_us"] > stream_us else "hbm"
    log(f"floors: {floors}")

    extras = {"floors": floors}
    table_host = ids_np = uniq = None
    if not args.no_extras:
        # LM head: three tables in rotation, so a table is read again only
        # after 350 MB of others have passed the 256 MB Infinity Cache.
        log("LM head / embedding / GEMM extras")
        heads = [qweights(20_000 + i, VOCAB, HIDDEN) for i in range(3)]
        logits = torch.empty(VOCAB, dtype=torch.float32, device=dev)

        def lm_launch(i):
            capi.gemv_f32(logits, heads[i % 3], x_h, VOCAB, HIDDEN, stream=sp)
        med, _ = per_launch(lm_launch, 72)
        b = qbytes(VOCAB, HIDDEN) + 2 * HIDDEN + 4 * VOCAB
        kernels["lm_head_f32_151936x2048"] = {"us": round(med, 3), "GBps": round(b / med / 1e3, 1)}

        # Embedding gather: 4096 Zipf(1.1) ids over the vocabulary.
        rng = np.random.default_rng(5)
        ranks = np.arange(1, VOCAB + 1, dtype=np.float64)
        cdf = np.cumsum(ranks ** -1.1)
        cdf /= cdf[-1]
        perm = rng.permutation(VOCAB)
        ids_np = perm[np.minimum(np.searchsorted(cdf, rng.random(4096)), VOCAB - 1)].astype(np.int32)
        ids = torch.from_numpy(ids_np).to(dev)
        emb = torch.empty((4096, HIDDEN), dtype=torch.float16, device=dev)

        def emb_launch(i):
            capi.embed_rows_f16(emb, heads[i % 3], VOCAB, ids, HIDDEN, stream=sp)
        med, _ = per_launch(emb_launch, 72)
        uniq = int(np.unique(ids_np).size)
        table_host = heads[0].cpu().numpy() if not args.no_cpu_baseline else None
        b = uniq * qbytes(1, HIDDEN) + 4096 * HIDDEN * 2 + 4096 * 4
        kernels["embed_gather_4096_zipf"] = {"us": round(med, 3), "GBps": round(b / med / 1e3, 1),
                                             "unique_rows": uniq}
        del heads

        # Q6_K (ggml type 14): LM head, embedding gather and ffn_down as a
        # Q4_K_M file stores them, and the Qwen3-4B-style mixed QKV triple
        # (Q4_K q, k + Q6_K v), on weights from ggml's reference quantiser.
        def q6_blocks(seed, rows, K):
            return qweights(seed, rows, K, ggml_type=14)

        q6b = lambda rows, K: rows * (K // 256) * 210  # noqa: E731
        heads6 = [q6_blocks(60_000 + i, VOCAB, HIDDEN) for i in range(3)]  # 574 MB

        def lm6_launch(i):
            capi.gemv_f32(logits, heads6[i % 3], x_h, VOCAB, HIDDEN, stream=sp, ggml_type=14)
        med, _ = per_launch(lm6_launch, 72)
        b = q6b(VOCAB, HIDDEN) + 2 * HIDDEN + 4 * VOCAB
        kernels["q6k_lm_head_f32_151936x2048"] = {"us": round(med, 3), "GBps": round(b / med / 1e3, 1)}

        def emb6_launch(i):
            capi.embed_rows_f16(emb, heads6[i % 3], VOCAB, ids, HIDDEN, stream=sp, ggml_type=14)
        med, _ = per_launch(emb6_launch, 72)
        b = uniq * q6b(1, HIDDEN) + 4096 * HIDDEN * 2 + 4096 * 4
        kernels["q6k_embed_gather_4096_zipf"] = {"us": round(med, 3), "GBps": round(b / med / 1e3, 1)}
        del heads6

        downs6 = [q6_blocks(61_000 + i, HIDDEN, FFN) for i in range(36)]  # 558 MB

        def d6_launch(i):
            capi.gemv_add_f16(y_d, downs6[i % 36], x_f, res, HIDDEN, FFN, stream=sp, ggml_type=14)
        med, _ = per_launch(d6_launch, 72)
        b = q6b(HIDDEN, FFN) + 2 * FFN + 4 * HIDDEN
        kernels["q6k_down_add_2048x11008"] = {"us": round(med, 3), "GBps": round(b / med / 1e3, 1)}
        del downs6

        vs6 = [q6_blocks(62_000 + i, 256, HIDDEN) for i in range(8)]

        def mixed_launch(i):
            q = layers[i % N_LAYERS]["qkv"]
            capi.gemv_multi_f16([(y_qkv[:2048], q[:2048], 2048), (y_qkv[2048:2304], q[2048:2304], 256),
                                 (y_qkv[2304:], vs6[i % 8], 256, 14)], x_h, HIDDEN, stream=sp)
        med, _ = per_launch(mixed_launch, 40)
        b = qbytes(2304, HIDDEN) + q6b(256, HIDDEN) + 2 * HIDDEN + 2 * 2560
        kernels["qkv_q4q4q6_2560x2048"] = {"us": round(med, 3), "GBps": round(b / med / 1e3, 1),
                                           "launches": 1}
        del vs6

        # Attention (decode at 4096 positions, prefill of 512 tokens) with
        # Qwen3-4B-like heads: 32 query heads, 8 KV heads, head_dim 128.
        AH, AKV, AD = 32, 8, 128
        # 36 K/V pairs of 16.8 MB (604 MB)
        caches = [(gen(70_000 + i, (4096, AKV, AD), 1.0).half(), gen(71_000 + i, (4096, AKV, AD), 1.0).half())
                  for i in range(36)]
        qa = gen(72_000, (AH * AD,), 1.0).half()
        oa = torch.empty(AH * AD, dtype=torch.float16, device=dev)

        def attn_launch(i):
            k, v = caches[i % 36]
            capi.attention_decode_f16(oa, qa, k, v, AH, AKV, AD, 4096, AD ** -0.5, stream=sp)
        med, _ = per_launch(attn_launch, 72)
        b = 2 * 4096 * AKV * AD * 2
        kernels["attn_decode_fp16_4096"] = {"us": round(med, 3), "GBps": round(b / med / 1e3, 1)}
        qp = gen(73_000, (512, AH * AD), 1.0).half()
        op = torch.empty_like(qp)

        def prefill_launch(i):
            k, v = caches[i % 36]
            capi.attention_prefill_f16(op, qp, k, v, AH, AKV, AD, 512, 0, AD ** -0.5, stream=sp)
        med, _ = per_launch(prefill_launch, 72)
        fl = 4.0 * AH * AD * sum(t + 1 for t in range(512))
        kernels["attn_prefill_fp16_512"] = {"us": round(med, 3), "TFLOPs": round(fl / med / 1e6, 2)}
        del caches
        # Reference point outside the path: the framework's fused causal
        # attention on the same problem (torch SDPA restricted to its flash
        # backend, which raises rather than fall back; K/V expanded to the
        # 32 query heads, its GQA form), timed the same way.
        try:
            from torch.nn.attention import SDPBackend, sdpa_kernel
            vq = [gen(76_000 + i, (1, AH, 512, AD), 1.0).half() for i in range(8)]
            vkv = [tuple(gen(s0 + i, (1, AKV, 512, AD), 1.0).half()
                         .repeat_interleave(AH // AKV, dim=1).contiguous() for s0 in (77_000, 78_000))
                   for i in range(8)]

            def sdpa_launch(i):
                k, v = vkv[i % 8]
                torch.nn.functional.scaled_dot_product_attention(vq[i % 8], k, v, is_causal=True)
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
                med, _ = per_launch(sdpa_launch, 72)
            extras["vendor_sdpa_prefill_512"] = {"us": round(med, 3), "TFLOPs": round(fl / med / 1e6, 2)}
            del vq, vkv
        except Exception as ex:  # no flash backend on this build: report, do not fall back
            extras["vendor_sdpa_prefill_512"] = {"unavailable": f"{type(ex).__name__}: {str(ex)[:120]}"}
        # 9 K/V pairs of 67 MB (604 MB)
        long_kv = [(gen(74_000 + i, (16384, AKV, AD), 1.0).half(), gen(75_000 + i, (16384, AKV, AD), 1.0).half())
                   for i in range(9)]

        def attn_long(i):
            k, v = long_kv[i % 9]
            capi.attention_decode_f16(oa, qa, k, v, AH, AKV, AD, 16384, AD ** -0.5, stream=sp)
        med, _ = per_launch(attn_long, 72)
        b = 2 * 16384 * AKV * AD * 2
        kernels["attn_decode_fp16_16384"] = {"us": round(med, 3), "GBps": round(b / med / 1e3, 1)}
        del long_kv

        # Small-batch decode: m tokens through
        # gemm_quant_batched's C-ABI form with fp16 x / y on the decode
        # set's gate+up and down weights (distinct layers per launch).
        small = {}
        for name, key, M, K in (("gate_up", "gu", 2 * FFN, HIDDEN), ("down", "down", HIDDEN, FFN)):
            for m in (1, 2, 4, 8, 16):
                xs_m = gen(50_000 + m + K, (m, K), 1.0).half()
                ys_m = torch.empty((m, M), dtype=torch.float16, device=dev)

                def sb_launch(i, xs_m=xs_m, ys_m=ys_m, key=key, M=M, K=K, m=m):
                    capi.gemm_f16(ys_m, layers[i % N_LAYERS][key], xs_m, M, m, K, stream=sp)
                med, _ = per_launch(sb_launch, N_LAYERS)
                b = qbytes(M, K) + m * K * 2 + m * M * 2
                small[f"{name}_{M}x{K}_m{m}"] = {"us": round(med, 3), "GBps": round(b / med / 1e3, 1),
                                                 "GFLOPs": round(2 * m * M * K / med / 1e3, 1)}
        extras["small_batch_decode"] = small

        # Prefill GEMM at m = 512 and 2048 (bf16
        # activations, bf16 out).
        for (M, K) in ((FFN, HIDDEN), (HIDDEN, FFN)):
            ws = [qweights(30_000 + M + i, M, K) for i in range(42)]  # 533 MB
            for m in (512, 2048):
                xb = gen(40_000 + K + m, (m, K), 1.0).to(torch.bfloat16)
                yb = torch.empty((m, M), dtype=torch.bfloat16, device=dev)

                def gm_launch(i, xb=xb, yb=yb, m=m):
                    capi.gemm(yb, ws[i % 42], xb, M, m, K, stream=sp)
                med, _ = per_launch(gm_launch, 42 if m == 512 else 21)
                tf = 2 * m * M * K / med / 1e6
                kernels[f"gemm_bf16_m{m}_{M}x{K}"] = {"us": round(med, 3), "TFLOPs": round(tf, 1),
                                                      "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)}
                del xb, yb
            del ws
        extras["gemm_m512_tflops"] = min(v["TFLOPs"] for k, v in kernels.items()
                                         if k.startswith("gemm_bf16_m512"))
        # The same prefill GEMM on Q6_K and Q5_K weights (Q4_K_M files keep
        # some FFN and V tensors in these formats).
        for t, tname in ((14, "q6k"), (13, "q5k")):
            for (M, K) in ((FFN, HIDDEN), (HIDDEN, FFN)):
                ws = [qweights(31_000 + M + i, M, K, ggml_type=t) for i in range(36)]
                xb = gen(41_000 + K, (512, K), 1.0).to(torch.bfloat16)
                yb = torch.empty((512, M), dtype=torch.bfloat16, device=dev)

                def kq_launch(i, ws=ws, xb=xb, yb=yb, M=M, K=K, t=t):
                    capi.gemm(yb, ws[i % 36], xb, M, 512, K, stream=sp, ggml_type=t)
                med, _ = per_launch(kq_launch, 36)
                tf = 2 * 512 * M * K / med / 1e6
                kernels[f"{tname}_gemm_bf16_m512_{M}x{K}"] = {"us": round(med, 3), "TFLOPs": round(tf, 1)}
                del ws
        # Reference point outside the path: the vendor library's dense bf16
        # GEMM (2-D torch.mm, hipBLASLt) on the same shapes,
        # weights already bf16 (no dequantisation) and laid out like the
        # Q4_K rows ([M x K], the library's faster layout of the two: [K x M]
        # measured 43 / 76 us at m = 512); copies rotate over > 512 MB.
        vendor = {}
        for (M, K) in ((FFN, HIDDEN), (HIDDEN, FFN)):
            n_w = max(2, -(-600_000_000 // (M * K * 2)))
            wts = [gen(32_000 + M + i, (M, K), 0.02).to(torch.bfloat16) for i in range(n_w)]
            for m in (512, 2048):
                xb = gen(42_000 + K + m, (m, K), 1.0).to(torch.bfloat16)
                yb = torch.empty((m, M), dtype=torch.bfloat16, device=dev)

                def vd_launch(i, xb=xb, yb=yb):
                    torch.mm(xb, wts[i % n_w].t(), out=yb)
                med, _ = per_launch(vd_launch, 2 * n_w)
                tf = 2 * m * M * K / med / 1e6
                vendor[f"m{m}_{M}x{K}"] = {"us": round(med, 3), "TFLOPs": round(tf, 1),
                                           "q4k_gemm_us": kernels[f"gemm_bf16_m{m}_{M}x{K}"]["us"]}
                del xb, yb
            del wts
        extras["vendor_bf16_gemm"] = vendor

    # ------------------------------------------------------- CPU baseline
    cpu = None
    cpu_cfg = None
    if not args.no_cpu_baseline:
        from oracle import oracle as orc
        log("CPU baseline: oracle restatement of gemv_quant_cpu, 1 thread, median of 5")
        xs = {HIDDEN: x_h.cpu().numpy().view(np.uint16), FFN: x_f.cpu().numpy().view(np.uint16)}
        hostw = [{k: v.cpu().numpy() for k, v in L.items()} for L in layers]

        def median_s(fn, runs=5):
            t = []
            for _ in range(runs):
                t0 = time.perf_counter()
                fn()
                t.append(time.perf_counter() - t0)
            return float(np.median(t))

        def step_cpu():
            for L in hostw:
                orc.gemv_f32(L["qkv"], HIDDEN, xs[HIDDEN])
                orc.gemv_f32(L["o"], HIDDEN, xs[HIDDEN])
                orc.gemv_f32(L["gu"], HIDDEN, xs[HIDDEN])
                orc.gemv_f32(L["down"], FFN, xs[FFN])
        cpu_s = median_s(step_cpu)
        host = host_cpu()
        cpu = {"value": round(step_bytes / cpu_s / 1e9, 3), "unit": "GB/s", "cores": 1,
               "kind": "port",
               "sample": "full 36-layer decode set (one step), fp32 outputs, single thread, "
                         f"median of 5: {cpu_s:.3f} s; host {host['model']}, "
                         f"{host['nproc']} cores visible",
               "ms_per_step": round(cpu_s * 1e3, 1)}
        log(f"CPU baseline {cpu['value']} GB/s ({cpu_s:.2f} s per step)")
        cpu_cfg = {"host": host, "threads": 1, "runs": 5, "statistic": "median",
                   "kind": "port (oracle/q4k_oracle.c, the reference gemv_quant_cpu loop)"}
        # W[2048 x 2048], x fp32 -> fp16, y fp32
        w1 = hostw[0]["o"]
        t = median_s(lambda: orc.gemv_f32(w1, HIDDEN, xs[HIDDEN]))
        b = qbytes(HIDDEN, HIDDEN) + 2 * HIDDEN + 4 * HIDDEN
        cpu_cfg["cfg1_gemv_2048x2048"] = {"us": round(t * 1e6, 1), "GBps": round(b / t / 1e9, 3)}
        # m independent GEMVs (the reference's batched host path
        # is per-token GEMV, q4_gemm.cu:1735-1739)
        cfg3 = {}
        for name, key, M, K in (("gate_up", "gu", 2 * FFN, HIDDEN), ("down", "down", HIDDEN, FFN)):
            W = hostw[0][key]
            for m in (1, 2, 4, 8, 16):
                xm = np.random.default_rng(60 + m).standard_normal((m, K)).astype(np.float16).view(np.uint16)
                t = median_s(lambda: orc.gemm_tokens_f32(W, K, xm))
                b = qbytes(M, K) + m * K * 2 + m * M * 2
                cfg3[f"{name}_{M}x{K}_m{m}"] = {"us": round(t * 1e6, 1), "GBps": round(b / t / 1e9, 3)}
        cpu_cfg["cfg3_small_batch"] = cfg3
        # a 16-token subset, extrapolated linearly to m tokens
        cfg4 = {}
        for M, K, key in ((FFN, HIDDEN, None), (HIDDEN, FFN, "down")):
            W = hostw[0]["down"] if key else hostw[0]["gu"][:FFN]
            x16 = np.random.default_rng(70).standard_normal((16, K)).astype(np.float16).view(np.uint16)
            t16 = median_s(lambda: orc.gemm_tokens_f32(W, K, x16))
            for m in (512, 2048):
                t = t16 * m / 16
                cfg4[f"gemm_m{m}_{M}x{K}"] = {"us": round(t * 1e6, 1),
                                              "GFLOPs": round(2 * m * M * K / t / 1e9, 3),
                                              "measured_tokens": 16, "extrapolated": True}
        cpu_cfg["cfg4_prefill_gemm"] = cfg4
        # embedding gather (restated row dequant; the reference
        # has no CPU embedding path) and the LM head GEMV, full size
        if table_host is not None:
            t = median_s(lambda: orc.embed_rows_f16(table_host, HIDDEN, ids_np))
            b = uniq * qbytes(1, HIDDEN) + 4096 * HIDDEN * 2 + 4096 * 4
            cpu_cfg["cfg5a_embed_gather_4096"] = {"us": round(t * 1e6, 1),
                                                  "GBps": round(b / t / 1e9, 3)}
            t = median_s(lambda: orc.gemv_f32(table_host, HIDDEN, xs[HIDDEN]))
            b = qbytes(VOCAB, HIDDEN) + 2 * HIDDEN + 4 * VOCAB
            cpu_cfg["cfg5b_lm_head_151936x2048"] = {"us": round(t * 1e6, 1),
                                                    "GBps": round(b / t / 1e9, 3)}
        log(f"CPU per-config baseline done ({host['model']})")

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "decode36: 36 layers x {QKV triple [2048|256|256]x2048, O add "
                        "[2048x2048], gate+up pair [11008|11008]x2048, down add [2048x11008]}, "
                        "Q4_K weights = ggml reference quantisation of N(0,0.02), fp16 N(0,1) activations, M=1, fp32 acc, fp16 out",
            "launches_per_step": len(calls),
            "bytes_per_step": step_bytes,
            "issue": "eager" if graph is None else "hip_graph",
        },
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "eager_ms_per_step": round(eager_ms, 4),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_baseline_per_config": cpu_cfg,
        "per_kernel": kernels,
    }
    out.update(extras)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
