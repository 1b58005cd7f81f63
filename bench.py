"""Benchmark of the quantized-linear hot path on one MI355X, every configuration in one run.

Headline (the `value` of the JSON line): batch-1 greedy decode of a Qwen3-4B-shaped Fish
s2-pro slow AR -- 36 layers, dim 2560, 32/8 heads x 128, SwiGLU 9728, tied 155776-row
head, every projection Q4_K -- with an f32 KV cache prefilled to 1024 positions (N(0,1)),
generating `--steps` tokens.  Weights are random N(0, 0.02) quantized with Candle's
from_float (synthetic data).  A step is one decode token (embedding -> 36 layers -> head
-> argmax fed back on the device), replayed as a captured HIP graph; `value` is tokens
per second over the timed steps.

`roofline` is the headline's dominant kernel family, the Q4_K decode GEMV: every
projection of a token launched back to back over 2.27 GB of weights, captured as a HIP
graph like the decode step and replayed, timed with HIP events on the stream the kernels
run on: algorithmic bytes (weight blocks + activation blocks + f32 outputs) per launch
over the average launch duration, against 8 TB/s.  `roofline.traffic` is the HBM bytes
per launch that rocprofv3's FETCH_SIZE / WRITE_SIZE report for the same pass (read from
the committed summary under profiles/, which gives the commands and the copy-kernel
scale factor).

The other configurations are objects in the same line, each with its own roofline and
CPU baseline:
  gemv_q8_0     one Q8_0 GEMV [4864 x 896] (the Qwen2-0.5B MLP up-projection) per
                QMatMul call, 64 weight copies rotated (296 MB > the 256 MB MALL);
  cv2_decode    the CosyVoice2 LM (Qwen2-0.5B shape, 24 layers, Q8_0, KV 512) decode;
  q8_0_decode   the headline model with Q8_0 projections;
  prefill       one Qwen3-4B layer's four projections at a 512-token prompt through
                QMatMul.forward (the f16 MFMA GEMM with its conversion of x and split-K
                sums), graph-replayed, against the 2.5 PFLOP/s dense f16 peak;
  skinny_batch  16 concurrent streams, ragged KV lengths uniform over 256..2048;
  fish_frame    Fish s2-pro dual-AR frames at batch 1: the slow step + the semantic draw +
                the 4-layer fast AR's 10 codebook positions with nine device draws;
  cv_generate   CosyVoice2 speech-token generation (Qwen2Lm::generate) on the device: the
                assembled prompt prefilled, then per token the RAS draw and the decode step
                on the drawn id, 24 layers, Q8_0.

CPU baselines (`cpu_baseline`: all threads this GPU's share of the host allows, at most
16; `cpu_baseline_1thread`): the oracle -- the CPU restatement of Candle 0.8's generic
quantized matmul (per-row activation quantization, then a vec-dot per output on a pool
of threads over output columns) -- on a bounded sample of each workload, median of 20
timed iterations after 3 warm-ups, scaled to the workload's unit as each `sample` says.

Usage: python bench.py [--gpus 1] [--steps 256] [--warmup 16] [--no-cpu] [--only LINE,...]
       python bench.py --mode gemv [--dtype q4k|q8_0] [--gemv-iters N] [--rows N]   (GEMV pass, counter runs)
       python bench.py --mode copy        (plain 1 GiB device copy: the counter scale)
       python bench.py --mode prefill     (the prefill line alone)
       python bench.py --mode frame [--frames N]   (the fish_frame line alone)
       python bench.py --mode decode1     (only the headline decode, for kernel traces)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense f16/bf16 MFMA, MI355X
Q4K, Q8_0 = 12, 8
LINES = ("gemv_q8_0", "cv2_decode", "q8_0_decode", "prefill", "skinny_batch", "fish_frame", "cv_generate")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--dtype", default="q4k", choices=["q4k", "q8_0"], help="--mode gemv only")
    ap.add_argument("--rows", type=int, default=1, help="--mode gemv: activation rows (streams)")
    ap.add_argument("--kv", type=int, default=1024)
    ap.add_argument("--gemv-iters", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--only", default=",".join(LINES), help="comma-separated extra lines to run")
    ap.add_argument("--mode", default="decode",
                    choices=["decode", "decode1", "gemv", "copy", "prefill", "frame", "generate", "hash"])
    ap.add_argument("--prefill-tokens", type=int, default=512)
    ap.add_argument("--prefill-iters", type=int, default=20)
    ap.add_argument("--skinny-batch", type=int, default=16)
    ap.add_argument("--skinny-steps", type=int, default=64)
    ap.add_argument("--frames", type=int, default=64, help="fish_frame line: timed frames")
    ap.add_argument("--gen-tokens", type=int, default=256, help="cv_generate line: generated tokens")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------------ CPU baseline helpers
def cpu_threads():
    """Threads for the all-cores CPU baseline: the cores this process may use, at most 16
    (one GPU's share of the host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_median(fn, iters=20, warm=3):
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_entry(value, unit, threads, sample):
    return {"value": round(value, 4), "unit": unit, "cores": threads, "kind": "port", "cpu_model": cpu_model(),
            "host_logical_cores": os.cpu_count(), "sample": sample}


def oracle_mod():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle  # the CPU oracle, timed as the CPU baseline
    return oracle


def quantized_blocks(torch, dev, n, k, dt, seed):
    """Random N(0, 0.02) [n, k] weights quantized on the GPU, as host canonical blocks."""
    from syrinx_amd import GgmlDType, QTensor
    g = torch.Generator(device=dev).manual_seed(seed)
    w = torch.randn(n, k, device=dev, generator=g) * 0.02
    b = QTensor.quantize(w, GgmlDType(dt)).data().cpu().numpy().reshape(n, -1)
    del w
    return b


def cpu_layer_token(torch, dev, cfg, dt, head_rows_div, label, rows=(1, 1)):
    """tok/s of one step's GEMV work on the CPU: median time of one layer's projections
    (as the reference calls them) x n_layers + the head (timed on 1/head_rows_div of its
    rows, scaled up), at all threads (rows[0] activation rows) and at 1 thread (rows[1]);
    tokens per second = rows / step time."""
    import numpy as np
    ora = oracle_mod()
    hd, nh, nkv = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    if cfg.qkv_bias:  # Qwen2: q, k, v, o, gate, up, down as separate QMatMuls
        shapes = [(nh * hd, cfg.dim), (nkv * hd, cfg.dim), (nkv * hd, cfg.dim), (cfg.dim, nh * hd),
                  (cfg.intermediate, cfg.dim), (cfg.intermediate, cfg.dim), (cfg.dim, cfg.intermediate)]
    else:            # Fish: fused wqkv, wo, w1, w3, w2
        shapes = [((nh + 2 * nkv) * hd, cfg.dim), (cfg.dim, nh * hd), (cfg.intermediate, cfg.dim),
                  (cfg.intermediate, cfg.dim), (cfg.dim, cfg.intermediate)]
    mats = [(k, quantized_blocks(torch, dev, n, k, dt, 11 + i)) for i, (n, k) in enumerate(shapes)]
    head_rows = cfg.vocab // head_rows_div
    head = quantized_blocks(torch, dev, head_rows, cfg.dim, dt, 99)
    rng = np.random.default_rng(0)
    out = {}
    for key, th, m in (("cpu_baseline", cpu_threads(), rows[0]), ("cpu_baseline_1thread", 1, rows[1])):
        xs = {k: rng.standard_normal((m, k)).astype(np.float32) for k, _ in mats}
        xh = rng.standard_normal((m, cfg.dim)).astype(np.float32)
        t_layer = cpu_median(lambda: [ora.matmul(dt, xs[k], b, threads=th) for k, b in mats])
        t_head = cpu_median(lambda: ora.matmul(dt, xh, head, threads=th)) * head_rows_div
        tok = m / (cfg.n_layers * t_layer + t_head)
        out[key] = cpu_entry(tok, "tok/s (GEMV share of a step)", th,
                             f"{label}: one layer's {len(mats)} projections at {m} activation row{'s' if m > 1 else ''} "
                             f"(median of 20 after 3 warm-ups: {t_layer * 1e3:.2f} ms) x {cfg.n_layers} layers + the "
                             f"head timed on {head_rows} of its {cfg.vocab} rows and scaled ({t_head * 1e3:.2f} ms), "
                             f"through the oracle's k_quants::matmul (generic vec-dot, {th} thread{'s' if th > 1 else ''})")
    return out


# ------------------------------------------------------------------ GPU measurements
def gemv_roofline(lm, torch, iters, rows=1):
    """Average duration of the GEMV launches of one step (every layer's four projections
    + the head) at `rows` activation rows, graph-replayed, timed with HIP events."""
    import ctypes
    from syrinx_amd._lib import check, lib
    s = torch.cuda.current_stream(lm.device)
    c = lm.cfg
    n_launch = 4 * c.n_layers + 1
    layer_b, head_b = lm.weight_bytes()
    qkv_n = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim
    outs = rows * (4 * (qkv_n + c.dim + 2 * c.intermediate + c.dim) * c.n_layers + 4 * c.vocab)
    act_blk = 292 if c.weight_dtype == Q4K else 34
    bs = 256 if c.weight_dtype == Q4K else 32
    acts = rows * act_blk * ((2 * c.dim + c.n_heads * c.head_dim + c.intermediate) // bs * c.n_layers + c.dim // bs)
    algo = layer_b + head_b + outs + acts

    def one(stream):
        check(lib().sxq_lm_gemv_pass(lm._h, rows, 1, ctypes.c_void_p(stream.cuda_stream)))

    for _ in range(2):
        one(s)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(iters):
        one(s)
    e1.record(s)
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / iters
    graph = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream(lm.device)
    cs.wait_stream(s)
    with torch.cuda.graph(graph, stream=cs):
        one(cs)
    s.wait_stream(cs)
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    e0.record(s)
    for _ in range(iters):
        graph.replay()
    e1.record(s)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / iters
    achieved = algo / (ms * 1e-3) / 1e9
    kernel = ("k_gemv_mma_q4k_rec" if rows > 4 else "k_gemv2_q4k") if c.weight_dtype == Q4K else "k_gemv2_q80"
    # counters were collected for the 16-row Qwen3-4B-shape pass (the skinny-batch line) and
    # for the one-row Q8_0 passes of the CosyVoice2 and Qwen3-4B shapes
    traffic, path = None, None
    if kernel == "k_gemv_mma_q4k_rec" and rows == 16 and c.dim == 2560 and c.n_layers == 36:
        path = SKINNY_TRAFFIC_FILE
    elif kernel == "k_gemv2_q80" and rows == 1 and c.dim == 896 and c.n_layers == 24:
        path = CV2_TRAFFIC_FILE
    elif kernel == "k_gemv2_q80" and rows == 1 and c.dim == 2560 and c.n_layers == 36:
        path = Q80_TRAFFIC_FILE
    if path:
        t = measured_traffic(path, kernel)
        traffic = None if t is None else round(t)
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "algorithmic_bytes_per_launch": round(algo / n_launch), "kernel": kernel, "rows": rows,
            "bytes_per_step": algo, "launches_per_step": n_launch, "avg_launch_us": round(ms * 1000.0 / n_launch, 3),
            "gemv_us_per_step": round(ms * 1000.0, 2), "replay": "hip graph",
            "eager_gemv_us_per_step": round(eager_ms * 1000.0, 2)}


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_gemv2_q4k_qwen3_4b_decode_traffic.txt")
SKINNY_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_gemv_mma_q4k_rec_qwen3_4b_16stream_traffic.txt")
CV2_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_gemv2_q80_qwen2_0_5b_decode_traffic.txt")
Q80_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_gemv2_q80_qwen3_4b_decode_traffic.txt")

# The sources each measured kernel is built from: a counter summary records their hash,
# and a summary whose hash differs from the sources in this tree is stale (not reported).
_CSRC = os.path.join(ROOT, "syrinx_amd", "csrc")
_COMMON = ("sxq_common.h", "sxq_kernels.h", "sxq_quant_dev.h", "sxq_sync_dev.h")
KERNEL_SOURCES = {
    "k_gemv2_q4k": ("sxq_gemv.hip", "sxq_gemv_dev.h") + _COMMON,
    "k_gemv_mma_q4k_rec": ("sxq_gemv.hip", "sxq_gemv_dev.h") + _COMMON,
    "k_gemv2_q80": ("sxq_gemv.hip", "sxq_gemv_dev.h") + _COMMON,
    "k_gemm_q4k": ("sxq_gemm.hip",) + _COMMON,
}


def kernel_sources_sha256(kernel):
    import hashlib
    h = hashlib.sha256()
    for name in KERNEL_SOURCES[kernel]:
        with open(os.path.join(_CSRC, name), "rb") as f:
            h.update(name.encode() + b"\0" + f.read())
    return h.hexdigest()


def measured_traffic(path=TRAFFIC_FILE, kernel="k_gemv2_q4k"):
    """HBM bytes per GEMV launch from a committed counter summary, or None when the
    summary is missing or was measured on other kernel sources than this tree's."""
    vals = {}
    try:
        with open(path) as f:
            for line in f:
                k, sep, v = line.partition(":")
                if sep and k in ("traffic_bytes_per_launch", "kernel_sources_sha256"):
                    vals[k] = v.strip()
    except OSError:
        return None
    if vals.get("kernel_sources_sha256") != kernel_sources_sha256(kernel):
        log(f"{os.path.basename(path)}: measured on other {kernel} sources than these; traffic not reported")
        return None
    return float(vals["traffic_bytes_per_launch"]) if "traffic_bytes_per_launch" in vals else None


def timed_decode(lm, torch, frame, kv, steps, warmup, batch=1):
    """Greedy decode from a KV cache holding `kv` positions: graph-replayed steps timed
    with HIP events on the stream they run on.  Returns ms per step."""
    lm.step(ids=frame, graph=True)  # captures the graph
    for _ in range(warmup):
        lm.step(n=batch, graph=True, want_logits=False)
    lm.set_lengths([kv] * batch)
    lm.step(ids=frame, graph=True, want_logits=False)
    lm.set_lengths([kv] * batch)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream(lm.device)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(steps):
        lm.step(n=batch, graph=True, want_logits=False)
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def fish_frame(lm, torch, n=1):
    f = torch.zeros((n, lm.ids_per), dtype=torch.int32)
    f[:, 0] = 151700
    f[:, 1:] = (torch.arange(n, dtype=torch.int32)[:, None] * 11 + torch.arange(lm.ids_per - 1)) * 37 % 4096
    return f


def q8_0_gemv(torch, cpu, copies=64, reps=20):
    """Config 1: one Q8_0 GEMV [4864 x 896] per QMatMul.forward (one launch: the GEMV
    quantizes x in its prologue), 64 weight copies rotated so the weights stream from HBM,
    not the MALL."""
    from syrinx_amd import GgmlDType, QMatMul, QTensor
    dev = torch.device("cuda:0")
    n, k = 4864, 896
    g = torch.Generator(device=dev).manual_seed(0)
    mats = []
    for _ in range(copies):
        w = torch.randn(n, k, device=dev, generator=g) * 0.02
        mats.append(QMatMul.from_qtensor(QTensor.quantize(w, GgmlDType.Q8_0)))
    x = torch.randn(1, k, device=dev, generator=g)
    ys = [q.forward(x) for q in mats]  # eager warm-up
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.current_stream(dev)
    cs = torch.cuda.Stream(dev)
    cs.wait_stream(s)
    with torch.cuda.graph(graph, stream=cs):
        ys = [q.forward(x) for q in mats]
    s.wait_stream(cs)
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        graph.replay()
    e1.record(s)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / (reps * copies)
    algo = n * (k // 32) * 34 + 4 * k + 4 * n  # weight blocks + f32 x + f32 y (4,653,568 B)
    gbs = algo / (us * 1e-6) / 1e9
    out = {"workload": f"one Q8_0 GEMV [{n} x {k}] (Qwen2-0.5B MLP up-projection) per QMatMul.forward, x [1 x {k}] "
                       f"N(0,1), weights N(0,0.02), {copies} weight copies rotated ({copies * n * (k // 32) * 34 / 1e6:.0f} MB)"
                       ", graph-replayed",
           "value": round(gbs, 1), "unit": "GB/s", "us_per_call": round(us, 3), "bytes_per_call": algo,
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                        "kernel": "k_gemv2_q80 (quantizing x in its prologue, one launch per call)"}}
    if cpu:
        import numpy as np
        ora = oracle_mod()
        blocks = mats[0].export_blocks().cpu().numpy().reshape(n, -1)
        xh = x.cpu().numpy()
        for key, th in (("cpu_baseline", cpu_threads()), ("cpu_baseline_1thread", 1)):
            t = cpu_median(lambda: ora.matmul(Q8_0, xh, blocks, threads=th))
            out[key] = cpu_entry(algo / t / 1e9, "GB/s", th,
                                 f"the same GEMV through the oracle's k_quants::matmul ({th} thread"
                                 f"{'s' if th > 1 else ''}), median of 20 after 3 warm-ups: {t * 1e6:.1f} us per call")
    out["host_ptr_drop_in"] = host_ptr_drop_in(torch)
    return out


def host_ptr_drop_in(torch, reps=20):
    """The per-projection drop-in with host buffers (SXQ_HOST_PTRS: x and y copied through
    pageable host memory, one synchronisation per call), PCIe-inclusive: the 169 QMatMul
    calls of one CosyVoice2 (Qwen2-0.5B, 24 layers, Q8_0) decode token -- q, k, v, o,
    gate, up, down per layer and the head -- from numpy buffers, median of `reps` tokens.
    Only the projections: the glue stays on the caller's CPU in this integration."""
    import numpy as np
    from syrinx_amd import GgmlDType, QMatMul, QTensor
    from syrinx_amd.quantized import qmatmul_host
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(5)
    dim, kvd, inter, vocab = 896, 128, 4864, 6564
    shapes = [(dim, dim), (kvd, dim), (kvd, dim), (dim, dim), (inter, dim), (inter, dim), (dim, inter)]
    layers = []
    for _ in range(24):
        layers.append([QMatMul.from_qtensor(QTensor.quantize(torch.randn(n, k, device=dev, generator=g) * 0.02,
                                                             GgmlDType.Q8_0)) for n, k in shapes])
    head = QMatMul.from_qtensor(QTensor.quantize(torch.randn(vocab, dim, device=dev, generator=g) * 0.02,
                                                 GgmlDType.Q8_0))
    rng = np.random.default_rng(5)
    xs = {k: rng.standard_normal((1, k)).astype(np.float32) for k in (dim, inter)}

    def token():
        for mats in layers:
            for q, (n, k) in zip(mats, shapes):
                qmatmul_host(q, xs[k])
        qmatmul_host(head, xs[dim])

    for _ in range(3):
        token()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        token()
        ts.append(time.perf_counter() - t0)
    t = float(np.median(ts))
    calls = 24 * len(shapes) + 1
    return {"workload": f"{calls} QMatMul.forward calls of one CosyVoice2 Q8_0 decode token (24 layers x q,k,v,o,"
                        "gate,up,down + head) with host (numpy) x and y via SXQ_HOST_PTRS, median of "
                        f"{reps} tokens", "us_per_token": round(t * 1e6, 1), "us_per_call": round(t * 1e6 / calls, 2),
            "tok_s_projection_share": round(1.0 / t, 1)}


def prefill_gemms(torch, tokens, iters, cpu=False):
    """Config 4: one Qwen3-4B layer's projections at a `tokens`-row prompt through
    QMatMul.forward (Q4_K weights, the f16 MFMA prefill GEMM incl. its f16 conversion)."""
    from syrinx_amd import GgmlDType, QMatMul, QTensor
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(3)
    shapes = [(6144, 2560), (2560, 4096), (2 * 9728, 2560), (2560, 9728)]  # wqkv, wo, w1|w3, w2
    mats, xs = [], []
    for n, k in shapes:
        w = torch.randn(n, k, device=dev, generator=g) * 0.02
        mats.append(QMatMul.from_qtensor(QTensor.quantize(w, GgmlDType.Q4K)))
        xs.append(torch.randn(tokens, k, device=dev, generator=g))
        del w
    flops = 2.0 * tokens * sum(n * k for n, k in shapes)
    for _ in range(3):
        for q, x in zip(mats, xs):
            q.forward(x)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(iters):
        for q, x in zip(mats, xs):
            q.forward(x)
    e1.record(s)
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / iters
    graph = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream(dev)
    cs.wait_stream(s)
    with torch.cuda.graph(graph, stream=cs):
        for q, x in zip(mats, xs):
            q.forward(x)
    s.wait_stream(cs)
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    e0.record(s)
    for _ in range(iters):
        graph.replay()
    e1.record(s)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / iters
    tflops = flops / (ms * 1e-3) / 1e12
    out = {"workload": f"Qwen3-4B layer projections (wqkv, wo, w1|w3, w2) at M={tokens}, Q4_K weights, "
                       "f16 MFMA with f32 accumulation",
           "us_per_layer": round(ms * 1000.0, 2), "flops_per_layer": flops, "value": round(tflops, 1),
           "unit": "TFLOP/s", "achieved": round(tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
           "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
           "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None,
                        "kernel": "k_gemm_q4k (+ k_x_to_f16_perm, k_gemm_splitk_sum)"},
           "replay": "hip graph", "eager_us_per_layer": round(eager_ms * 1000.0, 2),
           "ms_36_layers": round(36 * ms, 3)}
    if cpu:
        import numpy as np
        ora = oracle_mod()
        blocks = [(k, m.export_blocks().cpu().numpy().reshape(n, -1)) for (n, k), m in zip(shapes, mats)]
        rng = np.random.default_rng(1)
        for key, th, rows in (("cpu_baseline", cpu_threads(), 16), ("cpu_baseline_1thread", 1, 2)):
            xr = {k: rng.standard_normal((rows, k)).astype(np.float32) for k, _ in blocks}
            t = cpu_median(lambda: [ora.matmul(Q4K, xr[k], b, threads=th) for k, b in blocks])
            t_layer = t * tokens / rows  # the CPU path's cost is linear in the rows
            out[key] = cpu_entry(flops / t_layer / 1e12, "TFLOP/s", th,
                                 f"one layer's four projections at {rows} prompt rows through the oracle's "
                                 f"k_quants::matmul ({th} thread{'s' if th > 1 else ''}; per-row activation "
                                 f"quantization + a vec-dot per output, cost linear in the rows), median of 20 after "
                                 f"3 warm-ups ({t * 1e3:.1f} ms), scaled to {tokens} rows: "
                                 f"{t_layer * 1e3:.0f} ms per layer")
    return out


SKINNY_KV = (256, 2048)


def skinny_batch(lm, torch, n, steps, warmup, iters, cpu):
    """Config 5: greedy decode of n concurrent streams whose KV caches hold ragged lengths
    drawn uniformly from 256..2048 (seeded): the GEMVs see n activation rows, attention
    and the KV append run per stream at its own position."""
    import random
    rng = random.Random(5)
    lengths = [rng.randint(*SKINNY_KV) for _ in range(n)]
    lm.kv_fill_random([SKINNY_KV[1]] * n, seed=2)
    frame = fish_frame(lm, torch, n)
    lm.set_lengths(lengths)
    lm.step(ids=frame, graph=True, want_logits=False)  # captures the n-stream graph
    for _ in range(warmup):
        lm.step(n=n, graph=True, want_logits=False)
    lm.set_lengths(lengths)
    lm.step(ids=frame, graph=True, want_logits=False)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream(lm.device)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(steps):
        lm.step(n=n, graph=True, want_logits=False)
    e1.record(s)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    kv_bytes = 294912 * sum(L + steps // 2 for L in lengths)  # f32 K and V read per step, mid-run lengths
    out = {"workload": f"{n} concurrent streams, Qwen3-4B shape, Q4_K, ragged KV lengths uniform over "
                       f"{SKINNY_KV[0]}..{SKINNY_KV[1]} (seed 5), {steps} steps",
           "value": round(n * steps / (ms / 1000.0), 2), "unit": "tok/s (all streams)",
           "ms_per_step": round(ms / steps, 4), "kv_lengths": lengths, "kv_bytes_per_step": kv_bytes,
           "roofline": gemv_roofline(lm, torch, iters, rows=n)}
    if cpu:
        # all threads at the full 16 rows; one thread at 2 rows (the CPU path's cost is
        # linear in the rows: every row runs its own vec-dots over all the weights)
        out.update(cpu_layer_token(torch, lm.device, lm.cfg, Q4K, 16, f"{n} streams", rows=(n, 2)))
    return out


def fish_frames(D, torch, kv, frames, warmup, cpu, n=1):
    """Fish s2-pro dual-AR frames at batch n: per frame the slow AR step (36 layers, KV
    `kv`), the semantic draw, and the 4-layer fast AR over the 10 codebook positions with
    nine codebook draws, all on the device (syrinx_amd.dualar.generate_frames, the loop
    drive / drive_batch run: one graph per slow step and one per expansion, the host
    reading the streams' stop flags once per frame behind the next slow step).  Timed by
    the host clock around the loop (it synchronises with the host every frame)."""
    from syrinx_amd import dualar as DA
    from syrinx_amd.sampling import FishSampler, SamplingParams
    dev = torch.device("cuda:0")
    slow = build_model(D, torch, "fish", Q4K, kv + frames + warmup + 8, n)
    fast = D.FastAr(D.fish_s2_fast_ar_config(n_layers=4, max_batch=n), device=dev)
    fast.init_random(seed=3, std=0.02)
    slow.kv_fill_random([kv] * n, seed=1)
    logits, _, hidden = slow.step(ids=fish_frame(slow, torch, n), graph=True, want_hidden=True)
    smp = FishSampler([42 + i for i in range(n)], SamplingParams(), semantic=(151678, 155773, -1), device=dev)
    frame = torch.zeros((n, 1 + slow.cfg.n_codebooks), dtype=torch.int32, device=dev)
    active = torch.ones(n, dtype=torch.int32, device=dev)
    DA.generate_frames(slow, fast, smp, logits, hidden.reshape(n, 1, -1), warmup, kv + 1, active, frame)  # captures
    slow.set_lengths([kv + 1] * n)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out, _ = DA.generate_frames(slow, fast, smp, logits, hidden.reshape(n, 1, -1), frames, kv + 1, active, frame)
    sec = time.perf_counter() - t0
    assert len(out) == frames
    sl, sh = slow.weight_bytes()
    fl, fh = fast.weight_bytes()
    per_frame = sl + sh + fast.cfg.max_seq * (fl + fh)  # weight bytes streamed per frame
    achieved = per_frame * frames / sec / 1e9
    res = {"workload": f"Fish s2-pro dual-AR frames: slow AR (Qwen3-4B shape, 36 layers, Q4_K, f32 KV {kv}) + "
                       f"semantic draw + fast AR (4 layers of the same block, Q4_K, 10 codebook positions, nine "
                       f"codebook draws), batch {n}, {frames} frames",
           "value": round(n * frames / sec, 2), "unit": "frames/s", "ms_per_frame": round(sec * 1000.0 / frames, 4),
           "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                        "bytes_per_frame": per_frame, "kernel": "whole frame (weights streamed once per step)"}}
    if cpu:
        a = cpu_layer_token(torch, dev, slow.cfg, Q4K, 16, "slow AR")
        b = cpu_layer_token(torch, dev, fast.cfg, Q4K, 1, "fast AR")
        for key in ("cpu_baseline", "cpu_baseline_1thread"):
            ts, tf = 1.0 / a[key]["value"], 1.0 / b[key]["value"]
            res[key] = cpu_entry(1.0 / (ts + fast.cfg.max_seq * tf), "frames/s (GEMV share of a frame)",
                                 a[key]["cores"], f"one slow-AR step + 10 fast-AR steps of GEMV work: "
                                 f"{a[key]['sample']}; {b[key]['sample']}")
    del slow, fast
    return res


def cv_generate(D, torch, tokens, cpu):
    """CosyVoice2 Qwen2Lm::generate on the device (syrinx_amd.generate): the step-0 input
    [sos, 64 text rows, task_id, 160 prompt-speech rows] prefilled, then `tokens` tokens,
    each a RAS draw on the device followed by a graph-replayed decode step on the drawn
    id (the stop ids masked throughout -- min_len = max_len -- so the length is fixed).
    Timed by the host clock around the whole call (prefill included; the loop reads one
    id per token)."""
    from syrinx_amd.generate import COSYVOICE2, CosyVoiceLm
    dev = torch.device("cuda:0")
    n_text, n_prompt = 64, 160
    lm = build_model(D, torch, "cv2", Q8_0, 2 + n_text + n_prompt + tokens + 8, 1)
    g = torch.Generator(device=dev).manual_seed(9)
    c = lm.cfg
    speech = torch.randn(c.embed_rows, c.dim, device=dev, generator=g) * 0.02
    lm.set_vector(-1, D.EMBED, speech)
    cv = CosyVoiceLm(lm, torch.randn(4096, c.dim, device=dev, generator=g) * 0.02, speech,
                     torch.randn(2, c.dim, device=dev, generator=g) * 0.02, COSYVOICE2)
    text = [(i * 37) % 4096 for i in range(n_text)]
    prompt = [(i * 53) % 6561 for i in range(n_prompt)]
    cv.generate(text, prompt, 16, 16, 1)  # warm-up: captures the step graph
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks = cv.generate(text, prompt, tokens, tokens, 1)
    sec = time.perf_counter() - t0
    assert len(toks) == tokens
    lb, hb = lm.weight_bytes()
    achieved = (lb + hb) * tokens / sec / 1e9
    out = {"workload": f"CosyVoice2 LM (Qwen2-0.5B shape, 24 layers, Q8_0) speech-token generation: step-0 input of "
                       f"{2 + n_text + n_prompt} rows prefilled, {tokens} tokens, each a device RAS draw (top_p 0.8, "
                       f"top_k 25, window 10) + a graph-replayed decode step on the drawn id",
           "value": round(tokens / sec, 2), "unit": "tok/s (prefill included)", "ms_per_token": round(sec * 1e3 / tokens, 4),
           "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "bytes_per_token": lb + hb,
                        "kernel": "whole token (weights streamed once per step)"}}
    if cpu:
        out.update(cpu_layer_token(torch, dev, c, Q8_0, 1, "CosyVoice2 Q8_0"))
    del cv, lm
    return out


def copy_calibration(torch, iters=8):
    """A plain device-to-device copy of 1 GiB: its counters give the FETCH/WRITE scale."""
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"mode": "copy", "bytes_read_per_copy": n, "bytes_written_per_copy": n, "copies": iters}))


def build_model(D, torch, kind, dtype, max_seq, max_batch):
    dev = torch.device("cuda:0")
    if kind == "cv2":
        lm = D.Qwen2Lm(D.cosyvoice2_lm_config(n_layers=24, max_seq=max_seq, max_batch=max_batch, dtype=dtype),
                       device=dev)
    else:
        lm = D.SlowAr(D.fish_s2_slow_ar_config(n_layers=36, max_seq=max_seq, max_batch=max_batch, dtype=dtype),
                      device=dev)
    lm.init_random(seed=0, std=0.02)
    return lm


def decode_line(D, torch, kind, dtype, kv, args, cpu, label):
    t0 = time.time()
    lm = build_model(D, torch, kind, dtype, kv + args.steps + args.warmup + 8, 1)
    lm.kv_fill_random([kv], seed=1)
    frame = fish_frame(lm, torch) if kind == "fish" else torch.tensor([[100]], dtype=torch.int32)
    ms = timed_decode(lm, torch, frame, kv, args.steps, args.warmup)
    roof = gemv_roofline(lm, torch, args.gemv_iters)
    c = lm.cfg
    out = {"workload": label, "value": round(1000.0 / ms, 2), "unit": "tok/s", "ms_per_step": round(ms, 4),
           "config": {"n_layers": c.n_layers, "dim": c.dim, "heads": f"{c.n_heads}/{c.n_kv_heads}x{c.head_dim}",
                      "intermediate": c.intermediate, "vocab": c.vocab, "kv_len": kv, "batch": 1, "graph": True},
           "roofline": roof}
    log(f"{label}: {out['value']} tok/s, GEMV {roof['gemv_us_per_step']} us ({roof['frac']:.3f}) "
        f"[{time.time() - t0:.1f}s]")
    if cpu:
        out.update(cpu_layer_token(torch, lm.device, c, dtype, 16 if kind == "fish" else 1, label))
    del lm
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the GEMVs would shard "
              "by output rows, one shard per GPU)", file=sys.stderr)
        sys.exit(2)
    if args.mode == "hash":
        print(json.dumps({k: kernel_sources_sha256(k) for k in KERNEL_SOURCES}))
        return
    import torch
    if args.mode == "copy":
        copy_calibration(torch)
        return
    if args.mode == "prefill":
        print(json.dumps({"mode": "prefill", "prefill": prefill_gemms(torch, args.prefill_tokens, args.prefill_iters)}))
        return
    from syrinx_amd import decoder as D
    cpu = not args.no_cpu
    if args.mode == "frame":
        print(json.dumps({"mode": "frame", "fish_frame": fish_frames(D, torch, args.kv, args.frames, 8, cpu)}))
        return
    if args.mode == "generate":
        print(json.dumps({"mode": "generate", "cv_generate": cv_generate(D, torch, args.gen_tokens, cpu)}))
        return
    if args.mode == "gemv":
        dt = Q4K if args.dtype == "q4k" else Q8_0
        lm = build_model(D, torch, "fish", dt, args.kv + 16, max(1, args.rows))
        lm.kv_fill_random([args.kv] * args.rows, seed=1)
        lm.step(ids=fish_frame(lm, torch, args.rows), graph=False, want_logits=False)  # fills the activation blocks
        roof = gemv_roofline(lm, torch, args.gemv_iters, rows=args.rows)
        print(json.dumps({"mode": "gemv", "passes": 2 * (args.gemv_iters + 2), "roofline": roof}))
        return
    only = set(x for x in args.only.split(",") if x) if args.mode == "decode" else set()
    skinny = args.skinny_batch if "skinny_batch" in only else 0

    # headline: Qwen3-4B shape, Q4_K, batch 1, KV 1024
    t0 = time.time()
    max_seq = max(args.kv, SKINNY_KV[1] if skinny else 0) + max(args.steps, args.skinny_steps) + args.warmup + 8
    lm = build_model(D, torch, "fish", Q4K, max_seq, max(1, skinny))
    lm.kv_fill_random([args.kv], seed=1)
    log(f"model ready in {time.time() - t0:.1f}s")
    ms = timed_decode(lm, torch, fish_frame(lm, torch), args.kv, args.steps, args.warmup)
    log(f"{args.steps} steps: {ms * 1000:.1f} us/token")
    if args.mode == "decode1":
        print(json.dumps({"mode": "decode1", "ms_per_step": ms}))
        return
    roof = gemv_roofline(lm, torch, args.gemv_iters)
    traffic = measured_traffic()
    roof["traffic"] = None if traffic is None else round(traffic)
    log(f"GEMV: {roof['gemv_us_per_step']} us/token, {roof['achieved']} GB/s")
    lines = {}
    if skinny:
        lines["skinny_batch"] = skinny_batch(lm, torch, skinny, args.skinny_steps, args.warmup, args.gemv_iters, cpu)
        log(f"skinny batch: {lines['skinny_batch']['value']} tok/s")
    cpu_head = cpu_layer_token(torch, lm.device, lm.cfg, Q4K, 16, "Qwen3-4B shape, Q4_K") if cpu else {}
    del lm
    if "q8_0_decode" in only:
        lines["q8_0_decode"] = decode_line(D, torch, "fish", Q8_0, args.kv, args, cpu,
                                           f"Fish s2-pro slow AR (Qwen3-4B shape) greedy decode, Q8_0 projections, "
                                           f"batch 1, f32 KV prefilled to {args.kv}, {args.steps} tokens")
    if "cv2_decode" in only:
        lines["cv2_decode"] = decode_line(D, torch, "cv2", Q8_0, 512, args, cpu,
                                          f"CosyVoice2 LM (Qwen2-0.5B shape, 24 layers) greedy decode, Q8_0 "
                                          f"projections, batch 1, f32 KV prefilled to 512, {args.steps} tokens")
    if "gemv_q8_0" in only:
        lines["gemv_q8_0"] = q8_0_gemv(torch, cpu)
        log(f"Q8_0 GEMV: {lines['gemv_q8_0']['value']} GB/s")
    if "fish_frame" in only:
        lines["fish_frame"] = fish_frames(D, torch, args.kv, args.frames, 8, cpu)
        log(f"fish frames: {lines['fish_frame']['value']} frames/s")
    if "cv_generate" in only:
        lines["cv_generate"] = cv_generate(D, torch, args.gen_tokens, cpu)
        log(f"cv generate: {lines['cv_generate']['value']} tok/s")
    if "prefill" in only:
        lines["prefill"] = prefill_gemms(torch, args.prefill_tokens, args.prefill_iters, cpu)
        log(f"prefill: {lines['prefill']['us_per_layer']} us/layer, {lines['prefill']['value']} TFLOP/s")
    out = {
        "metric": "decode tok/s Qwen3-4B-shape Q4_K bs=1; quant-GEMV HBM GB/s as % of peak",
        "value": round(1000.0 / ms, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4k-weight x q8k-activation int dot, f32",
        "data": "synthetic (random N(0,0.02) weights quantized by from_float; KV N(0,1))",
        "config": {"workload": f"Fish s2-pro slow AR (Qwen3-4B shape) greedy decode, Q4_K projections, batch 1, "
                               f"f32 KV prefilled to {args.kv}, {args.steps} tokens",
                   "n_layers": 36, "dim": 2560, "heads": "32/8x128", "intermediate": 9728, "vocab": 155776,
                   "kv_len": args.kv, "batch": 1, "graph": True},
        "roofline": roof,
        "cpu_baseline": cpu_head.get("cpu_baseline"),
        "cpu_baseline_1thread": cpu_head.get("cpu_baseline_1thread"),
    }
    out.update({k: lines.get(k) for k in LINES})
    print(json.dumps(out))


if __name__ == "__main__":
    main()
