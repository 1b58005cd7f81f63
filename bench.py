"""Decode benchmark of the quantized-linear hot path on one MI355X.

Workload (the headline metric's configuration): batch-1 greedy decode of a
Qwen3-4B-shaped Fish s2-pro slow AR -- 36 layers, dim 2560, 32/8 heads x 128,
SwiGLU 9728, tied 155776-row head, every projection Q4_K -- with an f32 KV cache
prefilled to 1024 positions (N(0,1)), generating `--steps` tokens (default 256).
Weights are random N(0, 0.02) quantized with Candle's from_float (synthetic data).

A step is one decode token (embedding -> 36 layers -> head -> argmax fed back on the
device), replayed as a captured HIP graph.  `value` is tokens per second over the
timed steps.  `roofline` is the Q4_K GEMV family (every projection of a token,
launched back to back over 2.27 GB of weights, captured as a HIP graph like the decode
step and replayed; the eager-launch time is reported beside it) timed with HIP events
on the stream the kernels run on: algorithmic bytes (weight blocks + activations + outputs) per
launch over the average launch duration, against 8 TB/s.  `cpu_baseline` times the
oracle (the CPU restatement of Candle's quantized matmul) on one layer's projections
plus the head, on this host's cores, and scales it to one token's GEMV work.

`roofline.traffic` is the HBM bytes per GEMV launch that rocprofv3's FETCH_SIZE and
WRITE_SIZE counters report for the same GEMV pass (read from the committed summary
under profiles/, whose header gives the commands and the copy-kernel scale factor).

`prefill` is a second line in the same object: one Qwen3-4B layer's four projections
(wqkv, wo, w1|w3, w2; Q4_K) applied to a 512-token prompt through QMatMul.forward, i.e.
the f16 MFMA GEMM including its conversion of x and split-K sums, captured as a HIP
graph and replayed (the eager time is reported beside it), against the 2.5 PFLOP/s
dense f16 MFMA peak.

`skinny_batch` is a third line: 16 concurrent streams decoding at once with ragged
KV lengths drawn uniformly from 256..2048 (the GEMVs run 16 activation rows, attention
and the KV append run per stream), tokens per second over all streams.

Usage: python bench.py [--gpus 1] [--steps 256] [--warmup 16] [--dtype q4k|q8_0] [--no-cpu] [--no-prefill] [--skinny-batch 16|0]
       python bench.py --model cv2 --dtype q8_0 --kv 512   (the CosyVoice2 Qwen2-0.5B LM decode step)
       python bench.py --mode gemv [--gemv-iters N]   (GEMV pass only, for counter runs)
       python bench.py --mode copy                     (plain 1 GiB device copy, the counter scale)
       python bench.py --mode prefill                  (the prefill line alone)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--dtype", default="q4k", choices=["q4k", "q8_0"])
    ap.add_argument("--model", default="fish", choices=["fish", "cv2"],
                    help="fish: the Qwen3-4B-shaped slow AR (the headline); cv2: the CosyVoice2 Qwen2-0.5B LM "
                         "(24 layers, dim 896; pass --dtype q8_0 --kv 512 for its configuration)")
    ap.add_argument("--kv", type=int, default=1024)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--gemv-iters", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--mode", default="decode", choices=["decode", "gemv", "copy", "prefill"],
                    help="decode: the benchmark; gemv: only the per-token GEMV pass (for counter runs); "
                         "copy: a plain device copy of known size (the counter scale); prefill: the "
                         "512-token prefill GEMMs of one Qwen3-4B layer on MFMA")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill-GEMM line of the decode bench")
    ap.add_argument("--prefill-tokens", type=int, default=512)
    ap.add_argument("--prefill-iters", type=int, default=20)
    ap.add_argument("--skinny-batch", type=int, default=16,
                    help="streams of the skinny-batch line (ragged KV lengths uniform over 256..2048); 0 skips it")
    ap.add_argument("--skinny-steps", type=int, default=64)
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_gemv2_q4k_qwen3_4b_decode_traffic.txt")


def measured_traffic():
    """HBM bytes per GEMV launch from the committed counter summary (None if absent)."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def gemv_roofline(lm, torch, iters):
    """Average duration of the GEMV launches of one token (all 36 layers + head)."""
    dev = lm.device
    from syrinx_amd._lib import check, lib
    import ctypes
    s = torch.cuda.current_stream(dev)
    n_launch = 4 * lm.cfg.n_layers + 1
    layer_b, head_b = lm.weight_bytes()
    # algorithmic bytes per token of GEMV: weight blocks + f32 outputs + activation blocks
    c = lm.cfg
    qkv_n = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim
    outs = 4 * (qkv_n + c.dim + 2 * c.intermediate + c.dim) * c.n_layers + 4 * c.vocab
    act_blk = 292 if c.weight_dtype == 12 else 34
    bs = 256 if c.weight_dtype == 12 else 32
    acts = act_blk * ((2 * c.dim + c.n_heads * c.head_dim + c.intermediate) // bs * c.n_layers + c.dim // bs)
    algo = layer_b + head_b + outs + acts
    for _ in range(2):
        check(lib().sxq_lm_gemv_pass(lm._h, 1, 1, ctypes.c_void_p(s.cuda_stream)))
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # eager launches (reported alongside): each launch adds the host-queue dispatch cost
    e0.record(s)
    for _ in range(iters):
        check(lib().sxq_lm_gemv_pass(lm._h, 1, 1, ctypes.c_void_p(s.cuda_stream)))
    e1.record(s)
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / iters
    # the measured pass: the same launches captured once as a HIP graph and replayed, as
    # the decode step runs them
    graph = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream(dev)
    cs.wait_stream(s)
    with torch.cuda.graph(graph, stream=cs):
        check(lib().sxq_lm_gemv_pass(lm._h, 1, 1, ctypes.c_void_p(cs.cuda_stream)))
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
    avg_us = ms * 1000.0 / n_launch
    achieved = algo / (ms * 1e-3) / 1e9
    traffic = measured_traffic() if c.weight_dtype == 12 else None
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None if traffic is None else round(traffic),
            "algorithmic_bytes_per_launch": round(algo / n_launch),
            "kernel": "k_gemv2_q4k" if c.weight_dtype == 12 else "k_gemv2_q80",
            "bytes_per_token": algo, "launches_per_token": n_launch, "avg_launch_us": round(avg_us, 3),
            "gemv_us_per_token": round(ms * 1000.0, 2), "replay": "hip graph",
            "eager_gemv_us_per_token": round(eager_ms * 1000.0, 2)}


def cpu_threads():
    """The host cores this process may use, capped at 16 (one GPU's share of the host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_baseline(lm, torch, budget_s=12.0):
    """Oracle (CPU port of Candle's quantized matmul) on whole tokens' GEMV work.

    One token = the four projections 36 times (layer 0's weights stand in for every
    layer: 57 MB per layer, far beyond the host caches) + the head; tokens are run until
    `budget_s` seconds have passed (at least one)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle  # the CPU oracle, timed as the CPU baseline
    from syrinx_amd import GgmlDType, QTensor
    c = lm.cfg
    dt = GgmlDType(c.weight_dtype)
    dev = lm.device
    rng = np.random.default_rng(0)
    qkv_n = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim
    shapes = [(qkv_n, c.dim), (c.dim, c.n_heads * c.head_dim), (2 * c.intermediate, c.dim), (c.dim, c.intermediate)]
    blocks = []
    g = torch.Generator(device=dev).manual_seed(1)
    for n, k in shapes + [(c.vocab, c.dim)]:
        w = torch.randn(n, k, device=dev, generator=g) * 0.02
        blocks.append((k, QTensor.quantize(w, dt).data().cpu().numpy().reshape(n, -1)))
        del w
    xs = {k: rng.standard_normal((1, k)).astype(np.float32) for k, _ in blocks}
    threads = cpu_threads()
    tokens = 0
    t0 = time.perf_counter()
    while tokens == 0 or time.perf_counter() - t0 < budget_s:
        for _ in range(c.n_layers):
            for k, b in blocks[:4]:
                oracle.matmul(int(dt), xs[k], b, threads=threads)
        k, b = blocks[4]
        oracle.matmul(int(dt), xs[k], b, threads=threads)
        tokens += 1
    total = time.perf_counter() - t0
    return {"value": round(tokens / total, 3), "unit": "tok/s (GEMV share of a token)", "cores": threads,
            "kind": "port",
            "sample": f"{tokens} tokens of GEMV work ({c.n_layers} x layer-0's four projections + the head, "
                      f"batch 1) through the oracle's k_quants::matmul (generic vec-dot, {threads} threads) "
                      f"in {total:.1f} s"}


MFMA_F16_PEAK_TFLOPS = 2500.0  # dense f16/bf16 MFMA, MI355X


def prefill_gemms(torch, tokens, iters):
    """One Qwen3-4B layer's projections at a `tokens`-row prompt through QMatMul.forward
    (Q4_K weights, the f16 MFMA prefill GEMM incl. its f16 conversion of x)."""
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
    # the measured layer: the same four forwards captured once as a HIP graph and
    # replayed, as the decode step runs (the eager time is reported beside it)
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
    return {"workload": f"Qwen3-4B layer projections (wqkv, wo, w1|w3, w2) at M={tokens}, Q4_K weights, "
                        "f16 MFMA with f32 accumulation",
            "us_per_layer": round(ms * 1000.0, 2), "flops_per_layer": flops, "achieved": round(tflops, 1),
            "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "replay": "hip graph", "eager_us_per_layer": round(eager_ms * 1000.0, 2),
            "ms_36_layers": round(36 * ms, 3)}


SKINNY_KV = (256, 2048)


def skinny_batch(lm, torch, n, steps, warmup):
    """Greedy decode of n concurrent streams whose KV caches hold ragged lengths drawn
    uniformly from 256..2048 (seeded): the GEMVs see n activation rows, attention and the
    KV append run per stream at its own position."""
    import random
    rng = random.Random(5)
    lengths = [rng.randint(*SKINNY_KV) for _ in range(n)]
    lm.kv_fill_random([SKINNY_KV[1]] * n, seed=2)
    frame = torch.zeros((n, 1 + lm.cfg.n_codebooks), dtype=torch.int32)
    frame[:, 0] = 151700
    frame[:, 1:] = (torch.arange(n, dtype=torch.int32)[:, None] * 11 + torch.arange(lm.cfg.n_codebooks)) * 37 % 4096
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
    return {"workload": f"{n} concurrent streams, Qwen3-4B shape, Q4_K, ragged KV lengths uniform over "
                        f"{SKINNY_KV[0]}..{SKINNY_KV[1]} (seed 5), {steps} steps",
            "value": round(n * steps / (ms / 1000.0), 2), "unit": "tok/s (all streams)",
            "ms_per_step": round(ms / steps, 4), "kv_lengths": lengths}


def copy_calibration(torch, iters=8):
    """A plain device-to-device copy of 1 GiB: its counters give the FETCH/WRITE scale."""
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"mode": "copy", "bytes_read_per_copy": n, "bytes_written_per_copy": n, "copies": iters}))


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the GEMVs would shard "
              "by output rows, one shard per GPU)", file=sys.stderr)
        sys.exit(2)
    import torch
    if args.mode == "copy":
        copy_calibration(torch)
        return
    if args.mode == "prefill":
        print(json.dumps({"mode": "prefill", "prefill": prefill_gemms(torch, args.prefill_tokens, args.prefill_iters)}))
        return
    from syrinx_amd import GgmlDType
    from syrinx_amd import decoder as D

    dev = torch.device("cuda:0")
    dt = GgmlDType.Q4K if args.dtype == "q4k" else GgmlDType.Q8_0
    skinny = args.skinny_batch if args.mode == "decode" and args.model == "fish" else 0
    max_seq = max(args.kv, SKINNY_KV[1] if skinny else 0) + max(args.steps, args.skinny_steps) + args.warmup + 8
    t0 = time.time()
    if args.model == "cv2":
        cfg = D.cosyvoice2_lm_config(n_layers=24, max_seq=max_seq, max_batch=args.batch, dtype=dt)
        lm = D.Qwen2Lm(cfg, device=dev)
    else:
        cfg = D.fish_s2_slow_ar_config(n_layers=36, max_seq=max_seq, max_batch=max(args.batch, skinny), dtype=dt)
        lm = D.SlowAr(cfg, device=dev)
    lm.init_random(seed=0, std=0.02)
    lm.kv_fill_random([args.kv] * args.batch, seed=1)
    print(f"[bench] model ready in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    if args.mode == "gemv":
        roof = gemv_roofline(lm, torch, args.gemv_iters)
        print(json.dumps({"mode": "gemv", "passes": 2 * (args.gemv_iters + 2), "roofline": roof}))
        return
    rng_frame = torch.zeros((args.batch, lm.ids_per), dtype=torch.int32)
    rng_frame[:, 0] = 151700 if args.model == "fish" else 100
    rng_frame[:, 1:] = torch.arange(lm.ids_per - 1, dtype=torch.int32) * 37 % 4096
    lm.step(ids=rng_frame, graph=True)  # captures the graph
    for _ in range(args.warmup):
        lm.step(n=args.batch, graph=True, want_logits=False)
    torch.cuda.synchronize()
    lm.set_lengths([args.kv] * args.batch)
    lm.step(ids=rng_frame, graph=True, want_logits=False)
    lm.set_lengths([args.kv] * args.batch)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_host0 = time.perf_counter()
    e0.record(s)
    for _ in range(args.steps):
        lm.step(n=args.batch, graph=True, want_logits=False)
    e1.record(s)
    torch.cuda.synchronize()
    t_host = time.perf_counter() - t_host0
    ms = e0.elapsed_time(e1)
    ms_per_step = ms / args.steps
    tok_s = args.batch * args.steps / (ms / 1000.0)
    print(f"[bench] {args.steps} steps in {ms:.1f} ms ({ms_per_step * 1000:.1f} us/token, host {t_host * 1000:.1f} ms)",
          file=sys.stderr, flush=True)
    roof = gemv_roofline(lm, torch, args.gemv_iters)
    print(f"[bench] GEMV: {roof['gemv_us_per_token']} us/token, {roof['achieved']} GB/s", file=sys.stderr, flush=True)
    skinny_line = skinny_batch(lm, torch, skinny, args.skinny_steps, args.warmup) if skinny else None
    cpu = None if args.no_cpu else cpu_baseline(lm, torch)
    prefill = None
    if not args.no_prefill and args.model == "fish":
        prefill = prefill_gemms(torch, args.prefill_tokens, args.prefill_iters)
        print(f"[bench] prefill: {prefill['us_per_layer']} us/layer, {prefill['achieved']} TFLOP/s", file=sys.stderr,
              flush=True)
    out = {
        "metric": "decode tok/s Qwen3-4B-shape Q4_K bs=1; quant-GEMV HBM GB/s as % of peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("q4k-weight x q8k-activation int dot, f32" if dt == GgmlDType.Q4K
                  else "q8_0-weight x q8_0-activation int dot, f32"),
        "data": "synthetic (random N(0,0.02) weights quantized by from_float; KV N(0,1))",
        "config": {"workload": (f"Fish s2-pro slow AR (Qwen3-4B shape) greedy decode" if args.model == "fish" else
                                f"CosyVoice2 LM (Qwen2-0.5B shape) greedy decode") +
                               f", {args.dtype.upper()} projections, batch {args.batch}, f32 KV prefilled to "
                               f"{args.kv}, {args.steps} tokens",
                   "n_layers": cfg.n_layers, "dim": cfg.dim,
                   "heads": f"{cfg.n_heads}/{cfg.n_kv_heads}x{cfg.head_dim}", "intermediate": cfg.intermediate,
                   "vocab": cfg.vocab, "kv_len": args.kv, "batch": args.batch, "graph": True},
        "roofline": roof,
        "cpu_baseline": cpu,
        "prefill": prefill,
        "skinny_batch": skinny_line,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
