#!/usr/bin/env python
"""Benchmark of the batch-invariant kernels on one MI355X.

Default workload: 4-bit affine quantized matmul at
the Llama-3-8B MLP shape, x bf16 [M, 4096] @ W[14336, 4096]^T with W packed
4-bit, group 64, bf16 scales/biases; the headline is the decode GEMV, M = 1.
A step is one call of the op on one batch. Weights are rotated over >= 512 MB
of distinct copies so every step streams them from HBM (the 256 MB Infinity
Cache would otherwise hold them). Time is measured with HIP events on the
stream the kernels run on.

    python bench.py [--steps K] [--warmup W] [--op qmm4|qmm8|linear|rmsnorm|decode|prefill|gemm|llama|all]

Prints one JSON line per op (the default op only, unless --op is given).
`value` is the achieved fraction of the op's roofline in percent (HBM 8 TB/s,
or dense bf16 MFMA 2.5 PFLOP/s for the MFMA-bound ops), computed from the
algorithmic bytes/flops of one call over the measured call time.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "mlx-batch-invariant_amd"):
    sys.path.insert(0, str(p))

PEAK_HBM = 8.0e12          # B/s, MI355X HBM3E
# HBM traffic of the headline kernel per launch, from two rocprofv3 counter
# passes (FETCH_SIZE, WRITE_SIZE, KiB per dispatch) scaled by the same counters
# on a 256 MiB device copy (bench.py --op copycal): read x 2.000, write x 1.000.
# Source: profiles/qmatmul4_g64_llama_mlp_m1.txt. Re-measure after changing
# the kernel.
MEASURED_TRAFFIC_QMM4_M1 = {"fetch_kib": 16210.5, "fetch_scale": 2.000, "write_kib": 28, "write_scale": 1.000}
PEAK_BF16 = 2.5e15         # FLOP/s, dense bf16 MFMA
METRIC = "% of HBM/MFMA roofline per op at batch 1–256, with bitwise batch invariance"
ROTATE_BYTES = 512 << 20


def _sync():
    import torch
    torch.cuda.synchronize()


def _time_calls(fn, n, warmup, rotate, graph=True, replays=3):
    """Per-call device time (s) of fn(i), i cycling over `rotate` weight copies.

    graph=True: the n calls are captured into one HIP graph (so the host's
    per-call launch cost cannot leave the GPU idle between kernels), the graph
    is replayed, and each replay is bracketed by HIP events on the stream the
    kernels run on; the result is replay time / n, once per replay.
    graph=False: events around each eagerly launched call."""
    import torch
    for i in range(warmup):
        fn(i % rotate)
    _sync()
    if graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn(0)                         # allocator warm-up on the capture stream
        torch.cuda.current_stream().wait_stream(s)
        _sync()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                fn(i % rotate)
        g.replay()
        _sync()
        out = []
        for _ in range(replays):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            g.replay()
            b.record()
            _sync()
            out.append(a.elapsed_time(b) * 1e-3 / n)
        del g
        return out
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for i in range(n):
        evs[i][0].record()
        fn((warmup + i) % rotate)
        evs[i][1].record()
    _sync()
    return [a.elapsed_time(b) * 1e-3 for a, b in evs]


def _bits(t):
    import torch
    return t.contiguous().view(torch.uint8).cpu().numpy().tobytes()


# ---- workloads ------------------------------------------------------------------

def qmm_bytes(M, N, K, bits, gs):
    return N * K * bits // 8 + 2 * 2 * N * (K // gs) + 2 * M * K + 2 * M * N


# The kernel the M = 1 call launches (bi_quantized_matmul's policy for K = 4096,
# bf16 x, N / 16 >= 512): the barrier-free stream GEMV, in the instance the
# group count and scale-slice alignment select.
HEADLINE_KERNEL = {
    (4, 64): "gemv_stream<bf16,4,64,W=8,NB=2,MR=1,PD=1> (bi_quantized_matmul, M <= 4: one launch)",
    (8, 128): "gemv_stream<bf16,8,128,W=4,NB=4,MR=1,PD=1> (bi_quantized_matmul, M <= 4: one launch)",
}


def bench_qmm(args, bits=4, gs=64, Ms=(1, 2, 4, 8, 16, 32, 64)):
    import torch
    import mlx_batch_invariant_amd as bi
    N, K = 14336, 4096
    g = torch.Generator().manual_seed(0)
    W = 0.02 * torch.randn((N, K), generator=g)
    wq, s, b = bi.quantize(W, group_size=gs, bits=bits, dtype=torch.bfloat16)
    del W
    per = qmm_bytes(1, N, K, bits, gs)
    ncopy = max(1, math.ceil(ROTATE_BYTES / per))
    copies = [(wq.cuda(), s.cuda(), b.cuda())]
    for _ in range(ncopy - 1):
        copies.append(tuple(t.clone() for t in copies[0]))
    xs = (torch.randn((max(Ms), K), generator=g)).to(torch.bfloat16).cuda()

    def call(M):
        return lambda i: bi.batch_invariant_quantized_matmul(xs[:M], *copies[i], group_size=gs, bits=bits)

    # headline M = 1: `steps` calls captured in one graph, replayed three times
    # (each replay times exactly `steps` calls; the median replay is reported).
    # Timed before the M sweep: after the larger-M launches the same M = 1 graph
    # reads ~1 us per call slower for its first few hundred calls, then recovers.
    _sync()
    t0 = time.perf_counter()
    if args.profile_m != 1:                # profiling aid: only the calls at that M, no report
        _time_calls(call(args.profile_m), args.steps, args.warmup, ncopy, replays=3)
        return {"metric": METRIC, "op": f"qmm{bits} profile run at M={args.profile_m}", "value": None}
    durs = _time_calls(call(1), args.steps, args.warmup, ncopy, replays=3)
    wall = time.perf_counter() - t0
    table = {}
    for M in (() if args.headline_only else Ms):
        t = statistics.median(_time_calls(call(M), args.steps, args.warmup, ncopy))
        by = qmm_bytes(M, N, K, bits, gs)
        table[M] = {"us": round(t * 1e6, 3), "GBps": round(by / t / 1e9, 1),
                    "frac_hbm": round(by / t / PEAK_HBM, 4)}
    if args.headline_only:
        eager = stock_deq = stock_bf16 = None
        inv = None
    else:
        eager = statistics.median(_time_calls(call(1), args.steps, args.warmup, ncopy, graph=False))
        # bitwise invariance in the same run: row 0 at M = 1 vs inside M = 64
        inv = all(_bits(call(1)(0)[0]) == _bits(call(M)(0)[0]) for M in Ms)
        # stock, non-invariant baselines: dequantize + hipBLASLt, and bf16 GEMV on
        # the pre-dequantized weight
        Wd = bi.dequantize(copies[0][0], copies[0][1], copies[0][2], gs, bits, dtype=torch.bfloat16)
        stock_deq = statistics.median(_time_calls(
            lambda i: torch.matmul(xs[:1], bi.dequantize(*copies[i], gs, bits, dtype=torch.bfloat16).t()), 5, 2,
            ncopy, graph=False))
        stock_bf16 = statistics.median(_time_calls(lambda i: torch.matmul(xs[:1], Wd.t()), args.steps,
                                                   args.warmup, 1))
    t_med = statistics.median(durs)
    by1 = qmm_bytes(1, N, K, bits, gs)
    achieved = by1 / t_med
    cpu = None if args.no_cpu else cpu_baseline_qmm(bits, gs)
    cpu_oracle = None if args.no_cpu else cpu_oracle_qmm(bits, gs)
    traffic = None
    if bits == 4 and gs == 64:
        mt = MEASURED_TRAFFIC_QMM4_M1
        traffic = int(1024 * (mt["fetch_kib"] * mt["fetch_scale"] + mt["write_kib"] * mt["write_scale"]))
    return {
        "metric": METRIC,
        "value": round(100 * achieved / PEAK_HBM, 2),
        "unit": "% of HBM roofline (4-bit g64 qmatmul, M=1)" if bits == 4 else f"% of HBM roofline ({bits}-bit g{gs} qmatmul, M=1)",
        "ms_per_step": round(statistics.median(durs) * 1e3, 5),
        "replay_us_per_step": [round(d * 1e6, 3) for d in durs],
        "eager_us_per_call": None if eager is None else round(eager * 1e6, 2),
        "wall_s_timed": round(wall, 4),
        "dtype": "bf16",
        "config": {"workload": f"qmatmul {bits}-bit g{gs} affine, x[M,4096] @ W[14336,4096]^T, Llama-3-8B MLP shape",
                   "M": 1, "M_sweep": list(Ms), "weights_rotated_MB": round(ncopy * per / 2**20)},
        "roofline": {"bound": "hbm", "achieved": round(achieved / 1e9, 1), "peak": PEAK_HBM / 1e9,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM, 4), "traffic": traffic,
                     "traffic_source": None if traffic is None else
                     "rocprofv3 FETCH_SIZE + WRITE_SIZE per dispatch x copy-kernel scale (bytes per launch)",
                     "algorithmic_bytes": by1, "kernel": HEADLINE_KERNEL[(bits, gs)]},
        "per_m": table,
        "bitwise_invariant_M1_vs_all": inv,
        "stock_gpu": {"dequant_plus_matmul_us": None if stock_deq is None else round(stock_deq * 1e6, 2),
                      "bf16_hipblaslt_gemv_us": None if stock_bf16 is None else round(stock_bf16 * 1e6, 2),
                      "note": "non-invariant torch paths, reported only"},
        "cpu_baseline": cpu,
        "cpu_oracle": cpu_oracle,
    }


def cpu_threads() -> int:
    """Host threads the CPU legs use: all cores, capped by the job's CPU share
    (OMP_NUM_THREADS, which the GPU boxes set to their per-GPU share)."""
    n = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(n, int(cap))) if cap and cap.isdigit() else n


def cpu_baseline_qmm(bits, gs, warmup=3, runs=20):
    """Stock MLX's CPU backend is the planned CPU baseline; MLX does not exist
    for this platform, so the same op runs in PyTorch on the host cores: the
    full M = 1 call (dequantize the [14336, 4096] weight, then matmul), 3
    warm-ups + 20 timed runs, median (the reference's harness/bench.py:19-27
    protocol)."""
    import torch
    import mlx_batch_invariant_amd as bi
    N, K = 14336, 4096
    nthreads = cpu_threads()
    old = torch.get_num_threads()
    torch.set_num_threads(nthreads)
    try:
        g = torch.Generator().manual_seed(0)
        wq, s, b = bi.quantize(0.02 * torch.randn((N, K), generator=g), group_size=gs, bits=bits, dtype=torch.bfloat16)
        x = torch.randn((1, K), generator=g).to(torch.bfloat16)
        words = wq.view(torch.int32)
        per = 32 // bits
        shifts = torch.arange(0, 32, bits, dtype=torch.int32)
        sf, bf = s.float()[..., None], b.float()[..., None]

        def call():
            # codes low to high in each word; W = code * scale + bias per group, in fp32
            codes = ((words[..., None] >> shifts) & ((1 << bits) - 1)).reshape(N, K // gs, gs).float()
            W = (codes * sf + bf).reshape(N, K)
            return torch.matmul(x.float(), W.t()).to(torch.bfloat16)

        for _ in range(warmup):
            call()
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            call()
            ts.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(old)
    t = statistics.median(ts)
    return {"value": round(qmm_bytes(1, N, K, bits, gs) / t / 1e9, 3), "unit": "GB/s (algorithmic bytes)",
            "cores": nthreads, "kind": "substitute: torch CPU (MLX unavailable)",
            "sample": f"full M=1 call, x[1,4096] @ W[14336,4096]^T {bits}-bit g{gs}: unpack + fp32 dequantize + "
                      f"fp32 matmul in torch on {nthreads} threads (os.cpu_count() = {os.cpu_count()}), median of {runs} after "
                      f"{warmup} warm-ups: {t * 1e3:.1f} ms per call"}


def cpu_oracle_qmm(bits, gs, budget_s=10.0):
    """The oracle (numpy port of the same arithmetic) on a bounded sample of
    the M = 1 workload: as many 512-row slices of W as fit in ~budget_s."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import bi_oracle as ora
    N, K, rows = 14336, 4096, 512
    rng = np.random.default_rng(0)
    x = ora.round_to(rng.standard_normal((1, K)).astype(np.float32), "bf16")
    done_bytes, t_used, slices = 0, 0.0, 0
    with threadpool_limits(limits=1):
        while t_used < budget_s and slices * rows < N:
            codes = rng.integers(0, 1 << bits, size=(rows, K))
            w = ora.pack(codes, bits)
            sc = ora.round_to(rng.uniform(1e-3, 1e-2, size=(rows, K // gs)).astype(np.float32), "bf16")
            bs = ora.round_to(rng.uniform(-0.05, 0.05, size=(rows, K // gs)).astype(np.float32), "bf16")
            t0 = time.perf_counter()
            Wd = ora.dequantize(w, sc, bs, gs, bits, "bf16")
            ora.matmul(x, Wd, "bf16")
            t_used += time.perf_counter() - t0
            slices += 1
            done_bytes += qmm_bytes(1, rows, K, bits, gs)
    return {"value": round(done_bytes / t_used / 1e9, 4), "unit": "GB/s (algorithmic bytes)", "cores": 1,
            "kind": "port", "sample": f"M=1, {slices} x {rows} of the 14336 weight rows, K=4096, "
                                      f"{bits}-bit g{gs}; numpy oracle, 1 BLAS thread, {t_used:.1f} s"}


def bench_linear(args):
    """RMSNorm then linear, Qwen2-0.5B shape."""
    import torch
    import mlx_batch_invariant_amd as bi
    g = torch.Generator().manual_seed(0)
    N, K = 4864, 896
    per = N * K * 2
    ncopy = math.ceil(ROTATE_BYTES / per)
    Ws = [(0.02 * torch.randn((N, K), generator=g)).to(torch.bfloat16).cuda()]
    Ws += [Ws[0].clone() for _ in range(ncopy - 1)]
    gam = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16).cuda()
    out = {}
    for M in (1, 4, 16, 64, 256):
        x = torch.randn((M, K), generator=g).to(torch.bfloat16).cuda()
        tn = statistics.median(_time_calls(lambda i: bi.batch_invariant_rms_norm(x, gam, 1e-6), args.steps, args.warmup, 1))
        h = bi.batch_invariant_rms_norm(x, gam, 1e-6)
        tl = statistics.median(_time_calls(lambda i: bi.batch_invariant_matmul(h, Ws[i].t()), args.steps, args.warmup, ncopy))
        ts = statistics.median(_time_calls(lambda i: torch.nn.functional.linear(h, Ws[i]), args.steps, args.warmup, ncopy))
        by_l = per + 2 * M * (K + N)
        by_n = 4 * M * K + 2 * K
        out[M] = {"rmsnorm_us": round(tn * 1e6, 2), "rmsnorm_GBps": round(by_n / tn / 1e9, 1),
                  "linear_us": round(tl * 1e6, 2), "linear_GBps": round(by_l / tl / 1e9, 1),
                  "linear_frac_hbm": round(by_l / tl / PEAK_HBM, 4), "stock_linear_us": round(ts * 1e6, 2)}
    return {"metric": METRIC, "op": "rmsnorm+linear (config 1)", "per_m": out}


def bench_rmsnorm(args):
    """RMSNorm alone: the config-1 rows (D = 896, M = 1..256, launch-bound) and
    two HBM-bound shapes (D = 4096, 16384 / 65536 rows; inputs 128 / 512 MiB,
    so the 256 MB Infinity Cache cannot hold input and output)."""
    import torch
    import mlx_batch_invariant_amd as bi
    g = torch.Generator().manual_seed(0)
    shapes = [] if args.headline_only else [(M, 896) for M in (1, 4, 16, 64, 256)]
    shapes += [(16384, 4096), (65536, 4096)]
    res = {}
    for R, D in shapes:
        x = torch.randn((R, D), generator=g).to(torch.bfloat16).cuda()
        gam = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
        t = statistics.median(_time_calls(lambda i: bi.batch_invariant_rms_norm(x, gam, 1e-6), args.steps, args.warmup, 1))
        by = 4 * R * D + 2 * D
        e = {"us": round(t * 1e6, 2), "GBps": round(by / t / 1e9, 1), "frac_hbm": round(by / t / PEAK_HBM, 4)}
        if not args.headline_only:
            ts = statistics.median(_time_calls(lambda i: torch.nn.functional.rms_norm(x, (D,), gam, 1e-6),
                                               args.steps, args.warmup, 1))
            e["stock_us"] = round(ts * 1e6, 2)
        res[f"{R}x{D}"] = e
        del x
    return {"metric": METRIC, "op": "rms_norm (bf16, eps 1e-6)", "kernel": "rms_norm_kernel",
            "algorithmic_bytes": "4*R*D + 2*D (read x, write out, read gamma)", "per_shape": res}


def bench_layernorm(args):
    """LayerNorm (no kernel in the reference; its roadmap item) at the RMSNorm
    bench's HBM-bound shapes, weight and bias given, against F.layer_norm."""
    import torch
    import mlx_batch_invariant_amd as bi
    g = torch.Generator().manual_seed(0)
    res = {}
    for R, D in ((16384, 4096), (65536, 4096)):
        x = torch.randn((R, D), generator=g).to(torch.bfloat16).cuda()
        gam = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
        bet = (0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
        t = statistics.median(_time_calls(lambda i: bi.batch_invariant_layer_norm(x, gam, bet, 1e-5),
                                          args.steps, args.warmup, 1))
        by = 4 * R * D + 4 * D
        e = {"us": round(t * 1e6, 2), "GBps": round(by / t / 1e9, 1), "frac_hbm": round(by / t / PEAK_HBM, 4)}
        if not args.headline_only:
            ts = statistics.median(_time_calls(lambda i: torch.nn.functional.layer_norm(x, (D,), gam, bet, 1e-5),
                                               args.steps, args.warmup, 1))
            e["stock_us"] = round(ts * 1e6, 2)
        res[f"{R}x{D}"] = e
        del x
    return {"metric": METRIC, "op": "layer_norm (bf16, eps 1e-5, weight and bias)", "kernel": "layer_norm_kernel",
            "algorithmic_bytes": "4*R*D + 4*D (read x, write out, read gamma and beta)", "per_shape": res}


def bench_decode(args):
    """split-KV decode, GQA 32/8, D 128, ragged lengths."""
    import numpy as np
    import torch
    import mlx_batch_invariant_amd as bi
    g = torch.Generator().manual_seed(0)
    res = {}
    for B in ((256,) if args.headline_only else (1, 16, 64, 256)):
        rng = np.random.default_rng(B)
        lens = rng.integers(1, 8193, size=B)
        L = 8192
        k = torch.randn((B, 8, L, 128), generator=g).to(torch.bfloat16).cuda()
        v = torch.randn((B, 8, L, 128), generator=g).to(torch.bfloat16).cuda()
        q = torch.randn((B, 32, 1, 128), generator=g).to(torch.bfloat16).cuda()
        kl = torch.tensor(lens, dtype=torch.int32).cuda()
        t = statistics.median(_time_calls(lambda i: bi.batch_invariant_decode_attention(
            q, k, v, scale=128 ** -0.5, kv_lens=kl), args.steps, args.warmup, 1))
        tp = None if args.headline_only else statistics.median(_time_calls(
            lambda i: bi.batch_invariant_decode_attention(q, k, v, scale=128 ** -0.5, kv_lens=kl, order="per_key"),
            max(3, args.steps // 4), 2, 1))
        by = 4096 * int(lens.sum()) + 16384 * B
        res[B] = {"us": round(t * 1e6, 2), "GBps": round(by / t / 1e9, 1), "frac_hbm": round(by / t / PEAK_HBM, 4),
                  "sum_len": int(lens.sum()), "per_key_order_us": None if tp is None else round(tp * 1e6, 2)}
        del k, v
    return {"metric": METRIC, "op": "decode attention (config 3)", "per_b": res}


def bench_prefill(args):
    """causal prefill T=2048, GQA 32/8, D 128."""
    import torch
    import mlx_batch_invariant_amd as bi
    g = torch.Generator().manual_seed(0)
    res = {}
    T = 2048
    for B in ((16,) if args.headline_only else (1, 4, 16)):
        q = torch.randn((B, 32, T, 128), generator=g).to(torch.bfloat16).cuda()
        k = torch.randn((B, 8, T, 128), generator=g).to(torch.bfloat16).cuda()
        v = torch.randn((B, 8, T, 128), generator=g).to(torch.bfloat16).cuda()
        t = statistics.median(_time_calls(lambda i: bi.batch_invariant_prefill_attention(
            q, k, v, scale=128 ** -0.5, causal=True), max(3, args.steps // 4), 2, 1))
        ts = None if args.headline_only else statistics.median(_time_calls(
            lambda i: torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True),
            max(3, args.steps // 4), 2, 1))
        tp = None if args.headline_only else statistics.median(_time_calls(
            lambda i: bi.batch_invariant_prefill_attention(q, k, v, scale=128 ** -0.5, causal=True, order="per_key"),
            3, 1, 1))
        fl = 4 * B * 32 * 128 * T * (T + 1) / 2
        res[B] = {"ms": round(t * 1e3, 3), "TFLOPs": round(fl / t / 1e12, 1), "frac_mfma": round(fl / t / PEAK_BF16, 4),
                  "stock_sdpa_ms": None if ts is None else round(ts * 1e3, 3),
                  "per_key_order_ms": None if tp is None else round(tp * 1e3, 3)}
    return {"metric": METRIC, "op": "prefill attention (config 4)", "per_b": res}


def bench_gemm(args):
    """Large-M bf16 GEMM (config 5 prefill shape): [M,4096] x [14336,4096]^T."""
    import torch
    import mlx_batch_invariant_amd as bi
    g = torch.Generator().manual_seed(0)
    N, K = 14336, 4096
    W = (0.02 * torch.randn((N, K), generator=g)).to(torch.bfloat16).cuda()
    res = {}
    for M in ((4096,) if args.headline_only else (256, 4096)):
        x = torch.randn((M, K), generator=g).to(torch.bfloat16).cuda()
        t = statistics.median(_time_calls(lambda i: bi.batch_invariant_matmul(x, W.t()), max(3, args.steps // 2), 2, 1))
        ts = None if args.headline_only else statistics.median(
            _time_calls(lambda i: torch.matmul(x, W.t()), max(3, args.steps // 2), 2, 1))
        fl = 2 * M * N * K
        res[M] = {"ms": round(t * 1e3, 3), "TFLOPs": round(fl / t / 1e12, 1), "frac_mfma": round(fl / t / PEAK_BF16, 4),
                  "stock_ms": None if ts is None else round(ts * 1e3, 3),
                  "stock_TFLOPs": None if ts is None else round(fl / ts / 1e12, 1)}
    return {"metric": METRIC, "op": "bf16 GEMM (large M)", "per_m": res}


def _llama_generate(model, prompt, steps):
    """Prefill + `steps` greedy decode steps; returns (prefill s, decode s,
    bytes of row 0's logits at every step).

    Each decode step (one token per sequence at position T + s) is captured
    into its own HIP graph before the timed region (all graphs share one
    memory pool and replay in capture order); the graph also takes the argmax
    into the static token buffer the next step reads. The timed decode region
    replays the 128 graphs back to back, so tokens/s measure the kernels, not
    Python's per-layer launch cost. Prefill runs eagerly."""
    import torch
    B, T = prompt.shape
    cache = model.new_cache(B, T + steps)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    _sync()
    ev[0].record()
    logits = model(prompt, cache, 0)
    ev[1].record()
    rows = [logits[0:1].clone()]
    tok = logits.argmax(-1, keepdim=True)
    # warm-up of the decode path (library loads, allocator) on a throwaway cache
    scratch = model.new_cache(B, T + 1)
    model(tok, scratch, T)
    del scratch
    _sync()
    pool = torch.cuda.graph_pool_handle()
    graphs, outs = [], []
    for st in range(steps):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=pool):
            lg = model(tok, cache, T + st)
            outs.append(lg[0:1].clone())
            tok.copy_(lg.argmax(-1, keepdim=True))
        graphs.append(g)
    _sync()
    ev[2].record()
    for g in graphs:
        g.replay()
    ev[3].record()
    _sync()
    out = _bits(torch.cat(rows + outs))
    del graphs, outs, cache
    return ev[0].elapsed_time(ev[1]) * 1e-3, ev[2].elapsed_time(ev[3]) * 1e-3, out


def bench_llama(args):
    """random-init Llama-3-8B-shape decoder (32 layers),
    prefill of 512 random tokens then 128 greedy decode steps at batch 1, 4,
    16, 64; 4-bit g64 linears and bf16 linears. Row 0 holds the same prompt at
    every batch size; its logits at all 129 steps must be bitwise identical.
    Tokens/s under the mode next to the stock (non-invariant) torch path."""
    import torch
    import mlx_batch_invariant_amd as bi
    from mlx_batch_invariant_amd.llama import LlamaConfig, LlamaShaped
    T, steps, batches = args.llama_prompt, args.llama_steps, (1, 4, 16, 64)
    res = {}
    for bits in (4, None):
        tag = f"q{bits}g64" if bits else "bf16"
        cfg = LlamaConfig(layers=args.llama_layers, bits=bits)
        model = LlamaShaped(cfg, device="cuda", dtype=torch.bfloat16, seed=0)
        g = torch.Generator().manual_seed(0)
        row0 = torch.randint(0, cfg.vocab, (1, T), generator=g)
        per_b, ref = {}, {}
        for B in batches:
            fill = torch.randint(0, cfg.vocab, (B - 1, T), generator=torch.Generator().manual_seed(B))
            prompt = torch.cat([row0, fill]).cuda()
            entry = {}
            for label, on in (("invariant", True), ("stock", False)):
                bi.reset_stats()
                with bi.set_batch_invariant_mode(enabled=on, strict=on):
                    _llama_generate(model, prompt[:, :16], 2)          # warm-up
                    tp, td, lg = _llama_generate(model, prompt, steps)
                ref.setdefault(label, lg)
                entry[label] = {"prefill_tok_s": round(B * T / tp, 1), "decode_tok_s": round(B * steps / td, 1),
                                "prefill_s": round(tp, 3), "decode_s": round(td, 3),
                                "row0_logits_equal_B1": lg == ref[label]}
                if on:
                    entry[label]["fallbacks"] = sum(bi.stats()["fallbacks"].values())
                print(f"# llama {tag} B={B} {label}: {entry[label]}", file=sys.stderr, flush=True)
            per_b[B] = entry
        res[tag] = {"per_b": per_b,
                    "bitwise_invariant_all_b": all(e["invariant"]["row0_logits_equal_B1"] for e in per_b.values())}
        del model
        torch.cuda.empty_cache()
    return {"metric": METRIC, "op": "Llama-3-8B-shape forward (config 5)",
            "config": {"workload": f"{args.llama_layers}-layer Llama-3-8B-shape decoder, prefill {T} tokens + "
                                   f"{steps} greedy decode steps, batch 1/4/16/64", "dtype": "bf16 activations"},
            "models": res}


def bench_copycal(args):
    """Calibration for the HBM traffic counters: a plain device copy of a
    known size (256 MiB read, 256 MiB written per launch). rocprofv3's
    FETCH_SIZE / WRITE_SIZE for this kernel against 262144 KiB give the
    counter scale applied to the other kernels' readings."""
    import torch
    n = 256 << 20
    src = [torch.ones(n // 4, dtype=torch.float32, device="cuda") for _ in range(2)]
    dst = torch.empty_like(src[0])
    t = statistics.median(_time_calls(lambda i: dst.copy_(src[i]), max(3, args.steps // 4), 2, 2, graph=False))
    return {"metric": METRIC, "op": "copy calibration (256 MiB)", "bytes_read": n, "bytes_written": n,
            "us": round(t * 1e6, 2), "GBps": round(2 * n / t / 1e9, 1)}


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--op", default="qmm4", choices=["qmm4", "qmm8", "linear", "rmsnorm", "layernorm", "decode", "prefill", "gemm", "llama",
                                                     "copycal", "all"])
    p.add_argument("--llama-layers", type=int, default=32)
    p.add_argument("--llama-prompt", type=int, default=512)
    p.add_argument("--llama-steps", type=int, default=128)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--profile-m", type=int, default=1,
                   help="qmm4/qmm8: run only the graph-replayed calls at this M and print no result (for profilers)")
    p.add_argument("--headline-only", action="store_true",
                   help="time only each op's headline shape (qmm M=1, rmsnorm D=4096, decode B=256, "
                        "prefill B=16, gemm M=4096) without sweeps or stock legs; for profiling")
    a = p.parse_args(argv)
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: every kernel here is single-GPU and no multi-GPU "
              "path exists in this build (rows and heads would shard across GPUs without any "
              "exchange; a K split would all-gather per-group partials and fold them in order).",
              file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    import mlx_batch_invariant_amd as bi
    bi._lib.load()
    ops = ["qmm4", "qmm8", "linear", "rmsnorm", "layernorm", "decode", "prefill", "gemm"] if a.op == "all" else [a.op]
    for op in ops:
        if op == "qmm4":
            r = bench_qmm(a, 4, 64)
        elif op == "qmm8":
            r = bench_qmm(a, 8, 128)
        elif op == "linear":
            r = bench_linear(a)
        elif op == "rmsnorm":
            r = bench_rmsnorm(a)
        elif op == "layernorm":
            r = bench_layernorm(a)
        elif op == "decode":
            r = bench_decode(a)
        elif op == "prefill":
            r = bench_prefill(a)
        elif op == "llama":
            r = bench_llama(a)
        elif op == "copycal":
            r = bench_copycal(a)
        else:
            r = bench_gemm(a)
        r.setdefault("n_gpus", 1)
        r.setdefault("steps", a.steps)
        r.setdefault("warmup", a.warmup)
        r.setdefault("higher_is_better", True)
        r.setdefault("scaling", "weak")
        r.setdefault("vs_baseline", None)
        r.setdefault("data", "synthetic (seeded torch.Generator, random-init weights)")
        r.setdefault("gpu", torch.cuda.get_device_name(0))
        print(json.dumps(r), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
