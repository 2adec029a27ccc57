#!/usr/bin/env python
"""Benchmark of the batch-invariant kernels on one MI355X.

Default workload: 4-bit affine quantized matmul at
the Llama-3-8B MLP shape, x bf16 [M, 4096] @ W[14336, 4096]^T with W packed
4-bit, group 64, bf16 scales/biases; the headline is the decode GEMV, M = 1.
A step is one call of the op on one batch. Weights are rotated over >= 512 MB
of distinct copies so every step streams them from HBM (the 256 MB Infinity
Cache would otherwise hold them). Time is measured with HIP events on the
stream the kernels run on.

    python bench.py [--steps K] [--warmup W] [--op qmm4|qmm8|linear|rmsnorm|decode|prefill|gemm|llama|sweep|all]

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
# Source: profiles/qmatmul4_g64_llama_mlp_m1.txt (the repacked copy, the
# default) and the earlier take of the MLX-layout kernel recorded there.
# Re-measure after changing the kernel.
MEASURED_TRAFFIC_QMM4_M1 = {"fetch_kib": 16217.0, "fetch_scale": 2.000, "write_kib": 28, "write_scale": 1.000}
MEASURED_TRAFFIC_QMM4_M1_MLX = {"fetch_kib": 16217.5, "fetch_scale": 2.000, "write_kib": 28, "write_scale": 1.000}
PEAK_BF16 = 2.5e15         # FLOP/s, dense bf16 MFMA
METRIC = "% of HBM/MFMA roofline per op at batch 1–256, with bitwise batch invariance"
ROTATE_BYTES = 512 << 20


def _sync():
    import torch
    torch.cuda.synchronize()


def _time_calls(fn, n, warmup, rotate, graph=True, replays=3, warm_replays=1):
    """Per-call device time (s) of fn(i), i cycling over `rotate` weight copies.

    graph=True: the n calls are captured into one HIP graph (so the host's
    per-call launch cost cannot leave the GPU idle between kernels), the graph
    is replayed `warm_replays` times untimed and then `replays` times, each
    timed replay bracketed by HIP events on the stream the kernels run on; the
    result is replay time / n, once per timed replay.
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
        for _ in range(warm_replays):
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
# The same launch on the repacked copy (bi_quantized_matmul_packed).
HEADLINE_KERNEL_PACKED = {
    (4, 64): "gemv_stream<bf16,QuantPacked<4,64>,W=8,NB=2,MR=1,PD=1> (bi_quantized_matmul_packed, M <= 4: one launch)",
    (8, 128): "gemv_stream<bf16,QuantPacked<8,128>,W=8,NB=2,MR=1,PD=1> (bi_quantized_matmul_packed, M <= 4: one "
              "launch)",
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
    # The decode layout: every copy repacked once (cache_packed), so calls of
    # up to PACKED_MAX_M rows read the repacked codes (same bits).
    packed = args.qmm_layout == "packed"
    if packed:
        for c in copies:
            bi.cache_packed(*c, group_size=gs, bits=bits)

    def call(M):
        return lambda i: bi.batch_invariant_quantized_matmul(xs[:M], *copies[i], group_size=gs, bits=bits)

    # headline M = 1: `steps` calls captured in one graph, replayed (each
    # timed replay times exactly `steps` calls; the median replay is reported).
    # Timed before the M sweep: after the larger-M launches the same M = 1 graph
    # reads ~1 us per call slower for its first few hundred calls, then recovers.
    _sync()
    t0 = time.perf_counter()
    if args.profile_m != 1:                # profiling aid: only the calls at that M, no report
        _time_calls(call(args.profile_m), args.steps, args.warmup, ncopy, replays=3)
        return {"metric": METRIC, "op": f"qmm{bits} profile run at M={args.profile_m}", "value": None}
    # 9 timed replays after 20 untimed ones: single replays of a short graph
    # spread by several percent on one box, and the first few milliseconds of
    # replays run slower (per-step times fell 10.3 -> 9.2 us over the first
    # nine 1 ms replays after 3 untimed ones).
    durs = _time_calls(call(1), args.steps, args.warmup, ncopy, replays=9, warm_replays=20)
    wall = time.perf_counter() - t0
    mlx_layout = None
    if packed and not args.headline_only:
        # The same M = 1 graph on the MLX-layout operands (the copies dropped,
        # then repacked for the sweep), timed before any larger M.
        for c in copies:
            bi.drop_packed(c[0])
        d_mlx = _time_calls(call(1), args.steps, args.warmup, ncopy, replays=9, warm_replays=20)
        mlx_layout = {"us_per_step": round(statistics.median(d_mlx) * 1e6, 3),
                      "frac": round(qmm_bytes(1, N, K, bits, gs) / statistics.median(d_mlx) / PEAK_HBM, 4),
                      "kernel": HEADLINE_KERNEL[(bits, gs)]}
        for c in copies:
            bi.cache_packed(*c, group_size=gs, bits=bits)
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
    achievable = None if args.headline_only else stream_read_rate(per, args)
    traffic = None
    if bits == 4 and gs == 64:
        mt = MEASURED_TRAFFIC_QMM4_M1 if packed else MEASURED_TRAFFIC_QMM4_M1_MLX
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
                   "M": 1, "M_sweep": list(Ms), "weights_rotated_MB": round(ncopy * per / 2**20),
                   "weights": ("MLX packed codes with a copy repacked once at load (bi_quantized_pack: the same "
                               "codes, scales and biases in the decode GEMV's layout; M <= 16 reads it, bits equal "
                               "to the MLX-layout call)") if packed else "MLX packed codes"},
        "roofline": {"bound": "hbm", "achieved": round(achieved / 1e9, 1), "peak": PEAK_HBM / 1e9,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM, 4), "traffic": traffic,
                     "traffic_source": None if traffic is None else
                     "rocprofv3 FETCH_SIZE + WRITE_SIZE per dispatch x copy-kernel scale (bytes per launch)",
                     "algorithmic_bytes": by1,
                     "kernel": (HEADLINE_KERNEL_PACKED if packed else HEADLINE_KERNEL)[(bits, gs)],
                     "achievable": None if achievable is None else {
                         "value": round(achievable / 1e9, 1), "unit": "GB/s",
                         "frac_of_peak": round(achievable / PEAK_HBM, 4),
                         "frac_achieved_of_achievable": round(by1 / t_med / achievable, 4),
                         "kernel": "bi_stream_read: a plain read of the same bytes in one launch (1 KB per wave "
                                   "instruction), graph-replayed over the same rotation"}},
        "per_m": table,
        "mlx_layout_M1": mlx_layout,
        "bitwise_invariant_M1_vs_all": inv,
        "stock_gpu": {"dequant_plus_matmul_us": None if stock_deq is None else round(stock_deq * 1e6, 2),
                      "bf16_hipblaslt_gemv_us": None if stock_bf16 is None else round(stock_bf16 * 1e6, 2),
                      "note": "non-invariant torch paths, reported only"},
        "cpu_baseline": cpu,
        "cpu_oracle": cpu_oracle,
    }


def stream_read_rate(nbytes, args):
    """Achievable HBM read rate for one launch over `nbytes`: bi_stream_read
    (a plain read, 1 KB per wave instruction) graph-replayed like the op,
    over enough distinct buffers (>= 512 MB) that every launch reads HBM."""
    import torch
    from mlx_batch_invariant_amd import _lib
    lib = _lib.load()
    nbytes = nbytes // 16 * 16
    ncopy = max(1, math.ceil(ROTATE_BYTES / nbytes))
    bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device="cuda") for _ in range(ncopy)]
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")

    def call(i):
        _lib.check(lib.bi_stream_read(bufs[i].data_ptr(), nbytes, sink.data_ptr(), 0x9E3779B9,
                                      _lib.stream_of(sink)), "bi_stream_read")

    t = statistics.median(_time_calls(call, args.steps, args.warmup, ncopy))
    del bufs
    return nbytes / t


def cpu_threads() -> int:
    """Host threads the CPU legs use: all cores, capped by the job's CPU share
    (OMP_NUM_THREADS, which the GPU boxes set to their per-GPU share)."""
    n = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(n, int(cap))) if cap and cap.isdigit() else n


def _cpu_median(fn, warmup=3, runs=20):
    """Median wall time of fn() on the host after warm-ups (the reference's
    harness/bench.py:19-27 protocol: 3 warm-ups, 20 timed runs)."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


class _CpuThreads:
    """torch on every host core the job may use, restored on exit."""

    def __enter__(self):
        import torch
        self.old = torch.get_num_threads()
        self.n = cpu_threads()
        torch.set_num_threads(self.n)
        return self.n

    def __exit__(self, *exc):
        import torch
        torch.set_num_threads(self.old)


CPU_KIND = "substitute: torch CPU (MLX unavailable)"


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
    # The same linear with every weight copy repacked once (cache_packed_weight,
    # zero-filled to K = 1024): calls of up to 16 rows take the streaming GEMV,
    # with the bits of the row-major call.
    xs_h = {M: bi.batch_invariant_rms_norm(torch.randn((M, K), generator=g).to(torch.bfloat16).cuda(), gam, 1e-6)
            for M in (1, 4, 16)}
    plain = {M: bi.batch_invariant_matmul(xs_h[M], Ws[0].t()) for M in xs_h}
    for W in Ws:
        bi.cache_packed_weight(W)
    for M in (1, 4, 16):
        h = xs_h[M]
        tp = statistics.median(_time_calls(lambda i: bi.batch_invariant_matmul(h, Ws[i].t()), args.steps, args.warmup,
                                           ncopy))
        by_l = per + 2 * M * (K + N)
        out[M]["linear_packed_us"] = round(tp * 1e6, 2)
        out[M]["linear_packed_frac_hbm"] = round(by_l / tp / PEAK_HBM, 4)
        out[M]["linear_packed_bits_equal"] = bool(
            bi.batch_invariant_matmul(h, Ws[0].t()).view(torch.int16).equal(plain[M].view(torch.int16)))
    for W in Ws:
        bi.drop_packed_weight(W)
    cpu = None
    if not args.no_cpu:
        with _CpuThreads() as nth:
            gc = torch.Generator().manual_seed(0)
            Wc = (0.02 * torch.randn((N, K), generator=gc)).to(torch.bfloat16)
            gc_ = (1 + 0.1 * torch.randn(K, generator=gc)).to(torch.bfloat16)
            per_m = {}
            for M in (1, 4, 16, 64, 256):
                xc = torch.randn((M, K), generator=gc).to(torch.bfloat16)
                t = _cpu_median(lambda: torch.nn.functional.linear(
                    torch.nn.functional.rms_norm(xc, (K,), gc_, 1e-6), Wc))
                by = per + 2 * M * (K + N) + 4 * M * K + 2 * K
                per_m[M] = {"us": round(t * 1e6, 1), "GBps": round(by / t / 1e9, 2)}
        cpu = {"value": per_m[1]["GBps"], "unit": "GB/s (algorithmic bytes, M=1)", "cores": nth, "kind": CPU_KIND,
               "sample": f"full config-1 call (rms_norm then linear, bf16) at each M on {nth} threads, median of 20 "
                         "after 3 warm-ups", "per_m": per_m}
    return {"metric": METRIC, "op": "rmsnorm+linear (config 1)", "per_m": out, "cpu_baseline": cpu}


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
    cpu = None
    if not args.no_cpu:
        # bounded sample: the first sequences of the B = 256 batch's lengths, one at a time
        lens = np.random.default_rng(256).integers(1, 8193, size=256)[:4]
        gc = torch.Generator().manual_seed(0)
        with _CpuThreads() as nth:
            tot_t, tot_b = 0.0, 0
            for n in lens:
                n = int(n)
                qc = torch.randn((1, 32, 1, 128), generator=gc).to(torch.bfloat16)
                kc = torch.randn((1, 8, n, 128), generator=gc).to(torch.bfloat16)
                vc = torch.randn((1, 8, n, 128), generator=gc).to(torch.bfloat16)
                tot_t += _cpu_median(lambda: torch.nn.functional.scaled_dot_product_attention(
                    qc, kc, vc, scale=128 ** -0.5, enable_gqa=True))
                tot_b += 4096 * n + 16384
        cpu = {"value": round(tot_b / tot_t / 1e9, 3), "unit": "GB/s (algorithmic bytes)", "cores": nth,
               "kind": CPU_KIND, "sample": f"sdpa decode (GQA 32/8, D 128, bf16) of the first 4 sequences of the "
                                           f"B = 256 batch (lengths {[int(x) for x in lens]}), one call each, median "
                                           f"of 20 after 3 warm-ups, summed: {tot_t * 1e3:.2f} ms"}
    return {"metric": METRIC, "op": "decode attention (config 3)", "per_b": res, "cpu_baseline": cpu}


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
    cpu = None
    if not args.no_cpu:
        gc = torch.Generator().manual_seed(0)
        with _CpuThreads() as nth:
            qc = torch.randn((1, 32, T, 128), generator=gc).to(torch.bfloat16)
            kc = torch.randn((1, 8, T, 128), generator=gc).to(torch.bfloat16)
            vc = torch.randn((1, 8, T, 128), generator=gc).to(torch.bfloat16)
            t = _cpu_median(lambda: torch.nn.functional.scaled_dot_product_attention(
                qc, kc, vc, is_causal=True, enable_gqa=True), warmup=1, runs=5)
        fl = 4 * 32 * 128 * T * (T + 1) / 2
        cpu = {"value": round(fl / t / 1e12, 3), "unit": "TFLOP/s (causal half)", "cores": nth, "kind": CPU_KIND,
               "sample": f"sdpa causal prefill of one sequence (B = 1, T = {T}, GQA 32/8, D 128, bf16), median of "
                         f"5 after 1 warm-up: {t * 1e3:.1f} ms"}
    return {"metric": METRIC, "op": "prefill attention (config 4)", "per_b": res, "cpu_baseline": cpu}


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
    achievable = None
    if not args.headline_only:
        n = 8192
        a = torch.randn((n, n), generator=g).to(torch.bfloat16).cuda()
        b = torch.randn((n, n), generator=g).to(torch.bfloat16).cuda()
        t = statistics.median(_time_calls(lambda i: torch.matmul(a, b), 5, 2, 1))
        achievable = {"value": round(2 * n ** 3 / t / 1e12, 1), "unit": "TFLOP/s",
                      "frac_of_peak": round(2 * n ** 3 / t / PEAK_BF16, 4),
                      "kernel": "torch.matmul (hipBLASLt) bf16 8192 x 8192 x 8192, the achievable dense MFMA rate"}
    return {"metric": METRIC, "op": "bf16 GEMM (large M)", "per_m": res, "achievable": achievable}


def _llama_generate(model, prompt, steps):
    """Prefill + `steps` greedy decode steps; returns (prefill s, decode s,
    bytes of row 0's logits at every step).

    Each decode step (one token per sequence at position T + s) is captured
    into its own HIP graph before the timed region (all graphs share one
    memory pool and replay in capture order); the graph also takes the argmax
    into the static token buffer the next step reads. The timed decode region
    replays the 128 graphs back to back, so tokens/s measure the kernels, not
    Python's per-layer launch cost. Prefill runs eagerly, once untimed on a
    throwaway cache first (the first call of a shape loads its kernels and
    grows the allocator's pool)."""
    import torch
    B, T = prompt.shape
    warm = model.new_cache(B, T)
    model(prompt, warm, 0)
    del warm
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


def _dequantized_copy(model):
    """The stock 4-bit baseline as a serving stack runs it: every
    QuantizedLinear's weight dequantized once into a plain bf16 nn.Linear
    (hipBLASLt / rocBLAS per call), sharing everything else with ``model``."""
    import copy

    import torch
    import mlx_batch_invariant_amd as bi
    from mlx_batch_invariant_amd.nn import QuantizedLinear
    m = copy.copy(model)
    m._modules = dict(model._modules)

    def swap(mod):
        for name, child in list(mod._modules.items()):
            if isinstance(child, QuantizedLinear):
                lin = torch.nn.Linear(child.in_features, child.out_features, bias=child.bias is not None,
                                      device="meta", dtype=child.scales.dtype)
                W = bi.dequantize(child.weight, child.scales, child.biases, child.group_size, child.bits,
                                  dtype=child.scales.dtype)
                lin.weight = torch.nn.Parameter(W, requires_grad=False)
                if child.bias is not None:
                    lin.bias = torch.nn.Parameter(child.bias.detach(), requires_grad=False)
                mod._modules[name] = lin
            elif child is not None:
                c = copy.copy(child)
                c._modules = dict(child._modules)
                mod._modules[name] = c
                swap(c)

    swap(m)
    return m


def cpu_baseline_llama(layers=2, T=512, steps=4):
    """Bounded CPU sample of config 5: the bf16 Llama-3-8B-shape decoder with
    ``layers`` of its 32 layers (embedding, final norm and the 128256-row head
    included) in torch on the host cores: prefill of T random tokens at B = 1,
    then ``steps`` greedy decode steps. Also the per-token time scaled to 32
    layers from the measured per-layer cost (head and embedding once)."""
    import torch
    from mlx_batch_invariant_amd.llama import LlamaConfig, LlamaShaped
    with _CpuThreads() as nth:
        res = {}
        for L in (1, layers):
            cfg = LlamaConfig(layers=L, bits=None)
            m = LlamaShaped(cfg, device="cpu", dtype=torch.bfloat16, seed=0)
            prompt = torch.randint(0, cfg.vocab, (1, T), generator=torch.Generator().manual_seed(0))
            cache = m.new_cache(1, T + steps)
            t0 = time.perf_counter()
            lg = m(prompt, cache, 0)
            tp = time.perf_counter() - t0
            tok = lg.argmax(-1, keepdim=True)
            t0 = time.perf_counter()
            for st in range(steps):
                tok = m(tok, cache, T + st).argmax(-1, keepdim=True)
            td = (time.perf_counter() - t0) / steps
            res[L] = (tp, td)
            del m, cache
    (p1, d1), (pL, dL) = res[1], res[layers]
    per_p, per_d = (pL - p1) / (layers - 1), (dL - d1) / (layers - 1)
    p32, d32 = p1 + 31 * per_p, d1 + 31 * per_d
    return {"value": round(1 / d32, 3), "unit": "decode tok/s at B=1 (32 layers, from the per-layer cost)",
            "cores": nth, "kind": CPU_KIND,
            "sample": f"bf16 decoder with 1 and {layers} layers (+ embedding, norm, head) on {nth} threads: prefill "
                      f"{T} tokens {res[layers][0]:.2f} s, {steps} decode steps {res[layers][1] * 1e3:.0f} ms each "
                      f"at {layers} layers; scaled to 32 layers: prefill {T / p32:.1f} tok/s, decode {1 / d32:.2f} "
                      "tok/s",
            "prefill_tok_s_32_layers": round(T / p32, 2)}


def bench_llama(args):
    """random-init Llama-3-8B-shape decoder (32 layers),
    prefill of 512 random tokens then 128 greedy decode steps at batch 1, 4,
    16, 64; 4-bit g64 linears and bf16 linears. Row 0 holds the same prompt at
    every batch size; its logits at all 129 steps must be bitwise identical.
    Tokens/s under the mode next to the stock (non-invariant) torch path."""
    import torch
    import mlx_batch_invariant_amd as bi
    from mlx_batch_invariant_amd.llama import LlamaConfig, LlamaShaped
    from mlx_batch_invariant_amd.nn import QuantizedLinear, cache_packed_linears
    T, steps = args.llama_prompt, args.llama_steps
    batches = tuple(int(b) for b in args.llama_batches.split(","))
    weights = [w.strip() for w in args.llama_weights.split(",")]
    if not batches or batches[0] != 1 or any(b < 1 for b in batches) or set(weights) - {"q4", "bf16"}:
        raise SystemExit("--llama-batches must start at 1 (row 0 is checked against B = 1); "
                         "--llama-weights takes q4 and/or bf16")
    res = {}
    for bits in [4 if w == "q4" else None for w in weights]:
        tag = f"q{bits}g64" if bits else "bf16"
        cfg = LlamaConfig(layers=args.llama_layers, bits=bits)
        model = LlamaShaped(cfg, device="cuda", dtype=torch.bfloat16, seed=0)
        g = torch.Generator().manual_seed(0)
        row0 = torch.randint(0, cfg.vocab, (1, T), generator=g)
        stock_model = (_dequantized_copy(model) if bits else model) if args.llama_stock else None
        per_b, ref = {}, {}
        for B in batches:
            fill = torch.randint(0, cfg.vocab, (B - 1, T), generator=torch.Generator().manual_seed(B))
            prompt = torch.cat([row0, fill]).cuda()
            entry = {}
            # 4-bit also runs with every weight dequantized once next to its codes
            # (QuantizedLinear.cache_dequantized): prefill (M >= 256) then skips the
            # per-call dequantization, same bits; decode reads the codes either way.
            # And with every linear weight repacked once (nn.cache_packed_linears:
            # QuantizedLinear.cache_packed, cache_packed_weight for nn.Linear):
            # decode (M <= 16) then reads the decode GEMV's layout, same bits.
            runs = [("invariant", True, None), ("invariant_packed", True, "packed")]
            if args.llama_stock:
                runs.append(("stock", False, None))
                if bits:
                    runs.append(("invariant_dequantized_once", True, "dequantized"))
            for label, on, cached in runs:
                bi.reset_stats()
                mdl = model if on else stock_model
                qlins = [m for m in mdl.modules() if isinstance(m, QuantizedLinear)] if cached else []
                if cached == "packed":
                    cache_packed_linears(mdl)
                for m in qlins if cached == "dequantized" else []:
                    m.cache_dequantized()
                with bi.set_batch_invariant_mode(enabled=on, strict=on):
                    _llama_generate(mdl, prompt[:, :16], 2)            # warm-up
                    tp, td, lg = _llama_generate(mdl, prompt, steps)
                for m in qlins if cached == "dequantized" else []:
                    bi.drop_dequantized(m.weight)
                if cached == "packed":
                    for m in mdl.modules():
                        if isinstance(m, QuantizedLinear):
                            bi.drop_packed(m.weight)
                        elif isinstance(m, torch.nn.Linear):
                            bi.drop_packed_weight(m.weight)
                ref.setdefault(label, lg)
                if cached:
                    entry[label + "_bits_equal_invariant"] = lg == ref["invariant"]
                entry[label] = {"prefill_tok_s": round(B * T / tp, 1), "decode_tok_s": round(B * steps / td, 1),
                                "prefill_s": round(tp, 3), "decode_s": round(td, 3),
                                "row0_logits_equal_B1": lg == ref[label]}
                if on:
                    entry[label]["fallbacks"] = sum(bi.stats()["fallbacks"].values())
                print(f"# llama {tag} B={B} {label}: {entry[label]}", file=sys.stderr, flush=True)
            per_b[B] = entry
        res[tag] = {"per_b": per_b,
                    "bitwise_invariant_all_b": all(e["invariant"]["row0_logits_equal_B1"] for e in per_b.values()),
                    "stock": "torch bf16 linears (hipBLASLt / rocBLAS)" + (
                        " on weights dequantized once from the same 4-bit codes" if bits else "")
                    + ", F.rms_norm, F.scaled_dot_product_attention; not batch invariant"}
        del model, stock_model
        torch.cuda.empty_cache()
    cpu = None if args.no_cpu else cpu_baseline_llama()
    return {"metric": METRIC, "op": "Llama-3-8B-shape forward (config 5)", "cpu_baseline": cpu,
            "config": {"workload": f"{args.llama_layers}-layer Llama-3-8B-shape decoder, prefill {T} tokens + "
                                   f"{steps} greedy decode steps, batch {'/'.join(map(str, batches))}",
                       "dtype": "bf16 activations"},
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


def bench_sweep(args):
    """Batch-sweep conformance (mlx_batch_invariant_amd.conformance, the
    reference's harness/sweep.py): per op x dtype, stock torch and the
    invariant mode, first diverging batch and max|diff|. The table goes to
    stderr; the JSON line summarises it."""
    from mlx_batch_invariant_amd import conformance
    rep = conformance.run(file=sys.stderr)
    stock = {f"{r['op']}/{r['dtype']}": (None if r["passed"] else {"first_fail_B": r["first_fail"],
                                                                   "max_diff": r["max_diff"]})
             for r in rep["rows"] if r["mode"] == "STOCK"}
    return {"metric": METRIC, "op": "conformance sweep (stock vs invariant, batch 1-256)",
            "invariant_all_pass": rep["invariant_all_pass"], "stock_divergence": stock,
            "structure": rep["structure"], "batches": rep["batches"]}


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--op", default="qmm4", choices=["qmm4", "qmm8", "linear", "rmsnorm", "layernorm", "decode", "prefill", "gemm", "llama",
                                                     "copycal", "sweep", "all"])
    p.add_argument("--llama-layers", type=int, default=32)
    p.add_argument("--llama-prompt", type=int, default=512)
    p.add_argument("--llama-steps", type=int, default=128)
    p.add_argument("--llama-batches", default="1,4,16,64", help="llama: comma-separated batch sizes")
    p.add_argument("--llama-weights", default="q4,bf16", help="llama: comma-separated subset of q4, bf16")
    p.add_argument("--llama-stock", action=argparse.BooleanOptionalAction, default=True,
                   help="llama: also run the stock path and the dequantized-once run (off: the invariant run only)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--qmm-layout", default="packed", choices=["packed", "mlx"],
                   help="qmm4 / qmm8: weights with a copy repacked once for the decode GEMV (packed, the default; "
                        "the MLX-layout M=1 time is reported beside it) or the MLX layout alone")
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
        elif op == "sweep":
            r = bench_sweep(a)
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
