"""Benchmark of the MI355X fp32 GEMM backend (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary] [--no-cpu]

Headline (benchmark config 2): one step = one C[4096,4096] = A·B fp32 GEMM,
A,B ~ U(-1,1), all operands resident in HBM.  `value` is TFLOPS =
2·4096³ / (mean step time), timed with HIP events on the launch stream over
exactly K steps bracketed by device synchronisation.  The GEMM is a single
kernel launch per step, so the roofline figure uses the same events.

Secondary lines (the other benchmark configs: ms and TFLOPS, and HBM GB/s for
the batched one) are reported under "secondary".  Their kernels take 10-100
us, less than a Python/ctypes call, so `ms` is device time: 20 calls are
captured into a HIP graph and the graph is replayed between HIP events.
`ms_eager_python` is the same calls from a Python loop, for comparison.
The CPU baseline times the reference's own matmul_cpu (oracle/_ref, built
from the reference headers; the C restatement in oracle/ when that build is
absent) on a 64-row sample of the same GEMM, single-threaded.
Traffic (HBM bytes per launch) is read from the rocprofv3 FETCH_SIZE /
WRITE_SIZE summary committed under profiles/, or null when absent.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_TFLOPS = 157.3      # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0    # MI355X HBM3E
TRAFFIC_FILE = ROOT / "profiles" / "traffic_gemm_f32_4096.json"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--copy-probe", action="store_true",
                   help="also run a 256 MiB device copy (rocprof counter calibration)")
    p.add_argument("--only", default="",
                   help="comma list of secondary configs (c1,c3,c4,c5a,c5b): run just those "
                        "and print their JSON, without the headline and CPU legs "
                        "(per-workload profiles)")
    return p.parse_args()


def time_events(fn, iters: int, warmup: int) -> float:
    """Mean ms per call of fn over `iters` calls, HIP events on the current stream."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / iters


def time_graph(fn, calls: int = 20, replays: int = 10) -> float:
    """Mean device ms per call of fn: `calls` calls captured into one HIP graph,
    replayed `replays` times between HIP events.  Removes the Python/ctypes
    launch overhead, which exceeds the kernel time of the small configs."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / (replays * calls)
    del graph
    return ms


SECONDARY = ("c1", "c3", "c4", "c5a", "c5b")


def secondary(dev, only=SECONDARY) -> dict:
    """benchmark configs 1, 3, 4, 5 (ms, TFLOPS; GB/s for the HBM-near batched one)."""
    import ctypes
    import torch
    import minitensor_amd as mt

    g = torch.Generator(device=dev)
    g.manual_seed(42)

    def u(*shape):
        return torch.rand(*shape, device=dev, generator=g) * 2 - 1

    def n(*shape, std=1.0):
        return torch.randn(*shape, device=dev, generator=g) * std

    out = {}

    def both(fn, iters, warmup):
        """(device ms from graph replay, eager ms of the Python call loop)."""
        eager = time_events(fn, iters, warmup)
        return time_graph(fn), eager

    def rec(name, times, flops, bytes_=None, cfg=None):
        ms, eager = times
        d = {"ms": round(ms, 5), "ms_eager_python": round(eager, 5),
             "tflops": round(flops / ms / 1e9, 2),
             "frac_of_fp32_mfma_peak": round(flops / ms / 1e9 / PEAK_TFLOPS, 4)}
        if bytes_ is not None:
            d["hbm_gbs"] = round(bytes_ / ms / 1e6, 1)
            d["frac_of_hbm_peak"] = round(bytes_ / ms / 1e6 / PEAK_HBM_GBS, 4)
        if cfg:
            d["kernel"] = cfg
        out[name] = d

    def ws_for(A, B, C):
        return mt.workspace(mt.lib().mt_gemm_workspace_f32(mt.mat(A), mt.mat(B), mt.mat(C)), dev)

    if "c1" in only:  # MLP-Linear shape 256x512x512
        A, B = u(256, 512), u(512, 512)
        C = torch.empty(256, 512, device=dev)
        ws = ws_for(A, B, C)
        ms = both(lambda: mt.gemm(A, B, out=C, ws=ws), 200, 20)
        rec("c1_256x512x512", ms, 2 * 256 * 512 * 512, 4 * (256 * 512 + 512 * 512 + 256 * 512),
            mt.last_config())

    if "c3" in only:  # C = A·Bᵀ with B [2048,1024] as a transpose view; and the slice A[128:]
        A, B = n(2048, 1024), n(2048, 1024)
        C = torch.empty(2048, 2048, device=dev)
        ws = ws_for(A, B.t(), C)
        ms = both(lambda: mt.gemm(A, B.t(), out=C, ws=ws), 100, 10)
        rec("c3a_2048x2048x1024_bT_view", ms, 2 * 2048 * 2048 * 1024, None, mt.last_config())
        As = A[128:]
        C2 = torch.empty(1920, 2048, device=dev)
        ms = both(lambda: mt.gemm(As, B.t(), out=C2, ws=ws), 100, 10)
        rec("c3b_1920x2048x1024_slice_bT_view", ms, 2 * 1920 * 2048 * 1024, None,
            mt.last_config())

    if "c4" in only:  # Linear fwd + bwd, ResNet50-fc shape
        X = n(256, 2048)
        W = n(1000, 2048, std=(2.0 / 2048) ** 0.5)
        b = torch.zeros(1000, device=dev)
        dY = n(256, 1000, std=0.01)
        Y = torch.empty(256, 1000, device=dev)
        dX = torch.empty(256, 2048, device=dev)
        dW = torch.empty(1000, 2048, device=dev)
        db = torch.empty(1000, device=dev)
        lws = mt.workspace(mt.lib().mt_linear_workspace_f32(256, 2048, 1000), dev)
        f = 2 * 256 * 1000 * 2048
        ms = both(lambda: mt.linear(X, W, b, out=Y, ws=lws), 200, 20)
        rec("c4_linear_fwd", ms, f, None, mt.last_config())
        ms = both(lambda: mt.linear_backward(dY, X, W, True, False, False, dx=dX, ws=lws),
                  200, 20)
        rec("c4_linear_dx", ms, f, None, mt.last_config())
        ms = both(lambda: mt.linear_backward(dY, X, W, False, True, True, dw=dW, db=db,
                                             ws=lws), 200, 20)
        rec("c4_linear_dw_db", ms, f, None, mt.last_config())
        ms = both(lambda: (mt.linear(X, W, b, out=Y, ws=lws),
                           mt.linear_backward(dY, X, W, dx=dX, dw=dW, db=db, ws=lws)), 200, 20)
        rec("c4_linear_fwd_bwd_total", ms, 3 * f)

    if "c5a" in only:  # 3x3 conv as implicit GEMM, ResNet50 bottleneck shape
        x = n(32, 256, 14, 14)
        w = n(256, 256, 3, 3, std=(2.0 / 2304) ** 0.5)
        cb = torch.zeros(256, device=dev)
        d = mt.Conv2dDesc(32, 256, 14, 14, 256, 3, 3, 1, 1)
        cws = mt.workspace(mt.lib().mt_conv2d_workspace_f32(ctypes.byref(d)), dev)
        ms = both(lambda: mt.conv2d(x, w, cb, 1, 1, ws=cws), 100, 10)
        rec("c5a_conv3x3_n32_c256_14x14", ms, 2 * 6272 * 256 * 2304,
            4 * (x.numel() + w.numel() + cb.numel() + 32 * 256 * 196), mt.last_config())
        # the same layer's backward: dX (implicit, flipped weights) and dW (+ db)
        dy = n(32, 256, 14, 14, std=0.01)
        bws = mt.workspace(mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d)), dev)
        dwb = torch.empty_like(w)
        ms = both(lambda: mt.conv2d_backward(x, w, dy, 1, 1, need_dw=False, need_db=False,
                                             ws=bws), 100, 10)
        rec("c5a_conv_backward_dx", ms, 2 * 6272 * 256 * 2304, None, mt.last_config())
        ms = both(lambda: mt.conv2d_backward(x, w, dy, 1, 1, need_dx=False, ws=bws, dw=dwb),
                  100, 10)
        rec("c5a_conv_backward_dw_db", ms, 2 * 6272 * 256 * 2304, None, mt.last_config())

    if "c5b" in only:  # batched 64 x [512,64]·[64,512]
        A, B = u(64, 512, 64), u(64, 64, 512)
        C = torch.empty(64, 512, 512, device=dev)
        ws = ws_for(A, B, C)
        ms = both(lambda: mt.gemm(A, B, out=C, ws=ws), 200, 20)
        rec("c5b_bmm_64x512x512x64", ms, 2 * 64 * 512 * 512 * 64,
            4 * 64 * (512 * 64 + 64 * 512 + 512 * 512), mt.last_config())
    return out


def cpu_baseline() -> dict:
    """The reference CPU matmul on a bounded row sample of the 4096^3 GEMM, 1 thread."""
    import numpy as np
    import oracle

    rows = 64
    try:
        os.sched_setaffinity(0, {sorted(os.sched_getaffinity(0))[0]})
    except (AttributeError, OSError):
        pass
    a = oracle.uniform((rows, 4096), 42)
    b = oracle.uniform((4096, 4096), 43)
    c = np.empty((rows, 4096), np.float32)
    if oracle.ref_available():
        kind, fn = "reference", lambda: oracle.ref().ref_matmul_f32(
            oracle._fp(a), oracle._fp(b), oracle._fp(c), rows, 4096, 4096)
        what = "reference matmul_cpu (include/TensorOps.hpp:139-160, built from its headers)"
    else:
        kind, fn = "port", lambda: oracle.lib().ora_matmul(
            oracle._fp(a), oracle._fp(b), oracle._fp(c), rows, 4096, 4096)
        what = "C restatement of the reference matmul_cpu (oracle/oracle.c)"
    t0 = time.perf_counter()
    fn()
    dt = time.perf_counter() - t0
    flops = 2.0 * rows * 4096 * 4096
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(flops / dt / 1e12, 6), "unit": "TFLOPS", "cores": 1, "kind": kind,
            "sample": f"C[{rows},4096] = A[{rows},4096]·B[4096,4096] ({rows} of the 4096 rows of "
                      f"the headline GEMM), {what}, -O2 -ffp-contract=off, 1 thread pinned; "
                      f"{dt:.2f} s; host {cpu_model}, {os.cpu_count()} cpus visible",
            "seconds": round(dt, 3)}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(a GEMM shards by row or column blocks with no exchange). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import minitensor_amd as mt

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.only:
        names = tuple(x.strip() for x in args.only.split(",") if x.strip())
        unknown = [x for x in names if x not in SECONDARY]
        if unknown:
            print(f"bench.py: unknown --only entries {unknown}; choose from {SECONDARY}",
                  file=sys.stderr)
            sys.exit(2)
        print(json.dumps({"secondary": secondary(dev, names)}), flush=True)
        return
    M = N = K = 4096
    g = torch.Generator(device=dev)
    g.manual_seed(42)
    A = torch.rand(M, K, device=dev, generator=g) * 2 - 1
    B = torch.rand(K, N, device=dev, generator=g) * 2 - 1
    C = torch.empty(M, N, device=dev)
    ws = mt.workspace(mt.lib().mt_gemm_workspace_f32(mt.mat(A), mt.mat(B), mt.mat(C)), dev)

    def step():
        mt.gemm(A, B, out=C, ws=ws)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev0.elapsed_time(ev1) / args.steps
    kernel_cfg = mt.last_config()
    flops = 2.0 * M * N * K
    tflops = flops / ms / 1e9

    if args.copy_probe:  # 256 MiB device copy, for FETCH/WRITE_SIZE calibration
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()

    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

    line = {
        "metric": "fp32 matmul TFLOPS + % of fp32 MFMA peak at 4096³; strided/batched ms",
        "value": round(tflops, 3),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (U(-1,1), torch generator seed 42, resident in HBM)",
        "config": {"workload": "benchmark config 2: C[4096,4096] = A[4096,4096]·B[4096,4096] "
                               "fp32 row-major GEMM", "M": M, "N": N, "K": K,
                   "kernel": kernel_cfg, "wall_s_timed_region": round(wall, 4)},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 3), "peak": PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_TFLOPS, 4),
                     "traffic": traffic},
    }
    if not args.no_secondary:
        line["secondary"] = secondary(dev)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
