"""Benchmark of the MI355X fp32 GEMM backend (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary] [--no-cpu]

Headline (benchmark config 2): one step = one C[4096,4096] = A·B fp32 GEMM,
A,B ~ U(-1,1), all operands resident in HBM.  Protocol:
  1. W untimed warm-up steps;
  2. an untimed pre-roll of steps for about 200 ms of GPU time -- the length
     of the reference's adaptive trial window (test/benchmark.cpp:171-181) --
     so that the timed steps do not run on the clock ramp out of idle;
  3. exactly K timed steps, a HIP event recorded on the launch stream before
     the first and after every step.
`value` is TFLOPS = 2·4096³ / (mean step time), the mean being the span of
the K steps over K.  min and median of the per-step times are reported
beside it.  The GEMM is one kernel launch per step, so the roofline's
`achieved` uses the same events.  After the timed steps, `reference_window`
repeats the reference's own protocol (one timed call, then 200 ms / that
time trials) for comparison; it is not `value`.

Secondary lines (the other benchmark configs: ms and TFLOPS, HBM GB/s for
the batched one and the reference's HBM-bound "skinny" rows) are reported
under "secondary".  Their kernels take 7-100 us, less than a Python/ctypes
call, so `ms` is device time: 20 or more calls (about 1 ms of GPU work, at
most 200) are captured into a HIP graph and the graph is replayed between
HIP events; min / median / mean are over the replays.  `ms_eager_python` is
the same calls from a Python loop.  Config 3 is also timed with B
materialised (a strided copy into a dense Bᵀ, then the GEMM) to show what
the view saves.

`sustained`: the headline GEMM back to back for --sustained-seconds (2.5 s
by default), an event after every step, with the driver's clock, power and
temperature readings over the window (amdsmi, when importable).

CPU baselines (reported baselines only, never the target): the C
restatement of the reference CPU path in oracle/ (matmul_cpu,
matmul_cpu_strided, a per-batch matmul_cpu loop for bmm, conv2d_cpu;
-O2 -ffp-contract=off, bit-exact with the reference's own build), single
threaded and pinned to one core, on a bounded sample of each workload (rows,
batch entries or images), best of the stated repetitions, extrapolated
linearly to the full workload (each sampled unit does the same work).
Traffic (HBM bytes per launch) is read from the rocprofv3 FETCH_SIZE /
WRITE_SIZE summary committed under profiles/, or null when absent.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_TFLOPS = 157.3      # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0    # MI355X HBM3E
TRAFFIC_FILE = ROOT / "profiles" / "traffic_gemm_f32_4096.json"
PREROLL_MS = 200.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--sustained-seconds", type=float, default=SUSTAINED_S,
                   help="length of the sustained back-to-back window of the headline GEMM")
    p.add_argument("--copy-probe", action="store_true",
                   help="also run a 256 MiB device copy (rocprof counter calibration)")
    p.add_argument("--audit", default="",
                   help="SEED:COUNT: instead of the benchmark, time the planner's pick against "
                        "every forced tile configuration and split on COUNT random row-major "
                        "shapes (sizes 64-4700, seeded) and print one line per shape and a summary")
    p.add_argument("--only", default="",
                   help="comma list of secondary configs (c1,c3,c4,c5a,c5b,skinny), 'resnet' "
                        "(twelve ResNet-like conv layers, not in the default run), "
                        "'resnet_bwd' (their backward, two downsampling layers and the "
                        "stem) and/or "
                        "'sustained' (the headline GEMM back to back for 2.5 s): run just those "
                        "and print their JSON, without the headline and CPU legs "
                        "(per-workload profiles)")
    return p.parse_args()


def _stats(per_ms) -> dict:
    return {"min": round(min(per_ms), 5), "median": round(statistics.median(per_ms), 5),
            "mean": round(sum(per_ms) / len(per_ms), 5)}


def time_steps(step, steps: int, warmup: int, preroll_ms: float = PREROLL_MS):
    """Warm-up, ~preroll_ms of untimed steps, then `steps` timed steps with an
    event after each.  Returns (span ms of the timed steps, per-step ms list,
    pre-roll step count)."""
    import torch
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    n_pre = 0
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < preroll_ms:
        for _ in range(8):   # enqueue a few, then wait, so the queue stays short
            step()
        n_pre += 8
        torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    evs[0].record(stream)
    for i in range(steps):
        step()
        evs[i + 1].record(stream)
    torch.cuda.synchronize()
    per = [evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]
    return evs[0].elapsed_time(evs[-1]), per, n_pre


def reference_window(step) -> dict:
    """The reference's adaptive protocol (test/benchmark.cpp:171-181): one
    call timed by the host clock around two device syncs, trials = 200 ms /
    that time, min(5, trials) warm-up calls, then the mean over the trials."""
    import torch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    step()
    torch.cuda.synchronize()
    one_ms = (time.perf_counter() - t0) * 1e3
    trials = max(1, int(200.0 / max(one_ms, 0.01)))
    for _ in range(min(5, trials)):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(trials):
        step()
    e1.record()
    torch.cuda.synchronize()
    return {"trials": trials, "ms_mean": round(e0.elapsed_time(e1) / trials, 5)}


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


def time_graph(fn, calls: int = 20, replays: int = 10, preroll_ms: float = PREROLL_MS / 2,
               per_call_ms: float = 0.0) -> list:
    """Device ms per call of fn for each replay: `calls` calls captured into
    one HIP graph, replayed `replays` times with an event around each replay,
    after about preroll_ms of untimed replays (so that every workload is timed
    at the clocks of sustained work, not on the ramp out of the previous
    one's host-side set-up).  Removes the Python/ctypes launch overhead, which
    exceeds the kernel time of the small configs.  Given an estimate of the
    time per call, the graph holds enough calls (up to 200) for about 1 ms of
    GPU work per replay, so that the host's launch of the next replay never
    leaves the GPU idle inside a timed interval."""
    if per_call_ms > 0:
        calls = max(calls, min(200, int(1.0 / per_call_ms) + 1))
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
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(3):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    per_replay = max(t0.elapsed_time(t1) / 3, 1e-3)
    for _ in range(min(int(preroll_ms / per_replay), 5000)):
        graph.replay()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]
    evs[0].record()
    for i in range(replays):
        graph.replay()
        evs[i + 1].record()
    torch.cuda.synchronize()
    per = [evs[i].elapsed_time(evs[i + 1]) / calls for i in range(replays)]
    del graph
    return per


SECONDARY = ("c1", "c3", "c4", "c5a", "c5b", "skinny")
# Not in the default run (--only resnet): twelve ResNet-like convolution
# layers at batch 32, 3x3 and 1x1, 7x7 to 56x56 -- where the 64x112
# convolution tile on 16x16 MFMA blocks is or is not taken.
EXTRA = ("resnet", "resnet_bwd")
RESNET_LAYERS = [(56, 64, 64, 3), (56, 64, 256, 1), (56, 256, 64, 1),
                 (28, 128, 128, 3), (28, 128, 512, 1), (28, 512, 128, 1),
                 (14, 256, 256, 3), (14, 256, 1024, 1), (14, 1024, 256, 1),
                 (7, 512, 512, 3), (7, 512, 2048, 1), (7, 2048, 512, 1)]
# --only resnet_bwd: the backward (dX; dW + db in one call) of the same twelve
# layers, two downsampling layers and the 7x7 stem: (hw, c_in, c_out, k, stride, pad)
RESNET_BWD_LAYERS = [(hw, c, co, k, 1, k // 2) for hw, c, co, k in RESNET_LAYERS] + [
    (56, 128, 128, 3, 2, 1), (56, 256, 512, 1, 2, 0), (224, 3, 64, 7, 2, 3)]
SUSTAINED_S = 2.5


class ClockSampler:
    """Reads the GPU's clocks, socket power and hotspot temperature from the
    driver (amdsmi) every 100 ms on a side thread while a window runs; None
    when amdsmi is missing or refuses (the measurement never depends on it)."""

    def __init__(self):
        import threading
        self.samples, self.err = [], None
        self._stop = threading.Event()
        self._th = threading.Thread(target=self._run, daemon=True)

    def _run(self):
        try:
            import amdsmi
            amdsmi.amdsmi_init(amdsmi.AmdSmiInitFlags.INIT_AMD_GPUS)
            handles = amdsmi.amdsmi_get_processor_handles()
            if len(handles) != 1:
                self.err = f"{len(handles)} GPUs visible"
                return
            t0 = time.perf_counter()
            while not self._stop.is_set():
                m = amdsmi.amdsmi_get_gpu_metrics_info(handles[0])
                clks = [c for c in (m.get("current_gfxclks") or []) if isinstance(c, int)]
                # the driver refreshes its table about once a second: the first
                # second still shows the idle clocks before the window
                if time.perf_counter() - t0 >= 1.0:
                    self.samples.append((clks, m.get("current_socket_power"),
                                         m.get("temperature_hotspot")))
                self._stop.wait(0.1)
        except Exception as e:   # noqa: BLE001 -- optional instrumentation
            self.err = repr(e)[:120]

    def __enter__(self):
        self._th.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        self._th.join(timeout=5)

    def summary(self):
        if not self.samples:
            return {"error": self.err} if self.err else None
        clks = [c for s in self.samples for c in s[0]]
        pw = [s[1] for s in self.samples if isinstance(s[1], (int, float))]
        tp = [s[2] for s in self.samples if isinstance(s[2], (int, float))]
        rng = (lambda v: [min(v), statistics.median(v), max(v)] if v else None)  # noqa: E731
        return {"samples_after_first_second": len(self.samples),
                "gfxclk_mhz_per_xcd_min_median_max": rng(clks),
                "socket_power_w_min_median_max": rng(pw), "hotspot_c_min_median_max": rng(tp)}


def sustained(step, flops: float, seconds: float = SUSTAINED_S) -> dict:
    """The headline GEMM back to back for `seconds` of GPU time, an event
    after every step (the queue is kept about 64 steps deep, so the GPU never
    idles): min / median / mean of the per-step times over the whole window,
    the mean over its last second, and the mean of its first 100 steps (the
    regime of the short timed window); the driver's clock, power and
    temperature readings over the window beside them."""
    import torch
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    step()
    t1.record(stream)
    torch.cuda.synchronize()
    n = max(200, int(seconds * 1e3 / max(t0.elapsed_time(t1), 1e-3)))
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    with ClockSampler() as clocks:
        evs[0].record(stream)
        for i in range(n):
            step()
            evs[i + 1].record(stream)
            if i >= 64:
                evs[i - 63].synchronize()
        torch.cuda.synchronize()
    per = [evs[i].elapsed_time(evs[i + 1]) for i in range(n)]
    span = evs[0].elapsed_time(evs[-1])
    acc, last = 0.0, []
    for p in reversed(per):
        if acc >= 1000.0:
            break
        acc += p
        last.append(p)
    st = _stats(per)
    first = sum(per[:100]) / 100
    last_mean = sum(last) / len(last)
    by_second, acc, seg = [], 0.0, []
    for p in per:   # mean step time of each second of the window
        seg.append(p)
        acc += p
        if acc >= 1000.0:
            by_second.append(round(sum(seg) / len(seg), 4))
            acc, seg = 0.0, []
    return {"steps": n, "seconds": round(span / 1e3, 3), "ms_min": st["min"],
            "ms_median": st["median"], "ms_mean": st["mean"],
            "ms_mean_first_100": round(first, 5), "ms_mean_last_second": round(last_mean, 5),
            "tflops_mean": round(flops / st["mean"] / 1e9, 3),
            "tflops_last_second": round(flops / last_mean / 1e9, 3),
            "ms_mean_by_second": by_second[:60],
            "driver_readings": clocks.summary()}


def secondary(dev, only=SECONDARY) -> dict:
    """Benchmark configs 1, 3, 4, 5 (ms, TFLOPS; GB/s for the HBM-near batched one)."""
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
        """(per-replay device ms from graph replay, eager ms of the Python call loop)."""
        eager = time_events(fn, iters, warmup)
        return time_graph(fn, per_call_ms=eager), eager

    def rec(name, times, flops, bytes_=None, cfg=None):
        per, eager = times
        st = _stats(per)
        ms = st["mean"]
        d = {"ms": ms, "ms_min": st["min"], "ms_median": st["median"],
             "ms_eager_python": round(eager, 5),
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
        f3 = 2 * 2048 * 2048 * 1024
        ms = both(lambda: mt.gemm(A, B.t(), out=C, ws=ws), 100, 10)
        rec("c3a_2048x2048x1024_bT_view", ms, f3, None, mt.last_config())
        # the same product with Bᵀ materialised first: a strided copy into a
        # dense [1024,2048] buffer (what contiguous() does), then the GEMM
        Bt = torch.empty(1024, 2048, device=dev)
        ws_m = ws_for(A, Bt, C)
        ms = both(lambda: (mt.axpby(B.t(), Bt), mt.gemm(A, Bt, out=C, ws=ws_m)), 100, 10)
        rec("c3a_materialised_copy_plus_gemm", ms, f3, None, mt.last_config())
        ms = both(lambda: mt.gemm(A, Bt, out=C, ws=ws_m), 100, 10)
        rec("c3a_gemm_on_materialised_copy", ms, f3, None, mt.last_config())
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
        fc = 2 * 6272 * 256 * 2304
        ms = both(lambda: mt.conv2d(x, w, cb, 1, 1, ws=cws), 100, 10)
        rec("c5a_conv3x3_n32_c256_14x14", ms, fc,
            4 * (x.numel() + w.numel() + cb.numel() + 32 * 256 * 196), mt.last_config())
        # the same layer's backward: dX (implicit, flipped weights) and dW (+ db)
        dy = n(32, 256, 14, 14, std=0.01)
        bws = mt.workspace(mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d)), dev)
        dwb = torch.empty_like(w)
        ms = both(lambda: mt.conv2d_backward(x, w, dy, 1, 1, need_dw=False, need_db=False,
                                             ws=bws), 100, 10)
        rec("c5a_conv_backward_dx", ms, fc, None, mt.last_config())
        ms = both(lambda: mt.conv2d_backward(x, w, dy, 1, 1, need_dx=False, ws=bws, dw=dwb),
                  100, 10)
        rec("c5a_conv_backward_dw_db", ms, fc, None, mt.last_config())

    if "c5b" in only:  # batched 64 x [512,64]·[64,512]
        A, B = u(64, 512, 64), u(64, 64, 512)
        C = torch.empty(64, 512, 512, device=dev)
        ws = ws_for(A, B, C)
        ms = both(lambda: mt.gemm(A, B, out=C, ws=ws), 200, 20)
        rec("c5b_bmm_64x512x512x64", ms, 2 * 64 * 512 * 512 * 64,
            4 * 64 * (512 * 64 + 64 * 512 + 512 * 512), mt.last_config())

    if "resnet" in only:  # (hw, c_in, c_out, k): stride 1, "same" padding, batch 32
        for hw, c, co, k in RESNET_LAYERS:
            x = n(32, c, hw, hw)
            w = n(co, c, k, k, std=(2.0 / (c * k * k)) ** 0.5)
            cb = torch.zeros(co, device=dev)
            d = mt.Conv2dDesc(32, c, hw, hw, co, k, k, 1, k // 2)
            cws = mt.workspace(mt.lib().mt_conv2d_workspace_f32(ctypes.byref(d)), dev)
            ms = both(lambda: mt.conv2d(x, w, cb, 1, k // 2, ws=cws), 50, 5)
            rec(f"resnet_conv{k}x{k}_{hw}x{hw}_{c}to{co}", ms, 2 * 32 * hw * hw * co * c * k * k,
                4 * (x.numel() + w.numel() + co + 32 * co * hw * hw), mt.last_config())

    if "resnet_bwd" in only:  # batch 32; dX and dW + db of each layer
        for hw, c, co, k, st, pd in RESNET_BWD_LAYERS:
            ho = (hw + 2 * pd - k) // st + 1
            x = n(32, c, hw, hw)
            w = n(co, c, k, k, std=(2.0 / (c * k * k)) ** 0.5)
            dy = n(32, co, ho, ho, std=0.01)
            d = mt.Conv2dDesc(32, c, hw, hw, co, k, k, st, pd)
            bws = mt.workspace(mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d)), dev)
            dwb = torch.empty_like(w)
            f = 2 * 32 * ho * ho * co * c * k * k
            tag = f"resnet_bwd_conv{k}x{k}s{st}_{hw}x{hw}_{c}to{co}"
            ms = both(lambda: mt.conv2d_backward(x, w, dy, st, pd, need_dw=False, need_db=False,
                                                 ws=bws), 50, 5)
            rec(f"{tag}_dx", ms, f, None, mt.last_config())
            ms = both(lambda: mt.conv2d_backward(x, w, dy, st, pd, need_dx=False, ws=bws,
                                                 dw=dwb), 50, 5)
            rec(f"{tag}_dw_db", ms, f, None, mt.last_config())

    if "skinny" in only:
        # The reference's HBM-bound matmul rows (test/benchmark.cpp:732,737-738,
        # bench_matmul(M, N, K)): vector x matrix, the outer product and 63
        # rows, contiguous row-major, bytes = (MK + KN + MN)·4 as the
        # reference counts them (test/benchmark.cpp:168).
        for m, k, nn in ((1, 4096, 4096), (4096, 1, 4096), (63, 4096, 4096)):
            A, B = u(m, k), u(k, nn)
            C = torch.empty(m, nn, device=dev)
            ws = ws_for(A, B, C)
            ms = both(lambda: mt.gemm(A, B, out=C, ws=ws), 200, 20)
            rec(f"skinny_{m}x{k}x{nn}", ms, 2 * m * nn * k, 4 * (m * k + k * nn + m * nn),
                mt.last_config())
    return out


def attach_cpu(sec: dict, cpu: dict) -> None:
    """Adds each config's CPU baseline (and the GPU speed-up over it) to its entry."""
    for name, c in cpu.items():
        if name in sec:
            c = dict(c)
            c["gpu_speedup"] = round(c["ms_full_est"] / sec[name]["ms"], 1)
            sec[name]["cpu"] = c


def _pin_one_core():
    try:
        os.sched_setaffinity(0, {sorted(os.sched_getaffinity(0))[0]})
    except (AttributeError, OSError):
        pass


def _host_desc() -> str:
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return f"host {cpu_model}, {os.cpu_count()} cpus visible"


def _cpu_time(fn, reps: int) -> float:
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
    return best


def cpu_baseline() -> dict:
    """The C restatement of the reference matmul_cpu on a bounded row sample
    of the 4096^3 GEMM, 1 thread pinned (the headline's CPU baseline)."""
    import numpy as np
    import oracle

    rows = 64
    _pin_one_core()
    a = oracle.uniform((rows, 4096), 42)
    b = oracle.uniform((4096, 4096), 43)
    c = np.empty((rows, 4096), np.float32)
    dt = _cpu_time(lambda: oracle.lib().ora_matmul(oracle._fp(a), oracle._fp(b), oracle._fp(c),
                                                    rows, 4096, 4096), 1)
    flops = 2.0 * rows * 4096 * 4096
    return {"value": round(flops / dt / 1e12, 6), "unit": "TFLOPS", "cores": 1, "kind": "port",
            "sample": f"C[{rows},4096] = A[{rows},4096]·B[4096,4096] ({rows} of the 4096 rows "
                      f"of the headline GEMM), 1 rep, C restatement of the reference "
                      f"matmul_cpu (oracle/oracle.c, include/TensorOps.hpp:139-160; bit-exact "
                      f"with the reference's own build), -O2 -ffp-contract=off, 1 thread "
                      f"pinned; {dt:.2f} s; {_host_desc()}",
            "seconds": round(dt, 3),
            "ms_full_est": round(dt * 1e3 * 4096 / rows, 1)}


def cpu_config_baselines() -> dict:
    """CPU baselines of the secondary configs: the oracle's restatement of the
    reference CPU path on a bounded sample of each workload, best of `reps`,
    extrapolated linearly to the full workload.  About 15 s in total."""
    import numpy as np
    import oracle

    _pin_one_core()
    out = {}

    def rec(name, secs, scale, reps, sample, path):
        out[name] = {"ms_full_est": round(secs * 1e3 * scale, 2), "sample_ms": round(secs * 1e3, 2),
                     "reps": reps, "cores": 1, "kind": "port",
                     "sample": sample, "path": path}

    a = oracle.uniform((256, 512), 42)
    b = oracle.uniform((512, 512), 43)
    rec("c1_256x512x512", _cpu_time(lambda: oracle.matmul(a, b), 3), 1.0, 3,
        "the whole GEMM", "matmul_cpu (include/TensorOps.hpp:139-160)")

    A = oracle.normal((2048, 1024), 42)
    B = oracle.normal((2048, 1024), 43)
    rows = 256
    rec("c3a_2048x2048x1024_bT_view", _cpu_time(lambda: oracle.matmul(A[:rows], B.T), 3),
        2048 / rows, 3, f"{rows} of 2048 rows, B as a transpose view",
        "matmul_cpu_strided (include/TensorOps.hpp:162-189)")
    rec("c3b_1920x2048x1024_slice_bT_view",
        _cpu_time(lambda: oracle.matmul(A[128:128 + rows], B.T), 3), 1920 / rows, 3,
        f"{rows} of 1920 rows of the slice A[128:], B as a transpose view",
        "matmul_cpu_strided (include/TensorOps.hpp:162-189)")

    X = oracle.normal((256, 2048), 42)
    W = oracle.normal((1000, 2048), 43, std=(2.0 / 2048) ** 0.5)
    dY = oracle.normal((256, 1000), 44, std=0.01)
    t_f = _cpu_time(lambda: oracle.matmul(X[:64], W.T), 3)
    t_dx = _cpu_time(lambda: oracle.matmul(dY[:64], W), 3)
    t_dw = _cpu_time(lambda: oracle.matmul(dY.T[:250], X), 3)
    t_db = _cpu_time(lambda: oracle.colsum(dY), 3)
    path4 = "matmul_cpu_strided through transpose views (include/Autograd.hpp:117-147)"
    rec("c4_linear_fwd", t_f, 256 / 64, 3, "64 of 256 rows of Y = X·Wᵀ", path4)
    rec("c4_linear_dx", t_dx, 256 / 64, 3, "64 of 256 rows of dX = dY·W", path4)
    rec("c4_linear_dw_db", t_dw, 1000 / 250, 3, "250 of 1000 rows of dW = dYᵀ·X (db: whole)",
        path4 + " + sum_cpu for db (include/TensorOps.hpp:190-233)")
    out["c4_linear_dw_db"]["ms_full_est"] = round((t_dw * 1000 / 250 + t_db) * 1e3, 2)
    rec("c4_linear_fwd_bwd_total", 0.0, 1.0, 3, "sum of the three rows above", path4)
    out["c4_linear_fwd_bwd_total"]["ms_full_est"] = round(
        sum(out[k]["ms_full_est"] for k in ("c4_linear_fwd", "c4_linear_dx", "c4_linear_dw_db")),
        2)

    x = oracle.normal((32, 256, 14, 14), 42)
    w = oracle.normal((256, 256, 3, 3), 43, std=(2.0 / 2304) ** 0.5)
    imgs = 4
    rec("c5a_conv3x3_n32_c256_14x14",
        _cpu_time(lambda: oracle.conv2d(x[:imgs], w, np.zeros(256, np.float32), 1, 1), 1),
        32 / imgs, 1, f"{imgs} of 32 images", "conv2d_cpu (include/TensorOps.hpp:235-273)")

    Ab = oracle.uniform((64, 512, 64), 42)
    Bb = oracle.uniform((64, 64, 512), 43)
    nb = 16
    rec("c5b_bmm_64x512x512x64", _cpu_time(lambda: oracle.bmm(Ab[:nb], Bb[:nb]), 3), 64 / nb, 3,
        f"{nb} of 64 batch entries", "matmul_cpu per batch entry (bmm's loop, "
        "include/TensorOps.hpp:933-991)")
    return out


def copy_probe(dev) -> None:
    """Five copies of a 256 MiB tensor (__amd_rocclr_copyBuffer): reads and
    writes 256 MiB each, the calibration of FETCH_SIZE / WRITE_SIZE.  Then
    five fills of a 64 MiB tensor: a write-only stream, the reference for
    store-bound kernels."""
    import torch
    src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    out = torch.empty(16 << 20, dtype=torch.float32, device=dev)
    for _ in range(5):
        out.fill_(2.0)
    torch.cuda.synchronize()


def planner_audit(dev, seed: int, count: int) -> None:
    """The cost model's pick against the best forced plan (direct-to-LDS
    configurations at splits 1-16, wave-split configurations unsplit) on
    random row-major GEMMs: how far the planner is from the fastest kernel
    this library has for each shape."""
    import numpy as np
    import torch
    import minitensor_amd as mt

    rng = np.random.default_rng(seed)
    ws = mt.workspace(1 << 28, dev)

    def med(per):
        per = sorted(per)
        return per[len(per) // 2] * 1e3

    def dim():
        return int(2 ** rng.uniform(6, 12.2)) // 4 * 4

    cands = ([(mt.FAMILY_DL, c, s) for c in range(mt.config_count(mt.FAMILY_DL))
              for s in (1, 2, 3, 4, 6, 8, 12, 16)] +
             [(mt.FAMILY_KSW, c, 1) for c in range(mt.config_count(mt.FAMILY_KSW))])
    ratios = []
    for _ in range(count):
        M, N, K = dim(), dim(), dim()
        if M * N * K > 2 ** 33:
            K = max(64, 2 ** 33 // (M * N)) // 4 * 4
        A = torch.rand(M, K, device=dev) - 0.5
        B = torch.rand(K, N, device=dev) - 0.5
        C = torch.empty(M, N, device=dev)
        fn = lambda: mt.gemm(A, B, out=C, ws=ws)
        fn()
        torch.cuda.synchronize()
        auto_t, auto_c = med(time_graph(fn)), mt.last_config()
        best_t, best_c = auto_t, auto_c
        for fam, c, s in cands:
            with mt.forced_config(fam, c, s):
                try:
                    fn()
                    torch.cuda.synchronize()
                except RuntimeError:
                    continue
                name = mt.last_config()
                if not name.endswith(f"cfg={c}"):
                    continue   # the family cannot take these operands
                t = med(time_graph(fn, calls=20, replays=5, preroll_ms=5))
                if t < best_t:
                    best_t, best_c = t, name
        ratios.append(auto_t / best_t)
        print(f"{M}x{N}x{K}: auto {auto_t:.2f} us [{auto_c}], best {best_t:.2f} us [{best_c}], "
              f"ratio {auto_t / best_t:.3f}", flush=True)
    r = np.array(ratios)
    print(json.dumps({"shapes": count, "seed": seed, "within_5pct": int((r <= 1.05).sum()),
                      "within_10pct": int((r <= 1.10).sum()),
                      "geomean_ratio": round(float(np.exp(np.log(r).mean())), 4),
                      "worst_ratio": round(float(r.max()), 3)}), flush=True)


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
    M = N = K = 4096
    flops = 2.0 * M * N * K

    def headline_step():
        g = torch.Generator(device=dev)
        g.manual_seed(42)
        A = torch.rand(M, K, device=dev, generator=g) * 2 - 1
        B = torch.rand(K, N, device=dev, generator=g) * 2 - 1
        C = torch.empty(M, N, device=dev)
        ws = mt.workspace(mt.lib().mt_gemm_workspace_f32(mt.mat(A), mt.mat(B), mt.mat(C)), dev)
        return lambda: mt.gemm(A, B, out=C, ws=ws)

    if args.audit:
        seed, count = (int(x) for x in args.audit.split(":"))
        planner_audit(dev, seed, count)
        return
    if args.only:
        names = tuple(x.strip() for x in args.only.split(",") if x.strip())
        unknown = [x for x in names if x not in SECONDARY + EXTRA + ("sustained",)]
        if unknown:
            print(f"bench.py: unknown --only entries {unknown}; choose from "
                  f"{SECONDARY + EXTRA + ('sustained',)}", file=sys.stderr)
            sys.exit(2)
        res = {"secondary": secondary(dev, tuple(x for x in names if x != "sustained"))}
        if "sustained" in names:
            step = headline_step()
            for _ in range(args.warmup):
                step()
            res["sustained"] = sustained(step, flops, args.sustained_seconds)
            res["sustained"]["kernel"] = mt.last_config()
        if args.copy_probe:
            copy_probe(dev)
        print(json.dumps(res), flush=True)
        return
    step = headline_step()

    t0 = time.perf_counter()
    span_ms, per_ms, n_pre = time_steps(step, args.steps, args.warmup)
    wall = time.perf_counter() - t0
    ms = span_ms / args.steps
    kernel_cfg = mt.last_config()
    tflops = flops / ms / 1e9
    st = _stats(per_ms)
    ref_win = reference_window(step)
    ref_win["tflops"] = round(flops / ref_win["ms_mean"] / 1e9, 3)
    sus = sustained(step, flops, args.sustained_seconds)

    if args.copy_probe:
        copy_probe(dev)

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
        "ms_per_step_min": st["min"],
        "ms_per_step_median": st["median"],
        "tflops_at_min": round(flops / st["min"] / 1e9, 3),
        "tflops_at_median": round(flops / st["median"] / 1e9, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (U(-1,1), torch generator seed 42, resident in HBM)",
        "config": {"workload": "benchmark config 2: C[4096,4096] = A[4096,4096]·B[4096,4096] "
                               "fp32 row-major GEMM", "M": M, "N": N, "K": K,
                   "kernel": kernel_cfg, "preroll_steps": n_pre,
                   "wall_s_warmup_preroll_timed": round(wall, 4)},
        "reference_window": ref_win,
        "sustained": sus,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 3), "peak": PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_TFLOPS, 4),
                     "traffic": traffic},
    }
    if not args.no_secondary:
        line["secondary"] = secondary(dev)
    if not args.no_cpu:   # after every GPU leg, so the GPU never idles between them
        line["cpu_baseline"] = cpu_baseline()
        if not args.no_secondary:
            attach_cpu(line["secondary"], cpu_config_baselines())
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
