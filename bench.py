#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-inference hot path (one GPU).

Headline (the JSON `value`): INT4 group-128 dequant-GEMV, BASELINE config 3 at
M=1: W [14336, 4096] packed INT4 + f16 group scales, x bf16 [1, 4096], y f32.
A step is one decode GEMV over one token; inputs are resident in HBM and the
weights rotate over enough copies (> 2x the 256 MB MALL) that every step
streams them from HBM.  The timed region is a HIP graph of `--steps`
launches bracketed by events on the launch stream.

Secondary workloads (reported in `secondary`): INT8 and FP8 GEMV (config 2), INT4
GEMV at M=2..16, W8A8 GEMM at M=2048 (config 4) in INT8 and in FP8 e4m3,
per-row INT8 quantize /
dequantize round trip (config 1) and the INT4 FFN block (config 5).

`cpu_baseline` times the C restatement of the reference CPU path (oracle/,
f64 Linear::forward over the dequantized weight, which Linear::from_tensors
holds) on the headline workload, single-threaded; each secondary config carries
its own `cpu_baseline` timed the same way (configs 4 and 5 from row subsets,
extrapolated as gather + rows).  `measured_peaks` re-measures the roofline
denominators on the device (HBM stream over 4 GiB, i8 / bf16 MFMA loops) and
`read_ceiling_30mb` times a plain streaming read of the headline's bytes with
the headline's harness.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "neo-theano_amd"))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
I8_PEAK_TOPS = 5000.0        # dense int8 MFMA, 5.0 POP/s
FP8_PEAK_TFLOPS = 5000.0     # dense fp8 MFMA, 5.0 PFLOP/s
BF16_PEAK_TFLOPS = 2500.0    # dense bf16 MFMA
MALL_BYTES = 256 << 20
METRIC = "INT4/INT8 dequant-GEMV GB/s (% HBM peak) + W8A8 GEMM TOPS (% MFMA peak)"


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--only", default=None,
                   help="run one workload: gemv_w4, gemv_w8, gemv_fp8, gemv_w4_m, peaks, read_ceiling, read_sweep, "
                        "quant_i4, w8a8_decode, w8a8, fp8, mha, storage, roundtrip, mlp, mlp_mid, mlp_decode, copy")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="bound of the CPU baseline sample (0: skip)")
    p.add_argument("--eager", action="store_true", help="time eager launches instead of a HIP graph")
    p.add_argument("--reps", type=int, default=5, help="timed replays of the K launches (median reported)")
    return p.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timer:
    """Times `steps` calls of launch(i), bracketed by events on the stream the
    launches go to, and returns (ms per step, mode) in ONE fixed mode: "hip
    graph", the launches captured into a hipGraph by libtq_peaks.so's
    tqp_graph_time and replayed on its own stream (what a host that calls the C
    ABI directly sees).  Only when that capture fails does it fall back to a
    torch.cuda.graph replay ("torch graph"), and only with --eager to eager
    launches.  With `diagnostics=True`, `last` also holds the torch-graph and
    eager times of the same launches; they are never what `run` returns.
    Short kernels need a graph: a Python launch takes longer than the
    kernel."""

    def __init__(self, torch, eager=False, reps=1):
        self.torch = torch
        self.eager = eager
        self.reps = reps  # timed replays of the `steps` launches; the median is returned
        self.last = {}

    def run(self, launch, steps, warmup, diagnostics=False):
        self.last = {}
        if self.eager:
            res = self._run(launch, steps, warmup, graph=False)
            self.last[res[1]] = res[0]
            return res
        nat = self._native(launch, steps, warmup)
        if nat is not None:
            self.last["hip graph"] = nat
            if diagnostics:
                tg = self._run(launch, steps, 0, graph=True)
                self.last["torch graph" if tg[1] == "graph" else tg[1]] = tg[0]
                ea = self._run(launch, steps, 0, graph=False)
                self.last["eager"] = ea[0]
            return nat, "hip graph"
        res = self._run(launch, steps, warmup, graph=True)
        mode = "torch graph" if res[1] == "graph" else res[1]
        self.last[mode] = res[0]
        return res[0], mode

    def _native(self, launch, steps, warmup):
        """Median ms per step of a hipGraph replay (tqp_graph_time), or None
        when the launches cannot be captured that way."""
        import ctypes

        torch = self.torch
        try:
            L = _peaks_lib()
        except Exception as e:  # not built
            log(f"native graph timing unavailable ({e})")
            return None
        failed = []

        def cb(i, s):
            try:
                with torch.cuda.stream(torch.cuda.ExternalStream(s)):
                    launch(i)
                return 0
            except Exception as e:  # reported below, after the capture has ended
                failed.append(e)
                return 1

        fn = L.tqp_launch_fn(cb)
        us = (ctypes.c_float * self.reps)()
        rc = L.tqp_graph_time(fn, steps, warmup, self.reps, us)
        torch.cuda.synchronize()
        if rc != 0 or failed:
            log(f"native graph timing failed (hipError {rc}{', ' + str(failed[0]) if failed else ''}); "
                "using torch's graph")
            return None
        t = sorted(us[i] for i in range(self.reps))
        return t[len(t) // 2] * 1e-3

    def _run(self, launch, steps, warmup, graph):
        torch = self.torch
        for i in range(warmup):
            launch(i)
        torch.cuda.synchronize()
        mode = "eager"
        g = None
        if graph:
            try:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for i in range(steps):
                        launch(i)
                g.replay()
                torch.cuda.synchronize()
                mode = "graph"
            except Exception as e:  # capture unsupported: fall back to eager launches
                log(f"graph capture failed ({e}); timing eager launches")
                g = None
        times = []
        for _ in range(self.reps):
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            start.record()
            if g is not None:
                g.replay()
            else:
                for i in range(steps):
                    launch(i)
            end.record()
            end.synchronize()
            torch.cuda.synchronize()
            times.append(start.elapsed_time(end))
        times.sort()
        return times[len(times) // 2] / steps, mode


def _peaks_lib():
    import ctypes

    path = os.path.join(ROOT, "neo-theano_amd", "libtq_peaks.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run `python neo-theano_amd/build.py`")
    L = ctypes.CDLL(path)
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    L.tqp_hbm_read.argtypes = [vp, i64, vp, i32, vp]
    L.tqp_launch_fn = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_int, ctypes.c_void_p)
    L.tqp_graph_time.argtypes = [L.tqp_launch_fn, i32, i32, i32, ctypes.POINTER(ctypes.c_float)]
    L.tqp_graph_time.restype = i32
    L.tqp_hbm_read_chunks.argtypes = [vp, i64, vp, i32, vp]
    L.tqp_hbm_read_waves.argtypes = [vp, i64, vp, i32, i32, vp]
    L.tqp_gemv_w4_skeleton.argtypes = [vp, vp, vp, i64, i64, vp, vp]
    L.tqp_gemm_w8a8_phases.argtypes = [vp, vp, vp, vp, i32, i32, i32, vp, vp, vp]
    for fn in (L.tqp_mfma_i8, L.tqp_mfma_bf16, L.tqp_mfma_i8_random, L.tqp_mfma_bf16_random):
        fn.argtypes = [i32, i32, vp, vp]
    return L


def measured_peaks(torch, timer, dev, log):
    """HBM read rate over a 4 GiB buffer (16x the MALL) and the dense i8 / bf16
    MFMA rates of register-only loops, one 4-wave block per CU (the layout of
    the GEMM kernels) and four, on this device: with constant operands and
    with pseudo-random ones (`*_random_operands`), which draw the power real
    data does (the part then runs the matrix cores at a lower clock)."""
    import ctypes

    L = _peaks_lib()
    st = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    nb = 4 << 30
    buf = torch.empty(nb, dtype=torch.uint8, device=dev).fill_(1)
    out = torch.empty(1 << 20, dtype=torch.int32, device=dev)
    best = None
    for blocks in (4 * cus, 8 * cus, 16 * cus):
        ms, _ = timer.run(lambda i, b=blocks: L.tqp_hbm_read(buf.data_ptr(), nb, out.data_ptr(), b, st()), 5, 1)
        gbs = nb / (ms * 1e-3) / 1e9
        if best is None or gbs > best[0]:
            best = (gbs, blocks)
    del buf
    res = {"hbm_read_GB/s": round(best[0], 1), "hbm_read_blocks": best[1], "hbm_read_bytes": nb,
           "hbm_spec_GB/s": HBM_PEAK_GBS}
    iters = 400
    for name, fn, fr, per, spec in (("i8_mfma_TOPS", L.tqp_mfma_i8, L.tqp_mfma_i8_random, 65536, I8_PEAK_TOPS),
                                    ("bf16_mfma_TFLOPS", L.tqp_mfma_bf16, L.tqp_mfma_bf16_random, 32768,
                                     BF16_PEAK_TFLOPS)):
        for suffix, f in (("", fn), ("_random_operands", fr)):
            vals = {}
            for bpc in (1, 4):
                blocks = bpc * cus
                ms, _ = timer.run(lambda i, b=blocks, f=f: f(b, iters, out.data_ptr(), st()), 5, 1)
                vals[bpc] = blocks * 4 * 8 * iters * per / (ms * 1e-3) / 1e12
            res[name + suffix] = round(max(vals.values()), 1)
            res[name + suffix + "_1_block_per_cu"] = round(vals[1], 1)
        res[name.replace("_T", "_spec_T")] = spec
    log(f"measured peaks: {res}")
    return res


def read_ceiling(torch, timer, dev, nbytes, args, log):
    """A plain streaming read of `nbytes` per launch (16-byte nontemporal loads,
    no arithmetic), over copies rotating past the MALL, timed by the headline's
    harness: the rate one launch of this size reaches on this device."""
    import ctypes

    L = _peaks_lib()
    st = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    n16 = nbytes // 16 * 16
    copies = [torch.empty(n16, dtype=torch.uint8, device=dev).fill_(1) for _ in range(rotation(n16))]
    out = torch.empty(1 << 16, dtype=torch.int32, device=dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    res = {"bytes": n16, "variants": {}}
    best = None
    shapes = [("grid-stride", b) for b in (2 * cus, 4 * cus, 8 * cus, 16 * cus, 32 * cus)]
    shapes += [("one-pass", u) for u in (4, 8, 16)]
    shapes += [("waves", lw) for lw in ((8, 3), (8, 8), (16, 3))]
    for kind, a in shapes:
        if kind == "grid-stride":
            fn = lambda i, b=a: L.tqp_hbm_read(copies[i % len(copies)].data_ptr(), n16, out.data_ptr(), b, st())
            label = f"grid-stride, {a} blocks"
        elif kind == "one-pass":
            fn = lambda i, u=a: L.tqp_hbm_read_chunks(copies[i % len(copies)].data_ptr(), n16, out.data_ptr(), u,
                                                      st())
            label = f"one-pass, {(n16 // 16 + 256 * a - 1) // (256 * a)} blocks of {4096 * a} B"
        else:  # the INT4 GEMV's access pattern without its arithmetic
            fn = lambda i, lw=a: L.tqp_hbm_read_waves(copies[i % len(copies)].data_ptr(), n16, out.data_ptr(), lw[0],
                                                      lw[1], st())
            label = (f"GEMV pattern, {(n16 // 16 + 1024 * a[0] - 1) // (1024 * a[0])} blocks of 16 waves, "
                     f"{a[0]} KB per wave, {a[1]} loads in flight")
        ms, mode = timer.run(fn, args.steps, args.warmup)
        gbs = n16 / (ms * 1e-3) / 1e9
        res["variants"][label] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1)}
        log(f"  read {n16} B, {label}: {ms * 1e3:.2f} us  {gbs:.0f} GB/s")
        if best is None or gbs > best[1]:
            best = (ms, gbs, label, mode)
    res.update({"us": round(best[0] * 1e3, 3), "GB/s": round(best[1], 1), "best": best[2], "timing": best[3],
                "hbm_frac": round(best[1] / HBM_PEAK_GBS, 4)})
    log(f"read ceiling {n16} B per launch: {best[0] * 1e3:.2f} us  {best[1]:.0f} GB/s ({best[2]})")
    del copies
    return res


def read_sweep(torch, timer, dev, args, log, headline_bytes):
    """Plain streaming reads of 8-240 MB per launch (the best of five read
    kernels at each size, buffers rotating past the MALL, the headline's
    harness), fitted as t(B) = t0 + B / R by least squares: t0 is what every
    launch pays whatever its size (dispatch, first-byte latency, drain) and R
    the rate at which the bytes themselves stream.  The fit then gives the
    fastest any one launch of the headline's bytes can read them."""
    import ctypes

    L = _peaks_lib()
    st = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = torch.empty(1 << 16, dtype=torch.int32, device=dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    sizes = [8 << 20, 16 << 20, headline_bytes // 16 * 16, 60 << 20, 120 << 20, 240 << 20]
    points = []
    res = {"sizes": {}}
    for nb in sizes:
        copies = [torch.empty(nb, dtype=torch.uint8, device=dev).fill_(1) for _ in range(rotation(nb))]
        best = None
        for kind, a in [("grid-stride", b) for b in (8 * cus, 16 * cus, 32 * cus)] + [("one-pass", u) for u in (4, 16)]:
            if kind == "grid-stride":
                fn = lambda i, b=a: L.tqp_hbm_read(copies[i % len(copies)].data_ptr(), nb, out.data_ptr(), b, st())
                label = f"grid-stride, {a} blocks"
            else:
                fn = lambda i, u=a: L.tqp_hbm_read_chunks(copies[i % len(copies)].data_ptr(), nb, out.data_ptr(), u,
                                                          st())
                label = f"one-pass, {4096 * a} B per block"
            ms, _ = timer.run(fn, args.steps, args.warmup)
            if best is None or ms < best[0]:
                best = (ms, label)
        us = best[0] * 1e3
        points.append((nb, us))
        res["sizes"][str(nb)] = {"us": round(us, 3), "GB/s": round(nb / (us * 1e-6) / 1e9, 1),
                                 "hbm_frac": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "best": best[1],
                                 "copies": len(copies)}
        log(f"read sweep {nb / 1e6:.1f} MB per launch: {us:.2f} us  {nb / (us * 1e-6) / 1e9:.0f} GB/s ({best[1]})")
        del copies
    n = len(points)
    mx = sum(b for b, _ in points) / n
    my = sum(t for _, t in points) / n
    slope = sum((b - mx) * (t - my) for b, t in points) / sum((b - mx) ** 2 for b, _ in points)  # us per byte
    t0 = my - slope * mx
    rate = 1e-3 / slope  # GB/s: bytes per us / 1e3
    hb = headline_bytes
    t_hb = t0 + slope * hb
    res.update({"fixed_us": round(t0, 3), "sustained_GB/s": round(rate, 1),
                "sustained_hbm_frac": round(rate / HBM_PEAK_GBS, 4),
                "fit_max_abs_residual_us": round(max(abs(t - (t0 + slope * b)) for b, t in points), 3),
                "headline_bytes": hb, "headline_fit_us": round(t_hb, 3),
                "headline_fit_GB/s": round(hb / (t_hb * 1e-6) / 1e9, 1),
                "headline_fit_hbm_frac": round(hb / (t_hb * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                "target_70pct_us": round(hb / (0.7 * HBM_PEAK_GBS * 1e9) * 1e6, 3)})
    log(f"read sweep fit: t = {t0:.2f} us + B / {rate:.0f} GB/s; headline bytes -> {t_hb:.2f} us "
        f"({res['headline_fit_hbm_frac'] * 100:.1f} % of spec; the 70 % target needs {res['target_70pct_us']:.2f} us)")
    return res


def cpu_baselines(args, secondary, n3, k3, headline_bytes, log):
    """The reference CPU path restated in C (oracle/, f64, one thread), timed on
    the host beside the GPU legs.  A quantized Linear in the reference is
    Linear::from_tensors over the dequantized weight (linear.rs:65-75), so a
    forward is Linear::forward (linear.rs:111-121): Tensor::mm gathers the
    transposed weight and runs the i-p-j loop (tensor_ops.rs:379-410); the
    dequantization happens once at load and is not timed.  Configs 4 and 5 are
    timed as one forward at M=1 (the gather plus one row) and the i-p-j loop
    alone (tqo_mm on the already transposed weight) over a row subset of M'
    rows, and extrapolated as t(M) = t(1) + (M - 1) * t_loop(M') / M': the
    gather is paid once per forward, the loop per row.  (A difference of two
    whole forwards, t(M') - t(1), drowns the rows in the run-to-run spread of
    the gather, which takes seconds at the FFN's sizes.)  Each secondary config
    gets its own `cpu_baseline`; the headline's is returned."""
    import numpy as np

    import oracle as O  # the CPU restatement of the reference path, timed as the baseline
    from theano_quantize.synth import f32_to_bf16_bits, normal_f32

    O.lib()
    ncpu = os.cpu_count()
    model = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    # the reference path is single-threaded: pin this thread to one core (the
    # first this process may use), as `taskset -c 0` would, for the whole baseline
    allowed = sorted(os.sched_getaffinity(0))
    core = allowed[0]
    os.sched_setaffinity(0, {core})

    def timed(fn, budget):
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget or reps >= 50:
                return el / reps, reps

    def bf16_f64(bits):
        return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)

    def entry(value, unit, sample):
        return {"value": value, "unit": unit, "cores": 1, "kind": "port",
                "sample": sample + f"; 1 thread pinned to core {core} of {len(allowed)} allowed ({ncpu} host CPUs, "
                                   f"{model})"}

    # C3, the headline: INT4 g128 weight [14336, 4096] dequantized once, one token
    w = normal_f32(2, (n3, k3), 0.02)
    p, s = O.quantize_i4_g128(w)
    wh = O.dequantize_i4_g128(p, s).astype(np.float64)
    del w, p, s
    x = bf16_f64(f32_to_bf16_bits(normal_f32(2, (1, k3), 1.0, stream=1)))
    per, reps = timed(lambda: O.linear(x, wh), args.cpu_seconds)
    head = entry(round(headline_bytes / per / 1e9, 4), "GB/s",
                 f"config 3 at M=1: Linear::forward over the dequantized [14336, 4096] weight, {reps} calls, "
                 f"{per * 1e3:.0f} ms per call")
    log(f"cpu baseline C3: {per * 1e3:.1f} ms/call")
    del wh

    budget = max(1.0, args.cpu_seconds / 6)
    # C1: per-row INT8 quantize and dequantize of W [4096, 4096]
    w = normal_f32(0, (4096, 4096), 0.02)
    tq_, _ = timed(lambda: O.quantize_i8_rowwise(w), budget)
    q, sc = O.quantize_i8_rowwise(w)
    td, _ = timed(lambda: O.dequantize_i8_rowwise(q, sc), budget)
    b1 = 5 * 4096 * 4096 + 4 * 4096
    if "roundtrip_i8_4096x4096" in secondary:
        secondary["roundtrip_i8_4096x4096"]["cpu_baseline"] = entry(
            {"quantize_GB/s": round(b1 / tq_ / 1e9, 4), "dequantize_GB/s": round(b1 / td / 1e9, 4)}, "GB/s",
            f"config 1 in full: quantize_tensor per row (f64) {tq_ * 1e3:.0f} ms, dequantize_tensor {td * 1e3:.0f} ms")
    # C2: INT8 weight [4096, 4096] dequantized once, one f32 token
    wh = O.dequantize_i8_rowwise(q, sc).astype(np.float64)
    x = normal_f32(1, (1, 4096), 1.0, stream=1).astype(np.float64)
    t2, _ = timed(lambda: O.linear(x, wh), budget)
    if "gemv_w8_m1" in secondary:
        secondary["gemv_w8_m1"]["cpu_baseline"] = entry(
            round(secondary["gemv_w8_m1"]["bytes"] / t2 / 1e9, 4), "GB/s",
            f"config 2 in full: Linear::forward over the dequantized weight, {t2 * 1e3:.0f} ms per call")
    # C4: activations [M, 4096] quantized per row then dequantized, Linear over the dequantized weight
    xa = normal_f32(3, (32, 4096), 1.0)

    wht = np.ascontiguousarray(wh.T)  # the transposed weight Tensor::mm gathers per forward

    def c4(m):
        qa, sa = O.quantize_i8_rowwise(xa[:m])
        O.linear(O.dequantize_i8_rowwise(qa, sa).astype(np.float64), wh)

    def c4_rows(m):  # the per-row part: quantize, dequantize and the i-p-j loop, no gather
        qa, sa = O.quantize_i8_rowwise(xa[:m])
        O.mm(O.dequantize_i8_rowwise(qa, sa).astype(np.float64), wht)

    t41, _ = timed(lambda: c4(1), 0)
    t4r, _ = timed(lambda: c4_rows(32), 0)
    t4 = t41 + (2048 - 1) * t4r / 32
    if "w8a8_gemm_m2048" in secondary:
        secondary["w8a8_gemm_m2048"]["cpu_baseline"] = entry(
            round(2.0 * 2048 * 4096 * 4096 / t4 / 1e12, 6), "TOPS",
            f"config 4: per-row quantize + dequantize + Linear::forward at M=1 ({t41 * 1e3:.0f} ms) and the "
            f"per-row part (quantize, dequantize, i-p-j loop) of M'=32 rows ({t4r * 1e3:.0f} ms), extrapolated "
            f"to M=2048: {t4:.1f} s")
    del wh, wht, w, q, sc
    # C5: gate / up [14336, 4096] and down [4096, 14336], each dequantized once
    if "mlp_w4g128_m512" in secondary:
        d5, f5, m5, mp = 4096, 14336, 512, 32
        tot = 0.0
        parts = []
        for name, shape, count in (("gate/up", (f5, d5), 2), ("down", (d5, f5), 1)):
            p5, s5 = O.quantize_i4_g128(normal_f32(4, shape, 0.02))
            wh5 = O.dequantize_i4_g128(p5, s5).astype(np.float64)
            del p5, s5
            x5 = normal_f32(4, (mp, shape[1]), 1.0, stream=3).astype(np.float64)
            ta, _ = timed(lambda: O.linear(x5[:1], wh5), 0)
            wt5 = np.ascontiguousarray(wh5.T)
            tb, _ = timed(lambda: O.mm(x5, wt5), 0)
            tm = ta + (m5 - 1) * tb / mp
            tot += count * tm
            parts.append(f"{name} {ta * 1e3:.0f} ms at M=1, i-p-j loop {tb * 1e3:.0f} ms for M'={mp} rows")
            del wh5, wt5
        secondary["mlp_w4g128_m512"]["cpu_baseline"] = entry(
            round(m5 / tot, 4), "tokens/s",
            f"config 5: Linear::forward (" + "; ".join(parts) + f"), extrapolated to M=512 and summed over "
            f"gate, up and down (SiLU * up not timed): {tot:.1f} s")
    os.sched_setaffinity(0, set(allowed))
    head["cpu_model"] = model
    head["pinned_core"] = core
    log("cpu baselines done")
    return head


def w8a8_phases(torch, np, ops, y, m, n, k, log, launches=5):
    """Per-wave phases of single launches of the W8A8 GEMM kernel (the library's
    kernel instantiated with real-time stamps in libtq_peaks.so): each timed
    launch follows five untimed back-to-back launches and a synchronization, so
    it runs warm but alone, unlike the back-to-back launches of the timed leg.
    Microseconds from the first wave's start, percentiles (0, 50, 100) over the
    1024 waves, medians over the launches.  The caller adds `mfma_floor_us`, the GEMM's MFMA time at the
    measured random-operand i8 rate of one block per CU, when the peaks leg
    ran."""
    import ctypes

    L = _peaks_lib()
    st = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    waves = (m // 128) * (n // 256) * 4
    ts = torch.zeros(waves * 6, dtype=torch.int64, device=y.device)
    runs = []
    for r in range(launches):
        for i in range(5):
            qa, sa, qw, sw = ops[(r * 6 + i) % len(ops)]
            L.tqp_gemm_w8a8_phases(qa.data_ptr(), sa.data_ptr(), qw.data_ptr(), sw.data_ptr(), m, n, k, y.data_ptr(),
                                   ts.data_ptr(), st())
        qa, sa, qw, sw = ops[(r * 6 + 5) % len(ops)]
        torch.cuda.synchronize()
        rc = L.tqp_gemm_w8a8_phases(qa.data_ptr(), sa.data_ptr(), qw.data_ptr(), sw.data_ptr(), m, n, k, y.data_ptr(),
                                     ts.data_ptr(), st())
        torch.cuda.synchronize()
        if rc != 0:
            raise RuntimeError(f"tqp_gemm_w8a8_phases: hipError {rc}")
        a = ts.view(waves, 6).cpu().numpy().astype(np.int64)
        rel = (a[:, :4] - a[:, 0].min()) * 0.01  # 100 MHz ticks -> us
        runs.append({"span": rel[:, 3].max(), "start": rel[:, 0], "first_stage": rel[:, 1] - rel[:, 0],
                     "k_loop": rel[:, 2] - rel[:, 1], "epilogue": rel[:, 3] - rel[:, 2]})
    med = lambda v: round(float(np.median(v)), 2)
    out = {"launches": launches, "span_us": med([r["span"] for r in runs])}
    for key in ("start", "first_stage", "k_loop", "epilogue"):
        out[key + "_us_p0_p50_p100"] = [med([np.percentile(r[key], p) for r in runs]) for p in (0, 50, 100)]
    log(f"w8a8 one launch: span {out['span_us']} us; K loop {out['k_loop_us_p0_p50_p100']} us; "
        f"epilogue {out['epilogue_us_p0_p50_p100']} us")
    return out


def rotation(bytes_per_copy):
    return max(2, math.ceil(2 * MALL_BYTES / bytes_per_copy) + 1)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the hot path has no "
              "multi-GPU component in this build", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    import theano_quantize as tq
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream
    from theano_quantize.synth import f32_to_bf16_bits, normal_f32

    tq._abi.lib()
    dev = torch.device("cuda", 0)
    timer = Timer(torch, eager=args.eager, reps=max(1, args.reps))
    secondary = {}

    def dt(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    def bf16(a):
        return dt(f32_to_bf16_bits(a).view(np.int16)).view(torch.bfloat16)

    def quant_copies(w, fn, copies):
        """Quantizes w once and makes `copies` device copies of its buffers."""
        base = fn(dt(w))
        return [tuple(t.clone() for t in base) for _ in range(copies)]

    only = args.only
    want = (lambda name: only is None or only == name)
    headline = None

    # ---------------------------------------------------------- headline
    n3, k3 = 14336, 4096
    w4_bytes = n3 * k3 // 2 + 2 * n3 * (k3 // 128)         # packed + f16 scales
    w4_bytes_m = lambda m: w4_bytes + 2 * m * k3 + 4 * m * n3  # + x bf16 + y f32
    if want("gemv_w4") or want("gemv_w4_m") or only is None:
        log("setup: config 3 INT4 g128 weights [14336, 4096], decode kernel layout")
        w = normal_f32(2, (n3, k3), 0.02)
        p0, s0 = tq.quantize_i4_g128(dt(w))
        pt0, st0, tile = tq.repack_i4_g128_tiled(p0, s0)
        copies = [(pt0.clone(), st0.clone(), p0.clone(), s0.clone()) for _ in range(rotation(w4_bytes))]
        del w, p0, s0, pt0, st0
        x = bf16(normal_f32(2, (16, k3), 1.0, stream=1))
        y = torch.empty((16, n3), dtype=torch.float32, device=dev)

        def gemv_w4(m):
            def launch(i):  # same dispatch as QuantizedLinear
                pt, st, p, s = copies[i % len(copies)]
                if m <= tq.nn.TILED_MAX_M:
                    _abi.call("tq_gemv_w4g128_tiled", ptr(x), m, ptr(pt), ptr(st), None, n3, k3, tile, ptr(y),
                              stream())
                else:
                    _abi.call("tq_gemv_w4g128", ptr(x), m, ptr(p), ptr(s), None, n3, k3, ptr(y), stream())
            return launch

        if want("gemv_w4"):
            ms, mode = timer.run(gemv_w4(1), args.steps, args.warmup, diagnostics=True)
            gbs = w4_bytes_m(1) / (ms * 1e-3) / 1e9
            headline = {"ms": ms, "gbs": gbs, "mode": mode, "modes_us": {k: round(v * 1e3, 3) for k, v in timer.last.items()}}
            log(f"gemv_w4 M=1: {ms * 1e3:.2f} us/step  {gbs:.0f} GB/s  ({mode})")
            if tile == 64 and not args.no_secondary:
                # the same launch with its arithmetic left out (libtq_peaks.so): what the
                # loads, x staging and block reduction of this kernel cost on their own
                Lp = _peaks_lib()
                sk_out = torch.empty(2 * (n3 // 64) * 64, dtype=torch.int32, device=dev)

                def skeleton(i):
                    pt, st, _, _ = copies[i % len(copies)]
                    rc = Lp.tqp_gemv_w4_skeleton(ptr(x), ptr(pt), ptr(st), n3, k3, ptr(sk_out), stream())
                    if rc != 0:
                        raise RuntimeError(f"tqp_gemv_w4_skeleton: hipError {rc}")

                mss, modes = timer.run(skeleton, args.steps, args.warmup)
                secondary["gemv_w4g128_m1_loads_only"] = {
                    "us": round(mss * 1e3, 3), "GB/s": round(w4_bytes_m(1) / (mss * 1e-3) / 1e9, 1), "timing": modes,
                    "note": "the headline launch with the nibble unpack and MFMAs replaced by an xor fold: same loads, "
                            "x staging and block reduction"}
                log(f"gemv_w4 M=1 without arithmetic: {mss * 1e3:.2f} us/step")
        if not args.no_secondary and (only is None or only == "gemv_w4_m"):
            for m in (2, 4, 8, 16):
                ms, mode = timer.run(gemv_w4(m), args.steps, args.warmup)
                gbs = w4_bytes_m(m) / (ms * 1e-3) / 1e9
                secondary[f"gemv_w4g128_m{m}"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "timing": mode,
                                                  "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
                log(f"gemv_w4 M={m}: {ms * 1e3:.2f} us/step  {gbs:.0f} GB/s")
        del copies

    # ------------------------------------- roofline denominators, measured
    peaks = None
    if not args.no_secondary and (only is None or only == "peaks"):
        peaks = measured_peaks(torch, timer, dev, log)
        secondary["measured_peaks"] = peaks

    def of_random_peak(rate, key):
        # fraction of the matrix-core rate measured on random operands (None when
        # the peaks leg did not run)
        return round(rate / peaks[key], 4) if peaks else None

    # ----------------- plain streaming read of the headline's bytes per launch
    if not args.no_secondary and (only is None or only == "read_ceiling"):
        secondary["read_ceiling_30mb"] = read_ceiling(torch, timer, dev, w4_bytes_m(1), args, log)
    if not args.no_secondary and (only is None or only == "read_sweep"):
        secondary["read_sweep"] = read_sweep(torch, timer, dev, args, log, w4_bytes_m(1))

    # ------------------------------------- INT4 g128 quantize + pack (C3 weight)
    if not args.no_secondary and want("quant_i4"):
        nq = rotation(4 * n3 * k3)
        ins = [dt(normal_f32(2, (n3, k3), 0.02, stream=10 + i)) for i in range(nq)]
        pq = torch.empty((n3, k3 // 2), dtype=torch.uint8, device=dev)
        sq = torch.empty((n3, k3 // 128), dtype=torch.float16, device=dev)

        def launch_q4(i):
            _abi.call("tq_quantize_i4_g128", ptr(ins[i % nq]), n3, k3, ptr(pq), ptr(sq), stream())

        ms, mode = timer.run(launch_q4, args.steps // 4, 5)
        qb = 4 * n3 * k3 + n3 * k3 // 2 + 2 * n3 * (k3 // 128)
        gbs = qb / (ms * 1e-3) / 1e9
        secondary["quantize_i4_g128_14336x4096"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "timing": mode,
                                                    "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": qb}
        log(f"quantize_i4_g128 14336x4096: {ms * 1e3:.2f} us  {gbs:.0f} GB/s")
        del ins

    # ------------------------------------------------------ INT8 GEMV (C2)
    if not args.no_secondary and want("gemv_w8"):
        n2 = k2 = 4096
        b2 = n2 * k2 + 4 * n2 + 4 * k2 + 4 * n2
        w = normal_f32(1, (n2, k2), 0.02)
        copies = quant_copies(w, tq.quantize_per_channel_i8, rotation(n2 * k2))
        x = dt(normal_f32(1, (1, k2), 1.0, stream=1))
        y = torch.empty((1, n2), dtype=torch.float32, device=dev)

        def launch(i):
            q, s = copies[i % len(copies)]
            _abi.call("tq_gemv_w8", ptr(x), 1, ptr(q), ptr(s), None, n2, k2, ptr(y), stream())

        ms, mode = timer.run(launch, args.steps, args.warmup)
        gbs = b2 / (ms * 1e-3) / 1e9
        secondary["gemv_w8_m1"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "timing": mode,
                                   "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": b2}
        log(f"gemv_w8 M=1: {ms * 1e3:.2f} us/step  {gbs:.0f} GB/s")
        for mw in (2, 4):
            xm = dt(normal_f32(1, (mw, k2), 1.0, stream=1))
            ym = torch.empty((mw, n2), dtype=torch.float32, device=dev)

            def launch_m(i, mw=mw, xm=xm, ym=ym):
                q, s = copies[i % len(copies)]
                _abi.call("tq_gemv_w8", ptr(xm), mw, ptr(q), ptr(s), None, n2, k2, ptr(ym), stream())

            ms, mode = timer.run(launch_m, args.steps, args.warmup)
            bm = n2 * k2 + 4 * n2 + 4 * mw * k2 + 4 * mw * n2
            gbs = bm / (ms * 1e-3) / 1e9
            secondary[f"gemv_w8_m{mw}"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "timing": mode,
                                           "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": bm}
            log(f"gemv_w8 M={mw}: {ms * 1e3:.2f} us/step  {gbs:.0f} GB/s")
        del copies
        if only is None or only == "gemv_w8":
            secondary["gemv_w8_m1"]["read_ceiling"] = read_ceiling(torch, timer, dev, b2, args, log)

    # ------------------------- decode W8A8: fused activation quantization
    if not args.no_secondary and want("w8a8_decode"):
        n2 = k2 = 4096
        w = normal_f32(1, (n2, k2), 0.02)
        res = {}
        for kind, qfn, fused, quant, gemm in (
                ("w8a8", tq.quantize_per_channel_i8, "tq_gemv_w8a8", "tq_quantize_i8_rowwise", "tq_gemm_w8a8"),
                ("fp8", tq.quantize_per_channel_fp8, "tq_gemv_fp8a8", "tq_quantize_fp8_rowwise", "tq_gemm_fp8")):
            copies = quant_copies(w, qfn, rotation(n2 * k2))
            for md in ((1, 4, 16) if kind == "w8a8" else (1,)):
                x = dt(normal_f32(1, (md, k2), 1.0, stream=1))
                y = torch.empty((md, n2), dtype=torch.float32, device=dev)
                qa = torch.empty((md, k2), dtype=torch.int8 if kind == "w8a8" else torch.uint8, device=dev)
                sa = torch.empty(md, dtype=torch.float32, device=dev)

                def launch_fused(i, fused=fused, copies=copies, x=x, y=y, md=md):
                    q, s = copies[i % len(copies)]
                    _abi.call(fused, ptr(x), md, ptr(q), ptr(s), None, n2, k2, ptr(y), stream())

                def launch_two(i, quant=quant, gemm=gemm, copies=copies, x=x, y=y, qa=qa, sa=sa, kind=kind, md=md):
                    q, s = copies[i % len(copies)]
                    _abi.call(quant, ptr(x), md, k2, ptr(qa), ptr(sa), stream())
                    if kind == "w8a8":
                        _abi.call(gemm, ptr(qa), ptr(sa), ptr(q), ptr(s), None, md, n2, k2, None, ptr(y), stream())
                    else:
                        _abi.call(gemm, ptr(qa), ptr(sa), ptr(q), ptr(s), None, md, n2, k2, ptr(y), stream())

                ms_f, mode_f = timer.run(launch_fused, args.steps, args.warmup)
                ms_t, _ = timer.run(launch_two, args.steps, args.warmup)
                key = kind if md == 1 else f"{kind}_m{md}"
                res[key] = {"fused_us": round(ms_f * 1e3, 3), "quantize_plus_gemm_us": round(ms_t * 1e3, 3),
                            "timing": mode_f}
                log(f"decode {kind} M={md} 4096x4096: fused {ms_f * 1e3:.2f} us, quantize + GEMM {ms_t * 1e3:.2f} us")
            del copies
        secondary["a8_decode_m1_n4096_k4096"] = res

    # ------------------------------------------------ FP8 GEMV (C2 shape)
    if not args.no_secondary and want("gemv_fp8"):
        n2 = k2 = 4096
        b2 = n2 * k2 + 4 * n2 + 4 * k2 + 4 * n2
        w = normal_f32(1, (n2, k2), 0.02)
        copies = quant_copies(w, tq.quantize_per_channel_fp8, rotation(n2 * k2))
        x = dt(normal_f32(1, (1, k2), 1.0, stream=1))
        y = torch.empty((1, n2), dtype=torch.float32, device=dev)

        def launch(i):
            q, s = copies[i % len(copies)]
            _abi.call("tq_gemv_fp8", ptr(x), 1, ptr(q), ptr(s), None, n2, k2, ptr(y), stream())

        ms, mode = timer.run(launch, args.steps, args.warmup)
        gbs = b2 / (ms * 1e-3) / 1e9
        secondary["gemv_fp8_m1"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "timing": mode,
                                    "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": b2}
        log(f"gemv_fp8 M=1: {ms * 1e3:.2f} us/step  {gbs:.0f} GB/s")
        del copies

    # ---------------------------------------------------------- W8A8 (C4)
    if not args.no_secondary and want("w8a8"):
        m4, n4, k4 = 2048, 4096, 4096
        xd = dt(normal_f32(3, (m4, k4), 1.0))
        qa0, sa0 = tq.quantize_per_channel_i8(xd)
        qw0, sw0 = tq.quantize_per_channel_i8(dt(normal_f32(3, (n4, k4), 0.02, stream=1)))
        # every launch takes its own copy of the operands (codes and scales of
        # both sides), rotating over more than 2x the MALL
        ops = [(qa0.clone(), sa0.clone(), qw0.clone(), sw0.clone())
               for _ in range(rotation(m4 * k4 + n4 * k4 + 4 * (m4 + n4)))]
        y = torch.empty((m4, n4), dtype=torch.float32, device=dev)

        def launch(i):
            qa, sa, qw, sw = ops[i % len(ops)]
            _abi.call("tq_gemm_w8a8", ptr(qa), ptr(sa), ptr(qw), ptr(sw), None, m4, n4, k4, None, ptr(y), stream())

        steps = max(10, args.steps // 4)
        ms, mode = timer.run(launch, steps, max(2, args.warmup // 4))
        tops = 2.0 * m4 * n4 * k4 / (ms * 1e-3) / 1e12
        qbytes = 4 * m4 * k4 + m4 * k4 + 4 * m4
        xs = [xd] + [xd.clone() for _ in range(rotation(4 * m4 * k4) - 1)]
        qa1, sa1 = torch.empty_like(qa0), torch.empty_like(sa0)

        def launch_q(i):
            _abi.call("tq_quantize_i8_rowwise", ptr(xs[i % len(xs)]), m4, k4, ptr(qa1), ptr(sa1), stream())

        # 40 launches per graph at least: a replay's own launch cost (a few us) over
        # 10 launches of ~10 us added ~1.5 us per step
        msq, _ = timer.run(launch_q, max(40, steps), 2)
        secondary["w8a8_gemm_m2048"] = {
            "us": round(ms * 1e3, 3), "timing": mode, "TOPS": round(tops, 1), "i8_mfma_frac": round(tops / I8_PEAK_TOPS, 4),
            "i8_mfma_frac_of_random_operand_peak": of_random_peak(tops, "i8_mfma_TOPS_random_operands"),
            "operand_copies": len(ops),
            "act_quant_us": round(msq * 1e3, 3), "act_quant_GB/s": round(qbytes / (msq * 1e-3) / 1e9, 1),
            "act_quant_input_copies": len(xs)}
        log(f"w8a8 M=2048: {ms * 1e3:.2f} us  {tops:.0f} TOPS; act quant {msq * 1e3:.2f} us")
        ph = w8a8_phases(torch, np, ops, y, m4, n4, k4, log)
        if peaks:
            ph["mfma_floor_us"] = round(2.0 * m4 * n4 * k4 / (peaks["i8_mfma_TOPS_random_operands_1_block_per_cu"]
                                                          * 1e12) * 1e6, 2)
        secondary["w8a8_gemm_m2048"]["phases_one_launch"] = ph
        del ops, xs, y, xd, qa0, qw0, qa1

    # ------------------------------------------------ FP8 W8A8 (C4 shape)
    if not args.no_secondary and want("fp8"):
        m4, n4, k4 = 2048, 4096, 4096
        xd = dt(normal_f32(3, (m4, k4), 1.0))
        qa0, sa0 = tq.quantize_per_channel_fp8(xd)
        qw0, sw0 = tq.quantize_per_channel_fp8(dt(normal_f32(3, (n4, k4), 0.02, stream=1)))
        ops = [(qa0.clone(), sa0.clone(), qw0.clone(), sw0.clone())
               for _ in range(rotation(m4 * k4 + n4 * k4 + 4 * (m4 + n4)))]
        y = torch.empty((m4, n4), dtype=torch.float32, device=dev)

        def launch(i):
            qa, sa, qw, sw = ops[i % len(ops)]
            _abi.call("tq_gemm_fp8", ptr(qa), ptr(sa), ptr(qw), ptr(sw), None, m4, n4, k4, ptr(y), stream())

        steps = max(10, args.steps // 4)
        ms, mode = timer.run(launch, steps, max(2, args.warmup // 4))
        tf = 2.0 * m4 * n4 * k4 / (ms * 1e-3) / 1e12
        qbytes = 4 * m4 * k4 + m4 * k4 + 4 * m4
        xs = [xd] + [xd.clone() for _ in range(rotation(4 * m4 * k4) - 1)]
        qa1, sa1 = torch.empty_like(qa0), torch.empty_like(sa0)

        def launch_q(i):
            _abi.call("tq_quantize_fp8_rowwise", ptr(xs[i % len(xs)]), m4, k4, ptr(qa1), ptr(sa1), stream())

        msq, _ = timer.run(launch_q, max(40, steps), 2)
        secondary["fp8_gemm_m2048"] = {
            "us": round(ms * 1e3, 3), "timing": mode, "TFLOP/s": round(tf, 1), "fp8_mfma_frac": round(tf / FP8_PEAK_TFLOPS, 4),
            "operand_copies": len(ops),
            "act_quant_us": round(msq * 1e3, 3), "act_quant_GB/s": round(qbytes / (msq * 1e-3) / 1e9, 1),
            "act_quant_input_copies": len(xs)}
        log(f"fp8 M=2048: {ms * 1e3:.2f} us  {tf:.0f} TFLOP/s; act quant {msq * 1e3:.2f} us")
        del ops, xs, y, xd, qa0, qw0, qa1

    # ------------------------------ MultiheadAttention, INT4 projections
    if not args.no_secondary and want("mha"):
        b6, s6, e6, h6 = 1, 2048, 4096, 32
        ws6 = [dt(normal_f32(6, (e6, e6), 0.02, stream=i)) for i in range(4)]
        mha = tq.QuantizedMultiheadAttention.from_tensors(h6, *ws6, qconfig=tq.QConfig.default_int4())
        del ws6
        x6 = dt(normal_f32(6, (b6, s6, e6), 1.0, stream=9))
        qkv6 = mha.qkv(tq.convert(x6.reshape(b6 * s6, e6), torch.bfloat16))
        o6 = torch.empty((b6 * s6, e6), dtype=torch.float32, device=dev)

        def launch_core(i):
            _abi.call("tq_attention_f32", ptr(qkv6), 3 * e6, ptr(qkv6[:, e6:]), 3 * e6, ptr(qkv6[:, 2 * e6:]), 3 * e6,
                      None, 0, b6, s6, h6, e6 // h6, ptr(o6), e6, stream())

        ms_core, mode_core = timer.run(launch_core, 5, 1)
        ms_all, mode_all = timer.run(lambda i: mha(x6), 5, 1)
        core_tf = 4.0 * b6 * h6 * s6 * s6 * (e6 // h6) / (ms_core * 1e-3) / 1e12
        secondary["mha_w4_b1_s2048_e4096_h32"] = {
            "us": round(ms_all * 1e3, 1), "timing": mode_all, "attention_core_us": round(ms_core * 1e3, 1),
            "attention_core_TFLOP/s": round(core_tf, 1), "tokens/s": round(b6 * s6 / (ms_all * 1e-3), 1)}
        log(f"mha S=2048 E=4096 H=32 (int4): {ms_all * 1e3:.0f} us, attention core {ms_core * 1e3:.0f} us "
            f"({core_tf:.1f} TFLOP/s f32)")
        del mha, x6, qkv6, o6

    # ------------------------------------- device storage (C++ host layer)
    if not args.no_secondary and want("storage"):
        exe = os.path.join(ROOT, "neo-theano_amd", "bench_storage")
        if os.path.exists(exe):
            import subprocess

            r = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=300)
            if r.returncode == 0:
                secondary["device_storage"] = json.loads(r.stdout.strip().splitlines()[-1])
                log(f"device storage: {secondary['device_storage']}")
            else:
                log(f"bench_storage failed ({r.returncode}): {r.stderr[-500:]}")

    # ------------------------------------------------ round trip (C1)
    if not args.no_secondary and want("roundtrip"):
        n1 = k1 = 4096
        ins = [dt(normal_f32(0, (n1, k1), 0.02, stream=i)) for i in range(rotation(4 * n1 * k1))]
        q = torch.empty((n1, k1), dtype=torch.int8, device=dev)
        s = torch.empty(n1, dtype=torch.float32, device=dev)
        wh = torch.empty((n1, k1), dtype=torch.float32, device=dev)
        # dequantize input: codes rotating over copies as well, so that its reads come from HBM
        qs = [torch.randint(-127, 128, (n1, k1), dtype=torch.int8, device=dev) for _ in range(rotation(n1 * k1))]

        def lq(i):
            _abi.call("tq_quantize_i8_rowwise", ptr(ins[i % len(ins)]), n1, k1, ptr(q), ptr(s), stream())

        def ld(i):
            _abi.call("tq_dequantize_i8_rowwise", ptr(qs[i % len(qs)]), ptr(s), n1, k1, ptr(wh), stream())

        def lf(i):
            _abi.call("tq_fake_quantize_i8_rowwise", ptr(ins[i % len(ins)]), n1, k1, ptr(q), ptr(s), ptr(wh),
                      stream())

        res = {}
        for name, fn, nbytes in (("quantize", lq, 5 * n1 * k1 + 4 * n1), ("dequantize", ld, 5 * n1 * k1 + 4 * n1),
                                 ("fused", lf, 9 * n1 * k1 + 4 * n1)):
            ms, _ = timer.run(fn, args.steps, args.warmup)
            gbs = nbytes / (ms * 1e-3) / 1e9
            res[name] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
            log(f"roundtrip {name}: {ms * 1e3:.2f} us  {gbs:.0f} GB/s")
        secondary["roundtrip_i8_4096x4096"] = res
        del ins, qs

    # --------------------------------------------------------- MLP (C5)
    if not args.no_secondary and want("mlp"):
        d5, f5, m5 = 4096, 14336, 512
        mlp = tq.QuantizedMLP.from_tensors(dt(normal_f32(4, (f5, d5), 0.02)), dt(normal_f32(4, (f5, d5), 0.02, 1)),
                                           dt(normal_f32(4, (d5, f5), 0.02, 2)))
        wbytes = 3 * f5 * d5 // 2 + 3 * f5 * d5 // 128 * 2
        # every launch takes its own copy of the three weights, rotating over more than 2x the MALL
        mats = [(mlp.gate, mlp.up, mlp.down)] + [tuple(tuple(t.clone() for t in w) for w in (mlp.gate, mlp.up, mlp.down))
                                                 for _ in range(rotation(wbytes) - 1)]
        x = bf16(normal_f32(4, (m5, d5), 1.0, stream=3))
        ws = torch.empty((mlp.workspace_bytes(m5),), dtype=torch.uint8, device=dev)
        y = torch.empty((m5, d5), dtype=torch.float32, device=dev)

        def launch(i):
            g, u, dn = mats[i % len(mats)]
            _abi.call("tq_mlp_w4g128", ptr(x), m5, d5, f5, ptr(g[0]), ptr(g[1]), ptr(u[0]), ptr(u[1]), ptr(dn[0]),
                      ptr(dn[1]), ptr(ws), ws.numel(), ptr(y), stream())

        steps = max(5, args.steps // 10)
        ms, mode = timer.run(launch, steps, 2)
        flops = 6.0 * m5 * f5 * d5
        tf = flops / (ms * 1e-3) / 1e12
        secondary["mlp_w4g128_m512"] = {"us": round(ms * 1e3, 2), "timing": mode, "tokens/s": round(m5 / (ms * 1e-3), 1),
                                        "TFLOP/s": round(tf, 1), "bf16_mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4),
                                        "bf16_mfma_frac_of_random_operand_peak":
                                            of_random_peak(tf, "bf16_mfma_TFLOPS_random_operands"),
                                        "weight_copies": len(mats)}
        log(f"mlp M=512: {ms * 1e3:.1f} us  {m5 / (ms * 1e-3):.0f} tok/s  {tf:.0f} TFLOP/s")

        # prefill INT4 Linear on the gate weight alone: [512, 4096] x [14336, 4096]^T
        nbl = int(_abi.lib().tq_gemm_w4g128_bf16_workspace_bytes(m5, d5))
        wsl = torch.empty((nbl,), dtype=torch.uint8, device=dev)
        yl = torch.empty((m5, f5), dtype=torch.float32, device=dev)

        def launch_lin(i):
            g = mats[i % len(mats)][0]
            _abi.call("tq_gemm_w4g128_bf16_ws", ptr(x), m5, ptr(g[0]), ptr(g[1]), None, f5, d5, ptr(wsl), nbl,
                      ptr(yl), stream())

        ms, mode = timer.run(launch_lin, steps, 2)
        tf = 2.0 * m5 * f5 * d5 / (ms * 1e-3) / 1e12
        secondary["w4a16_linear_m512_n14336_k4096"] = {"us": round(ms * 1e3, 2), "timing": mode, "TFLOP/s": round(tf, 1),
                                                       "bf16_mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4),
                                                       "bf16_mfma_frac_of_random_operand_peak":
                                                           of_random_peak(tf, "bf16_mfma_TFLOPS_random_operands"),
                                                       "weight_copies": len(mats)}
        log(f"w4a16 linear M=512 N=14336 K=4096: {ms * 1e3:.1f} us  {tf:.0f} TFLOP/s")
        del mlp, mats, wsl, yl

    # --------------- mid-size M on the prefill kernels (C5 weights, M = 64, 128)
    if not args.no_secondary and want("mlp_mid"):
        d5, f5 = 4096, 14336
        base = tq.QuantizedMLP.from_tensors(dt(normal_f32(4, (f5, d5), 0.02)), dt(normal_f32(4, (f5, d5), 0.02, 1)),
                                            dt(normal_f32(4, (d5, f5), 0.02, 2)))
        wbytes = 3 * f5 * d5 // 2 + 3 * f5 * d5 // 128 * 2
        mats = [(base.gate, base.up, base.down)] + [tuple(tuple(t.clone() for t in w) for w in
                                                          (base.gate, base.up, base.down))
                                                    for _ in range(rotation(wbytes) - 1)]
        res = {}
        for mm in (64, 128):
            x = bf16(normal_f32(4, (mm, d5), 1.0, stream=3))
            nb = int(_abi.lib().tq_mlp_w4g128_workspace_bytes(mm, d5, f5))
            ws = torch.empty((nb,), dtype=torch.uint8, device=dev)
            y = torch.empty((mm, d5), dtype=torch.float32, device=dev)
            nbl = int(_abi.lib().tq_gemm_w4g128_bf16_workspace_bytes(mm, d5))
            wsl = torch.empty((nbl,), dtype=torch.uint8, device=dev)
            yl = torch.empty((mm, f5), dtype=torch.float32, device=dev)

            def launch_mid(i, mm=mm, x=x, ws=ws, nb=nb, y=y):
                g, u, dn = mats[i % len(mats)]
                _abi.call("tq_mlp_w4g128", ptr(x), mm, d5, f5, ptr(g[0]), ptr(g[1]), ptr(u[0]), ptr(u[1]),
                          ptr(dn[0]), ptr(dn[1]), ptr(ws), nb, ptr(y), stream())

            def launch_mid_lin(i, mm=mm, x=x, wsl=wsl, nbl=nbl, yl=yl):
                g = mats[i % len(mats)][0]
                _abi.call("tq_gemm_w4g128_bf16_ws", ptr(x), mm, ptr(g[0]), ptr(g[1]), None, f5, d5, ptr(wsl), nbl,
                          ptr(yl), stream())

            steps = max(10, args.steps // 5)
            ms, mode = timer.run(launch_mid, steps, 3)
            tf = 6.0 * mm * f5 * d5 / (ms * 1e-3) / 1e12
            msl, model = timer.run(launch_mid_lin, steps, 3)
            tfl = 2.0 * mm * f5 * d5 / (msl * 1e-3) / 1e12
            res[f"m{mm}"] = {"ffn_us": round(ms * 1e3, 2), "ffn_timing": mode, "ffn_tokens/s": round(mm / (ms * 1e-3), 1),
                             "ffn_TFLOP/s": round(tf, 1), "ffn_weights_GB/s": round(wbytes / (ms * 1e-3) / 1e9, 1),
                             "linear_n14336_k4096_us": round(msl * 1e3, 2), "linear_timing": model,
                             "linear_TFLOP/s": round(tfl, 1)}
            log(f"prefill FFN M={mm}: {ms * 1e3:.1f} us; INT4 Linear M={mm}: {msl * 1e3:.1f} us")
        secondary["prefill_mid_m"] = res
        del base, mats

    # ------------------------------- decode FFN (C5 weights, M = 1, 2, 4, 8, 16)
    if not args.no_secondary and want("mlp_decode"):
        d5, f5 = 4096, 14336
        base = tq.QuantizedMLP.from_tensors(dt(normal_f32(4, (f5, d5), 0.02)), dt(normal_f32(4, (f5, d5), 0.02, 1)),
                                            dt(normal_f32(4, (d5, f5), 0.02, 2)))
        wbytes = 3 * f5 * d5 // 2 + 3 * f5 * d5 // 128 * 2  # packed nibbles + f16 scales of the three weights
        copies = [base.decode] + [tuple(t.clone() if hasattr(t, "clone") else t for t in base.decode)
                                  for _ in range(rotation(wbytes) - 1)]
        res = {}
        for md in (1, 2, 4, 8, 16):
            x = bf16(normal_f32(4, (md, d5), 1.0, stream=3))
            ws = torch.empty((base.workspace_bytes(md),), dtype=torch.uint8, device=dev)
            y = torch.empty((md, d5), dtype=torch.float32, device=dev)

            def launch_dec(i, md=md, x=x, ws=ws, y=y):
                gu_t, gu_st, dn_t, dn_st, rows = copies[i % len(copies)]
                _abi.call("tq_mlp_w4g128_decode", ptr(x), md, d5, f5, ptr(gu_t), ptr(gu_st), ptr(dn_t), ptr(dn_st),
                          rows, ptr(ws), ws.numel(), ptr(y), stream())

            ms, mode = timer.run(launch_dec, args.steps, args.warmup)
            gbs = (wbytes + md * d5 * 2 + md * d5 * 4) / (ms * 1e-3) / 1e9
            res[f"m{md}"] = {"us": round(ms * 1e3, 2), "timing": mode, "GB/s": round(gbs, 1),
                             "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
            log(f"mlp decode M={md}: {ms * 1e3:.1f} us  {gbs:.0f} GB/s ({mode})")
        secondary["mlp_w4g128_decode"] = res
        del base, copies

    # ------------------------------------------ copy (PMC calibration)
    if only == "copy":
        nb = 1 << 30
        a = torch.empty(nb // 4, dtype=torch.float32, device=dev).fill_(1.0)
        b = torch.empty_like(a)
        ms, _ = timer.run(lambda i: b.copy_(a), 20, 3)
        log(f"copy 1 GiB: {ms * 1e3:.1f} us  {2 * nb / (ms * 1e-3) / 1e9:.0f} GB/s (read+write)")
        return

    if headline is None:
        return

    # ------------------------------------------------------ CPU baselines
    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baselines(args, secondary, n3, k3, w4_bytes_m(1), log)

    traffic = None
    tfile = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            traffic = json.load(f).get("gemv_w4g128_m1", {}).get("hbm_bytes_per_launch")

    gbs = headline["gbs"]
    rc30 = secondary.get("read_ceiling_30mb")
    out = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(headline["ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xbf16",
        "data": "synthetic (numpy PCG64 normals, seeded; weights rotate over copies > 2x MALL)",
        "config": {"workload": "int4_g128_dequant_gemv", "baseline_config": 3, "n": n3, "k": k3, "m": 1,
                   "group": 128, "weight_layout": "row-tiled",
                   "timing": f"{headline['mode']}, median of {max(1, args.reps)} timed replays of {args.steps} launches",
                   "us_per_launch_by_timing": headline["modes_us"]},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": w4_bytes_m(1),
                     "peak_measured": peaks["hbm_read_GB/s"] if peaks else None,
                     "frac_of_measured": round(gbs / peaks["hbm_read_GB/s"], 4) if peaks else None,
                     "read_ceiling_GB/s": rc30["GB/s"] if rc30 else None,
                     "frac_of_read_ceiling": round(gbs / rc30["GB/s"], 4) if rc30 else None},
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
