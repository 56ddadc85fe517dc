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

`cpu_baseline` times the C restatement of the reference CPU path
(oracle/, f64 dequantize + Linear::forward) on a bounded sample of the
headline workload, single-threaded.
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
                   help="run one workload: gemv_w4, gemv_w8, gemv_fp8, gemv_w4_m, w8a8_decode, w8a8, fp8, mha, storage, "
                        "roundtrip, mlp, mlp_decode, copy")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="bound of the CPU baseline sample (0: skip)")
    p.add_argument("--eager", action="store_true", help="time eager launches instead of a HIP graph")
    return p.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timer:
    """Times `steps` calls of launch(i) on the current stream, bracketed by
    events on that stream, as a HIP graph replay and as eager launches, and
    returns the faster of the two with its mode ("graph" / "eager"; only eager
    launches with --eager).  Short kernels need the graph (a Python launch
    takes longer than the kernel); long ones run back to back either way, and
    graph replay adds a few microseconds per node on this stack."""

    def __init__(self, torch, eager=False):
        self.torch = torch
        self.eager = eager

    def run(self, launch, steps, warmup):
        best = self._run(launch, steps, warmup, graph=not self.eager)
        if best[1] == "graph":
            eager = self._run(launch, steps, 0, graph=False)
            if eager[0] < best[0]:
                best = eager
        return best

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
        ms = start.elapsed_time(end)
        return ms / steps, mode


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
    timer = Timer(torch, eager=args.eager)
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
            ms, mode = timer.run(gemv_w4(1), args.steps, args.warmup)
            gbs = w4_bytes_m(1) / (ms * 1e-3) / 1e9
            headline = {"ms": ms, "gbs": gbs, "mode": mode}
            log(f"gemv_w4 M=1: {ms * 1e3:.2f} us/step  {gbs:.0f} GB/s  ({mode})")
        if not args.no_secondary and (only is None or only == "gemv_w4_m"):
            for m in (2, 4, 8, 16):
                ms, mode = timer.run(gemv_w4(m), args.steps, args.warmup)
                gbs = w4_bytes_m(m) / (ms * 1e-3) / 1e9
                secondary[f"gemv_w4g128_m{m}"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "timing": mode,
                                                  "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
                log(f"gemv_w4 M={m}: {ms * 1e3:.2f} us/step  {gbs:.0f} GB/s")
        del copies

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
        del copies

    # ------------------------- decode W8A8: fused activation quantization
    if not args.no_secondary and want("w8a8_decode"):
        n2 = k2 = 4096
        w = normal_f32(1, (n2, k2), 0.02)
        res = {}
        for kind, qfn, fused, quant, gemm in (
                ("w8a8", tq.quantize_per_channel_i8, "tq_gemv_w8a8", "tq_quantize_i8_rowwise", "tq_gemm_w8a8"),
                ("fp8", tq.quantize_per_channel_fp8, "tq_gemv_fp8a8", "tq_quantize_fp8_rowwise", "tq_gemm_fp8")):
            copies = quant_copies(w, qfn, rotation(n2 * k2))
            x = dt(normal_f32(1, (1, k2), 1.0, stream=1))
            y = torch.empty((1, n2), dtype=torch.float32, device=dev)
            qa = torch.empty((1, k2), dtype=torch.int8 if kind == "w8a8" else torch.uint8, device=dev)
            sa = torch.empty(1, dtype=torch.float32, device=dev)

            def launch_fused(i, fused=fused, copies=copies, x=x, y=y):
                q, s = copies[i % len(copies)]
                _abi.call(fused, ptr(x), 1, ptr(q), ptr(s), None, n2, k2, ptr(y), stream())

            def launch_two(i, quant=quant, gemm=gemm, copies=copies, x=x, y=y, qa=qa, sa=sa, kind=kind):
                q, s = copies[i % len(copies)]
                _abi.call(quant, ptr(x), 1, k2, ptr(qa), ptr(sa), stream())
                if kind == "w8a8":
                    _abi.call(gemm, ptr(qa), ptr(sa), ptr(q), ptr(s), None, 1, n2, k2, None, ptr(y), stream())
                else:
                    _abi.call(gemm, ptr(qa), ptr(sa), ptr(q), ptr(s), None, 1, n2, k2, ptr(y), stream())

            ms_f, mode_f = timer.run(launch_fused, args.steps, args.warmup)
            ms_t, _ = timer.run(launch_two, args.steps, args.warmup)
            res[kind] = {"fused_us": round(ms_f * 1e3, 3), "quantize_plus_gemm_us": round(ms_t * 1e3, 3),
                         "timing": mode_f}
            log(f"decode {kind} M=1 4096x4096: fused {ms_f * 1e3:.2f} us, quantize + GEMM {ms_t * 1e3:.2f} us")
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
        x = normal_f32(3, (m4, k4), 1.0)
        w = normal_f32(3, (n4, k4), 0.02, stream=1)
        xd = dt(x)
        qa, sa = tq.quantize_per_channel_i8(xd)
        qw, sw = tq.quantize_per_channel_i8(dt(w))
        y = torch.empty((m4, n4), dtype=torch.float32, device=dev)

        def launch(i):
            _abi.call("tq_gemm_w8a8", ptr(qa), ptr(sa), ptr(qw), ptr(sw), None, m4, n4, k4, None, ptr(y), stream())

        steps = max(10, args.steps // 4)
        ms, mode = timer.run(launch, steps, max(2, args.warmup // 4))
        tops = 2.0 * m4 * n4 * k4 / (ms * 1e-3) / 1e12
        qbytes = 4 * m4 * k4 + m4 * k4 + 4 * m4

        def launch_q(i):
            _abi.call("tq_quantize_i8_rowwise", ptr(xd), m4, k4, ptr(qa), ptr(sa), stream())

        msq, _ = timer.run(launch_q, steps, 2)
        secondary["w8a8_gemm_m2048"] = {
            "us": round(ms * 1e3, 3), "timing": mode, "TOPS": round(tops, 1), "i8_mfma_frac": round(tops / I8_PEAK_TOPS, 4),
            "act_quant_us": round(msq * 1e3, 3), "act_quant_GB/s": round(qbytes / (msq * 1e-3) / 1e9, 1)}
        log(f"w8a8 M=2048: {ms * 1e3:.2f} us  {tops:.0f} TOPS; act quant {msq * 1e3:.2f} us")
        del qa, qw, y, xd

    # ------------------------------------------------ FP8 W8A8 (C4 shape)
    if not args.no_secondary and want("fp8"):
        m4, n4, k4 = 2048, 4096, 4096
        xd = dt(normal_f32(3, (m4, k4), 1.0))
        qa, sa = tq.quantize_per_channel_fp8(xd)
        qw, sw = tq.quantize_per_channel_fp8(dt(normal_f32(3, (n4, k4), 0.02, stream=1)))
        y = torch.empty((m4, n4), dtype=torch.float32, device=dev)

        def launch(i):
            _abi.call("tq_gemm_fp8", ptr(qa), ptr(sa), ptr(qw), ptr(sw), None, m4, n4, k4, ptr(y), stream())

        steps = max(10, args.steps // 4)
        ms, mode = timer.run(launch, steps, max(2, args.warmup // 4))
        tf = 2.0 * m4 * n4 * k4 / (ms * 1e-3) / 1e12
        qbytes = 4 * m4 * k4 + m4 * k4 + 4 * m4

        def launch_q(i):
            _abi.call("tq_quantize_fp8_rowwise", ptr(xd), m4, k4, ptr(qa), ptr(sa), stream())

        msq, _ = timer.run(launch_q, steps, 2)
        secondary["fp8_gemm_m2048"] = {
            "us": round(ms * 1e3, 3), "timing": mode, "TFLOP/s": round(tf, 1), "fp8_mfma_frac": round(tf / FP8_PEAK_TFLOPS, 4),
            "act_quant_us": round(msq * 1e3, 3), "act_quant_GB/s": round(qbytes / (msq * 1e-3) / 1e9, 1)}
        log(f"fp8 M=2048: {ms * 1e3:.2f} us  {tf:.0f} TFLOP/s; act quant {msq * 1e3:.2f} us")
        del qa, qw, y, xd

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
        x = bf16(normal_f32(4, (m5, d5), 1.0, stream=3))
        ws = torch.empty((mlp.workspace_bytes(m5),), dtype=torch.uint8, device=dev)
        y = torch.empty((m5, d5), dtype=torch.float32, device=dev)

        def launch(i):
            _abi.call("tq_mlp_w4g128", ptr(x), m5, d5, f5, ptr(mlp.gate[0]), ptr(mlp.gate[1]), ptr(mlp.up[0]),
                      ptr(mlp.up[1]), ptr(mlp.down[0]), ptr(mlp.down[1]), ptr(ws), ws.numel(), ptr(y), stream())

        steps = max(5, args.steps // 10)
        ms, mode = timer.run(launch, steps, 2)
        flops = 6.0 * m5 * f5 * d5
        tf = flops / (ms * 1e-3) / 1e12
        secondary["mlp_w4g128_m512"] = {"us": round(ms * 1e3, 2), "timing": mode, "tokens/s": round(m5 / (ms * 1e-3), 1),
                                        "TFLOP/s": round(tf, 1), "bf16_mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4)}
        log(f"mlp M=512: {ms * 1e3:.1f} us  {m5 / (ms * 1e-3):.0f} tok/s  {tf:.0f} TFLOP/s")

        # prefill INT4 Linear on the gate weight alone: [512, 4096] x [14336, 4096]^T
        nbl = int(_abi.lib().tq_gemm_w4g128_bf16_workspace_bytes(m5, d5))
        wsl = torch.empty((nbl,), dtype=torch.uint8, device=dev)
        yl = torch.empty((m5, f5), dtype=torch.float32, device=dev)

        def launch_lin(i):
            _abi.call("tq_gemm_w4g128_bf16_ws", ptr(x), m5, ptr(mlp.gate[0]), ptr(mlp.gate[1]), None, f5, d5,
                      ptr(wsl), nbl, ptr(yl), stream())

        ms, mode = timer.run(launch_lin, steps, 2)
        tf = 2.0 * m5 * f5 * d5 / (ms * 1e-3) / 1e12
        secondary["w4a16_linear_m512_n14336_k4096"] = {"us": round(ms * 1e3, 2), "timing": mode, "TFLOP/s": round(tf, 1),
                                                       "bf16_mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4)}
        log(f"w4a16 linear M=512 N=14336 K=4096: {ms * 1e3:.1f} us  {tf:.0f} TFLOP/s")
        del mlp, wsl, yl

    # ------------------------------------ decode FFN (C5 weights, M = 1, 4)
    if not args.no_secondary and want("mlp_decode"):
        d5, f5 = 4096, 14336
        base = tq.QuantizedMLP.from_tensors(dt(normal_f32(4, (f5, d5), 0.02)), dt(normal_f32(4, (f5, d5), 0.02, 1)),
                                            dt(normal_f32(4, (d5, f5), 0.02, 2)))
        wbytes = 3 * f5 * d5 // 2 + 3 * f5 * d5 // 128 * 2  # packed nibbles + f16 scales of the three weights
        copies = [base.decode] + [tuple(t.clone() if hasattr(t, "clone") else t for t in base.decode)
                                  for _ in range(rotation(wbytes) - 1)]
        res = {}
        for md in (1, 4):
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

    # ------------------------------------------------------ CPU baseline
    cpu = None
    if args.cpu_seconds > 0:
        import oracle as O  # the CPU restatement of the reference path, timed as the baseline

        O.lib()
        w = normal_f32(2, (n3, k3), 0.02)
        p, s = O.quantize_i4_g128(w)
        del w
        xb = f32_to_bf16_bits(normal_f32(2, (1, k3), 1.0, stream=1))
        reps, t0 = 0, time.perf_counter()
        while True:
            O.linear_w4g128_bf16(xb, p, s)
            reps += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds or reps >= 50:
                break
        per = el / reps
        cpu = {"value": round(w4_bytes_m(1) / per / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"config 3 at M=1 (full [14336, 4096] INT4 g128 weight), {reps} calls of the "
                         f"f64 dequantize + Linear::forward restatement, {per * 1e3:.0f} ms per call, "
                         f"1 thread on {os.cpu_count()} host CPUs"}
        log(f"cpu baseline: {per * 1e3:.1f} ms/call")

    traffic = None
    tfile = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            traffic = json.load(f).get("gemv_w4g128_m1", {}).get("hbm_bytes_per_launch")

    gbs = headline["gbs"]
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
                   "group": 128, "weight_layout": "row-tiled", "timing": headline["mode"]},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": w4_bytes_m(1)},
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
