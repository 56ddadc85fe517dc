"""Writes the golden fixtures of this directory.

Two kinds of data:

* reference_kats.json -- the known-answer values asserted by the reference's own
  unit tests (crates/theano-quantize/src/{quantize,observer,qconfig}.rs and
  crates/theano-core/src/tensor_ops.rs), transcribed as inputs / expected
  outputs with the file:line of each assert, plus round-half-away-from-zero
  tie and signed-zero cases whose answers follow from the rounding rule
  quantize.rs:15 states (f64::round).  These need no program to produce.
* *.npz -- small cases of the build-defined formats (per-row INT8, INT4 g128,
  W8A8 accumulators) computed by the C restatement in oracle/ from seeded
  synthetic inputs, and the first 16 values of every synthetic-data seed (to
  pin the generator).  The oracle is itself pinned by tests/test_oracle.py;
  these files freeze its outputs so that the GPU kernels and any later change
  of the oracle are checked against the same bytes.
* checkpoint_int4_16x256.safetensors -- the INT4 case as a quantized Linear
  checkpoint, written by the independent `safetensors` package, for the
  checkpoint readers (Python and C++).

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "neo-theano_amd"))

import oracle  # noqa: E402
from theano_quantize import synth  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

INT8, UINT8, INT4, FP8 = oracle.INT8, oracle.UINT8, oracle.INT4, oracle.FP8

KATS = {
    "qdtype_ranges": {
        "cite": "crates/theano-quantize/src/qconfig.rs:82-108",
        "cases": [
            {"dtype": "Int8", "bits": 8, "signed": True, "qmin": -128.0, "qmax": 127.0},
            {"dtype": "UInt8", "bits": 8, "signed": False, "qmin": 0.0, "qmax": 255.0},
            {"dtype": "Int4", "bits": 4, "signed": True, "qmin": -8.0, "qmax": 7.0},
            {"dtype": "FP8", "bits": 8, "signed": False, "qmin": -448.0, "qmax": 448.0},
        ],
    },
    "quantize_tensor": {
        "cite": "crates/theano-quantize/src/quantize.rs:82-87 (clamps); ties and signed zeros "
                "follow quantize.rs:15 (f64::round, half away from zero)",
        "cases": [
            {"x": [1000.0, -1000.0], "scale": 1.0, "zp": 0.0, "dtype": "Int8", "q": [127.0, -128.0]},
            {"x": [2.5, -2.5, 0.5, -0.5, 1.5, -1.5], "scale": 1.0, "zp": 0.0, "dtype": "Int8",
             "q": [3.0, -3.0, 1.0, -1.0, 2.0, -2.0]},
            # -0.3 + 0.0 rounds to -0.0; -0.0 + 0.0 is +0.0 in IEEE, so x = -0.0 gives +0.0
            {"x": [-0.3, 0.3, "-0.0", 0.0], "scale": 1.0, "zp": 0.0, "dtype": "Int8",
             "q": ["-0.0", 0.0, 0.0, 0.0]},
            {"x": [7.5, -8.5, 100.0], "scale": 1.0, "zp": 0.0, "dtype": "Int4", "q": [7.0, -8.0, 7.0]},
            {"x": [0.25, 0.75], "scale": 0.5, "zp": 3.0, "dtype": "UInt8", "q": [4.0, 5.0]},
        ],
    },
    "dequantize_tensor": {
        "cite": "crates/theano-quantize/src/quantize.rs:89-99",
        "cases": [{"q": [0.0, 64.0, 127.0], "scale": 0.01, "zp": 0.0, "x": [0.0, 0.64, 1.27], "tol": 1e-10}],
    },
    "quantize_per_tensor_roundtrip": {
        "cite": "crates/theano-quantize/src/quantize.rs:61-72,128-136",
        "cases": [
            {"x": [0.0, 0.5, 1.0, -0.5, -1.0], "dtype": "Int8", "tol": 0.05},
            {"x": [0.5, -0.5], "dtype": "Int8", "tol": 0.05},
        ],
    },
    "quantize_per_tensor_range": {
        "cite": "crates/theano-quantize/src/quantize.rs:101-119",
        "cases": [
            {"x": [0.0, 0.5, 1.0], "dtype": "Int4", "lo": -8.0, "hi": 7.0},
            {"x": [0.0, 0.5, 1.0], "dtype": "UInt8", "lo": 0.0, "hi": 255.0},
        ],
    },
    "minmax_observer": {
        "cite": "crates/theano-quantize/src/observer.rs:142-188",
        "cases": [
            {"observe": [[1.0, 2.0, 3.0, -1.0]], "min": -1.0, "max": 3.0},
            {"observe": [[1.0, 2.0], [-5.0, 10.0]], "min": -5.0, "max": 10.0},
            {"observe": [], "dtype": "Int8", "scale": 1.0, "zp": 0.0},
            {"observe": [[0.0, 1.0]], "dtype": "UInt8", "scale": 1.0 / 255.0, "tol": 1e-6},
        ],
    },
    "matmul": {
        "cite": "crates/theano-core/src/tensor_ops.rs:841-865",
        "cases": [
            {"a": [[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], "b": [[7.0, 8.0], [9.0, 10.0], [11.0, 12.0]],
             "c": [[58.0, 64.0], [139.0, 154.0]]},
            {"a": [[1.0, 2.0, 3.0]], "b": [[7.0, 8.0], [9.0, 10.0], [11.0, 12.0]], "c": [[58.0, 64.0]]},
            {"a": [[1.0, 2.0, 3.0]], "b": [[4.0], [5.0], [6.0]], "c": [[32.0]]},
        ],
    },
    "sigmoid": {
        "cite": "crates/theano-core/src/tensor_ops.rs:793-798; crates/theano-nn/src/activation.rs:138-144",
        "cases": [{"x": 0.0, "y": 0.5, "tol": 1e-10}],
    },
}


def synth_prefixes():
    """First 16 values (f32 bits) of each seed's normal stream, std 1."""
    out = {}
    for name, seed in synth.SEEDS.items():
        for stream in (0, 1, 2):
            v = synth.normal_f32(seed, (16,), 1.0, stream=stream)
            out[f"{name}_s{stream}"] = v.view(np.uint32)
    return out


def main():
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(KATS, f, indent=1)

    # per-row INT8 (per output channel), 64 x 256; rows 0..3 carry edge cases
    w8 = synth.normal_f32(100, (64, 256), 0.02)
    w8[0] = 0.0                               # all-zero row: floor scale 1e-10
    w8[1, :] = np.float32(0.5)                # constant row
    w8[2, ::2] = np.float32(1.0)
    w8[2, 1::2] = np.float32(-1.0)           # codes +-127
    w8[3, 7] = np.float32(1000.0)            # one outlier
    q8, s8 = oracle.quantize_i8_rowwise(w8)
    d8 = oracle.dequantize_i8_rowwise(q8, s8)
    np.savez(os.path.join(HERE, "int8_rowwise_64x256.npz"), w=w8, q=q8, s=s8, w_hat=d8)

    # INT4 g128, 16 x 256 (two groups per row); rows 0..1 carry edge cases
    w4 = synth.normal_f32(101, (16, 256), 0.02)
    w4[0, :128] = 0.0                         # zero group: scale floor 2^-24
    w4[1, 128:] = np.linspace(-7.0, 7.0, 128, dtype=np.float32)  # exact codes -7..7
    p4, s4 = oracle.quantize_i4_g128(w4)
    d4 = oracle.dequantize_i4_g128(p4, s4)
    np.savez(os.path.join(HERE, "int4_g128_16x256.npz"), w=w4, packed=p4, s_f16=s4, w_hat=d4)

    # W8A8 accumulators 4 x 256 x 8 (plus the y the epilogue should approximate)
    xa = synth.normal_f32(102, (4, 256), 1.0)
    ww = synth.normal_f32(102, (8, 256), 0.02, stream=1)
    qa, sa = oracle.quantize_i8_rowwise(xa)
    qw, sw = oracle.quantize_i8_rowwise(ww)
    acc = oracle.gemm_w8a8_acc(qa, qw)
    y = oracle.linear_w8a8(qa, sa, qw, sw)
    np.savez(os.path.join(HERE, "w8a8_4x256x8.npz"), x=xa, w=ww, qa=qa, sa=sa, qw=qw, sw=sw, acc=acc, y=y)

    np.savez(os.path.join(HERE, "synth_prefixes.npz"), **synth_prefixes())

    # a quantized checkpoint written by the independent `safetensors` package:
    # the INT4 case above as a Linear "proj" (+ bias) and a few constants whose
    # values the C++ and Python readers assert
    from safetensors.numpy import save as st_save

    tensors = {
        "proj.weight": p4, "proj.weight_scale": s4.view(np.float16),
        "proj.bias": synth.normal_f32(103, (16,), 0.1),
        "const.f64": np.array([1.5, -2.0, 3.25]), "const.i8": np.array([-128, 0, 127], dtype=np.int8),
        "const.f16": np.array([0.5, -1.0, 65504.0], dtype=np.float16),
        "const.u8": np.array([[0, 255], [7, 128]], dtype=np.uint8),
    }
    meta = {"format": "theano-quantize/1", "proj.quant": "int4_g128", "proj.group_size": "128",
            "proj.in_features": "256", "proj.out_features": "16"}
    with open(os.path.join(HERE, "checkpoint_int4_16x256.safetensors"), "wb") as f:
        f.write(st_save(tensors, metadata=meta))
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
