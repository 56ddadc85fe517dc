"""quantize_tensor / dequantize_tensor / quantize_per_tensor / fake_quantize
(crates/theano-quantize/src/quantize.rs:8-55) on the GPU.

Codes come back as float32 device tensors: every code the reference returns
in its Vec<f64> (integral values within +-448, -0.0, NaN) is exact in f32, so
``codes.double()`` equals the reference's vector element for element.
"""
from __future__ import annotations

import torch

from . import _abi
from ._tensor import on_device, ptr, stream
from .qconfig import QuantDType

PER_TENSOR_WORKSPACE = 64  # TQ_PER_TENSOR_WORKSPACE


def quantize_tensor(tensor, scale: float, zero_point: float, dtype: QuantDType) -> torch.Tensor:
    """q = clamp(round(x / scale + zero_point), qmin, qmax) (quantize.rs:8-19)."""
    x = on_device(tensor, torch.float32, "quantize_tensor")
    q = torch.empty_like(x)
    _abi.call("tq_quantize_tensor", ptr(x), x.numel(), float(scale), float(zero_point), int(dtype),
              ptr(q), stream())
    return q


def dequantize_tensor(quantized, scale: float, zero_point: float) -> torch.Tensor:
    """x = (q - zero_point) * scale (quantize.rs:22-27), f64 arithmetic, f32 result."""
    q = on_device(quantized, torch.float32, "dequantize_tensor")
    out = torch.empty_like(q)
    _abi.call("tq_dequantize_tensor", ptr(q), q.numel(), float(scale), float(zero_point), ptr(out),
              stream())
    return out


def quantize_per_tensor(tensor, dtype: QuantDType):
    """Asymmetric per-tensor quantization (quantize.rs:30-48).

    Returns (codes, scale, zero_point) like the reference's tuple."""
    x = on_device(tensor, torch.float32, "quantize_per_tensor")
    q = torch.empty_like(x)
    szp = torch.empty(2, dtype=torch.float64, device=x.device)
    ws = torch.empty(PER_TENSOR_WORKSPACE, dtype=torch.uint8, device=x.device)
    _abi.call("tq_quantize_per_tensor", ptr(x), x.numel(), int(dtype), ptr(q), ptr(szp), ptr(ws),
              stream())
    s, z = szp.tolist()
    return q, s, z


def fake_quantize(tensor, scale: float, zero_point: float, dtype: QuantDType) -> torch.Tensor:
    """dequantize(quantize(x)) with the input's shape (quantize.rs:51-55)."""
    x = on_device(tensor, torch.float32, "fake_quantize")
    out = torch.empty_like(x)
    _abi.call("tq_fake_quantize", ptr(x), x.numel(), float(scale), float(zero_point), int(dtype),
              ptr(out), stream())
    return out
