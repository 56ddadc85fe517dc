"""quantize_tensor / dequantize_tensor / quantize_per_tensor / fake_quantize
(crates/theano-quantize/src/quantize.rs:8-55) on the GPU.

Each primitive takes float32 or float64 device data.  float64 (the element type
of the reference's Tensor storage and Vec<f64>) runs the libtq ``_f64`` entry
points and returns exactly the reference's f64 values.  float32 runs the
device-native forms; their codes come back as float32: every code the
reference returns (integral values within +-448, -0.0, NaN) is exact in f32,
so ``codes.double()`` equals the reference's vector element for element.
Other element types raise InvalidArgument.
"""
from __future__ import annotations

import torch

from . import _abi
from ._tensor import on_device, ptr, stream
from .errors import InvalidArgument
from .qconfig import QuantDType

PER_TENSOR_WORKSPACE = 64  # TQ_PER_TENSOR_WORKSPACE


def _float_input(tensor, name):
    """(device tensor, f64 suffix): float64 keeps the reference's element type."""
    t = tensor if isinstance(tensor, torch.Tensor) else torch.as_tensor(tensor)
    if t.dtype == torch.float64:
        return on_device(t, torch.float64, name), "_f64"
    if t.dtype == torch.float32:
        return on_device(t, torch.float32, name), ""
    raise InvalidArgument(f"{name}: expected float32 or float64, got {t.dtype}")


def quantize_tensor(tensor, scale: float, zero_point: float, dtype: QuantDType) -> torch.Tensor:
    """q = clamp(round(x / scale + zero_point), qmin, qmax) (quantize.rs:8-19)."""
    x, f64 = _float_input(tensor, "quantize_tensor")
    q = torch.empty_like(x)
    _abi.call("tq_quantize_tensor" + f64, ptr(x), x.numel(), float(scale), float(zero_point), int(dtype),
              ptr(q), stream())
    return q


def dequantize_tensor(quantized, scale: float, zero_point: float) -> torch.Tensor:
    """x = (q - zero_point) * scale (quantize.rs:22-27) in f64; float32 codes
    give the f32 rounding of that value, float64 codes the f64 value itself."""
    q, f64 = _float_input(quantized, "dequantize_tensor")
    out = torch.empty_like(q)
    _abi.call("tq_dequantize_tensor" + f64, ptr(q), q.numel(), float(scale), float(zero_point), ptr(out),
              stream())
    return out


def quantize_per_tensor(tensor, dtype: QuantDType):
    """Asymmetric per-tensor quantization (quantize.rs:30-48).

    Returns (codes, scale, zero_point) like the reference's tuple."""
    x, f64 = _float_input(tensor, "quantize_per_tensor")
    q = torch.empty_like(x)
    szp = torch.empty(2, dtype=torch.float64, device=x.device)
    ws = torch.empty(PER_TENSOR_WORKSPACE, dtype=torch.uint8, device=x.device)
    _abi.call("tq_quantize_per_tensor" + f64, ptr(x), x.numel(), int(dtype), ptr(q), ptr(szp), ptr(ws),
              stream())
    s, z = szp.tolist()
    return q, s, z


def fake_quantize(tensor, scale: float, zero_point: float, dtype: QuantDType) -> torch.Tensor:
    """dequantize(quantize(x)) with the input's shape (quantize.rs:51-55)."""
    x, f64 = _float_input(tensor, "fake_quantize")
    out = torch.empty_like(x)
    _abi.call("tq_fake_quantize" + f64, ptr(x), x.numel(), float(scale), float(zero_point), int(dtype),
              ptr(out), stream())
    return out
