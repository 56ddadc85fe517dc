"""theano_quantize -- MI355X (gfx950) implementation of neo-theano's
`theano-quantize` crate and its quantized Linear, over libtq.so's C ABI.

Same names as the reference crate (crates/theano-quantize/src/lib.rs:9-11):
QuantDType, QConfig, Observer, MinMaxObserver, PerChannelMinMaxObserver,
quantize_tensor, dequantize_tensor, quantize_per_tensor (+ fake_quantize).
Build-defined formats and modules: quantize_per_channel_i8, quantize_i4_g128,
quantize_per_channel_fp8 (OCP e4m3),
QuantizedLinear, QuantizedMLP; quantized checkpoints (save_quantized /
load_quantized over the safetensors container of crates/theano-serialize).
"""
from ._tensor import convert
from .checkpoint import load_quantized, load_safetensors, save_quantized, save_safetensors
from .errors import InvalidArgument, KernelError, OutOfMemory, TheanoError
from .formats import (
    dequantize_i4_g128,
    dequantize_per_channel_fp8,
    dequantize_per_channel_i8,
    fake_quantize_per_channel_fp8,
    fake_quantize_per_channel_i8,
    quantize_i4_g128,
    quantize_per_channel_fp8,
    quantize_per_channel_i8,
    repack_i4_g128_gate_up_tiled,
    repack_i4_g128_tiled,
    tile_rows_for,
)
from .nn import Module, QuantizedLinear, QuantizedMLP, QuantizedMultiheadAttention
from .observer import MinMaxObserver, Observer, PerChannelMinMaxObserver
from .qconfig import QConfig, QuantDType
from .quantize import dequantize_tensor, fake_quantize, quantize_per_tensor, quantize_tensor

__all__ = [
    "TheanoError", "InvalidArgument", "KernelError", "OutOfMemory",
    "QuantDType", "QConfig", "Observer", "MinMaxObserver", "PerChannelMinMaxObserver",
    "quantize_tensor", "dequantize_tensor", "quantize_per_tensor", "fake_quantize",
    "quantize_per_channel_i8", "dequantize_per_channel_i8", "fake_quantize_per_channel_i8",
    "quantize_per_channel_fp8", "dequantize_per_channel_fp8", "fake_quantize_per_channel_fp8",
    "quantize_i4_g128", "dequantize_i4_g128", "repack_i4_g128_tiled", "repack_i4_g128_gate_up_tiled", "tile_rows_for", "Module", "QuantizedLinear", "QuantizedMLP", "QuantizedMultiheadAttention",
    "save_safetensors", "load_safetensors", "save_quantized", "load_quantized", "convert",
]
