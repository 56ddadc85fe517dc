"""Device-memory plumbing: torch tensors supply HIP allocations and streams."""
from __future__ import annotations

import ctypes

import torch

from .errors import InvalidArgument


def device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("theano_quantize needs a ROCm GPU (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


def on_device(t, dtype: torch.dtype, name: str) -> torch.Tensor:
    """Returns `t` as a dense device tensor of `dtype` (copies only if needed)."""
    if not isinstance(t, torch.Tensor):
        t = torch.as_tensor(t)
    if t.dtype != dtype:
        raise InvalidArgument(f"{name}: expected dtype {dtype}, got {t.dtype}")
    if t.device.type != "cuda":
        t = t.to(device())
    return t.contiguous()


def ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(None if t is None else t.data_ptr())


def stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


# DType order of the reference (crates/theano-types/src/dtype.rs:5-25) -> the
# torch element type holding it on the device (F16 / BF16 / Bool as their bits)
DTYPE_CODES = {"float16": 0, "bfloat16": 1, "float32": 2, "float64": 3, "uint8": 4, "int8": 5, "int16": 6,
               "int32": 7, "int64": 8, "bool": 9}
_TORCH_OF = {0: torch.float16, 1: torch.bfloat16, 2: torch.float32, 3: torch.float64, 4: torch.uint8, 5: torch.int8,
             6: torch.int16, 7: torch.int32, 8: torch.int64, 9: torch.bool}
_CODE_OF = {v: k for k, v in _TORCH_OF.items()}


def convert(t: torch.Tensor, dtype) -> torch.Tensor:
    """Tensor::to for element types on the device (libtq tq_convert): the f64
    value of each element cast to `dtype` (a torch dtype or a DType name) with
    round-to-nearest-even for floats and Rust `as` (toward zero, saturating,
    NaN -> 0) for integers."""
    from . import _abi

    dst = DTYPE_CODES[dtype] if isinstance(dtype, str) else _CODE_OF.get(dtype)
    src = _CODE_OF.get(t.dtype)
    if dst is None or src is None:
        raise InvalidArgument(f"convert: unsupported dtype {t.dtype} -> {dtype}")
    if t.device.type != "cuda":
        t = t.to(device())
    t = t.contiguous()
    out = torch.empty(t.shape, dtype=_TORCH_OF[dst], device=t.device)
    _abi.call("tq_convert", ptr(t), src, ptr(out), dst, t.numel(), stream())
    return out
