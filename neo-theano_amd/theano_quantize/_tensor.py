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
