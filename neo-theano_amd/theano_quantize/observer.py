"""MinMaxObserver / PerChannelMinMaxObserver (crates/theano-quantize/src/observer.rs:6-136).

The running min/max live on the device; the scale/zero-point arithmetic is the
reference's scalar f64 code, run on the host by libtq.so (tq_observer_scale_zp).
The state starts as float32 (exact for f32 data).  The first float64 input
widens it to float64 (exact) and from then on every input is folded in f64
(f32 inputs widen exactly), so f64 data get the reference's f64 min/max.
"""
from __future__ import annotations

import ctypes

import torch

from . import _abi
from ._tensor import device, on_device, ptr, stream
from .errors import InvalidArgument
from .qconfig import QuantDType


def _scale_zp(mn: float, mx: float, initialized: bool, dtype: QuantDType):
    s, z = ctypes.c_double(), ctypes.c_double()
    _abi.call("tq_observer_scale_zp", float(mn), float(mx), int(initialized), int(dtype),
              ctypes.byref(s), ctypes.byref(z))
    return s.value, z.value


def _observe_input(obs, values, name):
    """Device input in the state's element type; widens the state to float64
    on the first float64 input.  Returns (tensor, libtq suffix)."""
    t = values if isinstance(values, torch.Tensor) else torch.as_tensor(values)
    if t.dtype not in (torch.float32, torch.float64):
        raise InvalidArgument(f"{name}: expected float32 or float64, got {t.dtype}")
    if t.dtype == torch.float64 and obs._state.dtype == torch.float32:
        obs._state = obs._state.double()
    if obs._state.dtype == torch.float64:
        return on_device(t, t.dtype, name).double(), "_f64"
    return on_device(t, torch.float32, name), ""


class Observer:
    """Observer trait (observer.rs:6-10)."""

    def observe(self, values) -> None:
        raise NotImplementedError

    def compute_scale_zero_point(self, dtype: QuantDType):
        raise NotImplementedError

    def reset(self) -> None:
        raise NotImplementedError


class MinMaxObserver(Observer):
    """Running min/max of everything observed (observer.rs:12-73)."""

    def __init__(self):
        self._state = torch.empty(2, dtype=torch.float32, device=device())
        self.reset()

    def observe(self, values) -> None:
        x, f64 = _observe_input(self, values, "MinMaxObserver.observe")
        _abi.call("tq_minmax_observe" + f64, ptr(x), x.numel(), ptr(self._state), stream())
        self._initialized = True

    def min_val(self) -> float:
        return float(self._state[0].item())

    def max_val(self) -> float:
        return float(self._state[1].item())

    def compute_scale_zero_point(self, dtype: QuantDType):
        mn, mx = self._state.double().tolist()
        return _scale_zp(mn, mx, self._initialized, dtype)

    def reset(self) -> None:
        f64 = "_f64" if self._state.dtype == torch.float64 else ""
        _abi.call("tq_minmax_reset" + f64, ptr(self._state), 1, stream())
        self._initialized = False


class PerChannelMinMaxObserver(Observer):
    """Per-channel running min/max over a [channels, ...] layout (observer.rs:75-136)."""

    def __init__(self, num_channels: int):
        self.num_channels = int(num_channels)
        self._state = torch.empty(2 * self.num_channels, dtype=torch.float32, device=device())
        self.reset()

    def observe(self, values) -> None:
        x, f64 = _observe_input(self, values, "PerChannelMinMaxObserver.observe")
        _abi.call("tq_minmax_observe_per_channel" + f64, ptr(x), x.numel(), self.num_channels,
                  ptr(self._state), stream())
        self._initialized = True

    def min_vals(self):
        return self._state.view(-1, 2)[:, 0].double().tolist()

    def max_vals(self):
        return self._state.view(-1, 2)[:, 1].double().tolist()

    def scales_and_zero_points(self, dtype: QuantDType):
        """One (scale, zero_point) per channel (observer.rs:93-106); no
        `initialized` check, exactly like the reference."""
        st = self._state.view(-1, 2).double().tolist()
        return [_scale_zp(mn, mx, True, dtype) for mn, mx in st]

    def compute_scale_zero_point(self, dtype: QuantDType):
        """Average of the per-channel scales and zero points (observer.rs:123-129)."""
        sz = self.scales_and_zero_points(dtype)
        s = 0.0
        z = 0.0
        for a, b in sz:
            s += a
            z += b
        return s / len(sz), z / len(sz)

    def reset(self) -> None:
        f64 = "_f64" if self._state.dtype == torch.float64 else ""
        _abi.call("tq_minmax_reset" + f64, ptr(self._state), self.num_channels, stream())
        self._initialized = False
