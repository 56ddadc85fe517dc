"""QuantDType and QConfig (crates/theano-quantize/src/qconfig.rs:5-76)."""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass

from . import _abi


class QuantDType(enum.IntEnum):
    """Quantized data types, same order as the reference enum (qconfig.rs:5-10)."""

    Int8 = 0
    UInt8 = 1
    Int4 = 2
    FP8 = 3

    def _info(self):
        bits, signed = ctypes.c_int(), ctypes.c_int()
        qmin, qmax = ctypes.c_double(), ctypes.c_double()
        _abi.call("tq_qdtype_info", int(self), ctypes.byref(bits), ctypes.byref(signed),
                  ctypes.byref(qmin), ctypes.byref(qmax))
        return bits.value, bool(signed.value), qmin.value, qmax.value

    def bits(self) -> int:  # qconfig.rs:13-18
        return self._info()[0]

    def is_signed(self) -> bool:  # qconfig.rs:20-22
        return self._info()[1]

    def qmin(self) -> float:  # qconfig.rs:24-31
        return self._info()[2]

    def qmax(self) -> float:  # qconfig.rs:33-40
        return self._info()[3]


@dataclass
class QConfig:
    """Quantization configuration for a layer (qconfig.rs:44-76).

    As in the reference, `symmetric` and `per_channel` are recorded; the
    quantized Linear here always uses symmetric per-output-channel INT8 or
    symmetric group-128 INT4 weights, selected by `weight_dtype`."""

    weight_dtype: QuantDType
    activation_dtype: QuantDType
    symmetric: bool
    per_channel: bool

    @staticmethod
    def default_int8() -> "QConfig":  # qconfig.rs:53-60
        return QConfig(QuantDType.Int8, QuantDType.UInt8, True, False)

    @staticmethod
    def default_int4() -> "QConfig":  # qconfig.rs:62-69
        return QConfig(QuantDType.Int4, QuantDType.Int8, True, True)

    @staticmethod
    def default() -> "QConfig":  # qconfig.rs:72-76
        return QConfig.default_int8()
