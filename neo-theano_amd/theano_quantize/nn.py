"""Quantized modules: drop-in replacements for the reference's Linear and an
FFN block built from Linear + SiLU.

`QuantizedLinear` keeps the Module contract of crates/theano-nn/src/module.rs:8-55
(forward / parameters / named_parameters / num_parameters / state_dict) and
computes what `Linear::from_tensors(dequantize(W), b).forward(x)` computes
(linear.rs:65-75, 111-121): y = x . dequant(W)^T + b.

Modes (chosen from the QConfig):
  * "w8"   weight-only INT8 per output channel, f32 activations
           (QConfig.default_int8(): activations are not quantized);
  * "w8a8" INT8 weights and per-row dynamic INT8 activations
           (QConfig with activation_dtype Int8 and weight_dtype Int8);
  * "w4"   weight-only INT4 group-128, bf16 activations
           (QConfig.default_int4());
  * "fp8"  FP8 e4m3 weights per output channel and per-row dynamic FP8
           activations (QConfig with weight_dtype and activation_dtype FP8);
  * "fp8_weight"  FP8 e4m3 weight-only, f32 activations (weight_dtype FP8,
           activations not FP8).
Decode shapes (M <= 16 tokens) run the dequant-GEMV kernels (in "fp8" mode on
the fake-quantized activations, the same product as the GEMM); prefill shapes
run the i8-MFMA W8A8 GEMM, the fp8-MFMA GEMM or the bf16-MFMA W4A16 GEMM.
"""
from __future__ import annotations

import torch

from . import _abi
from ._tensor import on_device, ptr, stream
from .errors import InvalidArgument
from .formats import quantize_i4_g128, quantize_per_channel_fp8, quantize_per_channel_i8, repack_i4_g128_tiled
from .qconfig import QConfig, QuantDType

DECODE_MAX_M = 16
TILED_MAX_M = 16  # decode shapes run on the row-tiled copy of an INT4 weight


class Module:
    """Module contract (crates/theano-nn/src/module.rs:8-55)."""

    def forward(self, x):
        raise NotImplementedError

    def __call__(self, x):
        return self.forward(x)

    def parameters(self):
        return [t for _, t in self.named_parameters()]

    def named_parameters(self):
        return [(f"param_{i}", p) for i, p in enumerate(self.parameters())]

    def num_parameters(self) -> int:
        return sum(int(p.numel()) for p in self.parameters())

    def state_dict(self):
        return dict(self.named_parameters())


def _mode_of(qconfig: QConfig) -> str:
    if qconfig.weight_dtype == QuantDType.Int4:
        return "w4"
    if qconfig.weight_dtype == QuantDType.Int8:
        return "w8a8" if qconfig.activation_dtype == QuantDType.Int8 else "w8"
    if qconfig.weight_dtype == QuantDType.FP8:
        return "fp8" if qconfig.activation_dtype == QuantDType.FP8 else "fp8_weight"
    raise InvalidArgument(f"QuantizedLinear: unsupported weight dtype {qconfig.weight_dtype!r}")


class QuantizedLinear(Module):
    """y = x . dequant(W)^T + b with W quantized on the device."""

    def __init__(self, mode, in_features, out_features, qweight, scales, bias=None):
        self.mode = mode
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.qweight = qweight
        self.scales = scales
        self.bias = bias
        self.tiled = None
        if mode == "w4" and self.in_features <= 16384:
            # row-tiled copy (a permutation of qweight) for the decode GEMV, M <= 16
            self.tiled = repack_i4_g128_tiled(qweight, scales)

    @staticmethod
    def from_tensors(weight, bias=None, qconfig: QConfig | None = None) -> "QuantizedLinear":
        """Quantizes a [out, in] f32 weight (cf. Linear::from_tensors, linear.rs:65-75)."""
        qconfig = qconfig or QConfig.default_int8()
        mode = _mode_of(qconfig)
        w = on_device(weight, torch.float32, "QuantizedLinear.from_tensors")
        if w.dim() != 2:
            raise InvalidArgument("QuantizedLinear.from_tensors: weight must be [out, in]")
        out_f, in_f = w.shape
        if mode == "w4":
            q, s = quantize_i4_g128(w)
        elif mode in ("fp8", "fp8_weight"):
            q, s = quantize_per_channel_fp8(w)
        else:
            q, s = quantize_per_channel_i8(w)
        b = None if bias is None else on_device(bias, torch.float32, "bias")
        return QuantizedLinear(mode, in_f, out_f, q, s, b)

    def named_parameters(self):
        out = [("weight", self.qweight), ("weight_scale", self.scales)]
        if self.bias is not None:
            out.append(("bias", self.bias))
        return out

    def num_parameters(self) -> int:
        return self.in_features * self.out_features + (0 if self.bias is None else self.out_features)

    def _act_dtype(self):
        return torch.bfloat16 if self.mode == "w4" else torch.float32

    def forward(self, x):
        x = on_device(x, self._act_dtype(), "QuantizedLinear.forward")
        squeeze = x.dim() == 1
        if squeeze:
            x = x.unsqueeze(0)
        if x.dim() != 2 or x.shape[1] != self.in_features:
            raise InvalidArgument(
                f"QuantizedLinear.forward: shape mismatch, expected [*, {self.in_features}], "
                f"got {tuple(x.shape)}")
        m = x.shape[0]
        y = torch.empty((m, self.out_features), dtype=torch.float32, device=x.device)
        n, k = self.out_features, self.in_features
        if self.mode == "w4":
            if m <= TILED_MAX_M and self.tiled is not None:
                pt, st, t = self.tiled
                _abi.call("tq_gemv_w4g128_tiled", ptr(x), m, ptr(pt), ptr(st), ptr(self.bias), n, k, t,
                          ptr(y), stream())
            elif m <= DECODE_MAX_M:
                _abi.call("tq_gemv_w4g128", ptr(x), m, ptr(self.qweight), ptr(self.scales), ptr(self.bias), n, k,
                          ptr(y), stream())
            else:
                # prefill: pipelined kernels with x's k-order and group sums in a workspace
                nb = int(_abi.lib().tq_gemm_w4g128_bf16_workspace_bytes(m, k))
                ws = torch.empty((max(nb, 1),), dtype=torch.uint8, device=x.device)
                _abi.call("tq_gemm_w4g128_bf16_ws", ptr(x), m, ptr(self.qweight), ptr(self.scales), ptr(self.bias),
                          n, k, ptr(ws), nb, ptr(y), stream())
        elif self.mode == "w8":
            for m0 in range(0, m, DECODE_MAX_M):
                mm = min(DECODE_MAX_M, m - m0)
                _abi.call("tq_gemv_w8", ptr(x[m0:m0 + mm]), mm, ptr(self.qweight), ptr(self.scales),
                          ptr(self.bias), n, k, ptr(y[m0:m0 + mm]), stream())
        elif self.mode == "fp8" and m > DECODE_MAX_M:
            qa = torch.empty((m, k), dtype=torch.uint8, device=x.device)
            sa = torch.empty(m, dtype=torch.float32, device=x.device)
            _abi.call("tq_quantize_fp8_rowwise", ptr(x), m, k, ptr(qa), ptr(sa), stream())
            _abi.call("tq_gemm_fp8", ptr(qa), ptr(sa), ptr(self.qweight), ptr(self.scales),
                      ptr(self.bias), m, n, k, ptr(y), stream())
        elif self.mode in ("fp8", "fp8_weight"):
            if self.mode == "fp8":  # x -> e4m3(qa) * sa, the GEMM's activation values
                qa = torch.empty((m, k), dtype=torch.uint8, device=x.device)
                sa = torch.empty(m, dtype=torch.float32, device=x.device)
                xq = torch.empty_like(x)
                _abi.call("tq_fake_quantize_fp8_rowwise", ptr(x), m, k, ptr(qa), ptr(sa), ptr(xq), stream())
                x = xq
            for m0 in range(0, m, DECODE_MAX_M):
                mm = min(DECODE_MAX_M, m - m0)
                _abi.call("tq_gemv_fp8", ptr(x[m0:m0 + mm]), mm, ptr(self.qweight), ptr(self.scales),
                          ptr(self.bias), n, k, ptr(y[m0:m0 + mm]), stream())
        else:
            qa = torch.empty((m, k), dtype=torch.int8, device=x.device)
            sa = torch.empty(m, dtype=torch.float32, device=x.device)
            _abi.call("tq_quantize_i8_rowwise", ptr(x), m, k, ptr(qa), ptr(sa), stream())
            _abi.call("tq_gemm_w8a8", ptr(qa), ptr(sa), ptr(self.qweight), ptr(self.scales),
                      ptr(self.bias), m, n, k, None, ptr(y), stream())
        return y.squeeze(0) if squeeze else y


class QuantizedMLP(Module):
    """Llama-style FFN on INT4 g128 weights: y = (SiLU(x Wg^T) * (x Wu^T)) Wd^T.

    The composition follows Linear (linear.rs:111-121), SiLU
    (crates/theano-nn/src/activation.rs:66-79) and Tensor::mul; the
    SiLU(gate)*up intermediate is kept in f32."""

    def __init__(self, d, f, gate, up, down):
        self.d, self.f = int(d), int(f)
        self.gate, self.up, self.down = gate, up, down  # (packed, scales) pairs

    @staticmethod
    def from_tensors(gate_w, up_w, down_w) -> "QuantizedMLP":
        g = quantize_i4_g128(gate_w)
        u = quantize_i4_g128(up_w)
        dn = quantize_i4_g128(down_w)
        f, d = g[0].shape[0], g[0].shape[1] * 2
        if u[0].shape != g[0].shape or dn[0].shape != (d, f // 2):
            raise InvalidArgument("QuantizedMLP: gate/up must be [F, D] and down [D, F]")
        return QuantizedMLP(d, f, g, u, dn)

    def named_parameters(self):
        return [("gate.weight", self.gate[0]), ("gate.weight_scale", self.gate[1]),
                ("up.weight", self.up[0]), ("up.weight_scale", self.up[1]),
                ("down.weight", self.down[0]), ("down.weight_scale", self.down[1])]

    def num_parameters(self) -> int:
        return 3 * self.d * self.f

    def workspace_bytes(self, m: int) -> int:
        """Device bytes of intermediates forward() needs for m tokens."""
        return int(_abi.lib().tq_mlp_w4g128_workspace_bytes(m, self.d, self.f))

    def forward(self, x, workspace=None):
        """y = (SiLU(x Wg^T) * (x Wu^T)) Wd^T for x bf16 [M, D]; `workspace` is an
        optional uint8 device tensor of at least workspace_bytes(M) bytes."""
        x = on_device(x, torch.bfloat16, "QuantizedMLP.forward")
        if x.dim() != 2 or x.shape[1] != self.d:
            raise InvalidArgument(f"QuantizedMLP.forward: expected [M, {self.d}], got {tuple(x.shape)}")
        m = x.shape[0]
        need = self.workspace_bytes(m)
        if workspace is None:
            workspace = torch.empty((max(need, 1),), dtype=torch.uint8, device=x.device)
        y = torch.empty((m, self.d), dtype=torch.float32, device=x.device)
        _abi.call("tq_mlp_w4g128", ptr(x), m, self.d, self.f, ptr(self.gate[0]), ptr(self.gate[1]),
                  ptr(self.up[0]), ptr(self.up[1]), ptr(self.down[0]), ptr(self.down[1]),
                  ptr(workspace), workspace.numel() * workspace.element_size(), ptr(y), stream())
        return y
