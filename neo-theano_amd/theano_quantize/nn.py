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
Decode shapes (M <= 16 tokens) run the dequant-GEMV kernels; in "w8a8" and
"fp8" modes the GEMV quantizes the activation rows itself (the same codes and
product as quantize + GEMM, one launch).  "w4" runs the tiled GEMV in passes of
16 tokens up to M = 32, where it is faster than the prefill GEMM, whose 64-row
M tiles are mostly empty there.  Prefill shapes run the i8-MFMA W8A8 GEMM, the
fp8-MFMA GEMM or the bf16-MFMA W4A16 GEMM.
"""
from __future__ import annotations

import torch

from . import _abi
from ._tensor import on_device, ptr, stream
from .errors import InvalidArgument
from .formats import (quantize_i4_g128, quantize_per_channel_fp8, quantize_per_channel_i8, repack_i4_g128_gate_up_tiled,
                      repack_i4_g128_tiled)
from .qconfig import QConfig, QuantDType

DECODE_MAX_M = 16
# "w8a8" and "fp8": the GEMV with activation quantization inside up to this M (at
# 4096 x 4096: 5.4 / 7.0 us at M = 1 / 2 for INT8, 6.2 / 6.9 for FP8); beyond,
# quantize + the GEMM's skinny kernel (INT8 10.6 / 12.5 us at M = 3 / 16, FP8
# 10.0 / 11.3, against 12.0 / 52.3 and 12.9 / 54.0 us for the fused GEMV)
FUSED_A8_MAX_M = 2
TILED_MAX_M = 16  # tokens per launch of the INT4 GEMV on the row-tiled copy
# INT4 Linear: the tiled GEMV in passes of TILED_MAX_M tokens up to this M (at N =
# 14336, K = 4096: 19 us at M = 17-32 against 21-24 us for the prefill GEMM on
# its 64-row tiles; 28.5 / 37 against 24.5 / 25.5 us at M = 48 / 64)
TILED_PASSES_MAX_M = 32
# QuantizedMLP runs the decode kernels for up to 8 tokens, and, where D <= 4096
# (its gate/up then takes 16 tokens in one launch), up to 28 tokens in passes of
# 16; the prefill FFN beyond.  At D = 4096, F = 14336: 48 us at 16 tokens and
# 66-78 us for 17-24 (93 us at 32), against 85-88 us for the prefill FFN on its
# 64-row tiles at 16-32 tokens.
DECODE_MLP_MAX_M = 28
DECODE_MLP_PASS_M = 16
DECODE_MLP_ONE_PASS_D = 4096
MLP_DOWN_TILE_ROWS = 32  # tile height of the FFN's decode copy of down


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


def _fused_a8_ok(x, q, k) -> bool:
    """Shapes the fused-activation decode GEMVs take (tq_gemv_w8a8 / tq_gemv_fp8a8)."""
    return 0 < k <= 8192 and k % 16 == 0 and x.data_ptr() % 16 == 0 and q.data_ptr() % 16 == 0


class QuantizedLinear(Module):
    """y = x . dequant(W)^T + b with W quantized on the device."""

    def __init__(self, mode, in_features, out_features, qweight, scales, bias=None, tiled=True):
        self.mode = mode
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.qweight = qweight
        self.scales = scales
        self.bias = bias
        self.tiled = None
        if tiled and mode == "w4" and self.in_features <= 16384:
            # row-tiled copy (a permutation of qweight) for the decode GEMV (passes
            # of 16 tokens up to M = 32)
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
            if m <= TILED_PASSES_MAX_M and self.tiled is not None:
                pt, st, t = self.tiled
                for m0 in range(0, m, TILED_MAX_M):
                    mm = min(TILED_MAX_M, m - m0)
                    _abi.call("tq_gemv_w4g128_tiled", ptr(x[m0:m0 + mm]), mm, ptr(pt), ptr(st), ptr(self.bias), n,
                              k, t, ptr(y[m0:m0 + mm]), stream())
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
        elif self.mode in ("w8a8", "fp8") and m <= FUSED_A8_MAX_M and _fused_a8_ok(x, self.qweight, k):
            # activation quantization fused into the decode GEMV (one launch)
            _abi.call("tq_gemv_w8a8" if self.mode == "w8a8" else "tq_gemv_fp8a8", ptr(x), m, ptr(self.qweight),
                      ptr(self.scales), ptr(self.bias), n, k, ptr(y), stream())
        elif self.mode == "fp8" and m > FUSED_A8_MAX_M:
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

    def __init__(self, d, f, gate, up, down, tiled=True):
        self.d, self.f = int(d), int(f)
        self.gate, self.up, self.down = gate, up, down  # (packed, scales) pairs
        self.decode = None
        if tiled and self.d <= 16384 and self.f <= 16384:
            # row-tiled copies (permutations of the weights) for decode shapes:
            # gate and up interleaved in 64-row tiles, down in 32-row tiles (two K
            # halves per tile: 2 * D / 32 blocks, one round at D = 4096)
            gu = repack_i4_g128_gate_up_tiled(gate, up)
            dn = repack_i4_g128_tiled(down[0], down[1], MLP_DOWN_TILE_ROWS)
            self.decode = (gu[0], gu[1], dn[0], dn[1], dn[2])

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

    def _decode_path(self, m: int) -> bool:
        if self.decode is None or m < 1:
            return False
        return m <= 8 or (m <= DECODE_MLP_MAX_M and self.d <= DECODE_MLP_ONE_PASS_D)

    def workspace_bytes(self, m: int) -> int:
        """Device bytes of intermediates forward() needs for m tokens."""
        if self._decode_path(m):
            mm = min(m, DECODE_MLP_PASS_M)  # one pass at a time
            return int(_abi.lib().tq_mlp_w4g128_decode_workspace_bytes(mm, self.d, self.f))
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
        wsb = workspace.numel() * workspace.element_size()
        if self._decode_path(m):
            gu_t, gu_st, dn_t, dn_st, dn_rows = self.decode
            for m0 in range(0, m, DECODE_MLP_PASS_M):  # passes ordered on the stream share the workspace
                mm = min(DECODE_MLP_PASS_M, m - m0)
                _abi.call("tq_mlp_w4g128_decode", ptr(x[m0:m0 + mm]), mm, self.d, self.f, ptr(gu_t), ptr(gu_st),
                          ptr(dn_t), ptr(dn_st), dn_rows, ptr(workspace), wsb, ptr(y[m0:m0 + mm]), stream())
            return y
        _abi.call("tq_mlp_w4g128", ptr(x), m, self.d, self.f, ptr(self.gate[0]), ptr(self.gate[1]),
                  ptr(self.up[0]), ptr(self.up[1]), ptr(self.down[0]), ptr(self.down[1]),
                  ptr(workspace), wsb, ptr(y), stream())
        return y


class QuantizedMultiheadAttention(Module):
    """MultiheadAttention (crates/theano-nn/src/transformer.rs:9-162) with its
    q/k/v/out projections as QuantizedLinear consumers.

    The q, k and v weights are quantized row by row (per channel, or per row
    group for INT4), so their concatenation [3E, E] quantizes to exactly the
    three separate codes: self-attention runs the three projections as ONE
    fused GEMM / GEMV over the concatenated weight; cross-attention
    (forward_with_mask with distinct query / key / value) runs row slices of it.
    The attention core (scores, additive mask, softmax, P V) is libtq's
    tq_attention_f32 reading q, k and v in place in the fused [B*S, 3E] output.
    Inputs and outputs are f32 [batch, seq, embed_dim] device tensors."""

    def __init__(self, num_heads, qkv: QuantizedLinear, out_proj: QuantizedLinear):
        e = out_proj.in_features
        if qkv.out_features != 3 * e or qkv.in_features != e or out_proj.out_features != e or e % num_heads:
            raise InvalidArgument("QuantizedMultiheadAttention: qkv must be [3E, E], out_proj [E, E], E % heads == 0")
        self.embed_dim, self.num_heads, self.head_dim = e, int(num_heads), e // int(num_heads)
        self.qkv, self.out_proj = qkv, out_proj
        self._parts = []
        for i in range(3):  # row slices (views) of the fused weight
            rows = slice(i * e, (i + 1) * e)
            self._parts.append(QuantizedLinear(qkv.mode, e, e, qkv.qweight[rows], qkv.scales[rows],
                                               None if qkv.bias is None else qkv.bias[rows], tiled=False))

    @staticmethod
    def from_tensors(num_heads, wq, wk, wv, wo, bq=None, bk=None, bv=None, bo=None,
                     qconfig: QConfig | None = None) -> "QuantizedMultiheadAttention":
        """Quantizes [E, E] f32 weights (cf. MultiheadAttention::from_linears,
        transformer.rs:49-61); missing q/k/v biases are zeros when any is given."""
        ws = [on_device(w, torch.float32, "QuantizedMultiheadAttention.from_tensors") for w in (wq, wk, wv)]
        e = ws[0].shape[0]
        bias = None
        if any(b is not None for b in (bq, bk, bv)):
            bias = torch.cat([torch.zeros(e, dtype=torch.float32, device=ws[0].device) if b is None
                              else on_device(b, torch.float32, "bias") for b in (bq, bk, bv)])
        qkv = QuantizedLinear.from_tensors(torch.cat(ws, 0), bias, qconfig)
        out = QuantizedLinear.from_tensors(wo, bo, qconfig)
        return QuantizedMultiheadAttention(num_heads, qkv, out)

    def named_parameters(self):
        out = []
        for name, part in zip(("q_proj", "k_proj", "v_proj"), self._parts):
            out += [(f"{name}.{n}", t) for n, t in part.named_parameters()]
        out += [(f"out_proj.{n}", t) for n, t in self.out_proj.named_parameters()]
        return out

    def num_parameters(self) -> int:
        return self.qkv.num_parameters() + self.out_proj.num_parameters()

    def _act(self, x2d):
        from ._tensor import convert

        return convert(x2d, torch.bfloat16) if self.qkv.mode == "w4" else x2d

    def _attend(self, q, k, v, ldq, ldk, ldv, batch, seq, mask):
        from . import _abi

        e = self.embed_dim
        o = torch.empty((batch * seq, e), dtype=torch.float32, device=q.device)
        mb, mp = 0, None
        if mask is not None:
            mp = on_device(mask, torch.float32, "attention mask")
            if mp.dim() == 4:  # [Bm, 1, S, S]
                mp = mp.reshape(mp.shape[0], seq, seq)
            if mp.dim() != 3 or mp.shape[1:] != (seq, seq) or mp.shape[0] not in (1, batch):
                raise InvalidArgument(f"attention mask: expected [batch or 1, {seq}, {seq}], got {tuple(mask.shape)}")
            mb = 1 if mp.shape[0] == 1 and batch != 1 else mp.shape[0]
        _abi.call("tq_attention_f32", ptr(q), ldq, ptr(k), ldk, ptr(v), ldv, ptr(mp), mb, batch, seq,
                  self.num_heads, self.head_dim, ptr(o), e, stream())
        return o

    def forward_with_mask(self, query, key, value, mask=None):
        """query, key, value: [batch, seq, embed_dim]; mask additive [batch or 1,
        (1,) seq, seq] (transformer.rs:86-142).  Returns [batch, seq, embed_dim]."""
        xs = [on_device(t, torch.float32, "QuantizedMultiheadAttention.forward") for t in (query, key, value)]
        if any(t.dim() != 3 or t.shape[2] != self.embed_dim for t in xs) or len({tuple(t.shape) for t in xs}) != 1:
            raise InvalidArgument("QuantizedMultiheadAttention: query, key, value must be [batch, seq, embed_dim]")
        batch, seq, e = xs[0].shape
        flat = [t.reshape(batch * seq, e) for t in xs]
        if query is key and key is value:  # self-attention: one fused projection
            qkv = self.qkv(self._act(flat[0]))
            q, k, v = qkv, qkv[:, e:], qkv[:, 2 * e:]
            ld = 3 * e
            o = self._attend(q, k, v, ld, ld, ld, batch, seq, mask)
        else:
            q, k, v = (part(self._act(x)) for part, x in zip(self._parts, flat))
            o = self._attend(q, k, v, e, e, e, batch, seq, mask)
        return self.out_proj(self._act(o)).reshape(batch, seq, e)

    def forward_qkv(self, query, key, value):
        return self.forward_with_mask(query, key, value, None)

    def forward(self, x):
        return self.forward_with_mask(x, x, x, None)
