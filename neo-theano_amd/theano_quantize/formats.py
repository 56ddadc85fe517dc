"""Weight formats built from the reference primitives.

* per-row symmetric INT8: s_r = f32(max(absmax_r/127, 1e-10)),
  q = quantize_tensor(row, s_r, 0, Int8)  (quantize.rs:8-19, 39; observer.rs:110-121)
* INT4, groups of 128 along K: s = max(f16_rne(absmax/7), 2^-24),
  q = quantize_tensor(group, s, 0, Int4), two nibbles per byte, low nibble = even k.
* per-row symmetric FP8 (OCP e4m3, the 8-bit float behind QuantDType::FP8 and
  its [-448, 448] range, qconfig.rs:29,38): s_r = f32(max(absmax_r/448, 1e-10)),
  q = e4m3_rne(clamp(f32(x/s_r), -448, 448)), NaN -> 0x7F.  Codes are kept as
  uint8 bit patterns (``q.view(torch.float8_e4m3fn)`` reads them as floats).
"""
from __future__ import annotations

import torch

from . import _abi
from ._tensor import on_device, ptr, stream
from .errors import InvalidArgument

GROUP = 128


def _as_2d(w, name):
    w = on_device(w, torch.float32, name)
    if w.dim() != 2:
        raise InvalidArgument(f"{name}: expected a 2-D [rows, K] tensor, got shape {tuple(w.shape)}")
    return w


def quantize_per_channel_i8(weight):
    """Symmetric per-row INT8 -> (codes int8 [N, K], scales f32 [N])."""
    w = _as_2d(weight, "quantize_per_channel_i8")
    n, k = w.shape
    q = torch.empty((n, k), dtype=torch.int8, device=w.device)
    s = torch.empty(n, dtype=torch.float32, device=w.device)
    _abi.call("tq_quantize_i8_rowwise", ptr(w), n, k, ptr(q), ptr(s), stream())
    return q, s


def dequantize_per_channel_i8(q, s):
    """w_hat = f32(q * s[row]) (quantize.rs:22-27 per row)."""
    q = on_device(q, torch.int8, "dequantize_per_channel_i8")
    s = on_device(s, torch.float32, "dequantize_per_channel_i8")
    n, k = q.shape
    out = torch.empty((n, k), dtype=torch.float32, device=q.device)
    _abi.call("tq_dequantize_i8_rowwise", ptr(q), ptr(s), n, k, ptr(out), stream())
    return out


def fake_quantize_per_channel_i8(weight):
    """Codes, scales and the dequantized tensor in one pass."""
    w = _as_2d(weight, "fake_quantize_per_channel_i8")
    n, k = w.shape
    q = torch.empty((n, k), dtype=torch.int8, device=w.device)
    s = torch.empty(n, dtype=torch.float32, device=w.device)
    out = torch.empty((n, k), dtype=torch.float32, device=w.device)
    _abi.call("tq_fake_quantize_i8_rowwise", ptr(w), n, k, ptr(q), ptr(s), ptr(out), stream())
    return q, s, out


def quantize_per_channel_fp8(weight):
    """Symmetric per-row FP8 e4m3 -> (codes uint8 [N, K], scales f32 [N])."""
    w = _as_2d(weight, "quantize_per_channel_fp8")
    n, k = w.shape
    q = torch.empty((n, k), dtype=torch.uint8, device=w.device)
    s = torch.empty(n, dtype=torch.float32, device=w.device)
    _abi.call("tq_quantize_fp8_rowwise", ptr(w), n, k, ptr(q), ptr(s), stream())
    return q, s


def dequantize_per_channel_fp8(q, s):
    """w_hat = f32(e4m3(q) * s[row])."""
    q = on_device(q, torch.uint8, "dequantize_per_channel_fp8")
    s = on_device(s, torch.float32, "dequantize_per_channel_fp8")
    n, k = q.shape
    out = torch.empty((n, k), dtype=torch.float32, device=q.device)
    _abi.call("tq_dequantize_fp8_rowwise", ptr(q), ptr(s), n, k, ptr(out), stream())
    return out


def fake_quantize_per_channel_fp8(weight):
    """FP8 codes, scales and the dequantized tensor in one pass."""
    w = _as_2d(weight, "fake_quantize_per_channel_fp8")
    n, k = w.shape
    q = torch.empty((n, k), dtype=torch.uint8, device=w.device)
    s = torch.empty(n, dtype=torch.float32, device=w.device)
    out = torch.empty((n, k), dtype=torch.float32, device=w.device)
    _abi.call("tq_fake_quantize_fp8_rowwise", ptr(w), n, k, ptr(q), ptr(s), ptr(out), stream())
    return q, s, out


def quantize_i4_g128(weight):
    """Symmetric INT4 g128 -> (packed uint8 [N, K/2], scales f16 [N, K/128])."""
    w = _as_2d(weight, "quantize_i4_g128")
    n, k = w.shape
    if k % GROUP:
        raise InvalidArgument(f"quantize_i4_g128: K={k} is not a multiple of {GROUP}")
    p = torch.empty((n, k // 2), dtype=torch.uint8, device=w.device)
    s = torch.empty((n, k // GROUP), dtype=torch.float16, device=w.device)
    _abi.call("tq_quantize_i4_g128", ptr(w), n, k, ptr(p), ptr(s), stream())
    return p, s


def dequantize_i4_g128(packed, scales):
    """w_hat = f32(q * s) for the group-128 INT4 format."""
    p = on_device(packed, torch.uint8, "dequantize_i4_g128")
    s = on_device(scales, torch.float16, "dequantize_i4_g128")
    n, kh = p.shape
    out = torch.empty((n, 2 * kh), dtype=torch.float32, device=p.device)
    _abi.call("tq_dequantize_i4_g128", ptr(p), ptr(s), n, 2 * kh, ptr(out), stream())
    return out


def tile_rows_for(n: int) -> int:
    """Tile height of the decode kernel layout for an N-row weight on this device."""
    return int(_abi.lib().tq_w4g128_tile_rows(int(n)))


def repack_i4_g128_gate_up_tiled(gate, up):
    """Gate and up projections of an FFN (canonical INT4 g128 (packed, scales) pairs
    of [F, D]) as one row-tiled weight of 64-row tiles: tile t holds gate rows
    32t..32t+31 then up rows 32t..32t+31.  Returns (packed_t, s_t)."""
    gp = on_device(gate[0], torch.uint8, "repack_i4_g128_gate_up_tiled")
    gs = on_device(gate[1], torch.float16, "repack_i4_g128_gate_up_tiled")
    upk = on_device(up[0], torch.uint8, "repack_i4_g128_gate_up_tiled")
    us = on_device(up[1], torch.float16, "repack_i4_g128_gate_up_tiled")
    f, kh = gp.shape
    if tuple(upk.shape) != (f, kh):
        raise InvalidArgument("repack_i4_g128_gate_up_tiled: gate and up must have the same shape")
    d = 2 * kh
    tiles = (f + 31) // 32
    pt = torch.empty(tiles * 64 * kh, dtype=torch.uint8, device=gp.device)
    st = torch.empty(tiles * 64 * (d // GROUP), dtype=torch.float16, device=gp.device)
    _abi.call("tq_repack_w4g128_gate_up_tiled", ptr(gp), ptr(gs), ptr(upk), ptr(us), f, d, ptr(pt), ptr(st), stream())
    return pt, st


def repack_i4_g128_tiled(packed, scales, tile_rows=None):
    """Row-tiled kernel layout of a canonical INT4 g128 weight (a pure permutation,
    rows padded to a multiple of tile_rows).  Returns (packed_t, s_t, tile_rows)."""
    p = on_device(packed, torch.uint8, "repack_i4_g128_tiled")
    s = on_device(scales, torch.float16, "repack_i4_g128_tiled")
    n, kh = p.shape
    k = 2 * kh
    t = tile_rows_for(n) if tile_rows is None else int(tile_rows)
    tiles = (n + t - 1) // t
    pt = torch.empty(tiles * t * kh, dtype=torch.uint8, device=p.device)
    st = torch.empty(tiles * t * (k // GROUP), dtype=torch.float16, device=p.device)
    _abi.call("tq_repack_w4g128_tiled", ptr(p), ptr(s), n, k, t, ptr(pt), ptr(st), stream())
    return pt, st, t
