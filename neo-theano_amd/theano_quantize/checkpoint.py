"""Quantized checkpoints in the safetensors container.

The reference's serializer (crates/theano-serialize/src/safetensors.rs) writes
an 8-byte little-endian header length, a JSON header and a data section
(safetensors.rs:3, ``to_bytes`` :83-95), with every payload stored as f64
little-endian whatever the tensor's dtype name (``add_tensor`` :36-54), and
its parser recognises only float/int64/int32 names (:203-208).  Quantized
weights need their own element types so that a checkpoint loads straight into
the device buffers of ``QuantizedLinear`` / ``QuantizedMLP``.

Read: both dialects of the container.
* The reference dialect: dtype names as ``DType`` prints them ("float32",
  "float64", "int8", ...; crates/theano-types/src/dtype.rs:79-100).  A payload
  of 8 bytes per element is the reference's f64 encoding and decodes to f64; a
  payload of the named type's size decodes as that type.
* Standard safetensors: dtype codes F64, F32, F16, BF16, I64, I32, I16, I8, U8,
  BOOL, F8_E4M3 with payloads of that element type, and an optional
  ``__metadata__`` map of strings.  F8_E4M3 payloads are read as their uint8
  bit patterns.

Written: standard safetensors (tensors in name order, contiguous, header
padded with spaces to a multiple of 8 bytes).  A quantized Linear ``<name>``
becomes
    <name>.weight        I8 [N, K]    per-row INT8 codes
                         U8 [N, K/2]  INT4 g128, two nibbles per byte, low nibble = even k
                         F8_E4M3 [N, K]  per-row FP8 (OCP e4m3) codes
    <name>.weight_scale  F32 [N]      | F16 [N, K/128] (INT4)
    <name>.bias          F32 [N]      (when present)
with ``__metadata__`` entries ``<name>.quant`` ("int8_per_channel",
"int8_per_channel_a8" for W8A8, "int4_g128", "fp8_e4m3_per_channel" (FP8
weight-only) or "fp8_e4m3_per_channel_a8" (FP8 weights and activations)),
``<name>.group_size`` ("128",
INT4), ``<name>.in_features`` and
``<name>.out_features``; a ``QuantizedMLP`` ``<name>`` is the three INT4
Linears ``<name>.gate``, ``<name>.up``, ``<name>.down`` plus ``<name>.quant`` =
"mlp_int4_g128".  A ``QuantizedMultiheadAttention`` ``<name>`` is the Linears
``<name>.qkv`` (the fused [3E, E] projection) and ``<name>.out_proj`` plus
``<name>.attention`` = "multihead" and ``<name>.num_heads``.  ``format`` =
"theano-quantize/1".
"""
from __future__ import annotations

import json
import struct

import numpy as np

from .errors import InvalidArgument

FORMAT = "theano-quantize/1"

# standard safetensors codes -> numpy element type (BF16 kept as its 16-bit pattern)
_STD = {"F64": np.float64, "F32": np.float32, "F16": np.float16, "BF16": np.uint16, "I64": np.int64,
        "I32": np.int32, "I16": np.int16, "I8": np.int8, "U8": np.uint8, "BOOL": np.bool_,
        "F8_E4M3": np.uint8}
# the reference's DType names (dtype.rs:79-100) -> numpy element type of a raw payload
_REF = {"float64": np.float64, "float32": np.float32, "float16": np.float16, "bfloat16": np.uint16,
        "int64": np.int64, "int32": np.int32, "int16": np.int16, "int8": np.int8, "uint8": np.uint8,
        "bool": np.bool_, "qint8": np.int8, "quint8": np.uint8, "qint32": np.int32}
_CODE_OF = {np.dtype(np.float64): "F64", np.dtype(np.float32): "F32", np.dtype(np.float16): "F16",
            np.dtype(np.int64): "I64", np.dtype(np.int32): "I32", np.dtype(np.int16): "I16",
            np.dtype(np.int8): "I8", np.dtype(np.uint8): "U8", np.dtype(np.bool_): "BOOL"}


def _host_array(t):
    """numpy view of a numpy array or a (device) torch tensor; bfloat16 -> (uint16 bits, "BF16"),
    float8_e4m3fn -> (uint8 bits, "F8_E4M3")."""
    try:
        import torch
    except ImportError:  # pragma: no cover
        torch = None
    if torch is not None and isinstance(t, torch.Tensor):
        t = t.detach()
        if t.dtype == torch.bfloat16:
            return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16), "BF16"
        if t.dtype == torch.float8_e4m3fn:
            return t.contiguous().view(torch.uint8).cpu().numpy(), "F8_E4M3"
        t = t.contiguous().cpu().numpy()
    a = np.ascontiguousarray(t)
    code = _CODE_OF.get(a.dtype)
    if code is None:
        raise InvalidArgument(f"safetensors: unsupported element type {a.dtype}")
    return a, code


def save_safetensors(tensors, metadata=None) -> bytes:
    """tensors: {name: numpy array or torch tensor}; metadata: {str: str}."""
    header = {}
    chunks = []
    off = 0
    for name in sorted(tensors):
        if name == "__metadata__":
            raise InvalidArgument("safetensors: '__metadata__' is not a tensor name")
        a, code = _host_array(tensors[name])
        raw = a.astype(a.dtype.newbyteorder("<"), copy=False).tobytes()
        header[name] = {"dtype": code, "shape": [int(s) for s in a.shape], "data_offsets": [off, off + len(raw)]}
        chunks.append(raw)
        off += len(raw)
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * (-len(hb) % 8)
    return struct.pack("<Q", len(hb)) + hb + b"".join(chunks)


def load_safetensors(data: bytes):
    """-> ({name: numpy array}, {metadata}); reads both dialects (module docstring)."""
    out, meta, _ = _parse(data)
    return out, meta


def _parse(data: bytes):
    """-> (tensors, metadata, {name: header dtype string})."""
    data = memoryview(data)
    if len(data) < 8:
        raise InvalidArgument("safetensors: too short")
    (hlen,) = struct.unpack("<Q", data[:8])
    if hlen > len(data) - 8:
        raise InvalidArgument("safetensors: truncated header")
    try:
        header = json.loads(bytes(data[8:8 + hlen]).decode("utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise InvalidArgument(f"safetensors: bad header ({e})") from None
    if not isinstance(header, dict):
        raise InvalidArgument("safetensors: header is not an object")
    body = data[8 + hlen:]
    meta = header.pop("__metadata__", None) or {}
    if not isinstance(meta, dict):
        raise InvalidArgument("safetensors: __metadata__ is not an object")
    out, dtypes = {}, {}
    for name, info in header.items():
        try:
            dtype, shape, (b, e) = info["dtype"], [int(s) for s in info["shape"]], info["data_offsets"]
        except (KeyError, TypeError, ValueError):
            raise InvalidArgument(f"safetensors: bad entry for '{name}'") from None
        if not (0 <= b <= e <= len(body)):
            raise InvalidArgument(f"safetensors: '{name}' data_offsets [{b}, {e}] outside the data section")
        n = int(np.prod(shape)) if shape else 1
        nbytes = e - b
        if dtype in _STD:
            el = np.dtype(_STD[dtype])
        elif dtype in _REF:
            el = np.dtype(_REF[dtype])
            if nbytes == 8 * n and el.itemsize != 8:
                el = np.dtype(np.float64)  # the reference's f64 encoding of every payload
        else:
            raise InvalidArgument(f"safetensors: '{name}' has unknown dtype {dtype!r}")
        if nbytes != n * el.itemsize:
            raise InvalidArgument(f"safetensors: '{name}' holds {nbytes} bytes, shape {shape} of {dtype} "
                                  f"needs {n * el.itemsize}")
        out[name] = np.frombuffer(body[b:e], dtype=el.newbyteorder("<")).astype(el, copy=True).reshape(shape)
        dtypes[name] = dtype
    return out, {str(k): str(v) for k, v in meta.items()}, dtypes


# ------------------------------------------------------------ quantized modules
def _linear_entries(name, lin, tensors, meta):
    from .nn import QuantizedLinear

    if not isinstance(lin, QuantizedLinear):
        raise InvalidArgument(f"save_quantized: '{name}' is not a QuantizedLinear")
    if lin.mode == "w4":
        meta[f"{name}.quant"] = "int4_g128"
        meta[f"{name}.group_size"] = "128"
    elif lin.mode in ("w8", "w8a8"):
        meta[f"{name}.quant"] = "int8_per_channel" if lin.mode == "w8" else "int8_per_channel_a8"
    elif lin.mode in ("fp8", "fp8_weight"):
        meta[f"{name}.quant"] = "fp8_e4m3_per_channel_a8" if lin.mode == "fp8" else "fp8_e4m3_per_channel"
    else:
        raise InvalidArgument(f"save_quantized: '{name}' has mode {lin.mode!r}")
    meta[f"{name}.in_features"] = str(lin.in_features)
    meta[f"{name}.out_features"] = str(lin.out_features)
    import torch

    fp8 = lin.mode in ("fp8", "fp8_weight")
    tensors[f"{name}.weight"] = lin.qweight.view(torch.float8_e4m3fn) if fp8 else lin.qweight
    tensors[f"{name}.weight_scale"] = lin.scales
    if lin.bias is not None:
        tensors[f"{name}.bias"] = lin.bias


def save_quantized(modules) -> bytes:
    """{name: QuantizedLinear | QuantizedMLP | QuantizedMultiheadAttention} ->
    safetensors bytes (layout in the module docstring)."""
    from .nn import QuantizedMLP, QuantizedMultiheadAttention

    tensors, meta = {}, {"format": FORMAT}
    for name, mod in modules.items():
        if isinstance(mod, QuantizedMultiheadAttention):
            meta[f"{name}.attention"] = "multihead"
            meta[f"{name}.num_heads"] = str(mod.num_heads)
            _linear_entries(f"{name}.qkv", mod.qkv, tensors, meta)
            _linear_entries(f"{name}.out_proj", mod.out_proj, tensors, meta)
        elif isinstance(mod, QuantizedMLP):
            meta[f"{name}.quant"] = "mlp_int4_g128"
            meta[f"{name}.group_size"] = "128"
            meta[f"{name}.hidden"] = str(mod.d)
            meta[f"{name}.intermediate"] = str(mod.f)
            for part, (q, s) in (("gate", mod.gate), ("up", mod.up), ("down", mod.down)):
                tensors[f"{name}.{part}.weight"] = q
                tensors[f"{name}.{part}.weight_scale"] = s
        else:
            _linear_entries(name, mod, tensors, meta)
    return save_safetensors(tensors, meta)


def _need(tensors, key, dtype, shape):
    a = tensors.get(key)
    if a is None:
        raise InvalidArgument(f"load_quantized: missing tensor '{key}'")
    if a.dtype != np.dtype(dtype) or list(a.shape) != list(shape):
        raise InvalidArgument(f"load_quantized: '{key}' is {a.dtype} {list(a.shape)}, expected "
                              f"{np.dtype(dtype)} {list(shape)}")
    return a


def load_quantized(data: bytes, device="cuda"):
    """safetensors bytes -> {name: QuantizedLinear | QuantizedMLP |
    QuantizedMultiheadAttention} with the codes and scales copied into device
    buffers as stored (no re-quantization)."""
    tensors, meta, dtypes = _parse(data)
    if meta.get("format") != FORMAT:
        raise InvalidArgument(f"load_quantized: not a {FORMAT} checkpoint (format={meta.get('format')!r})")
    return _load(tensors, meta, dtypes, device)


def _load(tensors, meta, dtypes, device):
    import torch

    from .nn import QuantizedLinear, QuantizedMLP, QuantizedMultiheadAttention

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(device)

    out = {}
    for key, kind in meta.items():
        if not key.endswith(".quant"):
            continue
        name = key[:-len(".quant")]
        owner = name.rsplit(".", 1)[0] if "." in name else None
        if owner is not None and meta.get(f"{owner}.attention") == "multihead":
            continue  # the projections of an attention module, assembled below
        if kind == "mlp_int4_g128":
            d, f = int(meta[f"{name}.hidden"]), int(meta[f"{name}.intermediate"])
            parts = []
            for part, (rows, cols) in (("gate", (f, d)), ("up", (f, d)), ("down", (d, f))):
                q = _need(tensors, f"{name}.{part}.weight", np.uint8, (rows, cols // 2))
                s = _need(tensors, f"{name}.{part}.weight_scale", np.float16, (rows, cols // 128))
                parts.append((dev(q), dev(s.view(np.int16)).view(torch.float16)))
            out[name] = QuantizedMLP(d, f, *parts)
            continue
        k, n = int(meta[f"{name}.in_features"]), int(meta[f"{name}.out_features"])
        if kind == "int4_g128":
            if meta.get(f"{name}.group_size") != "128":
                raise InvalidArgument(f"load_quantized: '{name}' group size {meta.get(f'{name}.group_size')}")
            q = dev(_need(tensors, f"{name}.weight", np.uint8, (n, k // 2)))
            s = dev(_need(tensors, f"{name}.weight_scale", np.float16, (n, k // 128)).view(np.int16))
            s = s.view(torch.float16)
            mode = "w4"
        elif kind in ("fp8_e4m3_per_channel", "fp8_e4m3_per_channel_a8"):
            if dtypes.get(f"{name}.weight") != "F8_E4M3":
                raise InvalidArgument(f"load_quantized: '{name}.weight' is not F8_E4M3")
            q = dev(_need(tensors, f"{name}.weight", np.uint8, (n, k)))
            s = dev(_need(tensors, f"{name}.weight_scale", np.float32, (n,)))
            mode = "fp8" if kind.endswith("_a8") else "fp8_weight"
        elif kind in ("int8_per_channel", "int8_per_channel_a8"):
            q = dev(_need(tensors, f"{name}.weight", np.int8, (n, k)))
            s = dev(_need(tensors, f"{name}.weight_scale", np.float32, (n,)))
            mode = "w8" if kind == "int8_per_channel" else "w8a8"
        else:
            raise InvalidArgument(f"load_quantized: '{name}' has unknown scheme {kind!r}")
        b = tensors.get(f"{name}.bias")
        bias = None if b is None else dev(_need(tensors, f"{name}.bias", np.float32, (n,)))
        out[name] = QuantizedLinear(mode, k, n, q, s, bias)
    for key, kind in meta.items():
        if key.endswith(".attention") and kind == "multihead":
            name = key[:-len(".attention")]
            pre = name + "."
            sub = _load({k[len(pre):]: v for k, v in tensors.items() if k.startswith(pre)},
                        {k[len(pre):]: v for k, v in meta.items() if k.startswith(pre)},
                        {k[len(pre):]: v for k, v in dtypes.items() if k.startswith(pre)}, device)
            out[name] = QuantizedMultiheadAttention(int(meta[f"{name}.num_heads"]), sub["qkv"], sub["out_proj"])
    return out
