"""Safetensors container (crates/theano-serialize/src/safetensors.rs) for
quantized checkpoints: the standard dialect is checked against the
independent `safetensors` package in both directions; the reference's own
dialect (f64 payloads under DType names, safetensors.rs:36-54, 83-135) is
checked on the reference's test tensors (safetensors.rs:246-284)."""
import json
import os
import struct
import sys
import tempfile

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "neo-theano_amd"))
from theano_quantize.checkpoint import load_safetensors, save_safetensors  # noqa: E402
from theano_quantize.errors import InvalidArgument  # noqa: E402

st_numpy = pytest.importorskip("safetensors.numpy")


def sample():
    rng = np.random.default_rng(7)
    return {
        "a.weight": rng.integers(-127, 128, (6, 16), dtype=np.int8),
        "a.weight_scale": rng.random(6, dtype=np.float32),
        "b.weight": rng.integers(0, 256, (4, 64), dtype=np.uint8),
        "b.weight_scale": rng.random((4, 1)).astype(np.float16),
        "c.bias": rng.standard_normal(5),
        "d.index": rng.integers(-5, 5, 3, dtype=np.int64),
        "e.flags": np.array([True, False, True]),
        "f.empty": np.zeros((0, 3), dtype=np.float32),
    }


def test_standard_dialect_read_by_the_safetensors_package():
    t = sample()
    blob = save_safetensors(t, {"format": "x", "a.quant": "int8_per_channel"})
    got = st_numpy.load(blob)
    assert set(got) == set(t)
    for k in t:
        assert got[k].dtype == t[k].dtype and np.array_equal(got[k], t[k]), k
    with tempfile.NamedTemporaryFile(suffix=".safetensors") as f:
        f.write(blob)
        f.flush()
        from safetensors import safe_open

        with safe_open(f.name, framework="numpy") as h:
            assert h.metadata() == {"format": "x", "a.quant": "int8_per_channel"}
    (hlen,) = struct.unpack("<Q", blob[:8])
    assert hlen % 8 == 0


def test_standard_dialect_written_by_the_safetensors_package():
    t = sample()
    blob = st_numpy.save(t, metadata={"k": "v"})
    got, meta = load_safetensors(blob)
    assert meta == {"k": "v"}
    for k in t:
        assert got[k].dtype == t[k].dtype and np.array_equal(got[k], t[k]), k


def _reference_bytes(tensors, dtype_names, order):
    """Bytes as the reference's SafeTensorsFile writes them: f64 LE payloads in
    insertion order, header keys sorted, no metadata."""
    data, info = b"", {}
    for name in order:
        v = np.asarray(tensors[name], dtype="<f8")
        info[name] = (len(data), len(data) + v.nbytes)
        data += v.tobytes()
    parts = []
    for name in sorted(tensors):
        shape = ",".join(str(s) for s in np.shape(tensors[name]))
        parts.append(f'"{name}":{{"dtype":"{dtype_names[name]}","shape":[{shape}],'
                     f'"data_offsets":[{info[name][0]},{info[name][1]}]}}')
    header = ("{" + ",".join(parts) + "}").encode()
    return struct.pack("<Q", len(header)) + header + data


def test_reference_dialect_roundtrip_vectors():
    # safetensors.rs:246-260: weight [[1, 2], [3, 4]], bias [5, 6] (f64 storage)
    t = {"weight": np.array([[1.0, 2.0], [3.0, 4.0]]), "bias": np.array([5.0, 6.0])}
    for order in (["weight", "bias"], ["bias", "weight"]):  # HashMap order is arbitrary
        got, meta = load_safetensors(_reference_bytes(t, {"weight": "float64", "bias": "float64"}, order))
        assert meta == {}
        assert got["weight"].shape == (2, 2) and got["weight"].tolist() == [[1.0, 2.0], [3.0, 4.0]]
        assert got["bias"].tolist() == [5.0, 6.0]


def test_reference_dialect_f64_payload_under_narrow_names():
    # a float32 (or int) tensor of the reference still carries 8-byte f64 values
    t = {"x": np.ones((3, 3)), "i": np.array([1.0, -2.0, 3.0])}
    got, _ = load_safetensors(_reference_bytes(t, {"x": "float32", "i": "int32"}, ["x", "i"]))
    assert got["x"].dtype == np.float64 and got["x"].shape == (3, 3) and np.all(got["x"] == 1.0)
    assert got["i"].tolist() == [1.0, -2.0, 3.0]


def test_reference_dialect_empty():
    # safetensors.rs:277-284: an empty map round-trips ("{}" header)
    got, meta = load_safetensors(struct.pack("<Q", 2) + b"{}")
    assert got == {} and meta == {}
    got, meta = load_safetensors(save_safetensors({}))
    assert got == {} and meta == {}


@pytest.mark.parametrize("blob", [
    b"\x01\x00",                                                     # too short
    struct.pack("<Q", 100) + b"{}",                                 # truncated header
    struct.pack("<Q", 4) + b"\xff\xfe{}",                           # not UTF-8
    struct.pack("<Q", 2) + b"[]",                                   # not an object
])
def test_malformed_containers_are_rejected(blob):
    with pytest.raises(InvalidArgument):
        load_safetensors(blob)


def _one(entry, data):
    h = json.dumps({"t": entry}).encode()
    return struct.pack("<Q", len(h)) + h + data


@pytest.mark.parametrize("entry,data", [
    ({"dtype": "F32", "shape": [2], "data_offsets": [0, 12]}, bytes(8)),      # past the data section
    ({"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}, bytes(8)),       # size != shape x element
    ({"dtype": "X9", "shape": [1], "data_offsets": [0, 4]}, bytes(4)),        # unknown dtype
    ({"dtype": "F32", "shape": [1]}, bytes(4)),                               # missing offsets
])
def test_malformed_entries_are_rejected(entry, data):
    with pytest.raises(InvalidArgument):
        load_safetensors(_one(entry, data))


def test_golden_checkpoint_fixture():
    """tests/golden/checkpoint_int4_16x256.safetensors (written by the
    `safetensors` package) decodes to the INT4 fixture's codes and scales."""
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    got, meta = load_safetensors(open(os.path.join(here, "checkpoint_int4_16x256.safetensors"), "rb").read())
    ref = np.load(os.path.join(here, "int4_g128_16x256.npz"))
    assert np.array_equal(got["proj.weight"], ref["packed"])
    assert np.array_equal(got["proj.weight_scale"].view(np.uint16), ref["s_f16"])
    assert meta["proj.quant"] == "int4_g128" and meta["proj.group_size"] == "128"
    assert got["const.f16"].tolist() == [0.5, -1.0, 65504.0]


def test_f8_e4m3_against_the_safetensors_torch_package():
    """F8_E4M3 tensors (FP8 codes) both ways through safetensors.torch."""
    torch = pytest.importorskip("torch")
    st_torch = pytest.importorskip("safetensors.torch")
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(16, 16)
    blob = save_safetensors({"w.weight": codes.view(torch.float8_e4m3fn), "w.weight_scale": np.ones(16, np.float32)},
                            {"format": "x"})
    got = st_torch.load(blob)
    assert got["w.weight"].dtype == torch.float8_e4m3fn
    assert torch.equal(got["w.weight"].view(torch.uint8), codes)
    back, _ = load_safetensors(st_torch.save({"w.weight": codes.view(torch.float8_e4m3fn)}))
    assert back["w.weight"].dtype == np.uint8 and np.array_equal(back["w.weight"], codes.numpy())
