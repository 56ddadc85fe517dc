"""GPU parity: element type conversion of device buffers (tq_convert, the device
half of Tensor::to) against the oracle on every source / destination pair of
the supported DTypes, bit-exact (NaN only required to stay NaN)."""
import numpy as np
import pytest

from test_oracle import conversion_probe_f64

pytestmark = pytest.mark.gpu

NAMES = ["float16", "bfloat16", "float32", "float64", "uint8", "int8", "int16", "int32", "int64", "bool"]


def _is_nan(a, t):
    if t == 0:
        return ((a & 0x7C00) == 0x7C00) & ((a & 0x3FF) != 0)
    if t == 1:
        return ((a & 0x7F80) == 0x7F80) & ((a & 0x7F) != 0)
    if t in (2, 3):
        return np.isnan(a)
    return np.zeros(a.shape, bool)


def same(got, ref, t):
    gn, rn = _is_nan(got, t), _is_nan(ref, t)
    if not np.array_equal(gn, rn):
        return False
    if t in (2, 3):
        return np.array_equal(got[~gn].view(np.uint32 if t == 2 else np.uint64),
                              ref[~rn].view(np.uint32 if t == 2 else np.uint64))
    return np.array_equal(got[~gn], ref[~rn])


@pytest.mark.parametrize("src", range(10), ids=NAMES)
def test_convert_all_pairs(tq, oracle, src):
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    probe = conversion_probe_f64()
    sv = oracle.convert(probe, 3, src)  # valid source values of this type
    sd = torch.from_numpy(sv.copy()).cuda()
    for dst in range(10):
        out = torch.empty(sv.size, dtype=torch.from_numpy(np.empty(0, oracle.NP_STORAGE[dst])).dtype, device="cuda")
        _abi.call("tq_convert", ptr(sd), src, ptr(out), dst, sv.size, stream())
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        ref = oracle.convert(sv, src, dst)
        assert same(got, ref, dst), (NAMES[src], NAMES[dst])


@pytest.mark.parametrize("n", [0, 1, 3, 4, 5, 1000, 1 << 20])
def test_convert_lengths_and_module_helper(tq, oracle, n):
    import torch

    x = torch.from_numpy(np.random.default_rng(n).standard_normal(n) * 3.0).cuda()
    for dt in (torch.float32, torch.bfloat16, torch.int8, "float16"):
        y = tq.convert(x, dt)
        code = tq._tensor.DTYPE_CODES[dt] if isinstance(dt, str) else tq._tensor._CODE_OF[dt]
        ref = oracle.convert(x.cpu().numpy(), 3, code)
        got = y.cpu().numpy() if y.dtype not in (torch.bfloat16, torch.float16) else y.view(torch.int16).cpu().numpy().view(np.uint16)
        assert same(got, ref, code)
