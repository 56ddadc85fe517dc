"""Quantized checkpoints on the GPU: save_quantized -> load_quantized restores the
codes and scales byte for byte, and the loaded modules give the same outputs;
a checkpoint assembled by the independent `safetensors` package from oracle
codes loads and matches the oracle's Linear."""
import numpy as np
import pytest

from conftest import assert_close

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-3, 1e-4


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def normal(seed, shape, std=1.0, stream=0):
    from theano_quantize.synth import normal_f32

    return normal_f32(seed, shape, std, stream)


def bf16(x):
    import torch

    from theano_quantize.synth import f32_to_bf16_bits

    return dev(f32_to_bf16_bits(x).view(np.int16)).view(torch.bfloat16)


def test_linear_and_mlp_roundtrip(tq):
    import torch

    n, k = 384, 512
    w = normal(81, (n, k), 0.02)
    b = normal(81, (n,), 0.1, stream=1)
    mods = {
        "l4": tq.QuantizedLinear.from_tensors(dev(w), dev(b), tq.QConfig.default_int4()),
        "l8": tq.QuantizedLinear.from_tensors(dev(w), dev(b), tq.QConfig.default_int8()),
        "l8a8": tq.QuantizedLinear.from_tensors(dev(w), None, tq.QConfig(tq.QuantDType.Int8, tq.QuantDType.Int8,
                                                                           True, True)),
        "lfp8": tq.QuantizedLinear.from_tensors(dev(w), dev(b), tq.QConfig(tq.QuantDType.FP8, tq.QuantDType.FP8,
                                                                            True, True)),
        "lfp8w": tq.QuantizedLinear.from_tensors(dev(w), None, tq.QConfig(tq.QuantDType.FP8, tq.QuantDType.UInt8,
                                                                           True, True)),
        "mlp": tq.QuantizedMLP.from_tensors(dev(normal(82, (512, 256), 0.02)), dev(normal(82, (512, 256), 0.02, 1)),
                                            dev(normal(82, (256, 512), 0.02, 2))),
    }
    blob = tq.save_quantized(mods)
    back = tq.load_quantized(blob)
    assert set(back) == set(mods)
    for name in ("l4", "l8", "l8a8", "lfp8", "lfp8w"):
        a, c = mods[name], back[name]
        assert (c.mode, c.in_features, c.out_features) == (a.mode, a.in_features, a.out_features)
        assert torch.equal(a.qweight, c.qweight) and torch.equal(a.scales.view(torch.int16) if a.scales.dtype ==
                                                                 torch.float16 else a.scales,
                                                                 c.scales.view(torch.int16) if c.scales.dtype ==
                                                                 torch.float16 else c.scales)
        assert (a.bias is None) == (c.bias is None)
        for m in (1, 5, 40):
            x = normal(83, (m, k), 1.0, stream=m)
            xi = bf16(x) if a.mode == "w4" else dev(x)
            assert np.array_equal(host(a(xi)), host(c(xi))), (name, m)
    x = bf16(normal(84, (7, 256), 1.0))
    assert np.array_equal(host(mods["mlp"](x)), host(back["mlp"](x)))


def test_checkpoint_from_the_safetensors_package(tq, oracle):
    st_numpy = pytest.importorskip("safetensors.numpy")
    n, k, m = 256, 1024, 3
    w = normal(85, (n, k), 0.02)
    b = normal(85, (n,), 0.1, stream=1)
    p, s = oracle.quantize_i4_g128(w)
    blob = st_numpy.save({"proj.weight": p, "proj.weight_scale": s.view(np.float16), "proj.bias": b},
                         metadata={"format": "theano-quantize/1", "proj.quant": "int4_g128", "proj.group_size": "128",
                                   "proj.in_features": str(k), "proj.out_features": str(n)})
    lin = tq.load_quantized(blob)["proj"]
    from theano_quantize.synth import f32_to_bf16_bits

    xb = f32_to_bf16_bits(normal(86, (m, k), 1.0))
    y = host(lin(bf16(normal(86, (m, k), 1.0))))
    assert_close(y, oracle.linear_w4g128_bf16(xb, p, s, b), RTOL, ATOL, "checkpoint w4")


def test_attention_roundtrip(tq):
    import torch

    E, H = 128, 4
    ws = [dev(normal(87, (E, E), 0.05, stream=i)) for i in range(4)]
    bs = [dev(normal(87, (E,), 0.1, stream=10 + i)) for i in range(4)]
    for cfg in (tq.QConfig.default_int4(), tq.QConfig(tq.QuantDType.FP8, tq.QuantDType.FP8, True, True)):
        mha = tq.QuantizedMultiheadAttention.from_tensors(H, *ws, *bs, qconfig=cfg)
        back = tq.load_quantized(tq.save_quantized({"layers.0.attn": mha}))["layers.0.attn"]
        assert isinstance(back, tq.QuantizedMultiheadAttention) and back.num_heads == H
        assert torch.equal(back.qkv.qweight, mha.qkv.qweight) and back.qkv.mode == mha.qkv.mode
        x = dev(normal(88, (2, 9, E), 1.0))
        assert np.array_equal(host(mha(x)), host(back(x)))
