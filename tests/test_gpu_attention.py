"""GPU parity: the attention core (tq_attention_f32) and QuantizedMultiheadAttention
(crates/theano-nn/src/transformer.rs) against the oracle: the core on its own,
the module end to end for the weight-only modes and stage by stage for the
modes that quantize activations.  f32 results, |got - ref| <= 1e-4 + 1e-3 |ref|."""
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


def run_core(tq, qkv, B, S, H, mask=None):
    """qkv: f32 [B*S, 3E] with q, k, v side by side (read in place)."""
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    E = qkv.shape[1] // 3
    d = dev(qkv)
    out = torch.empty((B * S, E), dtype=torch.float32, device="cuda")
    md = None if mask is None else dev(mask.astype(np.float32))
    mb = 0 if mask is None else mask.shape[0]
    _abi.call("tq_attention_f32", ptr(d), 3 * E, ptr(d[:, E:]), 3 * E, ptr(d[:, 2 * E:]), 3 * E, ptr(md), mb, B, S, H,
              E // H, ptr(out), E, stream())
    return host(out)


@pytest.mark.parametrize("B,S,H,D", [(1, 4, 4, 4), (2, 10, 8, 8), (2, 77, 4, 32), (1, 300, 8, 64), (2, 130, 2, 128),
                                     (3, 64, 1, 16), (1, 1, 2, 5)])
def test_attention_core_vs_oracle(tq, oracle, B, S, H, D):
    E = H * D
    qkv = normal(91, (B * S, 3 * E), 1.0)
    q, k, v = (qkv[:, i * E:(i + 1) * E].reshape(B, S, E).astype(np.float64) for i in range(3))
    rng = np.random.default_rng(S)
    causal = np.triu(np.full((1, S, S), -np.inf), k=1)
    rand = np.where(rng.random((B, S, S)) < 0.25, -np.inf, rng.standard_normal((B, S, S)))
    rand[:, :, -1] = 0.0  # every row keeps a key
    for mask in (None, causal, rand):
        got = run_core(tq, qkv, B, S, H, mask).reshape(B, S, E)
        ref = oracle.attention(q, k, v, H, None if mask is None else mask.astype(np.float32).astype(np.float64))
        assert_close(got, ref, RTOL, ATOL, f"attention B={B} S={S} H={H} D={D}")


@pytest.mark.parametrize("B,S,H,D", [(1, 77, 4, 128), (2, 40, 3, 64), (1, 33, 2, 32), (1, 64, 2, 12)])
def test_attention_quad_and_element_loads_agree(tq, B, S, H, D):
    """Row strides that are multiples of 4 floats take the quad-load kernel, a
    stride of 3E + 1 the per-element one: the same q, k, v and mask give the
    same bits (a partial last key tile included)."""
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    E = H * D
    qkv = normal(94, (B * S, 3 * E), 1.0)
    rng = np.random.default_rng(S + D)
    mask = np.where(rng.random((B, S, S)) < 0.25, -np.inf, rng.standard_normal((B, S, S))).astype(np.float32)
    mask[:, :, 0] = 0.0
    md = dev(mask)
    outs = []
    for pad in (0, 1):
        buf = np.zeros((B * S, 3 * E + pad), np.float32)
        buf[:, :3 * E] = qkv
        d = dev(buf)
        ld = 3 * E + pad
        out = torch.empty((B * S, E), dtype=torch.float32, device="cuda")
        _abi.call("tq_attention_f32", ptr(d), ld, ptr(d[:, E:]), ld, ptr(d[:, 2 * E:]), ld, ptr(md), B, B, S, H, D,
                  ptr(out), E, stream())
        outs.append(host(out))
    assert np.isfinite(outs[0]).all()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), f"B={B} S={S} H={H} D={D}"


def test_attention_wide_blocks_agree(tq):
    """At head dim 128 a launch with a block per CU or more runs 8-wave blocks
    (256 queries); the same batches one at a time run 4-wave blocks.  Every
    query row's arithmetic is the same in both: the same bits."""
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    B, S, H, D = 4, 256, 64, 128  # 4 x 64 blocks of 256 queries
    E = H * D
    assert B * H * ((S + 255) // 256) >= torch.cuda.get_device_properties(0).multi_processor_count
    d = dev(normal(95, (B * S, 3 * E), 1.0))
    causal = dev(np.triu(np.full((1, S, S), -np.inf, np.float32), k=1))

    def run(rows, nb):
        out = torch.empty((nb * S, E), dtype=torch.float32, device="cuda")
        x = d[rows]
        _abi.call("tq_attention_f32", ptr(x), 3 * E, ptr(x[:, E:]), 3 * E, ptr(x[:, 2 * E:]), 3 * E, ptr(causal), 1,
                  nb, S, H, D, ptr(out), E, stream())
        return host(out)

    wide = run(slice(0, B * S), B)
    for b in range(B):
        narrow = run(slice(b * S, (b + 1) * S), 1)
        assert np.isfinite(narrow).all()
        assert np.array_equal(wide[b * S:(b + 1) * S].view(np.uint32), narrow.view(np.uint32)), f"batch {b}"


def test_attention_fully_masked_row_is_nan(tq, oracle):
    B, S, H, D = 1, 70, 2, 8
    qkv = normal(92, (B * S, 3 * H * D), 1.0)
    mask = np.zeros((1, S, S))
    mask[0, 5, :] = -np.inf        # nothing to attend: NaN, as the reference's softmax
    mask[0, 6, :64] = -np.inf      # the whole first key tile masked: finite
    got = run_core(tq, qkv, B, S, H, mask)
    assert np.isnan(got[5]).all() and np.isfinite(np.delete(got, 5, axis=0)).all()
    q, k, v = (qkv[:, i * H * D:(i + 1) * H * D].reshape(B, S, H * D).astype(np.float64) for i in range(3))
    ref = oracle.attention(q, k, v, H, mask)
    assert_close(np.delete(got, 5, axis=0), np.delete(ref[0], 5, axis=0), RTOL, ATOL, "masked tiles")


# ------------------------------------------------------------------ module
def make_mha(tq, E, H, cfg, seed=93, bias=True):
    ws = [normal(seed, (E, E), 0.05, stream=i) for i in range(4)]
    bs = [normal(seed, (E,), 0.1, stream=10 + i) if bias else None for i in range(4)]
    mha = tq.QuantizedMultiheadAttention.from_tensors(H, *[dev(w) for w in ws],
                                                      *[None if b is None else dev(b) for b in bs], qconfig=cfg)
    return mha, ws, bs


def test_mha_reference_shapes_and_names(tq):
    # transformer.rs:188-268 (shape, parameters, named parameters, mask, state dict)
    import torch

    cfg = tq.QConfig.default_int8()
    mha, _, _ = make_mha(tq, 64, 8, cfg)
    assert tuple(mha(torch.ones(2, 10, 64, device="cuda")).shape) == (2, 10, 64)
    named = mha.named_parameters()
    assert [n for n, _ in named][:3] == ["q_proj.weight", "q_proj.weight_scale", "q_proj.bias"]
    assert named[3][0] == "k_proj.weight" and named[-1][0] == "out_proj.bias"
    assert len(named) == 12  # weight, weight_scale, bias for each of the four projections
    sd = mha.state_dict()
    assert "q_proj.weight" in sd and "q_proj.bias" in sd and "out_proj.weight" in sd
    mha16, _, _ = make_mha(tq, 16, 4, cfg)
    x = torch.ones(1, 4, 16, device="cuda")
    mask = torch.triu(torch.full((1, 4, 4), float("-inf")), diagonal=1).cuda()
    assert tuple(mha16.forward_with_mask(x, x, x, mask).shape) == (1, 4, 16)
    assert tuple(mha16.forward_qkv(x, x, x).shape) == (1, 4, 16)
    assert mha16.num_parameters() == 4 * (16 * 16 + 16)


def _oracle_projection(oracle, mode, x2d, w, b):
    """Linear over the quantized weight as the module computes it, from f32 activations."""
    from theano_quantize.synth import f32_to_bf16_bits

    x2d = x2d.astype(np.float32)
    if mode == "w8":
        q, s = oracle.quantize_i8_rowwise(w)
        return oracle.linear_w8(x2d, q, s, b)
    p, s = oracle.quantize_i4_g128(w)
    return oracle.linear_w4g128_bf16(f32_to_bf16_bits(x2d), p, s, b)


@pytest.mark.parametrize("mode", ["w8", "w4"])
@pytest.mark.parametrize("B,S,E,H", [(1, 8, 256, 4), (2, 40, 256, 8), (1, 129, 512, 4)])
def test_mha_weight_only_end_to_end(tq, oracle, mode, B, S, E, H):
    """Projections + attention against the oracle chain from the f32 input; the
    output projection against the oracle from the GPU's attention output (its
    bf16 rounding in the INT4 mode is defined on those f32 values)."""
    import torch

    cfg = tq.QConfig.default_int8() if mode == "w8" else tq.QConfig.default_int4()
    mha, ws, bs = make_mha(tq, E, H, cfg)
    act = (lambda t: tq.convert(t, torch.bfloat16)) if mode == "w4" else (lambda t: t)
    x = normal(94, (B, S, E), 1.0)
    mask = np.triu(np.full((1, S, S), -np.inf), k=1).astype(np.float32)
    xd = dev(x)
    y = host(mha.forward_with_mask(xd, xd, xd, dev(mask)))
    x2 = x.reshape(B * S, E)
    qkv = host(mha.qkv(act(dev(x2))))
    att = run_core(tq, qkv, B, S, H, mask)
    q, k, v = (_oracle_projection(oracle, mode, x2, ws[i], bs[i]).reshape(B, S, E) for i in range(3))
    assert_close(att.reshape(B, S, E), oracle.attention(q, k, v, H, mask.astype(np.float64)), RTOL, ATOL,
                 f"mha {mode} through attention")
    assert_close(y, _oracle_projection(oracle, mode, att, ws[3], bs[3]).reshape(B, S, E), RTOL, ATOL,
                 f"mha {mode} B={B} S={S}")
    # cross-attention through the row slices of the fused weight
    xk, xv = normal(95, (B, S, E), 1.0), normal(96, (B, S, E), 1.0)
    y2 = host(mha.forward_qkv(xd, dev(xk), dev(xv)))
    ins = [x2, xk.reshape(B * S, E), xv.reshape(B * S, E)]
    parts = [host(mha._parts[i](act(dev(ins[i])))) for i in range(3)]
    att2 = run_core(tq, np.concatenate(parts, 1), B, S, H)
    q, k, v = (_oracle_projection(oracle, mode, ins[i], ws[i], bs[i]).reshape(B, S, E) for i in range(3))
    assert_close(att2.reshape(B, S, E), oracle.attention(q, k, v, H), RTOL, ATOL, f"mha cross {mode} attention")
    assert_close(y2, _oracle_projection(oracle, mode, att2, ws[3], bs[3]).reshape(B, S, E), RTOL, ATOL,
                 f"mha cross {mode}")
    assert torch.isfinite(torch.from_numpy(y2)).all()


@pytest.mark.parametrize("mode", ["w8a8", "fp8"])
def test_mha_quantized_activations_stagewise(tq, oracle, mode):
    """Each stage against the oracle from the previous stage's GPU output (the
    activation codes are defined on the f32 values the GPU hands over)."""
    import torch

    B, S, E, H = 2, 24, 256, 4
    a8 = tq.QuantDType.Int8 if mode == "w8a8" else tq.QuantDType.FP8
    cfg = tq.QConfig(a8, a8, True, True)
    mha, ws, bs = make_mha(tq, E, H, cfg)
    x = normal(97, (B * S, E), 1.0)
    qkv = host(mha.qkv(dev(x)))
    wcat = np.concatenate(ws[:3], 0)
    bcat = np.concatenate(bs[:3])
    quant = oracle.quantize_i8_rowwise if mode == "w8a8" else oracle.quantize_fp8_rowwise
    lin = oracle.linear_w8a8 if mode == "w8a8" else oracle.linear_fp8
    qa, sa = quant(x)
    qw, sw = quant(wcat)
    assert_close(qkv, lin(qa, sa, qw, sw, bcat), RTOL, ATOL, "fused qkv")
    att = run_core(tq, qkv, B, S, H)
    q, k, v = (qkv[:, i * E:(i + 1) * E].reshape(B, S, E).astype(np.float64) for i in range(3))
    assert_close(att.reshape(B, S, E), oracle.attention(q, k, v, H), RTOL, ATOL, "attention")
    y = host(mha(dev(x.reshape(B, S, E)))).reshape(B * S, E)
    qa, sa = quant(att)
    qo, so = quant(ws[3])
    assert_close(y, lin(qa, sa, qo, so, bs[3]), RTOL, ATOL, "out_proj")
    assert torch.isfinite(torch.from_numpy(y)).all()
