"""GPU check of the allocation-free decode FFN entry point
(tq_mlp_w4g128_decode_noalloc): through the C ABI it gives the workspace
entry point's output bit for bit, on two calls in a row (the second with fewer
tokens and a smaller F, so stale scratch contents of the first call are
present), and it rejects shapes beyond its scratch."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(tq, m, d, f, seed):
    import torch
    from theano_quantize.synth import f32_to_bf16_bits, normal_f32

    wg = normal_f32(seed, (f, d), 0.02)
    wu = normal_f32(seed, (f, d), 0.02, stream=1)
    wd = normal_f32(seed, (d, f), 0.02, stream=2)
    xb = f32_to_bf16_bits(normal_f32(seed, (m, d), 1.0, stream=3))
    mlp = tq.QuantizedMLP.from_tensors(*(torch.from_numpy(w).cuda() for w in (wg, wu, wd)))
    x = torch.from_numpy(xb.view(np.int16)).cuda().view(torch.bfloat16)
    return mlp, x


def _run(tq, mlp, x, noalloc):
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    m = x.shape[0]
    gu_t, gu_st, dn_t, dn_st, dn_rows = mlp.decode
    y = torch.full((m, mlp.d), float("nan"), dtype=torch.float32, device="cuda")
    if noalloc:
        _abi.call("tq_mlp_w4g128_decode_noalloc", ptr(x), m, mlp.d, mlp.f, ptr(gu_t), ptr(gu_st), ptr(dn_t),
                  ptr(dn_st), dn_rows, ptr(y), stream())
    else:
        nb = int(_abi.lib().tq_mlp_w4g128_decode_workspace_bytes(m, mlp.d, mlp.f))
        ws = torch.empty((nb,), dtype=torch.uint8, device="cuda")
        _abi.call("tq_mlp_w4g128_decode", ptr(x), m, mlp.d, mlp.f, ptr(gu_t), ptr(gu_st), ptr(dn_t), ptr(dn_st),
                  dn_rows, ptr(ws), nb, ptr(y), stream())
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("cases", [((8, 4096, 14336), (3, 4096, 14336)), ((4, 512, 1536), (1, 256, 384))])
def test_noalloc_matches_workspace_entry_point(tq, cases):
    for i, (m, d, f) in enumerate(cases):
        print(f"noalloc decode FFN call {i}: M={m} D={d} F={f}", flush=True)
        mlp, x = _case(tq, m, d, f, seed=80 + i)
        ref = _run(tq, mlp, x, noalloc=False)
        got = _run(tq, mlp, x, noalloc=True)
        assert np.isfinite(ref).all()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"call {i}: M={m} D={d} F={f}"


def test_noalloc_rejects_beyond_scratch(tq):
    """The scratch holds M <= 16 tokens at F <= 16384 (h: 1 MiB, its block sums:
    64 KiB); larger shapes and a null output are rejected before anything is
    enqueued."""
    from theano_quantize import InvalidArgument, _abi

    lib = _abi.lib()
    assert lib.tq_mlp_w4g128_decode_workspace_bytes(16, 4096, 16384) == (1 << 20) + (1 << 16)
    with pytest.raises(InvalidArgument, match="M=17"):
        _abi.call("tq_mlp_w4g128_decode_noalloc", 16, 17, 256, 16384, 16, 16, 16, 16, 16, 16, None)
    with pytest.raises(InvalidArgument, match="F=16512"):
        _abi.call("tq_mlp_w4g128_decode_noalloc", 16, 16, 256, 16512, 16, 16, 16, 16, 16, 16, None)
    with pytest.raises(InvalidArgument, match="null"):
        _abi.call("tq_mlp_w4g128_decode_noalloc", 16, 2, 256, 256, 16, 16, 16, 16, 16, None, None)
