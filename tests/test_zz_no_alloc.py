"""dyninfer_mi355x_qlinear_multi_noalloc against dyninfer_mi355x_qlinear_multi,
through the C ABI: the same kernels with the prefill staging taken from the
device's static scratch array instead of a stream-ordered allocation, so the
outputs must be bit-identical, and both within the f16 bound of the oracle.
Two prefill calls in a row (the second smaller, over the first call's
leftover staging), decode calls (two in a row staging their activations in
the scratch array, the second smaller; bf16 outputs with long K, whose f32
accumulators the array also holds), a staging beyond the scratch size
(rejected host-side, after which calls still work), and a prefill captured in
a HIP graph (kernel nodes only) whose replays equal the eager call."""
import numpy as np
import pytest
import torch

import dyninfer_amd as d
import oracle

pytestmark = pytest.mark.gpu

F16X2 = 2.0 ** -10 + 2e-5


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def _weights(k, shapes, seed):
    datas = [oracle.synth_gguf(oracle.Q4_0, n, k, seed + i) for i, n in enumerate(shapes)]
    return [d.QWeight(d.ENC_Q4_0, n, k, dev(x)) for n, x in zip(shapes, datas)], datas


def _both(ctx, ws, x):
    ref = ctx.qlinear_multi(ws, x)
    outs = [torch.full_like(r, float("nan")) for r in ref]
    ctx.qlinear_multi(ws, x, outs, noalloc=True)
    torch.cuda.synchronize()
    return [r.cpu().numpy() for r in ref], [o.cpu().numpy() for o in outs]


def test_noalloc_matches_qlinear_multi_on_consecutive_calls(ctx):
    k, shapes = 1024, [512, 256, 256]
    ws, datas = _weights(k, shapes, seed=3)
    for rows, xbf16 in ((512, False), (100, True)):  # the second call smaller than the first
        x = oracle.randn(rows * k, seed=rows).reshape(rows, k)
        if xbf16:
            xb = oracle.f32_to_bf16_bits(x.reshape(-1)).reshape(rows, k)
            xd, x = dev(xb).view(torch.bfloat16), oracle.bf16_bits_to_f32(xb).reshape(rows, k)
        else:
            xd = dev(x)
        ref, got = _both(ctx, ws, xd)
        for r, g, data, n in zip(ref, got, datas, shapes):
            assert np.array_equal(r.view(np.uint32), g.view(np.uint32)), (rows, n)
            y64, absdot = oracle.linear_f64(x, oracle.dequant_gguf(oracle.Q4_0, data, n, k))
            assert oracle.normalized_error(g, y64, absdot) <= F16X2


@pytest.mark.parametrize("gtype", [oracle.Q4_K, oracle.Q5_K, oracle.IQ4_XS], ids=oracle.NAMES.get)
def test_noalloc_super_block_encodings(ctx, gtype):
    """The GGML super-block encodings through the no-allocation entry point:
    a prefill (the GEMM, staging in the scratch array) then a decode call."""
    enc = {oracle.Q4_K: d.ENC_Q4_K, oracle.Q5_K: d.ENC_Q5_K, oracle.IQ4_XS: d.ENC_IQ4_XS}[gtype]
    k, shapes = 1024, [512, 256]
    datas = [oracle.synth_gguf(gtype, n, k, 30 + i) for i, n in enumerate(shapes)]
    ws = [d.QWeight(enc, n, k, dev(x)) for n, x in zip(shapes, datas)]
    for rows in (200, 8):
        x = oracle.randn(rows * k, seed=rows + 5).reshape(rows, k)
        ref, got = _both(ctx, ws, dev(x))
        for r, g in zip(ref, got):
            assert np.array_equal(r.view(np.uint32), g.view(np.uint32)), rows
        y64, absdot = oracle.linear_f64(x, oracle.dequant_gguf(gtype, datas[0], shapes[0], k))
        assert oracle.normalized_error(got[0], y64, absdot) <= 2e-3


def test_noalloc_decode_staged_in_scratch(ctx):
    """16 then 9 activation rows on the MFMA GEMV (K >= 2048: the activations
    staged once per call, here in the scratch array): equal to the call with a
    workspace and to the one without, bit for bit, and within the f16 bound."""
    for k, rows, shapes, seed in ((4096, 16, [4096, 1024, 1024], 40), (2048, 9, [6144], 50)):
        ws, datas = _weights(k, shapes, seed=seed)
        x = oracle.randn(rows * k, seed=seed + 1).reshape(rows, k)
        ref, got = _both(ctx, ws, dev(x))
        own = [y.cpu().numpy() for y in ctx.qlinear_multi(ws, dev(x), workspace=False)]
        for r, g, o, data, n in zip(ref, got, own, datas, shapes):
            assert np.array_equal(r.view(np.uint32), g.view(np.uint32)), (k, rows, n)
            assert np.array_equal(o.view(np.uint32), g.view(np.uint32)), (k, rows, n)
            y64, absdot = oracle.linear_f64(x, oracle.dequant_gguf(oracle.Q4_0, data, n, k))
            assert oracle.normalized_error(g, y64, absdot) <= F16X2


def test_noalloc_decode_bf16_outputs_long_k(ctx):
    """bf16 outputs with K = 12288 at 16 rows (three LDS segments): the segments
    add into f32 accumulators in the scratch array after the staged activations,
    then one launch rounds them to bf16.  Every output is written (the outputs
    start as NaN) and lies within the f16 bound plus the bf16 rounding."""
    k, shapes, rows = 12288, [2048, 1024], 16
    ws, datas = _weights(k, shapes, seed=60)
    x = oracle.randn(rows * k, seed=61).reshape(rows, k)
    outs = [torch.full((rows, n), float("nan"), dtype=torch.bfloat16, device="cuda") for n in shapes]
    ctx.qlinear_multi(ws, dev(x), outs, noalloc=True)
    torch.cuda.synchronize()
    for o, data, n in zip(outs, datas, shapes):
        g = o.float().cpu().numpy().astype(np.float64)
        assert not np.isnan(g).any()
        y64, absdot = oracle.linear_f64(x, oracle.dequant_gguf(oracle.Q4_0, data, n, k))
        den = np.where(absdot > 0, absdot, 1)
        assert np.all(np.abs(g - y64) / den - np.abs(y64) * 2.0 ** -8 / den <= F16X2)


def test_noalloc_decode_and_size_limit(ctx):
    k = 1024
    ws, _ = _weights(k, [384], seed=9)
    x = dev(oracle.randn(8 * k, seed=1).reshape(8, k))
    ref, got = _both(ctx, ws, x)
    assert np.array_equal(ref[0].view(np.uint32), got[0].view(np.uint32))
    # 2048 rows x K 8192: a staging of 32 MiB + 8 KiB, beyond the scratch array
    kb = 8192
    wb, _ = _weights(kb, [64], seed=11)
    xb = torch.zeros((2048, kb), dtype=torch.float32, device="cuda")
    yb = [torch.empty((2048, 64), dtype=torch.float32, device="cuda")]
    with pytest.raises(d.DyninferError) as e:
        ctx.qlinear_multi(wb, xb, yb, noalloc=True)
    assert e.value.code == d.ERR_UNSUPPORTED and "static scratch" in e.value.message
    # the largest staging that fits (2048 rows x K 8128, K a multiple of 64) runs,
    # and calls keep working
    wf, dataf = _weights(8128, [64], seed=12)
    xf = oracle.randn(2048 * 8128, seed=2).reshape(2048, 8128)
    ref, got = _both(ctx, wf, dev(xf))
    assert np.array_equal(ref[0].view(np.uint32), got[0].view(np.uint32))
    ref, got = _both(ctx, ws, x)
    assert np.array_equal(ref[0].view(np.uint32), got[0].view(np.uint32))


def test_noalloc_prefill_graph_capture_replays(ctx, graph_node_types):
    """The callers this entry point is for capture it: a 200 x 768 x 1024 Q4_0
    prefill captured in a HIP graph holds kernel nodes only (no allocation or
    free node), and three replays, each after eager no-allocation calls of
    other sizes that overwrite the shared scratch array, equal the eager call
    bit for bit."""
    k, rows = 1024, 200
    ws, datas = _weights(k, [768], seed=21)
    x = oracle.randn(rows * k, seed=22).reshape(rows, k)
    xd = dev(x)
    eager = [torch.empty((rows, 768), dtype=torch.float32, device="cuda")]
    ctx.qlinear_multi(ws, xd, eager, noalloc=True)
    torch.cuda.synchronize()
    eager = eager[0].cpu().numpy()
    y64, absdot = oracle.linear_f64(x, oracle.dequant_gguf(oracle.Q4_0, datas[0], 768, k))
    assert oracle.normalized_error(eager, y64, absdot) <= F16X2
    y = [torch.empty((rows, 768), dtype=torch.float32, device="cuda")]
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        ctx.qlinear_multi(ws, xd, y, stream=st, noalloc=True)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(g, stream=st):
            ctx.qlinear_multi(ws, xd, y, stream=st, noalloc=True)
    torch.cuda.synchronize()
    types = graph_node_types(g)
    assert types and all(t == 0 for t in types), types
    g.instantiate()
    for i in range(3):
        other_rows = 300 + 150 * i
        xo = dev(oracle.randn(other_rows * k, seed=23 + i).reshape(other_rows, k))
        yo = [torch.empty((other_rows, 768), dtype=torch.float32, device="cuda")]
        ctx.qlinear_multi(ws, xo, yo, noalloc=True)  # overwrites the scratch staging
        y[0].fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y[0].cpu().numpy().view(np.uint32), eager.view(np.uint32)), i
    del g
