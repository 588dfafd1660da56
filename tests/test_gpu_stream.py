"""GPU parity of the batch-1 streaming GEMV (gemv_stream.hpp): one activation
row over weight streams too long for latency mode (more than 16384 row blocks,
or more chunks per lane than latency mode holds) and long enough for at least
three row steps per wave, through the C ABI, on 500 random output rows and
the last rows against the oracle.

The shapes select every chunks-per-lane count (CPL 1, 2, 3, 4, 6, 8) and
lanes-per-row L (8..64); weight bases 2 bytes past a 4-byte boundary (the
lanes' realignment); row counts that are not a multiple of the rows per step
(the last step moved back over rows already computed); grouped weights of
different N in one launch; and rows whose byte length is not a multiple of 4,
which the streaming kernel declines (the persistent pipeline runs them).
Bound: the f16 rounding of the activations, 2^-11 of sum|w||x| plus f32
accumulation.
"""
import numpy as np
import pytest
import torch

import dyninfer_amd as d
import oracle

pytestmark = pytest.mark.gpu

XF16 = 2.0 ** -11 + 2e-5
ENC = {oracle.Q4_0: d.ENC_Q4_0, oracle.Q4_1: d.ENC_Q4_1, oracle.Q8_0: d.ENC_Q8_0, oracle.Q6_K: d.ENC_Q6_K}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def weight(gtype, n, k, seed, off):
    data = oracle.synth_gguf(gtype, n, k, seed)
    if off:
        buf = torch.zeros(data.size + 16, dtype=torch.uint8, device="cuda")
        buf[off:off + data.size] = dev(data)
        w = d.QWeight(ENC[gtype], n, k, buf.data_ptr() + off)
        w._keep = buf
        return w, data
    return d.QWeight(ENC[gtype], n, k, dev(data)), data


def check_rows(y, x, gtype, data, n, k, seed):
    rows = np.unique(np.concatenate([np.random.default_rng(seed).choice(n, size=min(500, n), replace=False),
                                     np.arange(max(0, n - 6), n)]))  # the last rows (shifted last step)
    bw, bb = oracle.BLOCK[gtype]
    rb = (k // bw) * bb
    sub = np.concatenate([data[r * rb:(r + 1) * rb] for r in rows])
    wsub = oracle.dequant_gguf(gtype, sub, len(rows), k)
    y64, absdot = oracle.linear_f64(x, wsub)
    return oracle.normalized_error(np.ascontiguousarray(y[:, rows]), y64, absdot)


# (n, k) -> lanes per row L and chunks per lane CPL the launcher picks.  The
# streaming kernel runs when every wave gets at least 3 row steps of G = 64/L
# rows at 16 waves per CU (4096 waves on 256 CUs): at least 12288 G rows.
CW32 = [(17003, 4096),   # L 64, CPL 2
        (13000, 6144),   # L 64, CPL 3
        (16500, 8192),   # L 64, CPL 4
        (12400, 12288),  # L 64, CPL 6
        (12300, 16384),  # L 64, CPL 8
        (50001, 1024),   # L 16, CPL 2
        (33000, 3072)]   # L 32, CPL 3
Q6K = [(151936, 1024),   # L 8, CPL 2 (the Qwen3-0.6B lm_head)
       (30001, 4096),    # L 32, CPL 2
       (12500, 12288),   # L 64, CPL 3 (1024-thread workgroups)
       (12300, 8192),    # L 64, CPL 2
       (12300, 16384),   # L 64, CPL 4 at 1024 threads: would spill, persistent pipeline
       (100003, 512),    # L 8, CPL 1
       (5000, 1280)]     # 5 super-blocks per row (1050 bytes): not a multiple of 4, persistent pipeline


@pytest.mark.parametrize("gtype", [oracle.Q4_0, oracle.Q4_1, oracle.Q8_0], ids=oracle.NAMES.get)
@pytest.mark.parametrize("n,k", CW32)
@pytest.mark.parametrize("off", [0, 2])
def test_stream_cw32(ctx, gtype, n, k, off):
    if gtype == oracle.Q4_1 and off:
        pytest.skip("Q4_1 blocks are 4-byte aligned by contract")
    w, data = weight(gtype, n, k, seed=n + k, off=off)
    x = oracle.randn(k, seed=k + n).reshape(1, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    assert check_rows(y, x, gtype, data, n, k, seed=n) <= XF16


@pytest.mark.parametrize("n,k", Q6K)
@pytest.mark.parametrize("off", [0, 2])
def test_stream_q6_k(ctx, n, k, off):
    w, data = weight(oracle.Q6_K, n, k, seed=n + k, off=off)
    x = oracle.randn(k, seed=k + n + 1).reshape(1, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    assert check_rows(y, x, oracle.Q6_K, data, n, k, seed=n) <= XF16


@pytest.mark.parametrize("gtype", oracle.GGUF_TYPES, ids=oracle.NAMES.get)
@pytest.mark.parametrize("shapes,k", [([12288, 12288], 4096),        # Qwen3-8B gate/up
                                      ([9000, 5003, 3001], 4096),   # ragged, three weights
                                      ([60000, 16], 1024)])         # one weight of 16 rows (one wave)
def test_stream_grouped(ctx, gtype, shapes, k):
    made = [weight(gtype, n, k, seed=i + 7 * n, off=0) for i, n in enumerate(shapes)]
    x = oracle.randn(k, seed=len(shapes) + k).reshape(1, k)
    ys = ctx.qlinear_multi([m[0] for m in made], dev(x))
    for y, (_, data), n in zip(ys, made, shapes):
        assert check_rows(y.cpu().numpy(), x, gtype, data, n, k, seed=n) <= XF16


def test_stream_bf16_io(ctx):
    n, k = 24576, 4096
    w, data = weight(oracle.Q4_0, n, k, seed=3, off=2)
    xb = oracle.f32_to_bf16_bits(oracle.randn(k, seed=4)).reshape(1, k)
    x = oracle.bf16_bits_to_f32(xb).reshape(1, k)
    y = ctx.qlinear(w, dev(xb).view(torch.bfloat16), y_dtype=torch.bfloat16)
    y = oracle.bf16_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16)).reshape(1, n)
    rows = np.random.default_rng(1).choice(n, size=500, replace=False)
    rb = (k // 32) * 18
    wsub = oracle.dequant_gguf(oracle.Q4_0, np.concatenate([data[r * rb:(r + 1) * rb] for r in rows]), 500, k)
    y64, absdot = oracle.linear_f64(x, wsub)
    err = np.abs(y[:, rows].astype(np.float64) - y64) / absdot - np.abs(y64) * 2.0 ** -8 / absdot
    assert err.max() <= XF16
