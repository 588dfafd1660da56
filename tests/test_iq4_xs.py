"""GGUF IQ4_XS (GGML's block_iq4_xs) through the C ABI.

The reference declares IQ4_XS's schema only (gguf_block.rs:183-316: type 23,
256 weights, 136 bytes, components scale_f16 / scales_high_u16 /
scales_low_u8 / nonlinear_quants_u4; convention.rs:221,267), so the kernels
here decode GGML's layout and its kvalues_iq4nl codebook, which the oracle
restates and pins (tests/test_oracle.py: the packer-side scale layout, a
known-answer block, the closed form f32(d*(ls-32)*kvalue)).  The device holds
the codebook as its own constant, so the bit-exact dequantisation below checks
it against the oracle's independently typed table.

Bars, as max over outputs of |y - y64| / sum_k |w||x| (y64 the f64 contraction
of the exactly dequantised weights), each within the 2e-3 north-star tolerance:
  * dequantisation and embedding rows: bit-exact;
  * VALU GEMV (1..4 rows, and 5..16 rows of small weights): weights exact (a
    codebook byte times the f32 scale), activations rounded once to f16 after
    a power-of-two scaling: 2^-11 + 2e-5;
  * MFMA GEMV (5..16 rows): B = RNE_f16(kv*(ls-32)) plus the activation
    rounding: 2^-10 + 2e-5;
  * prefill GEMM: RNE_f16(kv*RNE_f16(d*(ls-32))) rounds the weight twice,
    plus the staged activation: 3 * 2^-11 + 2e-5.
"""
import struct

import numpy as np
import pytest

import dyninfer_amd as d
import oracle

TOL = 2e-3
IQ = oracle.IQ4_XS
BB = 136


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def weight(n, k, seed, off=0):
    import torch
    data = oracle.synth_gguf(IQ, n, k, seed)
    buf = torch.zeros(data.size + 16, dtype=torch.uint8, device="cuda")
    buf[off:off + data.size] = dev(data)
    w = d.QWeight(d.ENC_IQ4_XS, n, k, buf.data_ptr() + off, data_bytes=data.size)
    w._keep = buf
    return w, data


def err_of(y, x, wf):
    y64, absdot = oracle.linear_f64(x, wf)
    return oracle.normalized_error(y, y64, absdot)


# ---------------------------------------------------------------- host-side (no GPU)
def test_weight_rules():
    w = lambda **kw: d.QWeight(d.ENC_IQ4_XS, kw.pop("n", 8), kw.pop("k", 512), kw.pop("data", 0x1000), **kw)
    assert d.supports(w(), 1) and d.supports(w(), 16) and d.supports(w(), 512, d.DTYPE_BF16, d.DTYPE_BF16)
    assert not d.supports(w(k=384), 1)
    assert "multiple of the block size 256" in d.library().dyninfer_mi355x_last_error().decode()
    assert not d.supports(w(data=0x1002), 1)  # 136-byte super-blocks: 4-byte-aligned base
    assert d.supports(w(data_bytes=8 * 2 * BB), 1)
    assert not d.supports(w(data_bytes=8 * 2 * BB + 2), 1)
    assert d.block_geometry(d.ENC_IQ4_XS) == (256, BB)


def test_gguf_tensor_indexed_and_described():
    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    n, k = 5, 768
    raw = oracle.synth_gguf(IQ, n, k, 2).tobytes()
    body = b"GGUF" + struct.pack("<IQQ", 3, 1, 1) + s("general.architecture") + struct.pack("<I", 8) + s("qwen3")
    body += s("blk.0.attn_q.weight") + struct.pack("<I", 2) + struct.pack("<QQ", k, n) + struct.pack("<IQ", 23, 0)
    body += b"\0" * ((32 - len(body) % 32) % 32)
    g = d.GgufFile.from_bytes(body + raw)
    t = g.tensors[0]
    assert (t.type_code, t.nbytes, t.offset) == (23, len(raw), len(body))
    w = g.qweight("blk.0.attn_q.weight", 0x2000)
    assert (w.encoding, w.rows, w.cols, w.data_bytes) == (d.ENC_IQ4_XS, n, k, len(raw))


# ---------------------------------------------------------------- dequant / embedding
@pytest.mark.gpu
@pytest.mark.parametrize("n,k,off", [(1, 256, 0), (3, 512, 4), (64, 1024, 0), (33, 4096, 12)])
def test_dequant_bit_exact(ctx, n, k, off):
    w, data = weight(n, k, seed=n + k, off=off)
    got = ctx.dequant(w).cpu().numpy()
    ref = oracle.dequant_gguf(IQ, data, n, k)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))


@pytest.mark.gpu
def test_dequant_every_index_scale_and_special_d(ctx):
    """Every codebook index at every position of a sub-block, every 6-bit
    scale, and d over signed zeros, subnormals, max, inf and NaN."""
    specials = [0x8000, 0x0000, 0x0001, 0x03FF, 0x3C00, 0xC100, 0x7BFF, 0x7C00, 0xFC00, 0x7E00]
    rng = np.random.default_rng(4)
    blocks = []
    for i in range(64):
        b = rng.integers(0, 256, BB, dtype=np.uint8)
        dbits = specials[i % len(specials)] if i < 20 else int(np.frombuffer(np.float16(0.01 * (i + 1)).tobytes(), np.uint16)[0])
        b[0:2] = [dbits & 0xFF, dbits >> 8]
        ls = np.full(8, i)  # scale i on every sub-block: 0..63 over the blocks
        sl = [(ls[2 * j] & 15) | ((ls[2 * j + 1] & 15) << 4) for j in range(4)]
        sh = sum(int(ls[ib] >> 4) << (2 * ib) for ib in range(8))
        b[2:4] = [sh & 0xFF, sh >> 8]
        b[4:8] = sl
        b[8:136] = (np.arange(128) % 16) | (((np.arange(128) + i) % 16) << 4)
        blocks.append(b)
    data = np.concatenate(blocks)
    w = d.QWeight(d.ENC_IQ4_XS, 64, 256, dev(data))
    got = ctx.dequant(w).cpu().numpy()
    ref = oracle.dequant_gguf(IQ, data, 64, 256)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("vocab,k,n", [(1, 256, 1), (37, 512, 5), (300, 1024, 64), (9, 4096, 17)])
def test_embedding_bit_exact(ctx, vocab, k, n):
    w, data = weight(vocab, k, seed=vocab * 5 + k)
    rng = np.random.default_rng(n)
    ids = rng.integers(0, vocab, n).astype(np.int64)
    ids[:min(n, 2)] = [0, vocab - 1][:min(n, 2)]
    out = ctx.embedding(w, dev(ids)).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), oracle.dequant_gguf(IQ, data, vocab, k)[ids].view(np.uint32))


# ---------------------------------------------------------------- GEMV
SHAPES = [(1, 256), (67, 512), (1024, 1024), (3072, 1024), (1024, 3072), (513, 4096), (4096, 4096), (1024, 12288)]


@pytest.mark.gpu
@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 8, 16])
def test_gemv(ctx, n, k, batch):
    w, data = weight(n, k, seed=200 + n + k + batch)
    x = oracle.randn(batch * k, seed=n * 3 + batch).reshape(batch, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    err = err_of(y, x, oracle.dequant_gguf(IQ, data, n, k))
    # MFMA (5..16 rows of the larger weights) rounds each weight once more
    assert err <= TOL and err <= (2.0 ** -10 if batch > 4 else 2.0 ** -11) + 2e-5, err


@pytest.mark.gpu
@pytest.mark.parametrize("n,k,batch", [(20000, 1024, 12), (17000, 2048, 16)])
def test_gemv_mfma_whole_tiles(ctx, n, k, batch):
    """At least 1024 tiles: the MFMA GEMV's whole-tile mode (a wave per tile)."""
    w, data = weight(n, k, seed=n + batch)
    x = oracle.randn(batch * k, seed=batch + 7).reshape(batch, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    err = err_of(y, x, oracle.dequant_gguf(IQ, data, n, k))
    assert err <= TOL and err <= 2.0 ** -10 + 2e-5, err


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [1, 4, 16])
def test_multi_and_bf16(ctx, batch):
    import torch
    k = 4096
    ws = [weight(n, k, seed=n + batch, off=4) for n in (4096, 1024, 1024)]
    xt = torch.from_numpy(oracle.randn(batch * k, seed=batch).reshape(batch, k)).to(torch.bfloat16)
    ys = ctx.qlinear_multi([w for w, _ in ws], xt.cuda(), y_dtype=torch.bfloat16)
    x = xt.float().numpy()
    for (w, data), y in zip(ws, ys):
        y64, absdot = oracle.linear_f64(x, oracle.dequant_gguf(IQ, data, w.rows, k))
        err = np.abs(y.float().cpu().numpy() - y64) / absdot
        assert np.all(err <= 2.0 ** -10 + 2e-5 + 2.0 ** -9 * np.abs(y64) / absdot), err.max()


# ---------------------------------------------------------------- prefill GEMM
@pytest.mark.gpu
@pytest.mark.parametrize("rows,n,k,bf16", [(20, 512, 12288, False), (33, 256, 1024, False), (77, 3072, 1024, True),
                                           (200, 1024, 3072, False), (512, 3072, 1024, True), (512, 1024, 4096, False)])
def test_prefill_gemm(ctx, rows, n, k, bf16):
    import torch
    w, data = weight(n, k, seed=rows + n)
    xt = torch.from_numpy(oracle.randn(rows * k, seed=rows + 2).reshape(rows, k))
    if bf16:
        xt = xt.to(torch.bfloat16)
    y = ctx.qlinear(w, xt.cuda(), y_dtype=torch.bfloat16 if bf16 else torch.float32).float().cpu().numpy()
    x = xt.float().numpy()
    y64, absdot = oracle.linear_f64(x, oracle.dequant_gguf(IQ, data, n, k))
    err = np.abs(y - y64) / absdot
    bound = 3 * 2.0 ** -11 + 2e-5 + (2.0 ** -9 * np.abs(y64) / absdot if bf16 else 0.0)
    assert np.all(err <= bound), err.max()
    assert oracle.normalized_error(y, y64, absdot) <= TOL
