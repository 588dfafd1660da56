"""GGUF Q4_K and Q5_K (GGML's block_q4_K, block_q5_K) through the C ABI.

The reference declares their schemas only (gguf_block.rs:183-316: types 12
and 13, 256 weights, 144 and 176 bytes, components scale_min_f16 /
scales_and_mins_u6 / [high_bits /] quants_u4; convention.rs:210-211,240-241),
so the kernels here decode GGML's layouts, which the oracle restates and pins
(tests/test_oracle.py: the packer-side layouts, known-answer blocks, the
one-rounding closed forms).

Bars, as for the other encodings:
  * dequantisation and embedding rows: bit-exact (every f32 bit pattern)
    with the oracle, w = f32(d·sc)·q - f32(dmin·m) with one rounding;
  * GEMV outputs: max |y - y_ref| / Σ_k |w||x| <= 2e-3 and <= 2^-11 + 2e-5
    (one f16 rounding per activation after a power-of-two scaling per
    32-weight group, f32 accumulation), y_ref the f64 contraction of the
    exactly dequantised weights.
"""
import struct

import numpy as np
import pytest

import dyninfer_amd as d
import oracle

TOL = 2e-3
XF16 = 2.0 ** -11 + 2e-5
KQ = [oracle.Q4_K, oracle.Q5_K]
ENC = {oracle.Q4_K: d.ENC_Q4_K, oracle.Q5_K: d.ENC_Q5_K}
kinds = pytest.mark.parametrize("kind", KQ, ids=oracle.NAMES.get)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def weight(kind, n, k, seed, off=0):
    """A weight of synthetic super-blocks, `off` bytes into a device buffer."""
    import torch
    data = oracle.synth_gguf(kind, n, k, seed)
    buf = torch.zeros(data.size + 16, dtype=torch.uint8, device="cuda")
    buf[off:off + data.size] = dev(data)
    w = d.QWeight(ENC[kind], n, k, buf.data_ptr() + off, data_bytes=data.size)
    w._keep = buf
    return w, data


def assert_bits_equal(got, ref):
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    bad = (got.view(np.uint32) != ref.view(np.uint32)) & ~nan
    assert not bad.any(), f"{bad.sum()} differing, first at {np.argwhere(bad)[0]}"


def err_of(y, x, wf):
    y64, absdot = oracle.linear_f64(x, wf)
    return oracle.normalized_error(y, y64, absdot)


# ---------------------------------------------------------------- host-side (no GPU)
@kinds
def test_weight_rules(kind):
    w = lambda **kw: d.QWeight(ENC[kind], kw.pop("n", 8), kw.pop("k", 512), kw.pop("data", 0x1000), **kw)
    assert d.supports(w(), 1) and d.supports(w(), 16) and d.supports(w(), 512, d.DTYPE_BF16, d.DTYPE_BF16)
    assert not d.supports(w(k=384), 1)          # K a multiple of 256
    assert "multiple of the block size 256" in d.library().dyninfer_mi355x_last_error().decode()
    assert not d.supports(w(data=0x1002), 1)    # 4-byte-aligned super-blocks
    assert "4-byte aligned" in d.library().dyninfer_mi355x_last_error().decode()
    bb = oracle.BLOCK[kind][1]
    assert d.supports(w(data_bytes=8 * 2 * bb), 1)
    assert not d.supports(w(data_bytes=8 * 2 * bb - 4), 1)
    assert d.block_geometry(ENC[kind]) == (256, bb)


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


@kinds
def test_gguf_tensor_indexed_and_described(kind):
    """A GGUF file holding a tensor of the type: its exact byte range, and a
    QWeight of it (the reference indexes such tensors but has no kernel for them)."""
    n, k = 6, 512
    raw = oracle.synth_gguf(kind, n, k, 4).tobytes()
    body = b"GGUF" + struct.pack("<IQQ", 3, 1, 1) + _s("general.architecture") + struct.pack("<I", 8) + _s("llama")
    body += _s("blk.0.ffn_up.weight") + struct.pack("<I", 2) + struct.pack("<QQ", k, n) + struct.pack("<IQ", kind, 0)
    body += b"\0" * ((32 - len(body) % 32) % 32)
    g = d.GgufFile.from_bytes(body + raw)
    t = g.tensors[0]
    assert (t.type_code, t.nbytes, t.offset) == (kind, len(raw), len(body))
    w = g.qweight("blk.0.ffn_up.weight", 0x1000)
    assert (w.encoding, w.rows, w.cols, w.data_bytes) == (ENC[kind], n, k, len(raw))
    with pytest.raises(d.DyninferError):
        g.qweight("blk.0.ffn_up.weight", 0x1002)


# ---------------------------------------------------------------- dequant / embedding
@pytest.mark.gpu
@pytest.mark.parametrize("n,k,off", [(1, 256, 0), (3, 512, 4), (64, 1024, 0), (33, 4096, 12)])
@kinds
def test_dequant_bit_exact(ctx, kind, n, k, off):
    w, data = weight(kind, n, k, seed=n + k, off=off)
    assert_bits_equal(ctx.dequant(w).cpu().numpy(), oracle.dequant_gguf(kind, data, n, k))


@pytest.mark.gpu
@kinds
def test_dequant_special_fields(ctx, kind):
    """d, dmin over signed zeros, subnormals, max, inf and NaN; every scale and
    min byte pattern (0x00 / 0xFF / random) so the top-two-bit paths of
    sub-blocks 4..7 are all exercised."""
    specials = [0x8000, 0x0000, 0x0001, 0x03FF, 0x3C00, 0xC100, 0x7BFF, 0x7C00, 0xFC00, 0x7E00]
    rng = np.random.default_rng(9)
    blocks = []
    for i, dbits in enumerate(specials):
        for j, mbits in enumerate((0x0000, 0x3C00, specials[(i + 3) % len(specials)])):
            b = rng.integers(0, 256, oracle.BLOCK[kind][1], dtype=np.uint8)
            b[0:2] = [dbits & 0xFF, dbits >> 8]
            b[2:4] = [mbits & 0xFF, mbits >> 8]
            if j == 0:
                b[4:16] = 0xFF
            blocks.append(b)
    data = np.concatenate(blocks)
    rows = len(blocks)
    w = d.QWeight(ENC[kind], rows, 256, dev(data))
    assert_bits_equal(ctx.dequant(w).cpu().numpy(), oracle.dequant_gguf(kind, data, rows, 256))


@pytest.mark.gpu
@pytest.mark.parametrize("vocab,k,n", [(1, 256, 1), (37, 512, 5), (300, 1024, 64), (9, 4096, 17)])
@kinds
def test_embedding_bit_exact(ctx, kind, vocab, k, n):
    w, data = weight(kind, vocab, k, seed=vocab * 3 + k)
    rng = np.random.default_rng(n)
    ids = rng.integers(0, vocab, n).astype(np.int64)
    ids[:min(n, 2)] = [0, vocab - 1][:min(n, 2)]
    out = ctx.embedding(w, dev(ids)).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), oracle.dequant_gguf(kind, data, vocab, k)[ids].view(np.uint32))


@pytest.mark.gpu
@kinds
def test_embedding_out_of_range_ids_are_nan_rows(ctx, kind):
    w, data = weight(kind, 12, 512, seed=2)
    ids = np.array([3, -1, 12, 11], np.int64)
    out = ctx.embedding(w, dev(ids)).cpu().numpy()
    ref = oracle.dequant_gguf(kind, data, 12, 512)
    assert np.array_equal(out[0], ref[3]) and np.array_equal(out[3], ref[11])
    assert np.isnan(out[1]).all() and np.isnan(out[2]).all()


# ---------------------------------------------------------------- GEMV
# shapes reach every launch form: latency mode (few chunks per lane), the
# persistent pipeline, the batch-1 streaming kernel, 1024-thread workgroups
# for K > 8192, and several register passes for batches above 4
SHAPES = [(1, 256), (67, 512), (1024, 1024), (3072, 1024), (1024, 3072), (513, 4096), (4096, 4096), (1024, 12288)]


@pytest.mark.gpu
@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 8, 16])
@kinds
def test_gemv(ctx, kind, n, k, batch):
    w, data = weight(kind, n, k, seed=100 + n + k + batch)
    x = oracle.randn(batch * k, seed=n * 7 + batch).reshape(batch, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    err = err_of(y, x, oracle.dequant_gguf(kind, data, n, k))
    assert err <= TOL and err <= XF16, err


@pytest.mark.gpu
@kinds
@pytest.mark.parametrize("n,k", [(6144, 5120), (8192, 4096)])
def test_two_rows_many_row_blocks(ctx, kind, n, k):
    """Two activation rows over more row blocks than the 2-row latency mode takes
    for 64-weight chunks (2048 at 2 chunks per lane, 4096 at 1): the persistent
    pipeline.  Checked on the first 1024 rows."""
    w, data = weight(kind, n, k, seed=200 + n + k)
    x = oracle.randn(2 * k, seed=201).reshape(2, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    nc = 1024
    err = err_of(y[:, :nc], x, oracle.dequant_gguf(kind, data[:len(data) // n * nc], nc, k))
    assert err <= TOL and err <= XF16, err


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [17, 40])
@kinds
def test_more_than_16_rows(ctx, kind, rows):
    n, k = 768, 2048
    w, data = weight(kind, n, k, seed=rows)
    x = oracle.randn(rows * k, seed=rows + 1).reshape(rows, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    err = err_of(y, x, oracle.dequant_gguf(kind, data, n, k))
    assert err <= TOL and err <= XF16, err


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [1, 4])
@kinds
def test_bf16_activations_and_outputs_offset_base(ctx, kind, batch):
    import torch
    n, k = 2048, 4096
    w, data = weight(kind, n, k, seed=77, off=4)
    x = torch.from_numpy(oracle.randn(batch * k, seed=5).reshape(batch, k)).to(torch.bfloat16)
    xr = x.float().numpy()
    y = ctx.qlinear(w, x.cuda(), y_dtype=torch.bfloat16).float().cpu().numpy()
    y64, absdot = oracle.linear_f64(xr, oracle.dequant_gguf(kind, data, n, k))
    # bf16 outputs add one bf16 rounding of |y| (relative 2^-9)
    bound = XF16 + 2.0 ** -9 * np.max(np.abs(y64) / absdot)
    err = oracle.normalized_error(y, y64, absdot)
    assert err <= TOL and err <= bound, err


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [1, 2, 16])
@kinds
def test_multi_weights_share_activations(ctx, kind, batch):
    k = 4096
    ws = [weight(kind, n, k, seed=n + batch) for n in (4096, 1024, 1024)]
    x = oracle.randn(batch * k, seed=batch).reshape(batch, k)
    ys = ctx.qlinear_multi([w for w, _ in ws], dev(x))
    for (w, data), y in zip(ws, ys):
        err = err_of(y.cpu().numpy(), x, oracle.dequant_gguf(kind, data, w.rows, k))
        assert err <= TOL and err <= XF16, err


# ---------------------------------------------------------------- MFMA GEMV (5..16 rows)
# Large launches at 5..16 rows run on MFMA: B = sc·q exact in f16, d applied
# per weight row in f32, the offsets Σ_j dmin·m_j·X_j through one more MFMA
# whose activation sums X_j are rounded once to f16.  Per output the error is
# at most 2^-11·Σ|w||x| (activation rounding) + 2^-11·Σ|dmin·m||x| (sums)
# plus f32 accumulation.
def offsets_of(kind, data, n, k):
    """|dmin·m| per weight: the dequantisation with every d set to zero."""
    z = data.reshape(-1, oracle.BLOCK[kind][1]).copy()
    z[:, 0:2] = 0
    return np.abs(oracle.dequant_gguf(kind, z.ravel(), n, k))


MFMA_CASES = [  # (n, k, batch, y_bf16): split mode, whole tiles, K segments, a padded tile
    (4096, 4096, 5, False), (4096, 4096, 16, True), (12288, 4096, 8, False), (4096, 12288, 16, False),
    (20000, 1024, 12, False), (2056, 2048, 16, False), (2048, 4096, 7, True)]


@pytest.mark.gpu
@pytest.mark.parametrize("n,k,batch,ybf16", MFMA_CASES)
@kinds
def test_gemv_mfma(ctx, kind, n, k, batch, ybf16):
    import torch
    w, data = weight(kind, n, k, seed=n + k + batch, off=4 if ybf16 else 0)
    x = oracle.randn(batch * k, seed=batch * 3 + k).reshape(batch, k)
    y = ctx.qlinear(w, dev(x), y_dtype=torch.bfloat16 if ybf16 else torch.float32).float().cpu().numpy()
    wf = oracle.dequant_gguf(kind, data, n, k)
    y64, absdot = oracle.linear_f64(x, wf)
    absb = np.abs(x.astype(np.float64)) @ offsets_of(kind, data, n, k).astype(np.float64).T
    err = np.abs(y - y64) / absdot
    bound = 2.0 ** -11 + 2.0 ** -11 * absb / absdot + 2e-5
    if ybf16:
        bound = bound + 2.0 ** -9 * np.abs(y64) / absdot
    assert np.all(err <= bound), (err / bound).max()
    assert oracle.normalized_error(y, y64, absdot) <= TOL


@pytest.mark.gpu
@kinds
def test_gemv_mfma_large_offsets(ctx, kind):
    """Blocks whose offsets dominate (dmin·m far above d·sc·q): the offset
    MFMA's rounding stays within its bound."""
    n, k, batch = 4096, 2048, 16
    data = oracle.synth_gguf(kind, n, k, 8).reshape(-1, oracle.BLOCK[kind][1])
    data[:, 2:4] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)  # dmin = 0.5
    data = data.ravel()
    w = d.QWeight(ENC[kind], n, k, dev(data))
    x = oracle.randn(batch * k, seed=4).reshape(batch, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    y64, absdot = oracle.linear_f64(x, oracle.dequant_gguf(kind, data, n, k))
    absb = np.abs(x.astype(np.float64)) @ offsets_of(kind, data, n, k).astype(np.float64).T
    err = np.abs(y - y64) / absdot
    assert np.all(err <= 2.0 ** -11 + 2.0 ** -11 * absb / absdot + 2e-5)
    assert oracle.normalized_error(y, y64, absdot) <= TOL


# ---------------------------------------------------------------- prefill GEMM (33+ rows; 17+ for K > 8192)
# Staged f16 activations (one rounding each after a power-of-two row scaling)
# times weights decoded to f16 as RNE_f16(q·RNE_f16(d·sc) - RNE_f16(dmin·m)):
# per output at most 2^-10·Σ|w||x| + 2^-11·Σ(|q·d·sc| + |dmin·m|)|x| plus f32
# accumulation, and |q·d·sc| <= |w| + |dmin·m|.
GEMM_CASES = [  # (rows, n, k, x/y bf16, base offset); 33+ rows, or 17+ with K > 8192
    (20, 512, 12288, False, 0), (33, 256, 1024, False, 0), (64, 1000, 2048, False, 4), (77, 3072, 1024, True, 0), (200, 1024, 3072, False, 0),
    (512, 3072, 1024, True, 4), (512, 1024, 4096, False, 0)]


@pytest.mark.gpu
@pytest.mark.parametrize("rows,n,k,bf16,off", GEMM_CASES)
@kinds
def test_prefill_gemm(ctx, kind, rows, n, k, bf16, off):
    import torch
    w, data = weight(kind, n, k, seed=rows + n + k, off=off)
    xt = torch.from_numpy(oracle.randn(rows * k, seed=rows + 9).reshape(rows, k))
    if bf16:
        xt = xt.to(torch.bfloat16)
    y = ctx.qlinear(w, xt.cuda(), y_dtype=torch.bfloat16 if bf16 else torch.float32).float().cpu().numpy()
    x = xt.float().numpy()
    y64, absdot = oracle.linear_f64(x, oracle.dequant_gguf(kind, data, n, k))
    absb = np.abs(x.astype(np.float64)) @ offsets_of(kind, data, n, k).astype(np.float64).T
    bound = 2.0 ** -10 + 2.0 ** -11 * (1.0 + 2.0 * absb / absdot) + 2e-5
    if bf16:
        bound = bound + 2.0 ** -9 * np.abs(y64) / absdot
    err = np.abs(y - y64) / absdot
    assert np.all(err <= bound), (err / bound).max()
    assert oracle.normalized_error(y, y64, absdot) <= TOL


@pytest.mark.gpu
@kinds
def test_prefill_gemm_multi(ctx, kind):
    rows, k = 96, 2048
    ws = [weight(kind, n, k, seed=n) for n in (2048, 512, 512)]
    x = oracle.randn(rows * k, seed=3).reshape(rows, k)
    ys = ctx.qlinear_multi([w for w, _ in ws], dev(x))
    for (w, data), y in zip(ws, ys):
        y64, absdot = oracle.linear_f64(x, oracle.dequant_gguf(kind, data, w.rows, k))
        assert oracle.normalized_error(y.cpu().numpy(), y64, absdot) <= 2.0 ** -10 + 2.0 ** -10 + 2e-5


@pytest.mark.gpu
@kinds
def test_deterministic(ctx, kind):
    w, _ = weight(kind, 4096, 4096, seed=1)
    x = dev(oracle.randn(4096, seed=2).reshape(1, 4096))
    a = ctx.qlinear(w, x).cpu().numpy()
    for _ in range(3):
        assert np.array_equal(ctx.qlinear(w, x).cpu().numpy().view(np.uint32), a.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("gtype", [oracle.Q4_K, oracle.Q5_K, oracle.IQ4_XS], ids=oracle.NAMES.get)
@pytest.mark.parametrize("n,k", [(32768, 4096), (12400, 12288), (12300, 16384)])
def test_streaming_kernel_long_weight(ctx, gtype, n, k):
    """One activation row over a weight with enough row steps per wave for the
    batch-1 streaming kernel: 32768 x 4096 streams (lanes per row 32 for the
    64-weight chunks, 64 for IQ4_XS); at K = 12288 and 16384 (3 and 4 chunks
    per lane in 1024-thread workgroups) Q4_K and Q5_K would spill there and run
    the persistent pipeline instead.  Checked on 400 random rows, dequantised
    by the oracle from their own bytes."""
    enc = {oracle.Q4_K: d.ENC_Q4_K, oracle.Q5_K: d.ENC_Q5_K, oracle.IQ4_XS: d.ENC_IQ4_XS}[gtype]
    bb = oracle.BLOCK[gtype][1]
    data = oracle.synth_gguf(gtype, n, k, 17)
    w = d.QWeight(enc, n, k, dev(data))
    x = oracle.randn(k, seed=18).reshape(1, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    rows = np.sort(np.random.default_rng(19).choice(n, 400, replace=False))
    rb = k // 256 * bb
    sub = np.concatenate([data[r * rb:(r + 1) * rb] for r in rows])
    wf = oracle.dequant_gguf(gtype, sub, len(rows), k)
    y64, absdot = oracle.linear_f64(x, wf)
    err = oracle.normalized_error(y[:, rows], y64, absdot)
    assert err <= TOL and err <= 2.0 ** -11 + 2e-5, err


@pytest.mark.gpu
def test_gguf_file_mixed_super_blocks_upload_and_qlinear(ctx, tmp_path):
    """A GGUF file in the spirit of a Q4_K_M checkpoint: Q4_K, Q5_K, IQ4_XS
    and Q6_K tensors, indexed by path, each tensor's exact bytes uploaded and
    multiplied through the QWeight the index describes."""
    import torch
    specs = {"blk.0.attn_q.weight": (oracle.Q4_K, 512, 1024), "blk.0.attn_v.weight": (oracle.Q6_K, 256, 1024),
             "blk.0.ffn_down.weight": (oracle.Q5_K, 1024, 768), "blk.0.ffn_up.weight": (oracle.IQ4_XS, 768, 1024)}
    raws = {name: oracle.synth_gguf(t, n, k, 40 + i) for i, (name, (t, n, k)) in enumerate(specs.items())}
    body = b"GGUF" + struct.pack("<IQQ", 3, len(specs), 1) + _s("general.architecture") + struct.pack("<I", 8) + _s("qwen3")
    data = b""
    for name in sorted(specs):
        t, n, k = specs[name]
        data += b"\0" * ((32 - len(data) % 32) % 32)
        body += _s(name) + struct.pack("<I", 2) + struct.pack("<QQ", k, n) + struct.pack("<IQ", t, len(data))
        data += raws[name].tobytes()
    body += b"\0" * ((32 - len(body) % 32) % 32)
    path = tmp_path / "mixed.gguf"
    path.write_bytes(body + data)
    g = d.GgufFile(str(path))
    for name, (t, n, k) in specs.items():
        dev_bytes = g.upload(name)
        assert torch.equal(dev_bytes.cpu(), torch.from_numpy(raws[name]))
        w = g.qweight(name, dev_bytes)
        x = oracle.randn(3 * k, seed=n).reshape(3, k)
        y = ctx.qlinear(w, dev(x)).cpu().numpy()
        err = err_of(y, x, oracle.dequant_gguf(t, raws[name], n, k))
        assert err <= TOL and err <= 2.0 ** -11 + 2e-5, (name, err)

