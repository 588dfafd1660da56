"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Bars (written here as the tests use them):
  * dequantisation: bit-exact (every f32 bit pattern) with the oracle's
    restatement of the reference's MLIR dequant bodies;
  * GEMV / GEMM outputs: max over outputs of |y - y_ref| / Σ_k |w||x| <= 2e-3,
    y_ref the f64 contraction of the exactly dequantised weights (the
    north-star tolerance).  The GEMV rounds each activation once to f16 after
    an exact power-of-two scaling per scale group and accumulates in f32, so
    its error is bounded by the f16 unit roundoff 2^-11 of Σ|w||x| plus f32
    accumulation: the GEMV tests also hold it to XF16 = 2^-11 + 2e-5, which a
    dropped or mis-scaled block (an error of order 1/blocks per row) exceeds.
"""
import ctypes

import numpy as np
import pytest
import torch

import dyninfer_amd as d
import oracle

pytestmark = pytest.mark.gpu

TOL = 2e-3
XF16 = 2.0 ** -11 + 2e-5
ENC = {oracle.Q4_0: d.ENC_Q4_0, oracle.Q4_1: d.ENC_Q4_1, oracle.Q8_0: d.ENC_Q8_0, oracle.Q6_K: d.ENC_Q6_K,
       oracle.Q4_K: d.ENC_Q4_K, oracle.Q5_K: d.ENC_Q5_K, oracle.IQ4_XS: d.ENC_IQ4_XS}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def offset_bytes(data: np.ndarray, off: int):
    """Device copy of `data` starting `off` bytes into a larger buffer (keeps the buffer alive)."""
    buf = torch.zeros(data.size + 16, dtype=torch.uint8, device="cuda")
    buf[off:off + data.size] = dev(data)
    return buf, buf.data_ptr() + off


def gguf(gtype, n, k, seed, off=0):
    data = oracle.synth_gguf(gtype, n, k, seed)
    if off:
        buf, ptr = offset_bytes(data, off)
        w = d.QWeight(ENC[gtype], n, k, ptr)
        w._keep = buf
    else:
        w = d.QWeight(ENC[gtype], n, k, dev(data))
    return w, data


def assert_bits_equal(got: np.ndarray, ref: np.ndarray):
    g = got.view(np.uint32)
    r = ref.view(np.uint32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    bad = (g != r) & ~nan
    assert not bad.any(), f"{bad.sum()} differing elements, first at {np.argwhere(bad)[0]}: " \
                          f"got {got[tuple(np.argwhere(bad)[0])]} ref {ref[tuple(np.argwhere(bad)[0])]}"


def gemv_err(y: np.ndarray, x: np.ndarray, w: np.ndarray) -> float:
    y64, absdot = oracle.linear_f64(x, w)
    return oracle.normalized_error(y, y64, absdot)


# ----------------------------------------------------------------- dequant
@pytest.mark.parametrize("gtype", oracle.GGUF_TYPES, ids=oracle.NAMES.get)
@pytest.mark.parametrize("n,k,off", [(1, 256, 0), (3, 256, 0), (64, 512, 0), (5, 256, 2), (33, 768, 2), (7, 1024, 0)])
def test_dequant_gguf_bit_exact(ctx, gtype, n, k, off):
    if gtype == oracle.Q4_1 and off % 4:
        pytest.skip("Q4_1 blocks are 4-byte aligned by contract")
    w, data = gguf(gtype, n, k, seed=n * 7 + k, off=off)
    got = ctx.dequant(w).cpu().numpy()
    assert_bits_equal(got, oracle.dequant_gguf(gtype, data, n, k))


def _special_scale_blocks(gtype, scales):
    bw, bb = oracle.BLOCK[gtype]
    rows = len(scales)
    data = oracle.synth_gguf(gtype, rows, bw, 99).reshape(rows, bb)
    pos = 208 if gtype == oracle.Q6_K else 0
    for i, s in enumerate(scales):
        data[i, pos] = s & 0xFF
        data[i, pos + 1] = s >> 8
    if gtype == oracle.Q4_0:  # include code 8 (weight exactly zero) in every block
        data[:, 2] = (data[:, 2] & 0xF0) | 0x08
    return data.ravel(), rows, bw


@pytest.mark.parametrize("gtype", oracle.GGUF_TYPES, ids=oracle.NAMES.get)
def test_dequant_special_scales(ctx, gtype):
    # -0, +0, smallest subnormal, largest subnormal, 1.0, -2.5, max, +inf, -inf, NaN
    scales = [0x8000, 0x0000, 0x0001, 0x03FF, 0x3C00, 0xC100, 0x7BFF, 0x7C00, 0xFC00, 0x7E00]
    data, rows, k = _special_scale_blocks(gtype, scales)
    w = d.QWeight(ENC[gtype], rows, k, dev(data))
    assert_bits_equal(ctx.dequant(w).cpu().numpy(), oracle.dequant_gguf(gtype, data, rows, k))


@pytest.mark.parametrize("sdtype", [oracle.D_BF16, oracle.D_F16, oracle.D_F32])
@pytest.mark.parametrize("n,k,g", [(3, 64, 32), (17, 256, 64), (8, 512, 128)])
def test_dequant_mlx_bit_exact(ctx, sdtype, n, k, g):
    packed, sc, bi = oracle.synth_mlx_u4(n, k, g, sdtype, seed=n + k + g)
    w = d.QWeight(d.ENC_MLX_U4, n, k, dev(packed), dev(sc), dev(bi), g, sdtype)
    assert_bits_equal(ctx.dequant(w).cpu().numpy(), oracle.dequant_mlx_u4(packed, sc, bi, sdtype, n, k, g))


# ----------------------------------------------------------------- GEMV
GEMV_SHAPES = [(1, 256), (67, 512), (1024, 1024), (3072, 1024), (1024, 3072), (513, 4096)]


@pytest.mark.parametrize("gtype", oracle.GGUF_TYPES, ids=oracle.NAMES.get)
@pytest.mark.parametrize("n,k", GEMV_SHAPES)
@pytest.mark.parametrize("batch", [1, 4, 16])
def test_gemv_gguf(ctx, gtype, n, k, batch):
    w, data = gguf(gtype, n, k, seed=1000 + n + k + batch)
    x = oracle.randn(batch * k, seed=n * 31 + batch).reshape(batch, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    err = gemv_err(y, x, oracle.dequant_gguf(gtype, data, n, k))
    assert err <= TOL and err <= XF16, err


@pytest.mark.parametrize("gtype", oracle.GGUF_TYPES, ids=oracle.NAMES.get)
@pytest.mark.parametrize("batch", [2, 3, 5, 7, 9, 12, 15])
def test_gemv_gguf_odd_batches(ctx, gtype, batch):
    n, k = 300, 1024
    w, data = gguf(gtype, n, k, seed=77 + batch, off=2 if gtype != oracle.Q4_1 else 0)
    x = oracle.randn(batch * k, seed=batch).reshape(batch, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    err = gemv_err(y, x, oracle.dequant_gguf(gtype, data, n, k))
    assert err <= XF16, err


LATENCY8_CASES = [(g, n, k) for g in (oracle.Q4_0, oracle.Q4_1, oracle.Q8_0, oracle.IQ4_XS)
                  for n, k in ((1000, 2048), (700, 3072), (1024, 4096))]
LATENCY8_CASES += [(g, 6150, 1056) for g in (oracle.Q4_0, oracle.Q8_0)]


@pytest.mark.parametrize("gtype,n,k", LATENCY8_CASES, ids=[f"{oracle.NAMES[g]}-{n}x{k}" for g, n, k in LATENCY8_CASES])
@pytest.mark.parametrize("batch,xbf16", [(3, True), (4, False), (6, False), (8, False), (8, True)])
def test_gemv_latency_mode_eight_rows(ctx, gtype, n, k, batch, xbf16):
    """3-8 activation rows on small launches.  At 5-8 rows latency mode (one
    wave per row block with all of a lane's chunks loaded at once) at 1 chunk
    per lane (K = 2048) or 2 (K = 3072, where the lanes past the last chunk add
    zero, 4096, and 1056 in 32 lanes); at 3-4 rows latency mode at 1 chunk,
    the persistent pipeline at 2.  The 8-row kernel of 2 chunks is built for
    256-thread workgroups and must never be launched with 512, including at
    6150 rows, where 256 and 512 threads put the same number of waves on the
    busiest CU."""
    w, data = gguf(gtype, n, k, seed=500 + n + batch)
    x = oracle.randn(batch * k, seed=n + batch).reshape(batch, k)
    if xbf16:
        xb = oracle.f32_to_bf16_bits(x.reshape(-1)).reshape(batch, k)
        xd, x = dev(xb).view(torch.bfloat16), oracle.bf16_bits_to_f32(xb).reshape(batch, k)
    else:
        xd = dev(x)
    y = ctx.qlinear(w, xd).cpu().numpy()
    err = gemv_err(y, x, oracle.dequant_gguf(gtype, data, n, k))
    assert err <= XF16, err


@pytest.mark.parametrize("batch", [1, 4])
def test_gemv_multi_qkv(ctx, batch):
    # q/k/v of Qwen3-0.6B share one activation: one launch, three outputs
    k = 1024
    shapes = [2048, 1024, 1024]
    ws, datas = zip(*[gguf(oracle.Q4_0, n, k, seed=5 + i) for i, n in enumerate(shapes)])
    x = oracle.randn(batch * k, seed=11).reshape(batch, k)
    ys = ctx.qlinear_multi(list(ws), dev(x))
    for y, data, n in zip(ys, datas, shapes):
        err = gemv_err(y.cpu().numpy(), x, oracle.dequant_gguf(oracle.Q4_0, data, n, k))
        assert err <= XF16, err


# 5..16 activation rows on at least 384 tiles of 16 weight rows (K a
# multiple of 256) take the MFMA GEMV (every weight decoded once for all
# rows): ragged rows, task counts needing padding tasks (Q4_0 1280 = 5 tasks
# of 8 blocks, Q6_K 2304 = 9 super-blocks, rows alternating 4- and 2-byte
# alignment), K split over LDS segments (12288: three launches, the later
# ones adding with atomics), bf16 outputs, a weight base 2 bytes past a
# 4-byte boundary; K = 1056 (not whole tasks) stays on the VALU GEMV.
MFMA_CASES = [
    (oracle.Q4_0, 6144, 1024, 5, False, 0), (oracle.Q4_0, 6144, 1024, 16, False, 0),
    (oracle.Q4_0, 6150, 1280, 9, False, 2), (oracle.Q4_0, 6150, 1056, 9, False, 2),
    (oracle.Q4_0, 6144, 4096, 16, True, 0),
    (oracle.Q4_0, 6144, 12288, 7, False, 0), (oracle.Q4_0, 8000, 2048, 12, True, 0),
    (oracle.Q6_K, 6144, 1024, 5, False, 0), (oracle.Q6_K, 6144, 4096, 16, True, 0),
    (oracle.Q6_K, 6150, 2304, 9, False, 2), (oracle.Q6_K, 6144, 12288, 7, False, 0),
    (oracle.Q6_K, 8000, 4096, 12, True, 2),
    # whole tiles per wave (>= 1024 tiles) and few tiles shared by a workgroup's waves
    (oracle.Q4_0, 20480, 1024, 9, False, 0), (oracle.Q6_K, 17000, 1024, 16, True, 2),
    (oracle.Q6_K, 1040, 4096, 16, False, 0), (oracle.Q6_K, 4096, 12288, 16, False, 0),
    (oracle.Q4_0, 4096, 4096, 8, True, 0),
    # 3-4 rows: launches of >= 1024 tiles, and Q4_0 from 384 tiles (split mode)
    (oracle.Q6_K, 17000, 1024, 4, False, 0), (oracle.Q4_0, 20480, 1024, 3, True, 2),
    (oracle.Q4_0, 6144, 4096, 4, False, 0), (oracle.Q4_0, 6150, 4096, 3, True, 2),
    # more rows than one VALU register pass: whole tiles from 128 tiles
    (oracle.Q4_0, 2048, 1024, 12, False, 0), (oracle.Q6_K, 2570, 1024, 8, True, 2),
    # split mode, more tiles than resident workgroups: two 4-wave tile groups per
    # workgroup (an odd tile count leaves one group a recomputed, unstored tile)
    (oracle.Q4_0, 6160, 1024, 16, False, 0), (oracle.Q6_K, 6160, 1024, 16, True, 2),
    (oracle.Q4_0, 4104, 2048, 16, True, 0),
]


@pytest.mark.parametrize("gtype,n,k,batch,ybf16,off", MFMA_CASES,
                         ids=[f"{oracle.NAMES[c[0]]}-{c[1]}x{c[2]}-b{c[3]}{'-bf16' if c[4] else ''}{'-off2' if c[5] else ''}"
                              for c in MFMA_CASES])
def test_gemv_mfma(ctx, gtype, n, k, batch, ybf16, off):
    w, data = gguf(gtype, n, k, seed=n + k + batch, off=off)
    x = oracle.randn(batch * k, seed=batch).reshape(batch, k)
    y = ctx.qlinear(w, dev(x), y_dtype=torch.bfloat16 if ybf16 else torch.float32)
    if ybf16:
        y = oracle.bf16_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16))
    else:
        y = y.cpu().numpy()
    wf = oracle.dequant_gguf(gtype, data, n, k)
    y64, absdot = oracle.linear_f64(x, wf)
    den = np.where(absdot > 0, absdot, 1)
    # f16 weight and activation roundings: 2·2^-11 of Σ|w||x|; bf16 outputs add 2^-8 of |y|
    extra = np.abs(y64) * 2.0 ** -8 / den if ybf16 else 0.0
    err = np.abs(y.astype(np.float64) - y64) / den
    assert np.all(err <= 2.0 ** -10 + 2e-5 + extra), err.max()


# The optional workspace of the MFMA GEMV (K >= 2048, at 9..16 rows or when K
# takes several LDS segments): a prep kernel stages the activations once per
# call and every workgroup copies them into LDS, instead of staging them itself.
# The staged values and the order of the products are the same, so the outputs
# are identical (K segments add atomically, in either order: within 1e-6 of
# Σ|w||x|).  The workspace starts as 0xFF bytes (NaN in f16 and f32), so
# activation rows the prep kernel leaves unstaged (past the batch rounded up
# to 4, 8 or 16) must not reach a stored output.  3 rows take the MFMA GEMV
# on >= 1024 tiles only: 1025 tiles, the oracle on the first 2048 rows.
PRESTAGE_CASES = [c for c in MFMA_CASES if c[2] >= 2048 and (c[3] > 8 or c[2] > 4096)] + [
    (oracle.Q4_0, 16400, 8192, 3, False, 0), (oracle.Q4_K, 6144, 4096, 16, False, 0),
    (oracle.Q5_K, 4096, 12288, 9, False, 0), (oracle.IQ4_XS, 6144, 2048, 12, True, 0),
    # split mode, 16 tasks per segment: each wave's staged operands in registers
    (oracle.Q4_0, 4096, 4096, 16, False, 0), (oracle.Q4_K, 4096, 12288, 16, False, 0),
    (oracle.IQ4_XS, 2048, 4096, 12, True, 0)]


@pytest.mark.parametrize("gtype,n,k,batch,ybf16,off", PRESTAGE_CASES,
                         ids=[f"{oracle.NAMES[c[0]]}-{c[1]}x{c[2]}-b{c[3]}{'-bf16' if c[4] else ''}{'-off2' if c[5] else ''}"
                              for c in PRESTAGE_CASES])
def test_gemv_mfma_workspace_is_optional(ctx, gtype, n, k, batch, ybf16, off):
    w, data = gguf(gtype, n, k, seed=n + k + batch + 1, off=off)
    x = oracle.randn(batch * k, seed=batch + 1).reshape(batch, k)
    ydt = torch.bfloat16 if ybf16 else torch.float32
    need = d.prefill_workspace_bytes([w], batch, d.DTYPE_F32, d.DTYPE_BF16 if ybf16 else d.DTYPE_F32)
    per = 8192 + 64 + (256 if gtype in (oracle.Q4_K, oracle.Q5_K) else 0)
    assert need == (k // 256 * per + 255) // 256 * 256
    assert d.prefill_workspace_bytes([w], 1) == 0
    work = torch.full((need,), 0xFF, dtype=torch.uint8, device="cuda")
    y_pre = ctx.qlinear(w, dev(x), y_dtype=ydt, workspace=work)
    y_own = ctx.qlinear(w, dev(x), y_dtype=ydt, workspace=False)

    def host(y):
        if ybf16:
            return oracle.bf16_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16)).reshape(batch, n)
        return y.cpu().numpy()

    a, b = host(y_pre), host(y_own)
    nc = min(n, 2048)
    wf = oracle.dequant_gguf(gtype, data[:len(data) // n * nc], nc, k)
    y64, absdot = oracle.linear_f64(x, wf)
    den = np.where(absdot > 0, absdot, 1)
    if k <= 4096:  # one K segment: no atomics
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    else:
        assert np.max(np.abs(a[:, :nc].astype(np.float64) - b[:, :nc]) / den) <= 1e-6
    extra = np.abs(y64) * 2.0 ** -8 / den if ybf16 else 0.0
    bound = 2.0 ** -10 + 2e-5 if gtype in (oracle.Q4_0, oracle.Q6_K, oracle.IQ4_XS) else 2e-3
    err = np.abs(a[:, :nc].astype(np.float64) - y64) / den
    assert np.all(err <= bound + extra), err.max()


# bf16 outputs with K in several LDS segments: the MFMA GEMV adds the segments
# into f32 accumulators in the workspace (after the staged activations) and a
# last launch rounds them to bf16; without a workspace the VALU GEMV runs.
BF16_LONG_K = [(oracle.Q4_0, 4096, 12288, 16), (oracle.Q6_K, 2048, 8192, 9), (oracle.Q4_K, 1040, 12288, 12),
               (oracle.IQ4_XS, 3000, 8192, 16)]


@pytest.mark.parametrize("gtype,n,k,batch", BF16_LONG_K,
                         ids=[f"{oracle.NAMES[c[0]]}-{c[1]}x{c[2]}-b{c[3]}" for c in BF16_LONG_K])
def test_gemv_mfma_bf16_outputs_long_k(ctx, gtype, n, k, batch):
    w, data = gguf(gtype, n, k, seed=n + k + batch + 5)
    x = oracle.randn(batch * k, seed=batch + 5).reshape(batch, k)
    per = 8192 + 64 + (256 if gtype in (oracle.Q4_K, oracle.Q5_K) else 0)
    pre = (k // 256 * per + 255) // 256 * 256
    need = d.prefill_workspace_bytes([w], batch, d.DTYPE_F32, d.DTYPE_BF16)
    assert need == pre + (batch * n * 4 + 255) // 256 * 256
    assert d.prefill_workspace_bytes([w], batch, d.DTYPE_F32, d.DTYPE_F32) == pre
    work = torch.full((need,), 0xFF, dtype=torch.uint8, device="cuda")

    def host(y):
        return oracle.bf16_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16)).reshape(batch, n)

    a = host(ctx.qlinear(w, dev(x), y_dtype=torch.bfloat16, workspace=work))
    b = host(ctx.qlinear(w, dev(x), y_dtype=torch.bfloat16, workspace=False))
    f = ctx.qlinear(w, dev(x), y_dtype=torch.float32, workspace=work).cpu().numpy()
    nc = min(n, 1024)
    wf = oracle.dequant_gguf(gtype, data[:len(data) // n * nc], nc, k)
    y64, absdot = oracle.linear_f64(x, wf)
    den = np.where(absdot > 0, absdot, 1)
    bound = 2.0 ** -10 + 2e-5 if gtype in (oracle.Q4_0, oracle.Q6_K, oracle.IQ4_XS) else 2e-3
    for y in (a, b):  # MFMA through the f32 accumulators, and the VALU GEMV
        err = np.abs(y[:, :nc].astype(np.float64) - y64) / den - np.abs(y64) * 2.0 ** -8 / den
        assert np.all(err <= bound), err.max()
    # the MFMA launch's f32 sums rounded once (the segments' atomic order aside)
    assert np.all(np.abs(a[:, :nc].astype(np.float64) - f[:, :nc]) <= np.abs(f[:, :nc]) * 2.0 ** -8 + 1e-6 * den)


def test_gemv_mfma_workspace_checks(ctx):
    """A decode call's optional workspace: NULL runs without it; one that is given
    must be 256-byte aligned and at least the reported size, else
    ERR_INVALID_ARGUMENT before anything is enqueued (the outputs keep their
    sentinel)."""
    n, k, batch = 6144, 4096, 16
    w, data = gguf(oracle.Q4_0, n, k, seed=77)
    x = dev(oracle.randn(batch * k, seed=78).reshape(batch, k))
    need = d.prefill_workspace_bytes([w], batch)
    assert need == (k // 256 * 8256 + 255) // 256 * 256
    buf = torch.empty(need + 512, dtype=torch.uint8, device="cuda")
    y = torch.full((batch, n), 7.0, device="cuda")
    lib = d.library()
    wc = w.c()
    for ptr, nbytes in ((buf.data_ptr(), need - 256), (buf.data_ptr() + 16, need)):
        rc = lib.dyninfer_mi355x_qlinear(ctx._h, ctypes.byref(wc), x.data_ptr(), d.DTYPE_F32, batch, y.data_ptr(),
                                         d.DTYPE_F32, ptr, nbytes, torch.cuda.current_stream().cuda_stream)
        assert rc == d.ERR_INVALID_ARGUMENT, rc
        assert "decode" in lib.dyninfer_mi355x_last_error().decode()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
    rc = lib.dyninfer_mi355x_qlinear(ctx._h, ctypes.byref(wc), x.data_ptr(), d.DTYPE_F32, batch, y.data_ptr(),
                                     d.DTYPE_F32, None, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == d.OK
    y_null = y.cpu().numpy().copy()
    rc = lib.dyninfer_mi355x_qlinear(ctx._h, ctypes.byref(wc), x.data_ptr(), d.DTYPE_F32, batch, y.data_ptr(),
                                     d.DTYPE_F32, buf.data_ptr(), need, torch.cuda.current_stream().cuda_stream)
    assert rc == d.OK
    assert np.array_equal(y.cpu().numpy().view(np.uint32), y_null.view(np.uint32))
    assert gemv_err(y_null, x.cpu().numpy(), oracle.dequant_gguf(oracle.Q4_0, data, n, k)) <= 2.0 ** -10 + 2e-5


@pytest.mark.parametrize("n,k,g,sdtype,batch", [(1024, 3072, 64, oracle.D_F16, 12), (2048, 4096, 128, oracle.D_BF16, 9),
                                               (3072, 2048, 32, oracle.D_F32, 16), (1024, 8192, 64, oracle.D_BF16, 16),
                                               (2048, 4096, 64, oracle.D_F16, 16)])
def test_gemv_mfma_mlx_workspace_is_optional(ctx, n, k, g, sdtype, batch):
    """MLX affine U4 on the MFMA GEMV with its optional workspace and without: identical
    (K = 8192 takes two LDS segments adding into f32 outputs: equal up to the order of
    the atomic adds)."""
    packed, sc, bi = oracle.synth_mlx_u4(n, k, g, sdtype, seed=n + k + g)
    w = d.QWeight(d.ENC_MLX_U4, n, k, dev(packed), dev(sc), dev(bi), g, sdtype)
    xb = oracle.f32_to_bf16_bits(oracle.randn(batch * k, seed=batch + 11)).reshape(batch, k)
    xd = dev(xb).view(torch.bfloat16)
    need = d.prefill_workspace_bytes([w], batch, d.DTYPE_BF16, d.DTYPE_F32)
    assert need == (k // 256 * (8192 + 64) + 255) // 256 * 256
    work = torch.full((need,), 0xFF, dtype=torch.uint8, device="cuda")
    a = ctx.qlinear(w, xd, workspace=work).cpu().numpy()
    b = ctx.qlinear(w, xd, workspace=False).cpu().numpy()
    y64, absdot = oracle.linear_f64(oracle.bf16_bits_to_f32(xb), oracle.dequant_mlx_u4(packed, sc, bi, sdtype, n, k, g))
    if k <= 4096:
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    else:
        assert np.max(np.abs(a.astype(np.float64) - b) / np.where(absdot > 0, absdot, 1)) <= 1e-6
    assert oracle.normalized_error(a, y64, absdot) <= 2.0 ** -10 + 1e-4


def test_gemv_mfma_mlx_bf16_outputs_long_k(ctx):
    """MLX U4 with bf16 in/out and K = 12288 (three LDS segments) at 16 rows: on
    the MFMA GEMV through f32 accumulators in the workspace, and on the VALU GEMV
    without one; both against the oracle."""
    n, k, g, sdtype, batch = 2048, 12288, 64, oracle.D_BF16, 16
    packed, sc, bi = oracle.synth_mlx_u4(n, k, g, sdtype, seed=31)
    w = d.QWeight(d.ENC_MLX_U4, n, k, dev(packed), dev(sc), dev(bi), g, sdtype)
    xb = oracle.f32_to_bf16_bits(oracle.randn(batch * k, seed=32)).reshape(batch, k)
    xd = dev(xb).view(torch.bfloat16)
    pre = (k // 256 * (8192 + 64) + 255) // 256 * 256
    need = d.prefill_workspace_bytes([w], batch, d.DTYPE_BF16, d.DTYPE_BF16)
    assert need == pre + batch * n * 4
    work = torch.full((need,), 0xFF, dtype=torch.uint8, device="cuda")
    y64, absdot = oracle.linear_f64(oracle.bf16_bits_to_f32(xb), oracle.dequant_mlx_u4(packed, sc, bi, sdtype, n, k, g))
    den = np.where(absdot > 0, absdot, 1)
    for ws in (work, False):
        y = ctx.qlinear(w, xd, y_dtype=torch.bfloat16, workspace=ws)
        y = oracle.bf16_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16)).reshape(batch, n)
        err = np.abs(y.astype(np.float64) - y64) / den - np.abs(y64) * 2.0 ** -8 / den
        assert np.all(err <= 2.0 ** -10 + 2e-5), err.max()


@pytest.mark.parametrize("gtype,n,k", [(oracle.Q6_K, 4096, 12288), (oracle.Q4_0, 2048, 16384)],
                         ids=["q6_k-4096x12288", "q4_0-2048x16384"])
@pytest.mark.parametrize("staged", [True, False], ids=["workspace", "no-workspace"])
def test_gemv_mfma_segments_graph_replays(ctx, gtype, n, k, staged):
    """Long K at 16 rows: a kernel zeroes y (the prep kernel that stages the
    activations into the workspace, or a fill kernel), then every K segment adds
    into it atomically.  Captured in a HIP graph and replayed three times with
    eager launches between (over the same workspace): every replay must clear
    and re-accumulate (agreeing with the eager result up to the order of the
    atomic adds) and stay in the f16 bound."""
    w, data = gguf(gtype, n, k, seed=n + k)
    x = dev(oracle.randn(16 * k, seed=5).reshape(16, k))
    need = d.prefill_workspace_bytes([w], 16)
    assert need > 0
    work = torch.empty(need, dtype=torch.uint8, device="cuda") if staged else False
    eager = ctx.qlinear(w, x, workspace=work).cpu().numpy()
    y64, absdot = oracle.linear_f64(x.cpu().numpy(), oracle.dequant_gguf(gtype, data, n, k))
    assert oracle.normalized_error(eager, y64, absdot) <= 2.0 ** -10 + 2e-5
    y = torch.full((16, n), 7.0, device="cuda")
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        ctx.qlinear(w, x, y, stream=st, workspace=work)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            ctx.qlinear(w, x, y, stream=st, workspace=work)
    torch.cuda.synchronize()
    den = np.where(absdot > 0, absdot, 1)
    for _ in range(3):
        y.fill_(7.0)
        ctx.qlinear(w, x * 0.5, workspace=work)  # eager work between the replays
        g.replay()
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.max(np.abs(got.astype(np.float64) - eager) / den) <= 1e-6
    del g


@pytest.mark.parametrize("gtype", [oracle.Q4_0, oracle.Q6_K], ids=oracle.NAMES.get)
def test_gemv_mfma_grouped(ctx, gtype):
    # q/k/v of Qwen3-8B share one activation at batch 16: one MFMA launch, three outputs
    k, batch = 4096, 16
    shapes = [4096, 1024, 1024]
    ws, datas = zip(*[gguf(gtype, n, k, seed=21 + i) for i, n in enumerate(shapes)])
    x = oracle.randn(batch * k, seed=13).reshape(batch, k)
    ys = ctx.qlinear_multi(list(ws), dev(x))
    for y, data, n in zip(ys, datas, shapes):
        err = gemv_err(y.cpu().numpy(), x, oracle.dequant_gguf(gtype, data, n, k))
        assert err <= 2.0 ** -10 + 2e-5, err


@pytest.mark.parametrize("gtype", [oracle.Q4_0, oracle.Q6_K], ids=oracle.NAMES.get)
@pytest.mark.parametrize("lo,hi", [(6, 8), (-30, -28), (-8, 8)])
def test_gemv_mfma_activation_range(ctx, gtype, lo, hi):
    """The MFMA path's per-(row, task) power-of-two scaling over magnitudes f16
    cannot hold unscaled, mixed within a task, and a zero run."""
    n, k, batch = 6144, 2048, 8
    w, data = gguf(gtype, n, k, seed=17 + gtype)
    x = _ranged_x(batch, k, seed=(lo + 100) * 7 + (hi + 100), lo=lo, hi=hi)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    assert np.all(np.isfinite(y))
    err = gemv_err(y, x, oracle.dequant_gguf(gtype, data, n, k))
    assert err <= 2.0 ** -10 + 2e-5, err


@pytest.mark.parametrize("sdtype", [oracle.D_BF16, oracle.D_F16, oracle.D_F32])
@pytest.mark.parametrize("n,k,g", [(1, 64, 64), (1024, 1024, 64), (3072, 1024, 64), (1024, 3072, 64), (96, 512, 32),
                                   (40, 512, 128)])
@pytest.mark.parametrize("batch", [1, 8, 16])
def test_gemv_mlx_bf16_io(ctx, sdtype, n, k, g, batch):
    packed, sc, bi = oracle.synth_mlx_u4(n, k, g, sdtype, seed=n + k + batch)
    w = d.QWeight(d.ENC_MLX_U4, n, k, dev(packed), dev(sc), dev(bi), g, sdtype)
    xb = oracle.f32_to_bf16_bits(oracle.randn(batch * k, seed=batch + 3)).reshape(batch, k)
    x = oracle.bf16_bits_to_f32(xb)
    y = ctx.qlinear(w, dev(xb).view(torch.bfloat16), y_dtype=torch.bfloat16)
    y = y.view(torch.int16).cpu().numpy().view(np.uint16)
    # bf16 output: one RNE rounding of the f32 accumulation (relative 2^-9 of |y|)
    wf = oracle.dequant_mlx_u4(packed, sc, bi, sdtype, n, k, g)
    y64, absdot = oracle.linear_f64(x, wf)
    yf = oracle.bf16_bits_to_f32(y).reshape(batch, n)
    err = np.abs(yf - y64) / np.where(absdot > 0, absdot, 1)
    rounding = np.abs(y64) * 2.0 ** -8 / np.where(absdot > 0, absdot, 1)
    assert np.all(err <= TOL + rounding), err.max()


# MLX affine U4 on the MFMA GEMV (more than 8 rows, or 3-4 on >= 1024 tiles;
# K a multiple of 256):
# whole tiles per wave (>= 1024 tiles, or >= 384 with fewer than 8 tasks),
# split mode, group sizes 32 / 64 / 128, every scale dtype, bf16 and f32
# activations.
MLX_MFMA_CASES = [
    (6144, 1024, 64, oracle.D_BF16, 16, True), (20000, 1024, 64, oracle.D_F16, 12, True),
    (1024, 3072, 64, oracle.D_F16, 12, True), (3072, 2048, 32, oracle.D_F32, 16, True),
    (2048, 4096, 128, oracle.D_BF16, 9, False), (4100, 2048, 64, oracle.D_BF16, 9, False),
    (20000, 1024, 64, oracle.D_BF16, 4, True),
    (4096, 1024, 64, oracle.D_BF16, 16, True),  # 256 tiles, split (two VALU passes at 16 rows)
    (6160, 1024, 64, oracle.D_BF16, 16, True),  # 385 tiles: two 4-wave tile groups per workgroup
]


@pytest.mark.parametrize("n,k,g,sdtype,batch,xbf16", MLX_MFMA_CASES,
                         ids=[f"{c[0]}x{c[1]}-g{c[2]}-s{c[3]}-b{c[4]}{'-bf16io' if c[5] else '-f32io'}"
                              for c in MLX_MFMA_CASES])
def test_gemv_mfma_mlx(ctx, n, k, g, sdtype, batch, xbf16):
    packed, sc, bi = oracle.synth_mlx_u4(n, k, g, sdtype, seed=n + k + g + batch)
    w = d.QWeight(d.ENC_MLX_U4, n, k, dev(packed), dev(sc), dev(bi), g, sdtype)
    wf = oracle.dequant_mlx_u4(packed, sc, bi, sdtype, n, k, g)
    if xbf16:
        xb = oracle.f32_to_bf16_bits(oracle.randn(batch * k, seed=batch + 7)).reshape(batch, k)
        x = oracle.bf16_bits_to_f32(xb)
        y = ctx.qlinear(w, dev(xb).view(torch.bfloat16), y_dtype=torch.bfloat16)
        y = oracle.bf16_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16)).reshape(batch, n)
    else:
        x = oracle.randn(batch * k, seed=batch + 7).reshape(batch, k)
        y = ctx.qlinear(w, dev(x)).cpu().numpy()
    y64, absdot = oracle.linear_f64(x, wf)
    den = np.where(absdot > 0, absdot, 1)
    # f16 weights (one rounding of q·s + b; f32 scales and biases also rounded
    # to f16 first) and activations: 2^-10 plus slack; bf16 outputs 2^-8 of |y|
    extra = np.abs(y64) * 2.0 ** -8 / den if xbf16 else 0.0
    err = np.abs(y.astype(np.float64) - y64) / den
    assert np.all(err <= 2.0 ** -10 + 1e-4 + extra), err.max()


# f32 activations: one row of 2048 and 4096 (64 and 128 groups of 32: two
# staging threads per group), four rows of 2048 (256 groups: one thread)
@pytest.mark.parametrize("batch,k", [(1, 2048), (1, 4096), (4, 2048)])
def test_gemv_mlx_f32_io(ctx, batch, k):
    n, g = 257, 64
    packed, sc, bi = oracle.synth_mlx_u4(n, k, g, oracle.D_BF16, seed=4)
    w = d.QWeight(d.ENC_MLX_U4, n, k, dev(packed), dev(sc), dev(bi), g, oracle.D_BF16)
    x = oracle.randn(batch * k, seed=9).reshape(batch, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    assert gemv_err(y, x, oracle.dequant_mlx_u4(packed, sc, bi, oracle.D_BF16, n, k, g)) <= XF16


# ----------------------------------------------------------------- GEMM (MFMA prefill)
# Shapes that select every launch plan the GEMM's planner picks for Q4_0, Q4_1
# and Q8_0: TM = 2 or 4 activation row blocks and NB = 2 or 3 weight row
# blocks (of 32) per wave, S = 1, 2 or 4 K slices per 4-wave workgroup; plus
# ragged rows and columns, one-chunk K, and chunk counts no split divides.
# (m, n, k) -> (TM, NB, S) for Q4_0:
GEMM_SHAPES = [(17, 130, 64),      # one 64-k chunk: Q4_1/Q8_0 GEMM (Q4_0 takes 16-row GEMV chunks)
               (40, 256, 64),      # one chunk, every type on the GEMM (2, 2, 1)
               (64, 1000, 64),     # one chunk, ragged N
               (17, 256, 1024),    # (2, 2, 4)
               (20, 20000, 256),   # (2, 3, 2)
               (33, 512, 2048),    # (2, 2, 4)
               (50, 20000, 256),   # (2, 3, 2)
               (100, 300, 128),    # (2, 2, 2), two-chunk slices
               (200, 384, 1024),   # ragged last row tile
               (512, 3072, 1024),  # (2, 3, 4) (Qwen3-0.6B gate/up)
               (512, 1024, 3072),  # (2, 2, 4) (down)
               (512, 6144, 1024),
               (768, 2048, 1024),  # (4, 2, 4)
               (768, 3072, 1024),  # (2, 3, 2)
               (1536, 2048, 1024),  # (4, 2, 2)
               (2048, 3072, 1024),  # (4, 2, 1)
               (2000, 3000, 1024),  # ragged rows and columns
               (2048, 64, 8128),   # 127 chunks of 64 k: no K split divides them
               (300, 200, 4032),   # 63 chunks
               (48, 256, 12288),   # activation staging: 24 register slots per lane
               (40, 128, 16384)]   # activation staging: second pass reloads the row
GEMM_TYPES = [oracle.Q4_0, oracle.Q4_1, oracle.Q8_0]


@pytest.mark.parametrize("gtype", GEMM_TYPES, ids=oracle.NAMES.get)
@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
@pytest.mark.parametrize("ybf16", [False, True])
def test_gemm(ctx, gtype, m, n, k, ybf16):
    w, data = gguf(gtype, n, k, seed=m + n + k)
    xb = oracle.f32_to_bf16_bits(oracle.randn(m * k, seed=m)).reshape(m, k)
    x = oracle.bf16_bits_to_f32(xb)
    y = ctx.qlinear(w, dev(xb).view(torch.bfloat16), y_dtype=torch.bfloat16 if ybf16 else torch.float32)
    if ybf16:
        y = oracle.bf16_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16))
    else:
        y = y.cpu().numpy()
    wf = oracle.dequant_gguf(gtype, data, n, k)
    y64, absdot = oracle.linear_f64(x, wf)
    den = np.where(absdot > 0, absdot, 1)
    extra = np.abs(y64) * 2.0 ** -8 / den if ybf16 else 0.0
    err = np.abs(y.astype(np.float64) - y64) / den
    # bf16 activations are exact in f16 after the power-of-two staging: one
    # f16 rounding of each weight, 2^-11, plus f32 accumulation
    assert np.all(err <= 2.0 ** -11 + 1e-5 + extra), err.max()


# Q6_K: K a multiple of 256, the GEMM from 33 rows (shape -> TM, NB, S)
GEMM_SHAPES_Q6K = [(50, 20000, 256),
                   (64, 1000, 512),
                   (100, 300, 512),
                   (200, 384, 1024),
                   (512, 3072, 1024),  # (2, 3, 4)
                   (512, 1024, 3072),  # (2, 2, 4)
                   (512, 6144, 1024),
                   (768, 2048, 1024),  # (2, 2, 2)
                   (768, 3072, 1024),  # (4, 2, 2)
                   (2048, 3072, 1024),  # (4, 2, 1)
                   (2000, 3000, 1024),  # ragged
                   (300, 200, 4096)]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES_Q6K)
@pytest.mark.parametrize("ybf16", [False, True])
def test_gemm_q6_k(ctx, m, n, k, ybf16):
    """Q6_K weights round twice (d·sc, then (q-32)·ds): 2^-10 with exact bf16
    activations."""
    w, data = gguf(oracle.Q6_K, n, k, seed=m + n + k + 1)
    xb = oracle.f32_to_bf16_bits(oracle.randn(m * k, seed=m + 3)).reshape(m, k)
    x = oracle.bf16_bits_to_f32(xb)
    y = ctx.qlinear(w, dev(xb).view(torch.bfloat16), y_dtype=torch.bfloat16 if ybf16 else torch.float32)
    if ybf16:
        y = oracle.bf16_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16))
    else:
        y = y.cpu().numpy()
    y64, absdot = oracle.linear_f64(x, oracle.dequant_gguf(oracle.Q6_K, data, n, k))
    den = np.where(absdot > 0, absdot, 1)
    extra = np.abs(y64) * 2.0 ** -8 / den if ybf16 else 0.0
    err = np.abs(y.astype(np.float64) - y64) / den
    assert np.all(err <= 2.0 ** -10 + 1e-5 + extra), err.max()


@pytest.mark.parametrize("gtype", [oracle.Q4_0, oracle.Q8_0, oracle.Q6_K, oracle.IQ4_XS], ids=oracle.NAMES.get)
@pytest.mark.parametrize("k", [512, 768, 1280])
def test_gemm_four_slices_short_and_odd(ctx, gtype, k):
    """M512 N3072 takes four K slices per workgroup (TM4 S4), so every wave loads
    its own slice's activation fragments into registers two chunks ahead.
    These K give 2, 3 and 5 chunks per slice: the shortest slice, and odd
    counts that end on the unpaired step and re-copy the last chunk's window
    past the end."""
    m, n = 512, 3072
    data = oracle.synth_gguf(gtype, n, k, seed=k + 5)
    enc = {**ENC, oracle.IQ4_XS: d.ENC_IQ4_XS}[gtype]
    w = d.QWeight(enc, n, k, dev(data))
    xb = oracle.f32_to_bf16_bits(oracle.randn(m * k, seed=k)).reshape(m, k)
    x = oracle.bf16_bits_to_f32(xb)
    y = ctx.qlinear(w, dev(xb).view(torch.bfloat16)).cpu().numpy()
    y64, absdot = oracle.linear_f64(x, oracle.dequant_gguf(gtype, data, n, k))
    err = np.abs(y.astype(np.float64) - y64) / np.where(absdot > 0, absdot, 1)
    # one f16 rounding of each weight (Q6_K twice; IQ4_XS kv·RNE_f16(d·(ls-32)) then the
    # product: three halves of 2^-10), exact bf16 activations, f32 accumulation
    bound = {oracle.Q6_K: 2.0 ** -10 + 1e-5, oracle.IQ4_XS: 3 * 2.0 ** -11 + 2e-5}.get(gtype, 2.0 ** -11 + 1e-5)
    assert np.all(err <= bound), err.max()


@pytest.mark.parametrize("gtype", [oracle.Q4_0, oracle.Q8_0, oracle.Q6_K], ids=oracle.NAMES.get)
@pytest.mark.parametrize("m,n,k", [(200, 384, 1024), (512, 3072, 1024), (96, 1040, 2048), (512, 1024, 3072), (130, 2000, 768),
                                   (2048, 3072, 768), (20, 20000, 256), (33, 512, 2048)])
def test_gemm_offset_weights(ctx, gtype, m, n, k):
    # weight blocks starting 2 bytes past a 4-byte boundary (GGUF tensors are
    # only 2-byte aligned); ragged row and column tiles
    w, data = gguf(gtype, n, k, seed=m * 3 + n + k, off=2)
    xb = oracle.f32_to_bf16_bits(oracle.randn(m * k, seed=m + 1)).reshape(m, k)
    x = oracle.bf16_bits_to_f32(xb)
    y = ctx.qlinear(w, dev(xb).view(torch.bfloat16)).cpu().numpy()
    err = gemv_err(y, x, oracle.dequant_gguf(gtype, data, n, k))
    assert err <= (2.0 ** -10 if gtype == oracle.Q6_K else 2.0 ** -11) + 1e-5, err


# MLX affine U4 on the prefill GEMM: every wave tile and K split, group sizes
# 32 / 64 / 128, every scale dtype, scale and bias rows that start 2 bytes into
# a dword (K / group odd with 16-bit scales) and component bases 2 bytes into a
# dword.
GEMM_MLX_CASES = [
    (17, 130, 64, 32, oracle.D_BF16), (40, 256, 64, 64, oracle.D_F16),  # K of one 64-k chunk
    (17, 256, 1024, 64, oracle.D_BF16), (33, 512, 2048, 32, oracle.D_F16), (50, 20000, 256, 128, oracle.D_BF16),
    (100, 300, 1088, 64, oracle.D_BF16), (200, 384, 1024, 32, oracle.D_F32), (512, 3072, 1024, 64, oracle.D_BF16),
    (512, 1024, 3072, 64, oracle.D_F16), (2048, 3072, 1024, 128, oracle.D_BF16), (2000, 3000, 1024, 64, oracle.D_F32),
    (300, 200, 4032, 64, oracle.D_BF16), (768, 2048, 1024, 64, oracle.D_BF16), (1536, 2048, 1024, 32, oracle.D_F16),
]


def _mlx_offset(packed, sc, bi, off):
    """Device copies of the three components, each starting `off` bytes past a
    4-byte boundary (the packed words stay 4-byte aligned)."""
    keep = []
    def place(a, o):
        buf = torch.zeros(a.nbytes + 16, dtype=torch.uint8, device="cuda")
        buf[o:o + a.nbytes] = dev(a.view(np.uint8).reshape(-1))
        keep.append(buf)
        return buf.data_ptr() + o
    return place(packed, 0), place(sc, off), place(bi, off), keep


@pytest.mark.parametrize("m,n,k,g,sdtype", GEMM_MLX_CASES,
                         ids=[f"{c[0]}x{c[1]}x{c[2]}-g{c[3]}-s{c[4]}" for c in GEMM_MLX_CASES])
@pytest.mark.parametrize("off", [0, 2])
def test_gemm_mlx(ctx, m, n, k, g, sdtype, off):
    """w = RNE_f16(q·s + b) (s, b taken to f16: exact for bf16/f16 scales in
    f16's range, one more rounding for f32): 2^-11 with exact bf16
    activations, 2^-10 with f32 scales."""
    if off and sdtype == oracle.D_F32:
        pytest.skip("f32 scales and biases are 4-byte aligned by contract")
    packed, sc, bi = oracle.synth_mlx_u4(n, k, g, sdtype, seed=m + n + k + g)
    if off:
        pw, ps, pb, keep = _mlx_offset(packed, sc, bi, off)
        w = d.QWeight(d.ENC_MLX_U4, n, k, pw, ps, pb, g, sdtype)
        w._keep = keep
    else:
        w = d.QWeight(d.ENC_MLX_U4, n, k, dev(packed), dev(sc), dev(bi), g, sdtype)
    xb = oracle.f32_to_bf16_bits(oracle.randn(m * k, seed=m + 5)).reshape(m, k)
    x = oracle.bf16_bits_to_f32(xb)
    y = ctx.qlinear(w, dev(xb).view(torch.bfloat16)).cpu().numpy()
    err = gemv_err(y, x, oracle.dequant_mlx_u4(packed, sc, bi, sdtype, n, k, g))
    assert err <= (2.0 ** -10 + 1e-4 if sdtype == oracle.D_F32 else 2.0 ** -11 + 1e-5), err


def test_gemm_deterministic(ctx):
    """K-split partial tiles are summed in a fixed slice order: two calls give
    identical bits."""
    m, n, k = 512, 3072, 1024
    w, _ = gguf(oracle.Q4_0, n, k, seed=11)
    x = dev(oracle.randn(m * k, seed=12).reshape(m, k))
    y0 = ctx.qlinear(w, x)
    y1 = ctx.qlinear(w, x)
    assert torch.equal(y0, y1)


def _q4_0_blocks(codes: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    """GGUF Q4_0 bytes from codes [n, k] (0..15) and f16 scale bits [n, k/32]:
    byte l of a block holds k = l (low nibble) and k = 16 + l (high nibble)."""
    n, k = codes.shape
    c = codes.reshape(n, k // 32, 32).astype(np.uint8)
    blk = np.empty((n, k // 32, 18), np.uint8)
    blk[..., 0] = d_bits & 0xFF
    blk[..., 1] = d_bits >> 8
    blk[..., 2:] = c[..., :16] | (c[..., 16:] << 4)
    return blk.reshape(-1)


@pytest.mark.parametrize("m,n,k", [(128, 256, 1024), (512, 3072, 1024), (2048, 3072, 1024)])
def test_gemm_q4_0_bf16_neighbour_bits(ctx, m, n, k):
    """Each activation must be narrowed from its own bf16 alone.  Even k hold
    -3.0 (sign and top exponent bit set: the bits that sit just below an odd
    neighbour's mantissa when a dword is read as f32), odd k hold positive
    values, and only odd k carry weight (codes 15 against 8), so any leak of an
    even activation's bits into its odd neighbour is a one-signed error of up
    to 0.6% of Σ|w||x| in every output."""
    rng = np.random.default_rng(5)
    codes = np.full((n, k), 8, np.int64)
    codes[:, 1::2] = rng.integers(9, 16, size=(n, k // 2))
    d_bits = np.array([oracle.f32_to_f16(v) for v in rng.uniform(0.005, 0.02, 64)], np.uint16)
    data = _q4_0_blocks(codes, d_bits[rng.integers(0, 64, size=(n, k // 32))])
    x = np.empty((m, k), np.float32)
    x[:, 0::2] = -3.0
    x[:, 1::2] = rng.uniform(0.5, 2.0, size=(m, k // 2))
    xb = oracle.f32_to_bf16_bits(x.reshape(-1)).reshape(m, k)
    x = oracle.bf16_bits_to_f32(xb)
    w = d.QWeight(d.ENC_Q4_0, n, k, dev(data))
    y = ctx.qlinear(w, dev(xb).view(torch.bfloat16)).cpu().numpy()
    wf = oracle.dequant_gguf(oracle.Q4_0, data, n, k)
    y64, absdot = oracle.linear_f64(x, wf)
    err = np.abs(y.astype(np.float64) - y64) / absdot
    assert err.max() <= 2.0 ** -11 + 1e-5, err.max()


# ----------------------------------------------------------------- BASELINE full sizes
def _rows_subset(gtype, data, n, k, rows):
    bw, bb = oracle.BLOCK[gtype]
    rb = (k // bw) * bb
    return np.concatenate([data[r * rb:(r + 1) * rb] for r in rows])


@pytest.mark.parametrize("gtype,n,k,batch", [
    (oracle.Q6_K, 151936, 1024, 1),   # Qwen3-0.6B tied lm_head
    (oracle.Q6_K, 151936, 1024, 16),  # the same at batch 16 (MFMA path)
    (oracle.Q6_K, 151936, 4096, 1),   # Qwen3-8B lm_head (510 MB)
    (oracle.Q6_K, 151936, 4096, 4),
    (oracle.Q6_K, 151936, 4096, 16),
    (oracle.Q6_K, 4096, 12288, 4),    # Qwen3-8B down_proj
    (oracle.Q4_0, 12288, 4096, 16),   # Qwen3-8B gate/up
    (oracle.Q8_0, 1024, 3072, 4),     # Qwen3-0.6B down_proj
    (oracle.Q4_0, 1024, 2048, 1),     # Qwen3-0.6B o_proj (K = 2048), every GGUF type
    (oracle.Q4_1, 1024, 2048, 1),
    (oracle.Q8_0, 1024, 2048, 1),
    (oracle.Q6_K, 1024, 2048, 1),
])
def test_gemv_full_size_rows_subset(ctx, gtype, n, k, batch):
    """Full BASELINE shapes: 512 random output rows checked against the oracle,
    plus linearity in x over the whole output (size-independent property)."""
    w, data = gguf(gtype, n, k, seed=n + k)
    x1 = oracle.randn(batch * k, seed=1).reshape(batch, k)
    x2 = oracle.randn(batch * k, seed=2).reshape(batch, k)
    y1 = ctx.qlinear(w, dev(x1)).cpu().numpy()
    rows = np.sort(np.random.default_rng(0).choice(n, size=min(512, n), replace=False))
    sub = _rows_subset(gtype, data, n, k, rows)
    wsub = oracle.dequant_gguf(gtype, sub, len(rows), k)
    # 5..16 rows on Q4_0/Q6_K take the MFMA path: f16 weights add 2^-11
    tol = 2.0 ** -10 + 2e-5 if batch >= 5 and gtype in (oracle.Q4_0, oracle.Q6_K) else XF16
    assert gemv_err(np.ascontiguousarray(y1[:, rows]), x1, wsub) <= tol
    # linearity over every output: y(2 x1 - x2) == 2 y(x1) - y(x2) up to the
    # activation rounding of each of the three products
    x3 = (2 * x1 - x2).astype(np.float32)
    y2 = ctx.qlinear(w, dev(x2)).cpu().numpy()
    y3 = ctx.qlinear(w, dev(x3)).cpu().numpy()
    wabs = ctx.dequant(w).abs()
    bound = sum(c * (torch.abs(dev(xi)) @ wabs.T).cpu().numpy() for c, xi in ((2, x1), (1, x2), (1, x3)))
    assert np.all(np.abs(y3 - (2 * y1 - y2)) <= XF16 * bound + 1e-30)
    # zero activation gives exactly zero
    z = ctx.qlinear(w, torch.zeros((batch, k), dtype=torch.float32, device="cuda"))
    assert torch.count_nonzero(z).item() == 0


@pytest.mark.parametrize("gtype", oracle.GGUF_TYPES, ids=oracle.NAMES.get)
@pytest.mark.parametrize("n,k", [
    (300, 6144),    # one activation row: latency mode, 3 chunks per lane (Q6_K: 3, persistent)
    (300, 8192),    # latency mode, 4 chunks per lane (Q6_K: 2)
    (1024, 12288),  # persistent pipeline, one row per lane group (6 chunks per lane)
    (8448, 12288),  # persistent pipeline, 4 rows per lane group (Q6_K: 2); rows subset checked
                    # (K = 12288: 1024-thread workgroups)
])
def test_gemv_gguf_kernel_paths(ctx, gtype, n, k):
    """Batch-1 shapes that select each GEMV kernel path (latency mode with 3 and
    4 chunks per lane, the persistent pipeline with 1 and 4 rows per lane
    group), against the oracle on up to 512 output rows."""
    w, data = gguf(gtype, n, k, seed=n * 7 + k + gtype)
    x = oracle.randn(k, seed=n + k).reshape(1, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    rows = np.sort(np.random.default_rng(n).choice(n, size=min(512, n), replace=False))
    wsub = oracle.dequant_gguf(gtype, _rows_subset(gtype, data, n, k, rows), len(rows), k)
    assert gemv_err(np.ascontiguousarray(y[:, rows]), x, wsub) <= XF16


@pytest.mark.parametrize("batch", [1, 8, 16])
def test_gemv_mlx_lm_head_full_size(ctx, batch):
    """Qwen3-0.6B tied lm_head in MLX U4 g64 (151936 x 1024):
    512 random output rows against the oracle, linearity and zero input over
    every output."""
    n, k, g = 151936, 1024, 64
    packed, sc, bi = oracle.synth_mlx_u4(n, k, g, oracle.D_BF16, seed=151)
    w = d.QWeight(d.ENC_MLX_U4, n, k, dev(packed), dev(sc), dev(bi), g, oracle.D_BF16)
    x1 = oracle.randn(batch * k, seed=1).reshape(batch, k)
    x2 = oracle.randn(batch * k, seed=2).reshape(batch, k)
    y1 = ctx.qlinear(w, dev(x1)).cpu().numpy()
    rows = np.sort(np.random.default_rng(1).choice(n, size=512, replace=False))
    gpr = k // g
    sub = oracle.dequant_mlx_u4(packed.reshape(n, -1)[rows], sc.reshape(n, -1)[rows], bi.reshape(n, -1)[rows],
                                oracle.D_BF16, len(rows), k, g)
    tol = 2.0 ** -10 + 1e-4 if batch >= 5 else XF16
    assert gpr == 16 and gemv_err(np.ascontiguousarray(y1[:, rows]), x1, sub) <= tol
    x3 = (2 * x1 - x2).astype(np.float32)
    y2 = ctx.qlinear(w, dev(x2)).cpu().numpy()
    y3 = ctx.qlinear(w, dev(x3)).cpu().numpy()
    wabs = ctx.dequant(w).abs()
    bound = sum(c * (torch.abs(dev(xi)) @ wabs.T).cpu().numpy() for c, xi in ((2, x1), (1, x2), (1, x3)))
    assert np.all(np.abs(y3 - (2 * y1 - y2)) <= 2.0 ** -10 * bound + 1e-30)
    z = ctx.qlinear(w, torch.zeros((batch, k), dtype=torch.float32, device="cuda"))
    assert torch.count_nonzero(z).item() == 0


@pytest.mark.parametrize("n,k", [(300, 6144), (300, 8192), (1024, 12288)])
def test_gemv_mlx_kernel_paths(ctx, n, k):
    g = 64
    packed, sc, bi = oracle.synth_mlx_u4(n, k, g, oracle.D_BF16, seed=n + k)
    w = d.QWeight(d.ENC_MLX_U4, n, k, dev(packed), dev(sc), dev(bi), g, oracle.D_BF16)
    x = oracle.randn(k, seed=k).reshape(1, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    assert gemv_err(y, x, oracle.dequant_mlx_u4(packed, sc, bi, oracle.D_BF16, n, k, g)) <= XF16


# ----------------------------------------------------------------- activation range
def _ranged_x(batch, k, seed, lo, hi, zero_block=True):
    """N(0,1) activations scaled by 10^u per 16-element run, u uniform in [lo, hi];
    optionally one all-zero run."""
    rng = np.random.default_rng(seed)
    x = oracle.randn(batch * k, seed=seed).reshape(batch, k).astype(np.float64)
    runs = 10.0 ** rng.uniform(lo, hi, size=(batch, k // 16))
    x *= np.repeat(runs, 16, axis=1)
    if zero_block:
        x[:, 32:64] = 0.0
    return x.astype(np.float32)


@pytest.mark.parametrize("gtype", oracle.GGUF_TYPES, ids=oracle.NAMES.get)
@pytest.mark.parametrize("lo,hi", [(6, 8), (-30, -28), (-8, 8), (-36, 32)])
@pytest.mark.parametrize("batch", [1, 5])
def test_gemv_activation_range(ctx, gtype, lo, hi, batch):
    """Magnitudes f16 cannot hold unscaled (overflow above 65504, flush below
    6e-8), mixed across scale groups, and zero groups: the per-group
    power-of-two scaling keeps the error within the f16 bound.  (Up to 1e32:
    beyond ~1e36 an f32 contraction itself overflows.)"""
    n, k = 96, 1024
    w, data = gguf(gtype, n, k, seed=5 + batch)
    x = _ranged_x(batch, k, seed=(lo + 100) * 7 + (hi + 100) + batch, lo=lo, hi=hi)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    assert np.all(np.isfinite(y))
    err = gemv_err(y, x, oracle.dequant_gguf(gtype, data, n, k))
    assert err <= XF16, err


def test_gemv_mlx_activation_range(ctx):
    n, k, g = 80, 1024, 64
    packed, sc, bi = oracle.synth_mlx_u4(n, k, g, oracle.D_F32, seed=8)
    w = d.QWeight(d.ENC_MLX_U4, n, k, dev(packed), dev(sc), dev(bi), g, oracle.D_F32)
    for lo, hi in [(6, 8), (-30, -28), (-36, 32)]:
        x = _ranged_x(3, k, seed=hi + 100, lo=lo, hi=hi)
        y = ctx.qlinear(w, dev(x)).cpu().numpy()
        err = gemv_err(y, x, oracle.dequant_mlx_u4(packed, sc, bi, oracle.D_F32, n, k, g))
        assert err <= XF16, (lo, hi, err)


@pytest.mark.parametrize("gtype", oracle.GGUF_TYPES, ids=oracle.NAMES.get)
def test_gemv_nonfinite_activation_propagates(ctx, gtype):
    """A NaN or inf activation makes its batch row non-finite (every weight
    touches it) and leaves the other rows exact."""
    n, k = 40, 512
    w, data = gguf(gtype, n, k, seed=3)
    x = oracle.randn(3 * k, seed=4).reshape(3, k)
    x[0, 100] = np.nan
    x[1, 7] = np.inf
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    assert not np.any(np.isfinite(y[0])) and not np.any(np.isfinite(y[1]))
    err = gemv_err(np.ascontiguousarray(y[2:]), np.ascontiguousarray(x[2:]), oracle.dequant_gguf(gtype, data, n, k))
    assert err <= XF16


# ----------------------------------------------------------------- error paths (host-side checks, no kernel runs)
def test_errors_are_reported_not_faulted(ctx):
    data = torch.zeros(18 * 4, dtype=torch.uint8, device="cuda")
    x = torch.zeros((1, 100), dtype=torch.float32, device="cuda")
    with pytest.raises(d.DyninferError) as e:
        ctx.qlinear(d.QWeight(d.ENC_Q4_0, 1, 100, data), x)  # K not a multiple of 32
    assert e.value.code == d.ERR_UNSUPPORTED
    with pytest.raises(d.DyninferError) as e:
        ctx.qlinear(d.QWeight(99, 1, 128, data), x)
    assert e.value.code == d.ERR_UNSUPPORTED
    with pytest.raises(d.DyninferError) as e:
        ctx.qlinear(d.QWeight(d.ENC_Q4_0, 1, 128, data.data_ptr() + 1), torch.zeros((1, 128), device="cuda"))
    assert e.value.code == d.ERR_INVALID_ARGUMENT
