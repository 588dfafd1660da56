"""GPU parity for the routes a quantized linear takes beyond single-weight f32
decode, through the C ABI, against the CPU oracle:

  * prefill (rows >= 17) with f32 and bf16 activations for every encoding,
    through qlinear and qlinear_multi: the GGUF encodings run the
    staged-activation MFMA GEMM (x rounded once to f16 after a power-of-two
    scaling per row; Q4_0 and Q6_K from 33 rows, 17 when K > 8192 except Q6_K
    with f32 outputs), MLX and the
    shorter Q4_0 and Q6_K prefills the GEMV kernels over 16-row chunks (the chunks' x and y
    pointer arithmetic is what the 17/32/200/512 row counts check);
  * bf16 activations on the decode GEMV for every encoding;
  * grouped launches (q/k/v, gate/up) for every encoding at the Qwen3-0.6B
    shapes of BASELINE config 1, batches 1, 4 and 16;
  * the GEMM over activation magnitudes f16 cannot hold unscaled;
  * rows whose codes all sit at the zero point (w == 0 exactly, d != 0).

Tolerances, as max over outputs of |y - y64| / sum_k |w||x| (y64 the f64
contraction of the exactly dequantised weights): 2^-10 + 2e-5 (one f16
rounding of each weight and each activation, plus f32 accumulation), within
the 2e-3 north-star tolerance; bf16 outputs add their own rounding, 2^-8 of |y|.
"""
import numpy as np
import pytest
import torch

import dyninfer_amd as d
import oracle

pytestmark = pytest.mark.gpu

ENC = {oracle.Q4_0: d.ENC_Q4_0, oracle.Q4_1: d.ENC_Q4_1, oracle.Q8_0: d.ENC_Q8_0, oracle.Q6_K: d.ENC_Q6_K}
MLX = "mlx"
ALL = list(oracle.GGUF_TYPES) + [MLX]
IDS = {**oracle.NAMES, MLX: "mlx_u4"}
F16X2 = 2.0 ** -10 + 2e-5


def tol(kind):
    """F16X2, plus the Q6_K GEMM's second weight rounding (RNE_f16(d·sc), then
    the product): (2^-10 + 2^-11) + f32 accumulation."""
    return F16X2 + (2.0 ** -11 if kind == oracle.Q6_K else 0.0)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def make(kind, n, k, seed):
    """(QWeight, exactly dequantised f32 [n, k]) for a GGUF type or MLX U4 g64 bf16."""
    if kind == MLX:
        packed, sc, bi = oracle.synth_mlx_u4(n, k, 64, oracle.D_BF16, seed=seed)
        w = d.QWeight(d.ENC_MLX_U4, n, k, dev(packed), dev(sc), dev(bi), 64, d.DTYPE_BF16)
        return w, oracle.dequant_mlx_u4(packed, sc, bi, oracle.D_BF16, n, k, 64)
    data = oracle.synth_gguf(kind, n, k, seed)
    return d.QWeight(ENC[kind], n, k, dev(data)), oracle.dequant_gguf(kind, data, n, k)


def xs(rows, k, seed, bf16):
    """Activations as the device sees them (bf16 bits or f32) and their f32 values."""
    x = oracle.randn(rows * k, seed=seed).reshape(rows, k)
    if not bf16:
        return dev(x), x
    xb = oracle.f32_to_bf16_bits(x.reshape(-1)).reshape(rows, k)
    return dev(xb).view(torch.bfloat16), oracle.bf16_bits_to_f32(xb).reshape(rows, k)


def err_of(y, x, wf, ybf16=False):
    if ybf16:
        y = oracle.bf16_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16)).reshape(y.shape)
    else:
        y = y.cpu().numpy()
    y64, absdot = oracle.linear_f64(x, wf)
    den = np.where(absdot > 0, absdot, 1)
    err = np.abs(y.astype(np.float64) - y64) / den
    if ybf16:
        err = err - np.abs(y64) * 2.0 ** -8 / den
    return float(err.max())


# ----------------------------------------------------------------- prefill, every encoding
@pytest.mark.parametrize("kind", ALL, ids=IDS.get)
@pytest.mark.parametrize("rows", [17, 32, 200, 512])
@pytest.mark.parametrize("xbf16", [False, True], ids=["xf32", "xbf16"])
def test_prefill_rows(ctx, kind, rows, xbf16):
    n, k = 384, 1024
    w, wf = make(kind, n, k, seed=rows + 3)
    xd, x = xs(rows, k, seed=rows, bf16=xbf16)
    assert err_of(ctx.qlinear(w, xd), x, wf) <= tol(kind)


@pytest.mark.parametrize("kind", ALL, ids=IDS.get)
@pytest.mark.parametrize("rows", [17, 24, 33])
@pytest.mark.parametrize("ybf16", [False, True])
def test_prefill_long_k(ctx, kind, rows, ybf16):
    """K above 8192: the GEMM from 17 rows for every encoding (the MFMA GEMV
    would split K over launches), except Q6_K with f32 outputs, which keeps
    16-row MFMA GEMV chunks (their K split over launches) up to 32 rows."""
    n, k = 320, 12288
    w, wf = make(kind, n, k, seed=rows + 70)
    xd, x = xs(rows, k, seed=rows + 1, bf16=False)
    y = ctx.qlinear(w, xd, y_dtype=torch.bfloat16 if ybf16 else torch.float32)
    assert err_of(y, x, wf, ybf16=ybf16) <= tol(kind)


@pytest.mark.parametrize("kind", ALL, ids=IDS.get)
@pytest.mark.parametrize("rows", [17, 200])
def test_prefill_multi(ctx, kind, rows):
    """q/k/v sharing one activation, rows > 16: one staging of x, then one
    GEMM (or GEMV chunk sequence) per weight, outputs of different N."""
    k, shapes = 1024, [512, 256, 256]
    made = [make(kind, n, k, seed=40 + i) for i, n in enumerate(shapes)]
    xd, x = xs(rows, k, seed=9, bf16=False)
    ys = ctx.qlinear_multi([m[0] for m in made], xd)
    for y, (_, wf) in zip(ys, made):
        assert err_of(y, x, wf) <= tol(kind)


@pytest.mark.parametrize("m,n,k", [(17, 256, 1024), (128, 3072, 1024), (512, 3072, 1024), (512, 1024, 3072),
                                   (2048, 3072, 1024), (300, 1000, 768)])
@pytest.mark.parametrize("ybf16", [False, True], ids=["yf32", "ybf16"])
def test_gemm_q4_0_f32_activations(ctx, m, n, k, ybf16):
    """The Q4_0 GEMM with f32 activations (the candidates' advertised input
    type): each kernel path (K-split at M=128, 128x64 and 128x128 tiles),
    ragged tiles."""
    w, wf = make(oracle.Q4_0, n, k, seed=m + n)
    xd, x = xs(m, k, seed=m * 3 + k, bf16=False)
    y = ctx.qlinear(w, xd, y_dtype=torch.bfloat16 if ybf16 else torch.float32)
    assert err_of(y, x, wf, ybf16) <= F16X2


def _ranged_x(rows, k, seed, lo, hi):
    """N(0,1) activations scaled by 10^u per 16-element run, u uniform in
    [lo, hi], and one all-zero run."""
    rng = np.random.default_rng(seed)
    x = oracle.randn(rows * k, seed=seed).reshape(rows, k).astype(np.float64)
    x *= np.repeat(10.0 ** rng.uniform(lo, hi, size=(rows, k // 16)), 16, axis=1)
    x[:, 32:48] = 0.0
    return x.astype(np.float32)


@pytest.mark.parametrize("m", [128, 512, 2048])
@pytest.mark.parametrize("lo,hi", [(6, 8), (-30, -28), (-8, 8), (-36, 32)])
def test_gemm_q4_0_activation_range(ctx, m, lo, hi):
    """Magnitudes f16 cannot hold unscaled (above 65504, below 6e-8) and up to
    68 decades within a row: the per-row power-of-two staging keeps the large
    values at full f16 precision; values more than 2^29 below their row's
    largest become f16 subnormals, each at most 2^-40·max|x| off, a vanishing
    share of sum|w||x| here.  f32 and bf16 activations."""
    n, k = 512, 1024
    w, wf = make(oracle.Q4_0, n, k, seed=m + lo)
    x = _ranged_x(m, k, seed=(lo + 100) * 7 + hi + m, lo=lo, hi=hi)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    assert np.all(np.isfinite(y))
    y64, absdot = oracle.linear_f64(x, wf)
    assert oracle.normalized_error(y, y64, absdot) <= F16X2
    xb = oracle.f32_to_bf16_bits(x.reshape(-1)).reshape(m, k)
    y = ctx.qlinear(w, dev(xb).view(torch.bfloat16))
    assert err_of(y, oracle.bf16_bits_to_f32(xb).reshape(m, k), wf) <= F16X2


def test_gemm_q4_0_nonfinite_row_stays_in_its_row(ctx):
    n, k, m = 256, 1024, 64
    w, wf = make(oracle.Q4_0, n, k, seed=5)
    x = oracle.randn(m * k, seed=6).reshape(m, k)
    x[3, 10] = np.nan
    x[40, 900] = np.inf
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    assert not np.any(np.isfinite(y[3])) and not np.any(np.isfinite(y[40]))
    keep = [r for r in range(m) if r not in (3, 40)]
    y64, absdot = oracle.linear_f64(x[keep], wf)
    assert oracle.normalized_error(y[keep], y64, absdot) <= F16X2


# ----------------------------------------------------------------- decode with bf16 activations
@pytest.mark.parametrize("kind", ALL, ids=IDS.get)
@pytest.mark.parametrize("n,k", [(1024, 1024), (3072, 1024), (1024, 3072), (6144, 4096)])
@pytest.mark.parametrize("batch", [1, 2, 4, 8, 16])
def test_gemv_bf16_activations(ctx, kind, n, k, batch):
    w, wf = make(kind, n, k, seed=n + k + batch)
    xd, x = xs(batch, k, seed=batch + 17, bf16=True)
    assert err_of(ctx.qlinear(w, xd), x, wf) <= F16X2


# ----------------------------------------------------------------- grouped launches, every encoding
@pytest.mark.parametrize("kind", ALL, ids=IDS.get)
@pytest.mark.parametrize("batch", [1, 4, 16])
@pytest.mark.parametrize("group", ["qkv", "gate_up"])
def test_multi_config1_shapes(ctx, kind, batch, group):
    """Qwen3-0.6B q/k/v (2048, 1024, 1024 x 1024) and gate/up (2 x 3072 x 1024)
    in one launch, as BASELINE config 1's step issues them."""
    k = 1024
    shapes = [2048, 1024, 1024] if group == "qkv" else [3072, 3072]
    made = [make(kind, n, k, seed=100 + 7 * i + batch) for i, n in enumerate(shapes)]
    xd, x = xs(batch, k, seed=batch + 5, bf16=kind == MLX)
    ys = ctx.qlinear_multi([m[0] for m in made], xd)
    for y, (_, wf) in zip(ys, made):
        assert err_of(y, x, wf) <= tol(kind)


# ----------------------------------------------------------------- zero-point rows
def _zero_point(kind, n, k, seed):
    """Weights whose first 64 rows dequantise to exactly 0 everywhere, with
    non-zero scales: Q4_0 code 8, Q8_0 code 0, Q6_K q = 32 (ql 0, qh 2), Q4_1
    and MLX code 0 with a zero offset."""
    zr = 64
    if kind == MLX:
        packed, sc, bi = oracle.synth_mlx_u4(n, k, 64, oracle.D_BF16, seed=seed)
        packed.reshape(n, -1)[:zr] = 0
        bi.reshape(n, -1)[:zr] = 0
        wf = oracle.dequant_mlx_u4(packed, sc, bi, oracle.D_BF16, n, k, 64)
        w = d.QWeight(d.ENC_MLX_U4, n, k, dev(packed), dev(sc), dev(bi), 64, d.DTYPE_BF16)
        dmax = np.abs(oracle.bf16_bits_to_f32(sc).reshape(n, -1)).max(axis=1)
    else:
        data = oracle.synth_gguf(kind, n, k, seed)
        bw, bb = oracle.BLOCK[kind]
        blk = data.reshape(n, k // bw, bb)
        if kind == oracle.Q4_0:
            blk[:zr, :, 2:] = 0x88
        elif kind == oracle.Q4_1:
            blk[:zr, :, 2:4] = 0  # m = +0
            blk[:zr, :, 4:] = 0
        elif kind == oracle.Q8_0:
            blk[:zr, :, 2:] = 0
        else:
            blk[:zr, :, 0:128] = 0      # low 4 bits 0
            blk[:zr, :, 128:192] = 0xAA  # high 2 bits 2 in every field
        wf = oracle.dequant_gguf(kind, data, n, k)
        w = d.QWeight(ENC[kind], n, k, dev(data))
        dpos = 208 if kind == oracle.Q6_K else 0
        dbits = blk[:, :, dpos].astype(np.uint16) | (blk[:, :, dpos + 1].astype(np.uint16) << 8)
        dv = np.abs(dbits.view(np.float16).astype(np.float64))
        if kind == oracle.Q6_K:
            dv = dv * 128.0  # |d·sc| <= 128 |d|
        dmax = dv.max(axis=1)
    assert not np.any(wf[:zr]) and np.all(dmax[:zr] > 0)
    return w, wf, zr, dmax


@pytest.mark.parametrize("kind", ALL, ids=IDS.get)
@pytest.mark.parametrize("rows", [1, 4, 16, 200])
def test_zero_point_rows(ctx, kind, rows):
    """Rows that dequantise to exactly 0 give y = 0 in the reference.  Paths
    that decode each weight before multiplying (MFMA GEMV at 5..16 rows on
    large Q4_0/Q6_K/MLX weights, the prefill GEMM) return exactly 0.  The VALU
    GEMV computes sum P·v - C with C = sum coef·v formed in another order, so
    it leaves an f32 rounding residue, bounded in absolute terms by
    2^-8 · sum_k |x_k| · |scale of k's block| (|d·sc| for Q6_K): at most ~56
    roundings (two per v_dot2 if it rounds its product sum and its addition
    separately) of partial sums no larger than 1152·sum|v| per chunk.  x has
    magnitude ~1e3 so that any residue is visible."""
    n, k = 6144, 1024
    w, wf, zr, dmax = _zero_point(kind, n, k, seed=rows + 11)
    x = (oracle.randn(rows * k, seed=rows) * 1000.0).reshape(rows, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    y64, absdot = oracle.linear_f64(x, wf)
    assert oracle.normalized_error(y[:, zr:], y64[:, zr:], absdot[:, zr:]) <= tol(kind)
    bound = 2.0 ** -8 * np.abs(x).sum(axis=1, keepdims=True) * dmax[None, :zr]
    print(f"zero-point residue / bound: {np.max(np.abs(y[:, :zr]) / bound):.3e}")
    assert np.all(np.abs(y[:, :zr]) <= bound)
    # the prefill GEMM (GGUF encodings at 200 rows) and the MFMA GEMV (5..16 rows)
    # multiply exact zeros
    exact = (kind in oracle.GGUF_TYPES and rows >= 33) or (kind == MLX and rows >= 17) or \
        (rows >= 5 and rows <= 16 and kind in (oracle.Q4_0, oracle.Q6_K, MLX))
    if exact:
        assert not np.any(y[:, :zr]), np.abs(y[:, :zr]).max()


SUPER = {oracle.Q4_K: d.ENC_Q4_K, oracle.Q5_K: d.ENC_Q5_K, oracle.IQ4_XS: d.ENC_IQ4_XS}


def _zero_rows_super_block(kind, n, k, seed):
    """Weights whose first 64 rows dequantise to exactly 0 everywhere with
    d != 0.  Q4_K / Q5_K: every code 0 and every sub-block min m = 0, keeping
    the scales (GGML get_scale_min_k4: the mins are scale bytes 4..7 and the
    high nibbles of bytes 8..11, block bytes 8..16).  IQ4_XS: every sub-block
    scale ls = 32 (scales_h bits 0b10, scales_l nibbles 0), since its codebook
    holds no zero."""
    zr = 64
    data = oracle.synth_gguf(kind, n, k, seed)
    bw, bb = oracle.BLOCK[kind]
    blk = data.reshape(n, k // bw, bb)
    if kind == oracle.IQ4_XS:
        blk[:zr, :, 2:4] = 0xAA
        blk[:zr, :, 4:8] = 0
        scale_max = 32.0  # |ls - 32|
    else:
        blk[:zr, :, 8:12] = 0
        blk[:zr, :, 12:16] &= 0x0F
        blk[:zr, :, 16:] = 0  # Q4_K qs; Q5_K qh then qs
        scale_max = 63.0  # sc
    wf = oracle.dequant_gguf(kind, data, n, k)
    dbits = blk[:, :, 0].astype(np.uint16) | (blk[:, :, 1].astype(np.uint16) << 8)
    dmax = (np.abs(dbits.view(np.float16).astype(np.float64)) * scale_max).max(axis=1)
    assert not np.any(wf[:zr]) and np.all(dmax[:zr] > 0)
    return d.QWeight(SUPER[kind], n, k, dev(data)), wf, zr, dmax


@pytest.mark.parametrize("kind", list(SUPER), ids=oracle.NAMES.get)
@pytest.mark.parametrize("rows", [1, 4, 16, 200])
def test_zero_rows_super_block_encodings(ctx, kind, rows):
    """Zero rows of the super-block encodings (see test_zero_point_rows): the
    VALU GEMV leaves at most the same f32 residue, 2^-8 · sum_k |x_k| · max|d·sc|;
    the prefill GEMM decodes exact zeros.  IQ4_XS's group scale d·(ls - 32) is
    itself 0, so every path returns exactly 0."""
    n, k = 6144, 1024
    w, wf, zr, dmax = _zero_rows_super_block(kind, n, k, seed=rows + 23)
    x = (oracle.randn(rows * k, seed=rows + 1) * 1000.0).reshape(rows, k)
    y = ctx.qlinear(w, dev(x)).cpu().numpy()
    y64, absdot = oracle.linear_f64(x, wf)
    assert oracle.normalized_error(y[:, zr:], y64[:, zr:], absdot[:, zr:]) <= 2e-3
    bound = 2.0 ** -8 * np.abs(x).sum(axis=1, keepdims=True) * dmax[None, :zr]
    print(f"zero-row residue / bound: {np.max(np.abs(y[:, :zr]) / bound):.3e}")
    assert np.all(np.abs(y[:, :zr]) <= bound)
    if kind == oracle.IQ4_XS or rows >= 33:
        assert not np.any(y[:, :zr]), np.abs(y[:, :zr]).max()


# ----------------------------------------------------------------- the caller's prefill workspace
HIP_NODE_KERNEL, HIP_NODE_MEM_ALLOC, HIP_NODE_MEM_FREE = 0, 10, 11


def test_prefill_two_threads_two_streams_one_context(ctx):
    """One context, two host threads, each issuing prefill calls of several sizes
    (and a decode call) on a stream of its own with a workspace of its own,
    reused call after call: the context is immutable, so the calls need no
    lock, and every output matches the oracle."""
    import threading
    n, k = 512, 1024
    w, wf = make(oracle.Q4_0, n, k, seed=31)
    plans = {0: [(17, False), (2048, True), (64, False), (4, True)], 1: [(1500, True), (33, False), (3000, True)]}
    inputs = {t: [xs(rows, k, seed=100 + 10 * t + i, bf16=bf) for i, (rows, bf) in enumerate(p)]
              for t, p in plans.items()}
    need = {t: max(d.prefill_workspace_bytes([w], rows, d.DTYPE_F32, d.DTYPE_F32) for rows, _ in p)
            for t, p in plans.items()}
    assert need[0] == d.prefill_workspace_bytes([w], 2048) and need[1] == d.prefill_workspace_bytes([w], 3000)
    work = {t: torch.empty(need[t], dtype=torch.uint8, device="cuda") for t in plans}
    streams = {t: torch.cuda.Stream() for t in plans}
    outs, errors = {t: [] for t in plans}, []
    start = threading.Barrier(len(plans))
    torch.cuda.synchronize()

    def run(t):
        try:
            st = streams[t]
            with torch.cuda.stream(st):
                start.wait()
                for xd, _ in inputs[t]:
                    y = torch.empty((xd.shape[0], n), dtype=torch.float32, device="cuda")
                    ctx.qlinear(w, xd, y, stream=st, workspace=work[t])
                    outs[t].append(y)
            st.synchronize()
        except Exception as e:  # surfaced by the main thread
            errors.append(e)

    threads = [threading.Thread(target=run, args=(t,)) for t in plans]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    torch.cuda.synchronize()
    for t in plans:
        for y, (_, x) in zip(outs[t], inputs[t]):
            assert err_of(y, x, wf) <= F16X2, (t, y.shape)


def test_prefill_graph_capture_replays_without_allocations(ctx, graph_node_types):
    """A prefill captured in a HIP graph with a caller workspace allocated
    beforehand: the graph holds kernel nodes only (no allocation or free
    node), and three replays, with eager prefill calls of other sizes between
    them, each equal the eager result bit for bit."""
    n, k, rows = 768, 1024, 200
    w, wf = make(oracle.Q4_0, n, k, seed=41)
    xd, x = xs(rows, k, seed=42, bf16=False)
    eager = ctx.qlinear(w, xd).cpu().numpy()
    assert err_of(torch.from_numpy(eager), x, wf) <= F16X2
    y = torch.empty((rows, n), device="cuda")
    work = torch.empty(d.prefill_workspace_bytes([w], rows), dtype=torch.uint8, device="cuda")
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        ctx.qlinear(w, xd, y, stream=st, workspace=work)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(g, stream=st):
            ctx.qlinear(w, xd, y, stream=st, workspace=work)
    torch.cuda.synchronize()
    types = graph_node_types(g)
    assert types and all(t == HIP_NODE_KERNEL for t in types), types
    g.instantiate()
    for i in range(3):
        y.fill_(float("nan"))
        other, _ = xs(300 + 100 * i, k, seed=50 + i, bf16=True)
        ctx.qlinear(w, other)  # eager work between the replays (its own workspace)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), eager.view(np.uint32)), i
    del g


def test_context_close_after_prefills_on_two_streams():
    """A second context runs prefills on two streams, then closes with status OK
    (Context.close raises on any other status)."""
    n, k = 256, 1024
    w, wf = make(oracle.Q8_0, n, k, seed=61)
    c2 = d.Context(0)
    cases = []
    for i, st in enumerate((torch.cuda.Stream(), torch.cuda.Stream())):
        xd, x = xs(100 + 50 * i, k, seed=62 + i, bf16=i == 1)
        with torch.cuda.stream(st):
            cases.append((c2.qlinear(w, xd, stream=st), x))
    torch.cuda.synchronize()
    c2.close()
    assert c2._h is None
    for y, x in cases:
        assert err_of(y, x, wf) <= F16X2
