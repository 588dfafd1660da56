"""GPU parity of the quantized embedding gather (through the C ABI).

Bar: bit-exact (every f32 bit pattern) with the oracle's restatement of the
reference's dequant body applied to the gathered rows (gguf_codegen.rs:316-348
slices row `index` of the interleaved bytes and runs the :350-526 body on it;
mlx_affine.rs:628-675 does the same on the three MLX components).  Ids outside
[0, vocab) give a NaN row (the reference leaves them undefined).
"""
import numpy as np
import pytest
import torch

import dyninfer_amd as d
import oracle

pytestmark = pytest.mark.gpu

ENC = {oracle.Q4_0: d.ENC_Q4_0, oracle.Q4_1: d.ENC_Q4_1, oracle.Q8_0: d.ENC_Q8_0, oracle.Q6_K: d.ENC_Q6_K}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def ids_for(vocab, n, seed):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, vocab, n).astype(np.int64)
    ids[:min(n, 2)] = [0, vocab - 1][:min(n, 2)]  # first and last rows
    return ids


def assert_rows_equal(got, ref):
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("gtype", oracle.GGUF_TYPES, ids=oracle.NAMES.get)
@pytest.mark.parametrize("vocab,k,n", [(1, 256, 1), (37, 256, 5), (300, 1024, 64), (64, 4096, 3), (9, 768, 17)])
def test_gguf_gather_bit_exact(ctx, gtype, vocab, k, n):
    data = oracle.synth_gguf(gtype, vocab, k, seed=vocab + k)
    ref = oracle.dequant_gguf(gtype, data, vocab, k)
    ids = ids_for(vocab, n, seed=n)
    out = ctx.embedding(d.QWeight(ENC[gtype], vocab, k, dev(data)), dev(ids)).cpu().numpy()
    assert out.shape == (n, k)
    assert_rows_equal(out, ref[ids])


@pytest.mark.parametrize("gtype", [oracle.Q4_0, oracle.Q8_0, oracle.Q6_K], ids=oracle.NAMES.get)
def test_gguf_gather_two_byte_aligned_base(ctx, gtype):
    vocab, k = 23, 512
    data = oracle.synth_gguf(gtype, vocab, k, seed=5)
    buf = torch.zeros(data.size + 16, dtype=torch.uint8, device="cuda")
    buf[2:2 + data.size] = dev(data)
    ids = ids_for(vocab, 11, seed=3)
    out = ctx.embedding(d.QWeight(ENC[gtype], vocab, k, buf.data_ptr() + 2), dev(ids)).cpu().numpy()
    assert_rows_equal(out, oracle.dequant_gguf(gtype, data, vocab, k)[ids])


@pytest.mark.parametrize("sdtype", [oracle.D_F32, oracle.D_F16, oracle.D_BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_mlx_gather_bit_exact(ctx, sdtype, group):
    vocab, k = 151, 1024
    packed, sc, bi = oracle.synth_mlx_u4(vocab, k, group, sdtype, seed=group)
    ref = oracle.dequant_mlx_u4(packed, sc, bi, sdtype, vocab, k, group)
    dt = {oracle.D_F32: d.DTYPE_F32, oracle.D_F16: d.DTYPE_F16, oracle.D_BF16: d.DTYPE_BF16}[sdtype]
    w = d.QWeight(d.ENC_MLX_U4, vocab, k, dev(packed), dev(sc), dev(bi), group_size=group, scale_dtype=dt)
    ids = ids_for(vocab, 33, seed=group)
    assert_rows_equal(ctx.embedding(w, dev(ids)).cpu().numpy(), ref[ids])


def test_gather_out_of_range_ids_give_nan_rows(ctx):
    vocab, k = 16, 256
    data = oracle.synth_gguf(oracle.Q4_0, vocab, k, seed=1)
    ref = oracle.dequant_gguf(oracle.Q4_0, data, vocab, k)
    ids = np.array([3, -1, 16, 1 << 40, 15], np.int64)
    out = ctx.embedding(d.QWeight(d.ENC_Q4_0, vocab, k, dev(data)), dev(ids)).cpu().numpy()
    assert np.isnan(out[1:4]).all()
    assert_rows_equal(out[[0, 4]], ref[[3, 15]])


def test_gather_empty_and_error_paths(ctx):
    data = oracle.synth_gguf(oracle.Q4_0, 8, 64, seed=2)
    w = d.QWeight(d.ENC_Q4_0, 8, 64, dev(data))
    assert ctx.embedding(w, torch.empty(0, dtype=torch.int64, device="cuda")).shape == (0, 64)
    with pytest.raises(d.DyninferError):
        ctx.embedding(w, torch.zeros(2, dtype=torch.int32, device="cuda"))
    bad = d.QWeight(d.ENC_Q4_0, 8, 48, dev(data))  # K not a multiple of 32
    with pytest.raises(d.DyninferError) as e:
        ctx.embedding(bad, torch.zeros(2, dtype=torch.int64, device="cuda"))
    assert e.value.code == d.ERR_UNSUPPORTED


def test_gather_matches_golden_tiny_embedding(ctx):
    """token_embd of the reference's tiny MLX checkpoint (fixture.rs:236-260), all 32 rows."""
    with np.load("tests/golden/tiny_llama_quant.npz", allow_pickle=False) as z:
        packed, sc, bi, w = z["mlx0.packed"], z["mlx0.scales"], z["mlx0.biases"], z["mlx0.w"]
    qw = d.QWeight(d.ENC_MLX_U4, 32, 64, dev(packed), dev(sc), dev(bi), group_size=64, scale_dtype=d.DTYPE_F32)
    ids = np.arange(31, -1, -1, dtype=np.int64)
    assert_rows_equal(ctx.embedding(qw, dev(ids)).cpu().numpy(), w[ids])
