"""Pins of the CPU oracle (oracle/oracle.c) — host only.

Nothing here re-types the oracle's formula: each check comes from an
independent source —
  * numpy / torch conversions (RNE) for f16 and bf16, every f16 bit pattern;
  * the reference's own unit test pack_dequant_roundtrip_rough (q4.rs:317-329);
  * the reference's round-trip formulas (crates/dyninfer-runtime/src/reference.rs:106-193),
    restated in numpy f32, against pack -> bytes -> dequant;
  * hand-built known-answer blocks from the documented layouts
    (docs/quantization/gguf-q4.md:10-20; gguf_codegen.rs lane maps);
  * GGML's loop-form Q6_K decoder (a different formulation of the same
    layout) against the oracle's index-map form;
  * GGML's Q4_K scale/min packer (quantize_row_q4_K's 12-byte packing, the
    inverse of the decoder's unpacking) and the closed form
    f32(d*sc*q - dmin*m) with one rounding, on blocks built from chosen
    scales, mins and codes; Q5_K likewise with the high-bit packer of
    quantize_row_q5_K; IQ4_XS from the scale packer of quantize_row_iq4_xs and
    the codebook's closed form f32(d*(ls-32)*kvalue);
  * a numpy vectorised MLX decoder (LSB-first nibbles) and numpy f64 matmul.
A planted mistake (swapped nibble halves) is shown to fail the known answer.
"""
import numpy as np
import pytest

import oracle


# ---------------------------------------------------------------- f16 / bf16
def test_f16_decode_all_patterns():
    bits = np.arange(65536, dtype=np.uint32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _edge_f32():
    rng = np.random.default_rng(1)
    v = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1035156e-05, 6.0e-05, 5.9604645e-08,
         2.9802322e-08, 2.98e-08, 3.0e-08, 1e-30, np.inf, -np.inf, 0.1, 1 / 3]
    v += list(rng.standard_normal(4000) * 10.0 ** rng.integers(-9, 6, 4000))
    # exact halfway cases between f16 neighbours
    h = rng.integers(0, 0x7BFF, 2000).astype(np.uint16).view(np.float16).astype(np.float64)
    h2 = (h.astype(np.float16).view(np.uint16) + 1).view(np.float16).astype(np.float64)
    v += list(((h + h2) / 2).astype(np.float32))
    return np.array(v, np.float32)


def test_f16_encode_rne_matches_numpy():
    v = _edge_f32()
    got = np.array([oracle.f32_to_f16(float(x)) for x in v], np.uint16)
    ref = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_bf16_rne_matches_torch():
    import torch
    v = _edge_f32()
    got = oracle.f32_to_bf16_bits(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    assert all(oracle.f32_to_bf16(float(x)) == int(r) for x, r in zip(v[:200], ref[:200]))


# ---------------------------------------------------------------- LCG fill (q4.rs:212-223)
@pytest.mark.parametrize("seed", [0, 1, 9, 0xFFFFFFFF])
def test_fill_f32_closed_form(seed):
    n = 3000
    x = seed
    ref = np.empty(n, np.float32)
    for i in range(n):
        x = (x * 1664525 + 1013904223 + i) % 2**32
        ref[i] = np.float32(x % 1000) / np.float32(1000) - np.float32(0.5)
    assert np.array_equal(oracle.fill_f32(n, seed), ref)


# ---------------------------------------------------------------- reference round trips
def rust_round(v32):
    """Rust f32::round: half away from zero (exact in f64 for f32 inputs)."""
    v = v32.astype(np.float64)
    return (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.float32)


def f16_store(v32):
    return v32.astype(np.float16).astype(np.float32)


def rt_q4_0(values):
    """reference.rs:106-127 gguf_q4_0_roundtrip, numpy f32."""
    out = []
    for blk in values.reshape(-1, 32):
        amax = np.float32(np.max(np.abs(blk)))
        scale = amax / np.float32(7) if amax > 0 else np.float32(0)
        stored = f16_store(np.float32(scale))
        inv = np.float32(1) / scale if scale > 0 else np.float32(0)
        q = np.clip(rust_round((blk * inv).astype(np.float32)), -8, 7).astype(np.float32)
        out.append(q * stored)
    return np.concatenate(out)


def rt_q4_1(values):
    """reference.rs:129-154 gguf_q4_1_roundtrip."""
    out = []
    for blk in values.reshape(-1, 32):
        mn, mx = np.float32(blk.min()), np.float32(blk.max())
        scale = (mx - mn) / np.float32(15) if mx > mn else np.float32(0)
        ss, sm = f16_store(np.float32(scale)), f16_store(mn)
        inv = np.float32(1) / scale if scale > 0 else np.float32(0)
        q = np.clip(rust_round(((blk - mn) * inv).astype(np.float32)), 0, 15).astype(np.float32)
        out.append((q * ss).astype(np.float32) + sm)
    return np.concatenate(out)


def rt_q8_0(values):
    """reference.rs:156-175 gguf_q8_0_roundtrip."""
    out = []
    for blk in values.reshape(-1, 32):
        amax = np.float32(np.max(np.abs(blk)))
        scale = amax / np.float32(127) if amax > 0 else np.float32(0)
        stored = f16_store(np.float32(scale))
        inv = np.float32(1) / scale if scale > 0 else np.float32(0)
        q = np.clip(rust_round((blk * inv).astype(np.float32)), -127, 127).astype(np.float32)
        out.append(q * stored)
    return np.concatenate(out)


def rt_u4(values, cols, group=64):
    """reference.rs:177-193 affine_u4_roundtrip (f32 scale/bias, as the tiny fixture)."""
    out = []
    for row in values.reshape(-1, cols):
        for g in row.reshape(-1, group):
            mn, mx = np.float32(g.min()), np.float32(g.max())
            scale = np.maximum((mx - mn) / np.float32(15), np.float32(1e-7)).astype(np.float32)
            q = np.clip(rust_round(((g - mn) / scale).astype(np.float32)), 0, 15).astype(np.float32)
            out.append((q * scale).astype(np.float32) + mn)
    return np.concatenate(out)


def test_pack_dequant_roundtrip_rough():
    """q4.rs:317-329: w = i*0.01 - 0.3, max error < 0.15, 2 blocks of 18 bytes."""
    w = (np.arange(64, dtype=np.float32) * np.float32(0.01) - np.float32(0.3)).astype(np.float32)
    packed = oracle.pack(oracle.Q4_0, w)
    assert packed.size == 2 * 18
    back = oracle.dequant_gguf(oracle.Q4_0, packed, 2, 32).ravel()
    assert np.max(np.abs(w - back)) < 0.15


@pytest.mark.parametrize("gtype,rt", [(oracle.Q4_0, rt_q4_0), (oracle.Q4_1, rt_q4_1), (oracle.Q8_0, rt_q8_0)],
                         ids=["q4_0", "q4_1", "q8_0"])
@pytest.mark.parametrize("seed", [2, 5, 9])
def test_pack_then_dequant_equals_reference_roundtrip(gtype, rt, seed):
    # the tiny fixture's tensors (q4.rs:274-291): LCG fill, 64x64 and 128x64
    w = oracle.fill_f32(128 * 64, seed)
    got = oracle.dequant_gguf(gtype, oracle.pack(gtype, w), 128, 64).ravel()
    assert np.array_equal(got, rt(w))  # value equality (-0 == +0)


def test_quantize_affine_u4_then_dequant_equals_reference_roundtrip():
    rows, cols = 32, 128
    w = oracle.fill_f32(rows * cols, 3)
    packed, sc, bi = oracle.quantize_affine_u4(w, rows, cols, 64)
    got = oracle.dequant_mlx_u4(packed, sc, bi, oracle.D_F32, rows, cols, 64).ravel()
    assert np.array_equal(got, rt_u4(w, cols))


# ---------------------------------------------------------------- known answers
def test_q4_0_known_answer_block():
    """Low nibble of byte l is weight l, high nibble weight 16+l (gguf-q4.md:10-12)."""
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    for l in range(16):
        blk[2 + l] = (l & 0xF) | ((15 - l) << 4)
    w = oracle.dequant_gguf(oracle.Q4_0, blk, 1, 32).ravel()
    ref = np.array([(l - 8) * 0.5 for l in range(16)] + [(7 - l) * 0.5 for l in range(16)], np.float32)
    assert np.array_equal(w, ref)
    # the MLIR body adds +0.0 (gguf_codegen.rs:444): code 8 with a negative scale gives +0, not -0
    blk[0:2] = np.frombuffer(np.float16(-0.5).tobytes(), np.uint8)
    w = oracle.dequant_gguf(oracle.Q4_0, blk, 1, 32).ravel()
    assert w[8] == 0 and not np.signbit(w[8])


def test_planted_nibble_swap_fails_known_answer():
    """A decoder with the nibble halves swapped (a plausible mistake) disagrees."""
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:] = np.arange(16, dtype=np.uint8) | (np.uint8(3) << 4)
    good = oracle.dequant_gguf(oracle.Q4_0, blk, 1, 32).ravel()
    wrong = np.concatenate([(blk[2:] >> 4).astype(np.float32) - 8, (blk[2:] & 15).astype(np.float32) - 8])
    assert not np.array_equal(good, wrong)
    assert good[0] == -8.0 and good[16] == -5.0


def test_q4_1_known_answer_block():
    blk = np.zeros(20, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(-1.0).tobytes(), np.uint8)
    blk[4:] = np.arange(16, dtype=np.uint8) | ((15 - np.arange(16, dtype=np.uint8)) << 4)
    w = oracle.dequant_gguf(oracle.Q4_1, blk, 1, 32).ravel()
    ref = np.concatenate([np.arange(16) * 0.25 - 1.0, (15 - np.arange(16)) * 0.25 - 1.0]).astype(np.float32)
    assert np.array_equal(w, ref)


def test_q8_0_known_answer_block():
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(2.0).tobytes(), np.uint8)
    codes = np.array([-127, -128, -1, 0, 1, 127] + list(range(-13, 13)), np.int8)
    blk[2:] = codes.view(np.uint8)
    w = oracle.dequant_gguf(oracle.Q8_0, blk, 1, 32).ravel()
    assert np.array_equal(w, codes.astype(np.float32) * 2.0)


def ggml_q6_k(blk: np.ndarray) -> np.ndarray:
    """GGML's loop-form Q6_K decoder (one 128-weight half at a time, four
    outputs per l), written independently of the oracle's index maps."""
    d = float(blk[208:210].view(np.float16)[0])
    y = np.zeros(256, np.float64)
    for half in range(2):
        ql = blk[64 * half:64 * half + 64].astype(np.int64)
        qh = blk[128 + 32 * half:128 + 32 * half + 32].astype(np.int64)
        sc = blk[192 + 8 * half:192 + 8 * half + 8].view(np.int8).astype(np.int64)
        for l in range(32):
            is_ = l // 16
            q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32
            q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32
            q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32
            q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32
            y[128 * half + l] = d * sc[is_ + 0] * q1
            y[128 * half + l + 32] = d * sc[is_ + 2] * q2
            y[128 * half + l + 64] = d * sc[is_ + 4] * q3
            y[128 * half + l + 96] = d * sc[is_ + 6] * q4
    return y.astype(np.float32)  # every value is exact in f32


def test_q6_k_index_maps_equal_ggml_loop_form():
    data = oracle.synth_gguf(oracle.Q6_K, 6, 256, 11)
    rng = np.random.default_rng(5)
    extra = rng.integers(0, 256, (4, 210), dtype=np.uint8)  # unrestricted bytes, incl. sc = -128
    extra[:, 208:210] = np.frombuffer(np.float16(0.0123).tobytes(), np.uint8)
    data = np.concatenate([data, extra.ravel()])
    got = oracle.dequant_gguf(oracle.Q6_K, data, 10, 256)
    for r in range(10):
        assert np.array_equal(got[r], ggml_q6_k(data[r * 210:(r + 1) * 210])), r


def test_q6_k_known_answer_extremes():
    blk = np.zeros(210, np.uint8)
    blk[0:128] = 0xFF          # low 4 bits 15 everywhere
    blk[128:192] = 0xFF        # high 2 bits 3 everywhere -> q6 = 63
    blk[192:208] = np.array([127, -128] * 8, np.int8).view(np.uint8)
    blk[208:210] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    w = oracle.dequant_gguf(oracle.Q6_K, blk, 1, 256).ravel()
    sc = np.array([127, -128] * 8, np.float32)
    idx = np.arange(256)
    n, h, p, s = idx // 128, (idx // 64) % 2, (idx // 32) % 2, (idx // 16) % 2
    assert np.array_equal(w, (31 * sc[n * 8 + h * 4 + p * 2 + s] * 0.5).astype(np.float32))


def pack_q4_k_scales(sc, m) -> np.ndarray:
    """GGML's packing of eight 6-bit sub-block scales and mins into a Q4_K
    block's 12 scale bytes (quantize_row_q4_K): the inverse direction of the
    decoder's get_scale_min_k4, written from the packer's side."""
    out = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            out[j] |= sc[j]
            out[j + 4] |= m[j]
        else:
            out[j + 4] |= (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
            out[j - 4] |= (sc[j] >> 4) << 6
            out[j] |= (m[j] >> 4) << 6
    return out


def q4_k_block(d, dmin, sc, m, q) -> np.ndarray:
    """A Q4_K block from its fields: weight 64i + l is the low nibble of
    qs[32i + l] and weight 64i + 32 + l its high nibble."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    blk[4:16] = pack_q4_k_scales(sc, m)
    q = np.asarray(q, np.uint8).reshape(4, 2, 32)
    blk[16:144] = (q[:, 0, :] | (q[:, 1, :] << 4)).ravel()
    return blk


def test_q4_k_closed_form_from_chosen_fields():
    rng = np.random.default_rng(12)
    blocks, want = [], []
    for b in range(24):
        d = np.float16(rng.uniform(1e-4, 0.05) * (1 if b % 5 else 1e-3))  # some subnormal d
        dmin = np.float16(rng.uniform(0, 0.02)) if b % 7 else np.float16(0)
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        if b == 0:
            sc[:], m[:] = 63, 63  # every high bit set
        q = rng.integers(0, 16, 256)
        blocks.append(q4_k_block(d, dmin, sc, m, q))
        j = np.arange(256) // 32
        exact = float(d) * sc[j].astype(np.float64) * q - float(dmin) * m[j].astype(np.float64)
        want.append(exact.astype(np.float32))  # each term exact: one RNE rounding
    got = oracle.dequant_gguf(oracle.Q4_K, np.concatenate(blocks), 24, 256)
    assert np.array_equal(got.view(np.uint32), np.stack(want).view(np.uint32))


def test_q4_k_known_answer_block():
    # sc_j = j + 1, m_j = 2j (j < 8), codes = weight index mod 16, d = 0.5, dmin = 0.25
    sc, m = np.arange(1, 9), 2 * np.arange(8)
    q = np.arange(256) % 16
    blk = q4_k_block(0.5, 0.25, sc, m, q)
    w = oracle.dequant_gguf(oracle.Q4_K, blk, 1, 256).ravel()
    j = np.arange(256) // 32
    assert np.array_equal(w, (0.5 * (j + 1) * q - 0.25 * 2 * j).astype(np.float32))
    # the packed bytes themselves, from the layout: j<4 in the low 6 bits of bytes j / j+4,
    # j>=4 split into a nibble of byte j+4 and the top two bits of bytes j-4 / j
    assert list(blk[4:16]) == [1, 2, 3, 4, 0, 2, 4, 6, 5 | (8 << 4), 6 | (10 << 4), 7 | (12 << 4), 8 | (14 << 4)]


def test_q4_k_planted_scale_min_swap_fails():
    """A decoder that swaps the j >= 4 scale and min sources (a plausible
    slip) disagrees with the closed form on a block built by the packer."""
    rng = np.random.default_rng(3)
    sc, m = rng.integers(16, 64, 8), rng.integers(16, 64, 8)
    q = rng.integers(0, 16, 256)
    blk = q4_k_block(0.01, 0.005, sc, m, q)
    s = blk[4:16].astype(np.int64)
    wrong_sc = [(s[j + 4] >> 4) | ((s[j] >> 6) << 4) for j in range(4, 8)]
    assert wrong_sc != list(sc[4:])
    got = oracle.dequant_gguf(oracle.Q4_K, blk, 1, 256).ravel()
    j = np.arange(256) // 32
    assert np.array_equal(got, (np.float64(np.float16(0.01)) * sc[j] * q - np.float64(np.float16(0.005)) * m[j]).astype(np.float32))


def q5_k_block(d, dmin, sc, m, q) -> np.ndarray:
    """A Q5_K block from its fields, packed as GGML's quantize_row_q5_K does:
    code L of weight 64i + j (j < 32) and 64i + 32 + j go to the low and high
    nibbles of qs[32i + j], their bit 4 to bits 2i and 2i + 1 of qh[j]."""
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    blk[4:16] = pack_q4_k_scales(sc, m)
    q = np.asarray(q, np.int64)
    qh = np.zeros(32, np.int64)
    ql = np.zeros(128, np.int64)
    m1, m2 = 1, 2
    for n in range(0, 256, 64):
        for j in range(32):
            l1, l2 = q[n + j], q[n + j + 32]
            if l1 > 15:
                l1 -= 16
                qh[j] |= m1
            if l2 > 15:
                l2 -= 16
                qh[j] |= m2
            ql[n // 2 + j] = l1 | (l2 << 4)
        m1 <<= 2
        m2 <<= 2
    blk[16:48] = qh
    blk[48:176] = ql
    return blk


def test_q5_k_closed_form_from_chosen_fields():
    rng = np.random.default_rng(15)
    blocks, want = [], []
    for b in range(20):
        d = np.float16(rng.uniform(1e-4, 0.05))
        dmin = np.float16(rng.uniform(0, 0.02)) if b % 6 else np.float16(0)
        sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        if b == 0:
            sc[:], m[:] = 63, 63
        q = rng.integers(0, 32, 256)
        if b == 1:
            q[:] = 31  # every high bit set
        blocks.append(q5_k_block(d, dmin, sc, m, q))
        j = np.arange(256) // 32
        want.append((float(d) * sc[j].astype(np.float64) * q - float(dmin) * m[j].astype(np.float64)).astype(np.float32))
    got = oracle.dequant_gguf(oracle.Q5_K, np.concatenate(blocks), 20, 256)
    assert np.array_equal(got.view(np.uint32), np.stack(want).view(np.uint32))


def test_q5_k_known_answer_block():
    # q = index mod 32: weight 64i + l has bit 4 set for l >= 16 (and its high half for 32 + l >= 48)
    sc, m = np.arange(1, 9), np.arange(8)
    q = np.arange(256) % 32
    blk = q5_k_block(1.0, 0.5, sc, m, q)
    w = oracle.dequant_gguf(oracle.Q5_K, blk, 1, 256).ravel()
    j = np.arange(256) // 32
    assert np.array_equal(w, (1.0 * (j + 1) * q - 0.5 * j).astype(np.float32))
    # qh[l] for l >= 16 has every bit set (both halves of every step), else none
    assert list(blk[16:48]) == [0] * 16 + [255] * 16


KVALUES_IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.int64)


def iq4_xs_block(d, ls, q) -> np.ndarray:
    """An IQ4_XS block from d, the eight 6-bit scales ls and 256 codebook
    indices, packed as GGML's quantize_row_iq4_xs does: scales_l[ib/2] gets
    the low nibble of ls at 4*(ib%2), scales_h its high two bits at 2*ib; the
    sub-block's codes j and 16 + j share qs[16ib + j]."""
    blk = np.zeros(136, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    sh, sl = 0, np.zeros(4, np.int64)
    for ib in range(8):
        sl[ib // 2] |= (int(ls[ib]) & 15) << (4 * (ib % 2))
        sh |= (int(ls[ib]) >> 4) << (2 * ib)
    blk[2:4] = [sh & 0xFF, sh >> 8]
    blk[4:8] = sl
    q = np.asarray(q, np.int64).reshape(8, 2, 16)
    blk[8:136] = (q[:, 0, :] | (q[:, 1, :] << 4)).ravel()
    return blk


def test_iq4_xs_closed_form_from_chosen_fields():
    rng = np.random.default_rng(23)
    blocks, want = [], []
    for b in range(20):
        d = np.float16(rng.uniform(1e-5, 0.01))
        ls = rng.integers(0, 64, 8)
        if b == 0:
            ls[:] = [0, 63, 32, 31, 1, 62, 33, 16]
        q = rng.integers(0, 16, 256)
        blocks.append(iq4_xs_block(d, ls, q))
        ib = np.arange(256) // 32
        want.append((float(d) * (ls[ib] - 32).astype(np.float64) * KVALUES_IQ4NL[q]).astype(np.float32))
    got = oracle.dequant_gguf(oracle.IQ4_XS, np.concatenate(blocks), 20, 256)
    assert np.array_equal(got.view(np.uint32), np.stack(want).view(np.uint32))


def test_iq4_xs_known_answer_block():
    # ls = 33 everywhere (scale d), index = weight mod 16: each 16-weight run spans the codebook
    q = np.arange(256) % 16
    blk = iq4_xs_block(0.25, np.full(8, 33), q)
    assert list(blk[2:8]) == [0xAA, 0xAA, 0x11, 0x11, 0x11, 0x11]  # ls = 0b10_0001 per sub-block
    w = oracle.dequant_gguf(oracle.IQ4_XS, blk, 1, 256).ravel()
    assert np.array_equal(w, (0.25 * KVALUES_IQ4NL[q]).astype(np.float32))
    # the codebook (typed here and in the oracle independently): strictly increasing, -127..113
    assert np.all(np.diff(KVALUES_IQ4NL) > 0) and KVALUES_IQ4NL[0] == -127 and KVALUES_IQ4NL[-1] == 113


def test_mlx_u4_numpy_decoder():
    rows, cols, g = 5, 256, 64
    for sdt in (oracle.D_BF16, oracle.D_F16, oracle.D_F32):
        packed, sc, bi = oracle.synth_mlx_u4(rows, cols, g, sdt, 8)
        q = ((packed[:, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15).reshape(rows, cols).astype(np.float32)
        if sdt == oracle.D_BF16:
            s, b = oracle.bf16_bits_to_f32(sc), oracle.bf16_bits_to_f32(bi)
        elif sdt == oracle.D_F16:
            s, b = sc.view(np.float16).astype(np.float32), bi.view(np.float16).astype(np.float32)
        else:
            s, b = sc, bi
        s = np.repeat(s.reshape(rows, -1), g, axis=1)
        b = np.repeat(b.reshape(rows, -1), g, axis=1)
        ref = (q * s).astype(np.float32) + b
        got = oracle.dequant_mlx_u4(packed, sc, bi, sdt, rows, cols, g)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), sdt


# ---------------------------------------------------------------- contractions
def test_linear_f64_matches_numpy():
    x = oracle.randn(3 * 200, 1).reshape(3, 200)
    w = oracle.randn(50 * 200, 2).reshape(50, 200)
    y, a = oracle.linear_f64(x, w)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12)
    assert np.allclose(a, np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T, rtol=1e-12)


def test_linear_f32_sequential_within_f32_bound():
    x = oracle.randn(2 * 1000, 3).reshape(2, 1000)
    w = oracle.randn(30 * 1000, 4).reshape(30, 1000)
    y = oracle.linear_f32(x, w)
    y64, a = oracle.linear_f64(x, w)
    assert np.all(np.abs(y - y64) <= 1000 * 2.0 ** -24 * a)


@pytest.mark.parametrize("gtype", oracle.GGUF_TYPES + (oracle.Q4_K, oracle.Q5_K, oracle.IQ4_XS), ids=oracle.NAMES.get)
def test_cpu_baseline_contraction_within_tolerance(gtype):
    bw, _ = oracle.BLOCK[gtype]
    n, k = 40, 4 * bw * (2 if bw == 32 else 1)
    data = oracle.synth_gguf(gtype, n, k, 21)
    x = oracle.randn(3 * k, 22).reshape(3, k)
    y = oracle.qlinear_gguf_f32(gtype, data, x, n, k, threads=2)
    y64, a = oracle.linear_f64(x, oracle.dequant_gguf(gtype, data, n, k))
    assert oracle.normalized_error(y, y64, a) <= 1e-5


# ---------------------------------------------------------------- synthetic distributions
def test_synth_distributions():
    q40 = oracle.synth_gguf(oracle.Q4_0, 512, 256, 1).reshape(-1, 18)
    d = q40[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    assert np.all(d >= 0) and 0.005 < d.mean() < 0.011  # |N(0,1)|*0.01 has mean 0.008
    nib = np.concatenate([q40[:, 2:] & 15, q40[:, 2:] >> 4]).ravel()
    hist = np.bincount(nib, minlength=16) / nib.size
    assert np.all(np.abs(hist - 1 / 16) < 0.01)
    q80 = oracle.synth_gguf(oracle.Q8_0, 256, 256, 2).reshape(-1, 34)
    codes = q80[:, 2:].view(np.int8)
    assert codes.min() == -127 and codes.max() == 127
    q6 = oracle.synth_gguf(oracle.Q6_K, 256, 256, 3).reshape(-1, 210)
    sc = q6[:, 192:208].view(np.int8)
    assert sc.min() == -32 and sc.max() == 31
    w = oracle.dequant_gguf(oracle.Q6_K, q6.ravel(), 256, 256)
    q = np.round(w / (np.repeat(sc.astype(np.float32), 16, axis=1).reshape(256, 256) *
                      np.repeat(q6[:, 208:210].copy().view(np.float16).astype(np.float32), 256, axis=0).reshape(256, 256)))
    ok = np.isfinite(q)
    assert q[ok].min() == -32 and q[ok].max() == 31
    q4k = oracle.synth_gguf(oracle.Q4_K, 256, 256, 5).reshape(-1, 144)
    dd = q4k[:, 0:4].copy().view(np.float16).astype(np.float32)
    assert np.all(dd >= 0) and 0.005 < dd[:, 0].mean() < 0.011 and 0.0025 < dd[:, 1].mean() < 0.0055
    q41 = oracle.synth_gguf(oracle.Q4_1, 256, 256, 4).reshape(-1, 20)
    m = q41[:, 2:4].copy().view(np.float16).astype(np.float32)
    assert abs(m.mean()) < 0.002 and 0.007 < m.std() < 0.013


def test_normalized_error_metric():
    y64 = np.array([[1.0, -2.0]])
    a = np.array([[10.0, 4.0]])
    assert oracle.normalized_error(np.array([[1.01, -2.0]], np.float32), y64, a) == pytest.approx(0.001, rel=1e-3)
