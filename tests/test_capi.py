"""C-ABI boundary checks that need no GPU: the library loads, exports every
entry point include/*.h declares, and validates arguments host-side exactly
as documented (no compute call is made here)."""
import ctypes
import glob
import os
import re
import threading

import numpy as np
import pytest

import dyninfer_amd as d

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(dyninfer_mi355x_\w+)\s*\(", text))
    return names


def test_every_declared_symbol_is_exported():
    names = declared_symbols()
    assert len(names) >= 11
    lib = d.library()
    for n in names:
        assert hasattr(lib, n), n
    assert names == set(d.EXPORTED_SYMBOLS)


def test_nm_exports_are_c_linkage():
    out = os.popen(f"nm -D --defined-only {d.LIB_PATH}").read()
    for n in declared_symbols():
        assert re.search(rf"\bT {n}$", out, re.M), n


def test_version_and_candidates_json():
    assert b"gfx950" in d.library().dyninfer_mi355x_version()
    assert len(d.candidates()) == 40  # f32 and bf16-activation entries


def w(enc, rows=64, cols=256, data=0x1000, **kw):
    return d.QWeight(enc, rows, cols, data, **kw)


@pytest.mark.parametrize("enc,cols,ok", [
    (d.ENC_Q4_0, 256, True), (d.ENC_Q4_0, 100, False), (d.ENC_Q4_1, 64, True), (d.ENC_Q8_0, 96, True),
    (d.ENC_Q6_K, 256, True), (d.ENC_Q6_K, 384, False), (d.ENC_Q4_K, 512, True), (d.ENC_Q4_K, 288, False),
    (99, 256, False)])
def test_supports_block_multiples(enc, cols, ok):
    assert d.supports(w(enc, cols=cols), 1) == ok


def test_supports_alignment_rules():
    assert d.supports(w(d.ENC_Q4_0, data=0x1002), 1)          # GGUF: 2-byte aligned is enough
    assert not d.supports(w(d.ENC_Q4_0, data=0x1001), 1)
    assert not d.supports(w(d.ENC_Q4_1, data=0x1002), 1)      # Q4_1 blocks are 20 bytes: 4-byte base
    assert not d.supports(w(d.ENC_Q4_K, data=0x1002), 1)      # Q4_K super-blocks are 144 bytes: 4-byte base
    assert d.supports(w(d.ENC_Q4_K, data=0x1004), 1)
    assert not d.supports(w(d.ENC_Q4_0, data=0), 1)           # NULL


def test_supports_mlx_rules():
    good = w(d.ENC_MLX_U4, data=0x1000, scales=0x2000, biases=0x3000, group_size=64, scale_dtype=d.DTYPE_BF16)
    assert d.supports(good, 8, d.DTYPE_BF16, d.DTYPE_BF16)
    assert not d.supports(w(d.ENC_MLX_U4, scales=0x2000, biases=0x3000, group_size=48), 1)  # not a multiple of 32
    assert not d.supports(w(d.ENC_MLX_U4, cols=96, scales=0x2000, biases=0x3000, group_size=64), 1)
    assert not d.supports(w(d.ENC_MLX_U4, scales=0, biases=0x3000, group_size=64), 1)
    assert not d.supports(w(d.ENC_MLX_U4, scales=0x2001, biases=0x3000, group_size=64), 1)
    assert not d.supports(w(d.ENC_MLX_U4, scales=0x2000, biases=0x3000, group_size=64, scale_dtype=7), 1)


def test_supports_dtype_rules():
    # f32 or bf16 activations for every encoding, any row count; f16 activations are not qualified
    for enc in (d.ENC_Q4_0, d.ENC_Q4_1, d.ENC_Q8_0, d.ENC_Q6_K, d.ENC_Q4_K):
        for rows in (1, 4, 16, 17, 512):
            assert d.supports(w(enc), rows, d.DTYPE_BF16, d.DTYPE_BF16)
            assert d.supports(w(enc), rows, d.DTYPE_F32, d.DTYPE_F32)
    assert not d.supports(w(d.ENC_Q4_0), 1, d.DTYPE_F16)
    assert "activations must be f32 or bf16" in d.library().dyninfer_mi355x_last_error().decode()
    assert not d.supports(w(d.ENC_Q4_0), 1, d.DTYPE_F32, d.DTYPE_F16)
    assert not d.supports(w(d.ENC_Q4_0), 0)


@pytest.mark.parametrize("enc,rows,cols,nbytes", [
    (d.ENC_Q4_0, 64, 256, 64 * 8 * 18), (d.ENC_Q4_1, 3, 64, 3 * 2 * 20), (d.ENC_Q8_0, 5, 96, 5 * 3 * 34),
    (d.ENC_Q6_K, 7, 512, 7 * 2 * 210), (d.ENC_Q4_K, 3, 512, 3 * 2 * 144)])
def test_gguf_data_component_byte_total(enc, rows, cols, nbytes):
    """One interleaved data component of N·(K/B)·bytes_per_block bytes
    (gguf_block.rs:124-155): a short or long buffer is E_UNSUPPORTED_ENCODING."""
    assert d.supports(w(enc, rows, cols, data_bytes=nbytes), 1)
    for bad in (nbytes - 1, nbytes + 1, nbytes - 18, 0):
        assert not d.supports(w(enc, rows, cols, data_bytes=bad), 1)
        msg = d.library().dyninfer_mi355x_last_error().decode()
        assert f"requires one interleaved data component of {nbytes} bytes, got {bad} bytes" in msg
    lib = d.library()
    wc = w(enc, rows, cols, data_bytes=nbytes - 2).c()
    rc = lib.dyninfer_mi355x_qlinear(ctypes.c_void_p(1), ctypes.byref(wc), 0x1000, d.DTYPE_F32, 1, 0x2000,
                                     d.DTYPE_F32, None, 0, None)
    assert rc == d.ERR_UNSUPPORTED  # rejected host-side before any launch


def test_mlx_component_byte_lengths():
    """packed N·K/2, scales and biases N·(K/g)·sizeof(scale) (mlx_affine.rs:137-153)."""
    kw = dict(data=0x1000, scales=0x2000, biases=0x3000, group_size=64)
    n, k = 16, 256
    for dt, es in ((d.DTYPE_BF16, 2), (d.DTYPE_F16, 2), (d.DTYPE_F32, 4)):
        g = n * (k // 64) * es
        assert d.supports(w(d.ENC_MLX_U4, n, k, scale_dtype=dt, data_bytes=n * k // 2, scales_bytes=g,
                            biases_bytes=g, **kw), 1)
        for bad in (dict(data_bytes=n * k // 2 - 4), dict(scales_bytes=g - es), dict(biases_bytes=g + es)):
            assert not d.supports(w(d.ENC_MLX_U4, n, k, scale_dtype=dt, **kw, **bad), 1)
            assert "MLX component byte length is invalid" in d.library().dyninfer_mi355x_last_error().decode()


def test_calls_without_context_fail_cleanly():
    lib = d.library()
    wc = w(d.ENC_Q4_0).c()
    rc = lib.dyninfer_mi355x_qlinear(None, ctypes.byref(wc), 0x1000, d.DTYPE_F32, 1, 0x2000, d.DTYPE_F32, None, 0,
                                     None)
    assert rc == d.ERR_INVALID_ARGUMENT
    assert "context" in lib.dyninfer_mi355x_last_error().decode()
    rc = lib.dyninfer_mi355x_dequant(None, ctypes.byref(wc), 0x1000, None)
    assert rc == d.ERR_INVALID_ARGUMENT
    rc = lib.dyninfer_mi355x_embedding(None, ctypes.byref(wc), 0x1000, 1, 0x2000, None)
    assert rc == d.ERR_INVALID_ARGUMENT


def test_open_without_gpu_reports_hip_error():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(d.DyninferError) as e:
        d.Context(0)
    assert e.value.code in (d.ERR_HIP, d.ERR_INVALID_ARGUMENT)


def test_last_error_is_thread_local():
    lib = d.library()
    assert not d.supports(w(d.ENC_Q4_0, cols=100), 1)
    main_msg = lib.dyninfer_mi355x_last_error().decode()
    assert "multiple of the block size" in main_msg
    seen = []
    t = threading.Thread(target=lambda: seen.append(lib.dyninfer_mi355x_last_error().decode()))
    t.start()
    t.join()
    assert seen == [""]
    assert lib.dyninfer_mi355x_last_error().decode() == main_msg


def _ws_bytes(m, k):
    """The documented workspace size: round_up(round_up(m, 32)·k·2, 256) + 4·round_up(m, 256)."""
    return (((m + 31) // 32 * 32 * k * 2 + 255) // 256) * 256 + 4 * ((m + 255) // 256 * 256)


def _decode_ws_bytes(enc, k):
    """The documented optional workspace of a decode call on the MFMA GEMV (K >= 2048):
    K/256 tasks of 8 KiB of f16 fragments and 64 bytes of scales, plus 256 bytes of
    offset sums for Q4_K and Q5_K, rounded up to 256."""
    per = 8192 + 64 + (256 if enc in (d.ENC_Q4_K, d.ENC_Q5_K) else 0)
    return (k // 256 * per + 255) // 256 * 256


@pytest.mark.parametrize("enc,k", [(d.ENC_Q4_0, 1024), (d.ENC_Q4_1, 1024), (d.ENC_Q8_0, 3072), (d.ENC_Q6_K, 4096),
                                   (d.ENC_Q4_K, 4096), (d.ENC_IQ4_XS, 1024)])
def test_prefill_workspace_bytes_follows_the_routing(enc, k):
    """The documented staging size whenever the call runs the prefill GEMM; for GEMV
    calls 0, or the optional staging of 16-row chunks on the MFMA GEMV (these 256
    tiles of 16 weight rows take it at 16 rows, not at 1 or 4; K >= 2048 only)
    (host-only query, no device needed)."""
    ws = [w(enc, 3072, k), w(enc, 1024, k)]
    mfma16 = _decode_ws_bytes(enc, k) if enc in (d.ENC_Q6_K, d.ENC_Q4_K) else 0
    for rows in (1, 4):
        assert d.prefill_workspace_bytes(ws, rows) == 0
    assert d.prefill_workspace_bytes(ws, 16) == mfma16
    chunked = enc in (d.ENC_Q4_0, d.ENC_Q6_K, d.ENC_Q4_K, d.ENC_Q5_K, d.ENC_IQ4_XS) and k <= 8192
    for rows in (17, 32):
        assert d.prefill_workspace_bytes(ws, rows, d.DTYPE_BF16, d.DTYPE_BF16) == (mfma16 if chunked
                                                                                     else _ws_bytes(rows, k))
    for rows in (33, 128, 512, 2048, 3000):
        assert d.prefill_workspace_bytes(ws, rows, d.DTYPE_BF16, d.DTYPE_BF16) == _ws_bytes(rows, k)
        assert d.prefill_workspace_bytes(ws[:1], rows) == _ws_bytes(rows, k)


def test_prefill_workspace_bytes_validates_like_the_call():
    lib = d.library()
    arr = (d._QWeightC * 2)(w(d.ENC_Q4_0, 64, 1024).c(), w(d.ENC_Q4_0, 64, 512).c())
    n = ctypes.c_uint64(7)
    assert lib.dyninfer_mi355x_prefill_workspace_bytes(arr, 2, 64, d.DTYPE_F32, d.DTYPE_F32,
                                                       ctypes.byref(n)) == d.ERR_INVALID_ARGUMENT
    assert "grouped weights must share" in lib.dyninfer_mi355x_last_error().decode() and n.value == 0
    assert lib.dyninfer_mi355x_prefill_workspace_bytes(arr, 1, 64, d.DTYPE_F16, d.DTYPE_F32,
                                                       ctypes.byref(n)) == d.ERR_UNSUPPORTED
    assert lib.dyninfer_mi355x_prefill_workspace_bytes(arr, 1, 0, d.DTYPE_F32, d.DTYPE_F32,
                                                       ctypes.byref(n)) == d.ERR_INVALID_ARGUMENT
    assert lib.dyninfer_mi355x_prefill_workspace_bytes(arr, 5, 64, d.DTYPE_F32, d.DTYPE_F32,
                                                       ctypes.byref(n)) == d.ERR_INVALID_ARGUMENT
    assert lib.dyninfer_mi355x_prefill_workspace_bytes(arr, 1, 64, d.DTYPE_F32, d.DTYPE_F32,
                                                       None) == d.ERR_INVALID_ARGUMENT
    assert lib.dyninfer_mi355x_prefill_workspace_bytes(arr, 1, 64, d.DTYPE_F32, d.DTYPE_F32,
                                                       ctypes.byref(n)) == d.OK
    assert n.value == _ws_bytes(64, 1024)


def test_prefill_rejects_a_missing_or_short_workspace_before_launching():
    """A prefill call checks its workspace host-side (pointer, size, 256-byte alignment)
    and enqueues nothing when it is wrong; the context pointer is only checked for NULL
    here, so no device is touched."""
    lib = d.library()
    wc = w(d.ENC_Q4_0, 64, 1024).c()
    need = _ws_bytes(64, 1024)
    fake = ctypes.c_void_p(1)
    for ptr, nbytes in ((None, 0), (None, need), (0x10000, need - 1), (0x10000 + 128, need)):
        rc = lib.dyninfer_mi355x_qlinear(fake, ctypes.byref(wc), 0x1000, d.DTYPE_F32, 64, 0x2000, d.DTYPE_F32, ptr,
                                         nbytes, None)
        assert rc == d.ERR_INVALID_ARGUMENT, (ptr, nbytes)
        msg = lib.dyninfer_mi355x_last_error().decode()
        assert "workspace" in msg, msg
    assert f"needs a device workspace of {need} bytes" in (
        lib.dyninfer_mi355x_qlinear(fake, ctypes.byref(wc), 0x1000, d.DTYPE_F32, 64, 0x2000, d.DTYPE_F32, None, 0,
                                    None) and lib.dyninfer_mi355x_last_error().decode())


def test_close_of_null_context_is_ok():
    assert d.library().dyninfer_mi355x_close(None) == d.OK


def test_registry_output_buffer_too_small():
    lib = d.library()
    n = ctypes.c_size_t(0)
    buf = ctypes.create_string_buffer(8)
    req = b'{"operation_id":"o","operation":"linear","orientation":"native","mode":"decode"}'
    rc = lib.dyninfer_mi355x_registry_select(None, req, b'{"driver":"hip","architecture":"gfx950","features":[]}',
                                             ctypes.cast(buf, ctypes.c_void_p), 8, ctypes.byref(n))
    assert rc == d.ERR_BUFFER_TOO_SMALL and n.value > 8


def test_group_magic_division_is_exact():
    """The MLX kernels find a k's scale group as floor(k·magic / 2^32) with magic =
    ceil(2^32 / g) (one v_mul_hi_u32, group_magic in kernels.hpp): exact for every
    group size g (a multiple of 32) and every k below 2^16, the GEMV's bound on K."""
    n = np.arange(1 << 16, dtype=np.uint64)
    for g in range(32, 1 << 16, 32):
        magic = np.uint64(((1 << 32) + g - 1) // g)
        assert np.array_equal((n * magic) >> np.uint64(32), n // np.uint64(g)), g
