"""CPU oracle for the quantized weight-matmul path — TEST INFRASTRUCTURE ONLY.

numpy front end over ``oracle/_build/liboracle.so`` (built from ``oracle/oracle.c``
by ``oracle/Makefile``).  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only to check
or to time the CPU baseline; the product path in ``dyninfer_amd`` never does.

Each wrapper names the reference function it restates; the C source carries the
file:line citations.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")

Q4_0, Q4_1, Q8_0, Q6_K = 2, 3, 8, 14
# GGML's K-quants and IQ4_XS: the reference declares their schemas only (gguf_block.rs:183-316)
Q4_K, Q5_K, IQ4_XS = 12, 13, 23
GGUF_TYPES = (Q4_0, Q4_1, Q8_0, Q6_K)
# (weights per block, bytes per block): gguf_codegen.rs:23-38
BLOCK = {Q4_0: (32, 18), Q4_1: (32, 20), Q8_0: (32, 34), Q6_K: (256, 210), Q4_K: (256, 144), Q5_K: (256, 176),
         IQ4_XS: (256, 136)}
D_F32, D_F16, D_BF16 = 0, 1, 2
NAMES = {Q4_0: "q4_0", Q4_1: "q4_1", Q8_0: "q8_0", Q6_K: "q6_k", Q4_K: "q4_k", Q5_K: "q5_k", IQ4_XS: "iq4_xs"}

_lib = None


def build() -> str:
    """Compile the oracle library (gcc, OpenMP).  Returns its path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        P, U64, I, U32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_uint32
        sig = {
            "oracle_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "oracle_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "oracle_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "oracle_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "oracle_fill_f32": (None, [P, U64, U32]),
            "oracle_pack_q4_0": (I, [P, U64, P]),
            "oracle_pack_q4_1": (I, [P, U64, P]),
            "oracle_pack_q8_0": (I, [P, U64, P]),
            "oracle_quantize_affine_u4": (I, [P, U64, U64, U32, P, P, P]),
            "oracle_gguf_block": (I, [I, P, P]),
            "oracle_dequant_gguf": (I, [I, P, U64, U64, P]),
            "oracle_dequant_mlx_u4": (I, [P, P, P, I, U64, U64, U32, P]),
            "oracle_linear_f32": (None, [P, P, U64, U64, U64, P]),
            "oracle_linear_f64": (None, [P, P, U64, U64, U64, P, P]),
            "oracle_qlinear_gguf_f32": (I, [I, P, P, U64, U64, U64, P, I]),
            "oracle_randn_f32": (None, [P, U64, U64, ctypes.c_float]),
            "oracle_synth_gguf": (I, [I, U64, U64, U64, P]),
            "oracle_synth_mlx_u4": (I, [U64, U64, U32, I, U64, P, P, P]),
            "oracle_max_threads": (I, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments (rc={rc})")


# ---------------------------------------------------------------- scalars
def f16_to_f32(bits: int) -> float:
    return lib().oracle_f16_to_f32(bits)


def f32_to_f16(v: float) -> int:
    return lib().oracle_f32_to_f16(v)


def bf16_to_f32(bits: int) -> float:
    return lib().oracle_bf16_to_f32(bits)


def f32_to_bf16(v: float) -> int:
    return lib().oracle_f32_to_bf16(v)


# ---------------------------------------------------------------- fixtures
def fill_f32(n: int, seed: int) -> np.ndarray:
    """LCG fill: q4.rs:212-223 == fixture.rs:92-103."""
    out = np.empty(n, np.float32)
    lib().oracle_fill_f32(_p(out), n, seed)
    return out


def pack(gtype: int, w: np.ndarray) -> np.ndarray:
    """pack_q4_0 / pack_q4_1 / pack_q8_0 (q4.rs:16-96)."""
    w = np.ascontiguousarray(w, np.float32).ravel()
    bw, bb = BLOCK[gtype]
    out = np.zeros(w.size // bw * bb, np.uint8)
    fn = {Q4_0: lib().oracle_pack_q4_0, Q4_1: lib().oracle_pack_q4_1, Q8_0: lib().oracle_pack_q8_0}[gtype]
    _check(fn(_p(w), w.size, _p(out)), "pack")
    return out


def quantize_affine_u4(v: np.ndarray, rows: int, cols: int, group: int):
    """quantize_affine_u4 (fixture.rs:287-317): packed u32, f32 scales, f32 biases."""
    v = np.ascontiguousarray(v, np.float32).ravel()
    packed = np.zeros(rows * cols // 8, np.uint32)
    scales = np.zeros(rows * cols // group, np.float32)
    biases = np.zeros(rows * cols // group, np.float32)
    _check(lib().oracle_quantize_affine_u4(_p(v), rows, cols, group, _p(packed), _p(scales), _p(biases)),
           "quantize_affine_u4")
    return packed, scales, biases


# ---------------------------------------------------------------- dequant
def dequant_gguf(gtype: int, data: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """emit_dequant (gguf_codegen.rs:350-526) -> f32 [rows, cols]."""
    data = np.ascontiguousarray(data, np.uint8)
    bw, bb = BLOCK[gtype]
    assert data.size == rows * (cols // bw) * bb
    out = np.empty((rows, cols), np.float32)
    _check(lib().oracle_dequant_gguf(gtype, _p(data), rows, cols, _p(out)), "dequant_gguf")
    return out


def dequant_mlx_u4(packed, scales, biases, sdtype: int, rows: int, cols: int, group: int) -> np.ndarray:
    """emit_linear_u4's dequant body (mlx_affine.rs:593-598) -> f32 [rows, cols]."""
    packed = np.ascontiguousarray(packed, np.uint32)
    scales = np.ascontiguousarray(scales)
    biases = np.ascontiguousarray(biases)
    out = np.empty((rows, cols), np.float32)
    _check(lib().oracle_dequant_mlx_u4(_p(packed), _p(scales), _p(biases), sdtype, rows, cols, group, _p(out)),
           "dequant_mlx_u4")
    return out


# ---------------------------------------------------------------- contractions
def linear_f32(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """reference.rs:229-242 `linear`: sequential f32, y = x @ w.T."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    batch, k = x.shape
    n = w.shape[0]
    y = np.empty((batch, n), np.float32)
    lib().oracle_linear_f32(_p(x), _p(w), batch, k, n, _p(y))
    return y


def linear_f64(x: np.ndarray, w: np.ndarray):
    """f64 contraction and sum |x||w| per output (the tolerance normaliser)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    batch, k = x.shape
    n = w.shape[0]
    y = np.empty((batch, n), np.float64)
    a = np.empty((batch, n), np.float64)
    lib().oracle_linear_f64(_p(x), _p(w), batch, k, n, _p(y), _p(a))
    return y, a


def qlinear_gguf_f32(gtype: int, data: np.ndarray, x: np.ndarray, rows: int, cols: int, threads: int = 1):
    """CPU baseline: dequant adjacent to an f32 dot (gguf_codegen.rs:268-314)."""
    x = np.ascontiguousarray(x, np.float32)
    batch = x.shape[0]
    y = np.empty((batch, rows), np.float32)
    _check(lib().oracle_qlinear_gguf_f32(gtype, _p(np.ascontiguousarray(data)), _p(x), batch, rows, cols, _p(y),
                                         threads), "qlinear_gguf_f32")
    return y


# ---------------------------------------------------------------- synthetic data
def randn(n: int, seed: int, scale: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().oracle_randn_f32(_p(out), n, seed, scale)
    return out


def synth_gguf(gtype: int, rows: int, cols: int, seed: int) -> np.ndarray:
    bw, bb = BLOCK[gtype]
    out = np.empty(rows * (cols // bw) * bb, np.uint8)
    _check(lib().oracle_synth_gguf(gtype, rows, cols, seed, _p(out)), "synth_gguf")
    return out


def synth_mlx_u4(rows: int, cols: int, group: int, sdtype: int, seed: int):
    packed = np.empty(rows * cols // 8, np.uint32)
    dt = np.float32 if sdtype == D_F32 else np.uint16
    scales = np.empty(rows * (cols // group), dt)
    biases = np.empty(rows * (cols // group), dt)
    _check(lib().oracle_synth_mlx_u4(rows, cols, group, sdtype, seed, _p(packed), _p(scales), _p(biases)),
           "synth_mlx_u4")
    return packed, scales, biases


def max_threads() -> int:
    return lib().oracle_max_threads()


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (NaN quieted)."""
    u = np.ascontiguousarray(v, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def normalized_error(y: np.ndarray, y64: np.ndarray, absdot: np.ndarray) -> float:
    """max over outputs of |y - y_ref| / sum|W||x| (the 2e-3 tolerance metric)."""
    den = np.where(absdot > 0, absdot, 1.0)
    return float(np.max(np.abs(y.astype(np.float64) - y64) / den)) if y.size else 0.0
