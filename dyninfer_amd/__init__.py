"""dyninfer_amd — MI355X (gfx950) quantized weight-matmul path for dyninfer.

Python host mirror of the C ABI in ``include/dyninfer_mi355x.h`` (the drop-in
boundary).  Every compute call goes through ``libdyninfer_mi355x.so``; there
is no fallback of any kind: if the library is missing or the device is not
gfx950, calls raise.  torch is used only to own device memory and streams.

Reference correspondences:
  * ``QWeight`` — a quantized parameter binding: GGUF ``BlockQuantized`` data
    (crates/dyninfer-checkpoint-gguf/src/convention.rs:200-279) or MLX
    ``GroupQuantized`` packed/scales/biases (crates/dyninfer-checkpoint-safetensors/src/mlx.rs:152-261),
    in their exact on-disk bytes;
  * ``Context.qlinear`` — the helper the selected lowering calls for a
    Linear / OutputProjection (gguf_codegen.rs:268-314, mlx_affine.rs:557-626);
  * ``Context.dequant`` — ``emit_dequant`` (gguf_codegen.rs:350-526);
  * ``candidates`` / ``registry_select`` / ``registry_require`` — kernel
    candidates and ``KernelRegistry::{select,require}``
    (crates/dyninfer-kernel-registry/src/lib.rs:302-399).
"""
from __future__ import annotations

import ctypes
import json
import os
from dataclasses import dataclass
from typing import Optional, Sequence

__all__ = [
    "LIB_PATH", "DyninferError", "QWeight", "Context", "library", "candidates", "registry_select",
    "registry_require", "precision_check", "supports", "ENC_Q4_0", "ENC_Q4_1", "ENC_Q8_0", "ENC_Q6_K", "ENC_Q4_K", "ENC_Q5_K", "ENC_IQ4_XS", "ENC_MLX_U4",
    "DTYPE_F32", "DTYPE_F16", "DTYPE_BF16", "block_geometry", "weight_bytes", "prefill_workspace_bytes",
    "ERR_INVALID_ARGUMENT",
    "ERR_UNSUPPORTED", "ERR_HIP", "ERR_DEVICE", "ERR_BUFFER_TOO_SMALL",
]

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libdyninfer_mi355x.so")

OK, ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED, ERR_HIP, ERR_DEVICE, ERR_BUFFER_TOO_SMALL = 0, 1, 2, 3, 4, 5
ENC_Q4_0, ENC_Q4_1, ENC_Q8_0, ENC_Q6_K, ENC_MLX_U4 = 2, 3, 8, 14, 0x1004
# GGML's block_q4_K / block_q5_K / block_iq4_xs: schema-only types in the reference (gguf_block.rs:183-316)
ENC_Q4_K, ENC_Q5_K, ENC_IQ4_XS = 12, 13, 23
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
NOALLOC_SCRATCH_BYTES = 32 << 20  # DYNINFER_MI355X_NOALLOC_SCRATCH_BYTES
ENCODING_IDS = {ENC_Q4_0: "gguf.q4_0", ENC_Q4_1: "gguf.q4_1", ENC_Q8_0: "gguf.q8_0", ENC_Q6_K: "gguf.q6_k",
                ENC_Q4_K: "gguf.q4_k", ENC_Q5_K: "gguf.q5_k", ENC_IQ4_XS: "gguf.iq4_xs", ENC_MLX_U4: "mlx.affine.u4"}
# (weights per block, bytes per block): gguf_codegen.rs:23-38; K-quants: gguf_block.rs:207-226
_GGUF_BLOCK = {ENC_Q4_0: (32, 18), ENC_Q4_1: (32, 20), ENC_Q8_0: (32, 34), ENC_Q6_K: (256, 210),
               ENC_Q4_K: (256, 144), ENC_Q5_K: (256, 176), ENC_IQ4_XS: (256, 136)}

EXPORTED_SYMBOLS = (
    "dyninfer_mi355x_open", "dyninfer_mi355x_close", "dyninfer_mi355x_last_error", "dyninfer_mi355x_qlinear",
    "dyninfer_mi355x_qlinear_multi", "dyninfer_mi355x_dequant", "dyninfer_mi355x_embedding", "dyninfer_mi355x_supports",
    "dyninfer_mi355x_gguf_open", "dyninfer_mi355x_gguf_open_memory", "dyninfer_mi355x_gguf_close",
    "dyninfer_mi355x_gguf_tensor_count", "dyninfer_mi355x_gguf_metadata_json", "dyninfer_mi355x_gguf_tensor",
    "dyninfer_mi355x_gguf_find", "dyninfer_mi355x_gguf_upload", "dyninfer_mi355x_gguf_qweight",
    "dyninfer_mi355x_candidates_json", "dyninfer_mi355x_registry_select", "dyninfer_mi355x_registry_require",
    "dyninfer_mi355x_version", "dyninfer_mi355x_qlinear_multi_noalloc", "dyninfer_mi355x_precision_check",
    "dyninfer_mi355x_safetensors_open", "dyninfer_mi355x_safetensors_open_memory", "dyninfer_mi355x_safetensors_close",
    "dyninfer_mi355x_safetensors_tensor_count", "dyninfer_mi355x_safetensors_metadata_json",
    "dyninfer_mi355x_safetensors_tensor", "dyninfer_mi355x_safetensors_find", "dyninfer_mi355x_safetensors_upload",
    "dyninfer_mi355x_safetensors_mlx_qweight", "dyninfer_mi355x_prefill_workspace_bytes",
)


class DyninferError(RuntimeError):
    """Non-zero status from the C ABI; ``code`` is the status, the message is last_error."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class _QWeightC(ctypes.Structure):
    _fields_ = [
        ("encoding", ctypes.c_uint32), ("group_size", ctypes.c_uint32), ("rows", ctypes.c_uint64),
        ("cols", ctypes.c_uint64), ("data", ctypes.c_void_p), ("scales", ctypes.c_void_p),
        ("biases", ctypes.c_void_p), ("scale_dtype", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
        ("data_bytes", ctypes.c_uint64), ("scales_bytes", ctypes.c_uint64), ("biases_bytes", ctypes.c_uint64),
    ]


_lib: Optional[ctypes.CDLL] = None


class _GgufTensorC(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type_code", ctypes.c_uint32), ("n_dims", ctypes.c_uint32),
                ("dims", ctypes.c_uint64 * 16), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


class _StTensorC(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_char_p), ("n_dims", ctypes.c_uint32),
                ("dims", ctypes.c_uint64 * 16), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


def library() -> ctypes.CDLL:
    """Load the built library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python -m dyninfer_amd.build` "
                          "(the MI355X path has no fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    P, U32, I, SZ = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, ctypes.c_size_t
    W = ctypes.POINTER(_QWeightC)
    sig = {
        "dyninfer_mi355x_open": (I, [I, ctypes.POINTER(P)]),
        "dyninfer_mi355x_close": (I, [P]),
        "dyninfer_mi355x_last_error": (ctypes.c_char_p, []),
        "dyninfer_mi355x_qlinear": (I, [P, W, P, U32, U32, P, U32, P, ctypes.c_uint64, P]),
        "dyninfer_mi355x_qlinear_multi": (I, [P, W, U32, P, U32, U32, ctypes.POINTER(P), U32, P, ctypes.c_uint64, P]),
        "dyninfer_mi355x_prefill_workspace_bytes": (I, [W, U32, U32, U32, U32, ctypes.POINTER(ctypes.c_uint64)]),
        "dyninfer_mi355x_qlinear_multi_noalloc": (I, [P, W, U32, P, U32, U32, ctypes.POINTER(P), U32, P]),
        "dyninfer_mi355x_dequant": (I, [P, W, P, P]),
        "dyninfer_mi355x_embedding": (I, [P, W, P, U32, P, P]),
        "dyninfer_mi355x_gguf_open": (I, [ctypes.c_char_p, ctypes.POINTER(P)]),
        "dyninfer_mi355x_gguf_open_memory": (I, [P, ctypes.c_uint64, ctypes.POINTER(P)]),
        "dyninfer_mi355x_gguf_close": (I, [P]),
        "dyninfer_mi355x_gguf_tensor_count": (ctypes.c_uint64, [P]),
        "dyninfer_mi355x_gguf_metadata_json": (ctypes.c_char_p, [P]),
        "dyninfer_mi355x_gguf_tensor": (I, [P, ctypes.c_uint64, ctypes.POINTER(_GgufTensorC)]),
        "dyninfer_mi355x_gguf_find": (I, [P, ctypes.c_char_p, ctypes.POINTER(_GgufTensorC)]),
        "dyninfer_mi355x_gguf_upload": (I, [P, ctypes.c_char_p, P, ctypes.c_uint64, P]),
        "dyninfer_mi355x_gguf_qweight": (I, [P, ctypes.c_char_p, P, W]),
        "dyninfer_mi355x_supports": (I, [W, U32, U32, U32]),
        "dyninfer_mi355x_candidates_json": (ctypes.c_char_p, []),
        "dyninfer_mi355x_registry_select": (I, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, P, SZ,
                                                ctypes.POINTER(SZ)]),
        "dyninfer_mi355x_registry_require": (I, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, P, SZ,
                                                 ctypes.POINTER(SZ)]),
        "dyninfer_mi355x_version": (ctypes.c_char_p, []),
        "dyninfer_mi355x_precision_check": (I, [ctypes.c_char_p, ctypes.c_char_p]),
        "dyninfer_mi355x_safetensors_open": (I, [ctypes.c_char_p, ctypes.POINTER(P)]),
        "dyninfer_mi355x_safetensors_open_memory": (I, [P, ctypes.c_uint64, ctypes.c_char_p, ctypes.POINTER(P)]),
        "dyninfer_mi355x_safetensors_close": (I, [P]),
        "dyninfer_mi355x_safetensors_tensor_count": (ctypes.c_uint64, [P]),
        "dyninfer_mi355x_safetensors_metadata_json": (ctypes.c_char_p, [P]),
        "dyninfer_mi355x_safetensors_tensor": (I, [P, ctypes.c_uint64, ctypes.POINTER(_StTensorC)]),
        "dyninfer_mi355x_safetensors_find": (I, [P, ctypes.c_char_p, ctypes.POINTER(_StTensorC)]),
        "dyninfer_mi355x_safetensors_upload": (I, [P, ctypes.c_char_p, P, ctypes.c_uint64, P]),
        "dyninfer_mi355x_safetensors_mlx_qweight": (I, [P, ctypes.c_char_p, P, P, P, W]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _check(rc: int) -> None:
    if rc != OK:
        raise DyninferError(rc, library().dyninfer_mi355x_last_error().decode())


def block_geometry(encoding: int):
    """(weights per block, bytes per block) of a GGUF encoding."""
    return _GGUF_BLOCK[encoding]


def weight_bytes(encoding: int, rows: int, cols: int, group_size: int = 64, scale_bytes: int = 2) -> int:
    """On-disk weight bytes: the algorithmic HBM traffic of one GEMV pass."""
    if encoding in _GGUF_BLOCK:
        bw, bb = _GGUF_BLOCK[encoding]
        return rows * (cols // bw) * bb
    return rows * cols // 2 + 2 * rows * (cols // group_size) * scale_bytes


def _ptr(t) -> Optional[int]:
    if t is None:
        return None
    return t.data_ptr() if hasattr(t, "data_ptr") else int(t)


def _nbytes(t) -> Optional[int]:
    """Byte length of a tensor (None for a raw address)."""
    if t is None or not hasattr(t, "data_ptr"):
        return None
    return t.numel() * t.element_size()


@dataclass
class QWeight:
    """A quantized weight [rows = N out, cols = K in] in its on-disk bytes.

    GGUF: ``data`` holds the interleaved blocks.  MLX U4: ``data`` = packed u32
    words, ``scales``/``biases`` = [N, K/group] of ``scale_dtype``.  Tensors (or
    raw device addresses) must stay alive while kernels use them.

    Component byte lengths (``*_bytes``) default to the tensors' own sizes, so
    the C ABI checks the buffers actually bound against the encoding's byte
    totals; for a raw address they default to the encoding's expected length.
    """
    encoding: int
    rows: int
    cols: int
    data: object
    scales: object = None
    biases: object = None
    group_size: int = 0
    scale_dtype: int = DTYPE_BF16
    data_bytes: Optional[int] = None
    scales_bytes: Optional[int] = None
    biases_bytes: Optional[int] = None

    def _expected(self):
        if self.encoding in _GGUF_BLOCK:
            bw, bb = _GGUF_BLOCK[self.encoding]
            return self.rows * (self.cols // bw) * bb, 0, 0
        es = 4 if self.scale_dtype == DTYPE_F32 else 2
        g = self.rows * (self.cols // self.group_size) * es if self.group_size else 0
        return self.rows * self.cols // 2, g, g

    def c(self) -> _QWeightC:
        ed, es, eb = self._expected()
        pick = lambda given, t, exp: given if given is not None else (_nbytes(t) if _nbytes(t) is not None else exp)
        return _QWeightC(self.encoding, self.group_size, self.rows, self.cols, _ptr(self.data), _ptr(self.scales),
                         _ptr(self.biases), self.scale_dtype, 0, pick(self.data_bytes, self.data, ed),
                         pick(self.scales_bytes, self.scales, es), pick(self.biases_bytes, self.biases, eb))

    @property
    def nbytes(self) -> int:
        sb = 4 if self.scale_dtype == DTYPE_F32 else 2
        return weight_bytes(self.encoding, self.rows, self.cols, self.group_size or 64, sb)


def _dtype_code(t) -> int:
    import torch
    if t.dtype == torch.float32:
        return DTYPE_F32
    if t.dtype == torch.bfloat16:
        return DTYPE_BF16
    if t.dtype == torch.float16:
        return DTYPE_F16
    raise TypeError(f"unsupported dtype {t.dtype}")


def supports(w: QWeight, rows: int, x_dtype: int = DTYPE_F32, y_dtype: int = DTYPE_F32) -> bool:
    wc = w.c()
    return bool(library().dyninfer_mi355x_supports(ctypes.byref(wc), rows, x_dtype, y_dtype))


def prefill_workspace_bytes(ws: Sequence[QWeight], rows: int, x_dtype: int = DTYPE_F32,
                            y_dtype: int = DTYPE_F32) -> int:
    """Device workspace bytes of a qlinear / qlinear_multi call over ``ws`` with these rows
    and dtypes (dyninfer_mi355x_prefill_workspace_bytes): required by a call that runs the
    prefill GEMM, optional for a decode call on the MFMA GEMV (which then stages its
    activations once per call), 0 for every other call."""
    arr = (_QWeightC * len(ws))(*[w.c() for w in ws])
    n = ctypes.c_uint64(0)
    _check(library().dyninfer_mi355x_prefill_workspace_bytes(arr, len(ws), rows, x_dtype, y_dtype, ctypes.byref(n)))
    return n.value


class Context:
    """An open library context on one gfx950 device (dyninfer_mi355x_open/close)."""

    def __init__(self, device: int = 0):
        self._lib = library()
        self.device = device
        h = ctypes.c_void_p()
        _check(self._lib.dyninfer_mi355x_open(device, ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        """dyninfer_mi355x_close; raises DyninferError on a non-zero status."""
        if getattr(self, "_h", None):
            h, self._h = self._h, None
            _check(self._lib.dyninfer_mi355x_close(h))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _stream(stream) -> Optional[int]:
        if stream is None:
            import torch
            return torch.cuda.current_stream().cuda_stream
        return stream if isinstance(stream, int) else stream.cuda_stream

    def _workspace(self, ws, x, rows: int, ydt: int, stream, workspace):
        """(pointer, bytes, keep-alive) of the call's device workspace: the caller's
        ``workspace`` tensor, or a new torch allocation of the size the library asks
        for (torch's caching allocator, tied to the launch stream), or none (also when
        ``workspace`` is False: a decode call then runs without its optional one)."""
        import torch
        if workspace is False:
            return None, 0, None
        need = prefill_workspace_bytes(ws, rows, _dtype_code(x), ydt)
        if need == 0:
            return None, 0, None
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
            if stream is not None:
                st = stream if isinstance(stream, torch.cuda.Stream) else torch.cuda.ExternalStream(int(stream))
                workspace.record_stream(st)  # not reused before the call's work on `stream` completes
        return workspace.data_ptr(), workspace.numel() * workspace.element_size(), workspace

    def qlinear(self, w: QWeight, x, y=None, y_dtype=None, stream=None, workspace=None):
        """y = x · Wᵀ (f32 accumulation).  x: [rows, K] f32 or bf16 device tensor.
        workspace: a device tensor of at least prefill_workspace_bytes([w], rows, …)
        bytes (one is allocated through torch when omitted and that size is not 0), or
        False for none (decode calls only)."""
        import torch
        rows = x.shape[0] if x.dim() == 2 else 1
        if y is None:
            y = torch.empty((rows, w.rows), dtype=y_dtype or torch.float32, device=x.device)
        wp, wn, _keep = self._workspace([w], x, rows, _dtype_code(y), stream, workspace)
        wc = w.c()
        _check(self._lib.dyninfer_mi355x_qlinear(self._h, ctypes.byref(wc), x.data_ptr(), _dtype_code(x), rows,
                                                 y.data_ptr(), _dtype_code(y), wp, wn, self._stream(stream)))
        return y

    def qlinear_multi(self, ws: Sequence[QWeight], x, ys=None, y_dtype=None, stream=None, noalloc=False,
                      workspace=None):
        """One launch for several weights sharing activation x (same encoding and K).
        noalloc: dyninfer_mi355x_qlinear_multi_noalloc (prefill staging in the
        device's static scratch; the caller passes the outputs); otherwise the
        prefill workspace is ``workspace`` or a torch allocation as in qlinear."""
        import torch
        rows = x.shape[0] if x.dim() == 2 else 1
        if ys is None:
            ys = [torch.empty((rows, w.rows), dtype=y_dtype or torch.float32, device=x.device) for w in ws]
        arr = (_QWeightC * len(ws))(*[w.c() for w in ws])
        yp = (ctypes.c_void_p * len(ws))(*[y.data_ptr() for y in ys])
        if noalloc:
            _check(self._lib.dyninfer_mi355x_qlinear_multi_noalloc(self._h, arr, len(ws), x.data_ptr(), _dtype_code(x),
                                                                   rows, yp, _dtype_code(ys[0]), self._stream(stream)))
            return ys
        wp, wn, _keep = self._workspace(ws, x, rows, _dtype_code(ys[0]), stream, workspace)
        _check(self._lib.dyninfer_mi355x_qlinear_multi(self._h, arr, len(ws), x.data_ptr(), _dtype_code(x), rows, yp,
                                                       _dtype_code(ys[0]), wp, wn, self._stream(stream)))
        return ys

    def dequant(self, w: QWeight, out=None, stream=None):
        """Bit-exact f32 dequantisation of W on the device -> [rows, cols]."""
        import torch
        dev = torch.device("cuda", self.device)
        if out is None:
            out = torch.empty((w.rows, w.cols), dtype=torch.float32, device=dev)
        wc = w.c()
        _check(self._lib.dyninfer_mi355x_dequant(self._h, ctypes.byref(wc), out.data_ptr(), self._stream(stream)))
        return out

    def embedding(self, w: QWeight, ids, out=None, stream=None):
        """Gather rows ids (device int64 [n]) of W and dequantise them -> f32 [n, cols]."""
        import torch
        if ids.dtype != torch.int64 or not ids.is_cuda or not ids.is_contiguous():
            raise DyninferError(ERR_INVALID_ARGUMENT, "ids must be a contiguous int64 device tensor")
        n = ids.numel()
        if out is None:
            out = torch.empty((n, w.cols), dtype=torch.float32, device=ids.device)
        wc = w.c()
        _check(self._lib.dyninfer_mi355x_embedding(self._h, ctypes.byref(wc), ids.data_ptr() if n else None, n,
                                                   out.data_ptr() if n else None, self._stream(stream)))
        return out


def candidates() -> list:
    """This library's gfx950 KernelCandidateDescriptors (serde JSON)."""
    return json.loads(library().dyninfer_mi355x_candidates_json().decode())


def _registry(fn, request: dict, target: dict, cands) -> dict:
    lib = library()
    cj = None if cands is None else json.dumps(cands).encode()
    rq, tg = json.dumps(request).encode(), json.dumps(target).encode()
    n = ctypes.c_size_t(0)
    rc = getattr(lib, fn)(cj, rq, tg, None, 0, ctypes.byref(n))
    if rc not in (OK, ERR_BUFFER_TOO_SMALL):
        _check(rc)
    buf = ctypes.create_string_buffer(n.value + 1)
    _check(getattr(lib, fn)(cj, rq, tg, ctypes.cast(buf, ctypes.c_void_p), n.value + 1, ctypes.byref(n)))
    return json.loads(buf.value.decode())


def registry_select(request: dict, target: dict, cands=None) -> dict:
    """KernelRegistry::select over ``cands`` (default: this library's candidates) -> SelectionReport."""
    return _registry("dyninfer_mi355x_registry_select", request, target, cands)


def registry_require(request: dict, target: dict, cands=None) -> dict:
    """KernelRegistry::require -> SelectedKernelCandidate, or DyninferError(ERR_UNSUPPORTED, E_KERNEL_COVERAGE…)."""
    return _registry("dyninfer_mi355x_registry_require", request, target, cands)


def precision_check(selected: dict, activation_type: str = "f32") -> None:
    """The compiler's lower.precision gate (crates/dyninfer-compiler/src/lib.rs:289-306),
    relaxed for bf16 activations on this library's lowerings; raises DyninferError
    (ERR_UNSUPPORTED) when the selected kernel is not qualified."""
    _check(library().dyninfer_mi355x_precision_check(json.dumps(selected).encode(), activation_type.encode()))


@dataclass
class GgufTensor:
    name: str
    type_code: int
    shape: tuple
    offset: int
    nbytes: int


class GgufFile:
    """Index of a GGUF file: exact byte ranges of its tensors (dyninfer_mi355x_gguf_*).
    ``GgufFile(path)`` maps the file; ``GgufFile.from_bytes(b)`` indexes bytes in memory."""

    def __init__(self, path: Optional[str] = None, _data=None):
        self._lib = library()
        self._h = ctypes.c_void_p()
        self._keep = None
        if _data is not None:
            self._keep = ctypes.create_string_buffer(bytes(_data), len(_data))
            _check(self._lib.dyninfer_mi355x_gguf_open_memory(ctypes.addressof(self._keep), len(_data),
                                                              ctypes.byref(self._h)))
        else:
            _check(self._lib.dyninfer_mi355x_gguf_open(os.fsencode(path), ctypes.byref(self._h)))

    @classmethod
    def from_bytes(cls, data: bytes) -> "GgufFile":
        return cls(_data=data)

    def close(self) -> None:
        if self._h:
            self._lib.dyninfer_mi355x_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _py(t: "_GgufTensorC") -> GgufTensor:
        return GgufTensor(t.name.decode(), t.type_code, tuple(t.dims[:t.n_dims]), t.offset, t.nbytes)

    @property
    def tensors(self) -> list:
        out = []
        for i in range(self._lib.dyninfer_mi355x_gguf_tensor_count(self._h)):
            t = _GgufTensorC()
            _check(self._lib.dyninfer_mi355x_gguf_tensor(self._h, i, ctypes.byref(t)))
            out.append(self._py(t))
        return out

    @property
    def metadata(self) -> dict:
        return json.loads(self._lib.dyninfer_mi355x_gguf_metadata_json(self._h).decode())

    def find(self, name: str) -> GgufTensor:
        t = _GgufTensorC()
        _check(self._lib.dyninfer_mi355x_gguf_find(self._h, name.encode(), ctypes.byref(t)))
        return self._py(t)

    def upload(self, name: str, dst=None, stream=None):
        """Copy the tensor's exact bytes to the device (a new uint8 tensor unless dst is given)."""
        import torch
        if dst is None:
            dst = torch.empty(self.find(name).nbytes, dtype=torch.uint8, device="cuda")
        cap = dst.numel() * dst.element_size()
        _check(self._lib.dyninfer_mi355x_gguf_upload(self._h, name.encode(), dst.data_ptr(), cap,
                                                     Context._stream(stream)))
        return dst

    def qweight(self, name: str, device_data) -> QWeight:
        """QWeight of a rank-2 GGUF tensor (Q4_0/Q4_1/Q8_0/Q6_K/Q4_K/Q5_K/IQ4_XS) whose bytes are at device_data."""
        wc = _QWeightC()
        _check(self._lib.dyninfer_mi355x_gguf_qweight(self._h, name.encode(), _ptr(device_data), ctypes.byref(wc)))
        return QWeight(wc.encoding, wc.rows, wc.cols, device_data, data_bytes=wc.data_bytes)


@dataclass
class StTensor:
    name: str
    dtype: str
    shape: tuple
    offset: int
    nbytes: int


class SafeTensorsFile:
    """Index of a .safetensors file (dyninfer_mi355x_safetensors_*): exact byte ranges of its
    tensors and MLX affine weights from their three components.  ``SafeTensorsFile(path)``
    maps the file and reads config.json beside it; ``SafeTensorsFile.from_bytes(b, config)``
    indexes bytes in memory with the text of a config.json (or None)."""

    def __init__(self, path: Optional[str] = None, _data=None, _config: Optional[str] = None):
        self._lib = library()
        self._h = ctypes.c_void_p()
        self._keep = None
        if _data is not None:
            self._keep = ctypes.create_string_buffer(bytes(_data), len(_data))
            cfg = _config.encode() if _config is not None else None
            _check(self._lib.dyninfer_mi355x_safetensors_open_memory(ctypes.addressof(self._keep), len(_data), cfg,
                                                                     ctypes.byref(self._h)))
        else:
            _check(self._lib.dyninfer_mi355x_safetensors_open(os.fsencode(path), ctypes.byref(self._h)))

    @classmethod
    def from_bytes(cls, data: bytes, config: Optional[str] = None) -> "SafeTensorsFile":
        return cls(_data=data, _config=config)

    def close(self) -> None:
        if self._h:
            self._lib.dyninfer_mi355x_safetensors_close(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _py(t: "_StTensorC") -> StTensor:
        return StTensor(t.name.decode(), t.dtype.decode(), tuple(t.dims[:t.n_dims]), t.offset, t.nbytes)

    @property
    def tensors(self) -> list:
        out = []
        for i in range(self._lib.dyninfer_mi355x_safetensors_tensor_count(self._h)):
            t = _StTensorC()
            _check(self._lib.dyninfer_mi355x_safetensors_tensor(self._h, i, ctypes.byref(t)))
            out.append(self._py(t))
        return out

    @property
    def metadata(self) -> dict:
        return json.loads(self._lib.dyninfer_mi355x_safetensors_metadata_json(self._h).decode())

    def find(self, name: str) -> StTensor:
        t = _StTensorC()
        _check(self._lib.dyninfer_mi355x_safetensors_find(self._h, name.encode(), ctypes.byref(t)))
        return self._py(t)

    def upload(self, name: str, dst=None, stream=None):
        """Copy the tensor's exact bytes to the device (a new uint8 tensor unless dst is given)."""
        import torch
        if dst is None:
            dst = torch.empty(max(self.find(name).nbytes, 1), dtype=torch.uint8, device="cuda")
        cap = dst.numel() * dst.element_size()
        _check(self._lib.dyninfer_mi355x_safetensors_upload(self._h, name.encode(), dst.data_ptr(), cap,
                                                            Context._stream(stream)))
        return dst

    def mlx_qweight(self, weight_name: str, packed, scales, biases) -> QWeight:
        """QWeight of the MLX affine weight `weight_name` whose three components' bytes are at
        packed / scales / biases on the device (validated as the reference's MLX convention)."""
        wc = _QWeightC()
        _check(self._lib.dyninfer_mi355x_safetensors_mlx_qweight(self._h, weight_name.encode(), _ptr(packed),
                                                                 _ptr(scales), _ptr(biases), ctypes.byref(wc)))
        return QWeight(wc.encoding, wc.rows, wc.cols, packed, scales, biases, wc.group_size, wc.scale_dtype,
                       data_bytes=wc.data_bytes, scales_bytes=wc.scales_bytes, biases_bytes=wc.biases_bytes)
