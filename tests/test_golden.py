"""Committed golden fixtures (tests/golden/tiny_llama_quant.*).

The fixtures restate the reference's two tiny quantized checkpoints
(q4.rs:226-293 GGUF; fixture.rs:208-260 MLX affine U4) plus one synthetic
Q6_K tensor; make_golden.py documents their provenance.  CPU tests:
  * the oracle regenerates every byte stream (SHA-256 from the manifest), every
    dequantised weight bit for bit and every f64 contraction exactly;
  * independent pins on the fixture bytes: the reference's own round-trip
    formulas (reference.rs:106-193, numpy f32), GGML's loop-form Q6_K decoder,
    and a numpy f64 matmul for y64.
GPU tests run the HIP kernels through the C ABI on the fixture bytes: dequant
bit-exact, qlinear within the f16 activation bound of the fixture's y64.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from tests.golden import make_golden
from tests.test_oracle import ggml_q6_k, rt_q4_0, rt_q4_1, rt_q8_0, rt_u4

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
XF16 = 2.0 ** -11 + 2e-5


@pytest.fixture(scope="module")
def golden():
    with np.load(os.path.join(HERE, "tiny_llama_quant.npz"), allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    with open(os.path.join(HERE, "tiny_llama_quant.json")) as fh:
        manifest = json.load(fh)
    return arrays, manifest


def test_oracle_regenerates_fixtures_bit_for_bit(golden):
    arrays, manifest = golden
    fresh, fresh_manifest = make_golden.build()
    assert fresh_manifest == manifest
    assert sorted(fresh) == sorted(arrays)
    for k, v in arrays.items():
        assert fresh[k].dtype == v.dtype and fresh[k].shape == v.shape, k
        assert fresh[k].tobytes() == v.tobytes(), k


def test_fixture_hashes(golden):
    arrays, manifest = golden
    for t in manifest["gguf"]:
        assert hashlib.sha256(arrays[t["key"] + ".data"].tobytes()).hexdigest() == t["sha256"]
    for t in manifest["mlx"]:
        blob = b"".join(arrays[t["key"] + s].tobytes() for s in (".packed", ".scales", ".biases"))
        assert hashlib.sha256(blob).hexdigest() == t["sha256"]


def test_fixture_dequant_equals_reference_roundtrip(golden):
    """w in the fixture == the reference's quantize->dequant formulas applied to
    the same LCG values (reference.rs:106-193), and Q6_K == GGML's loop form."""
    arrays, manifest = golden
    rt = {"q4_0": rt_q4_0, "q4_1": rt_q4_1, "q8_0": rt_q8_0}
    for t in manifest["gguf"]:
        w = arrays[t["key"] + ".w"]
        if t["encoding"] == "q6_k":
            blocks = arrays[t["key"] + ".data"].reshape(-1, 210)
            ref = np.concatenate([ggml_q6_k(b) for b in blocks]).reshape(w.shape)
        else:
            ref = rt[t["encoding"]](oracle.fill_f32(t["rows"] * t["cols"], t["seed"])).reshape(w.shape)
            if t["encoding"] in ("q4_0", "q8_0"):
                # the round-trip formula keeps a rounded -0.0 code as a float; the stored
                # integer code is 0, which decodes to +0 (sitofp, and the `+ 0.0` of
                # gguf_codegen.rs:444, 465 for Q4_0)
                ref = ref + np.float32(0.0)
        assert np.array_equal(w.view(np.uint32), ref.astype(np.float32).view(np.uint32)), t["name"]
    for t in manifest["mlx"]:
        w = arrays[t["key"] + ".w"]
        ref = rt_u4(oracle.fill_f32(t["rows"] * t["cols"], t["seed"]), t["cols"], t["group_size"]).reshape(w.shape)
        assert np.array_equal(w.view(np.uint32), ref.view(np.uint32)), t["name"]


def test_fixture_contraction_equals_numpy_f64(golden):
    arrays, manifest = golden
    for t in manifest["gguf"] + manifest["mlx"]:
        k = t["key"]
        x, w = arrays[k + ".x"].astype(np.float64), arrays[k + ".w"].astype(np.float64)
        np.testing.assert_allclose(arrays[k + ".y64"], x @ w.T, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(arrays[k + ".absdot"], np.abs(x) @ np.abs(w).T, rtol=1e-12, atol=0)


# ---------------------------------------------------------------- GPU, through the C ABI
def _gpu_weight(d, arrays, t, kind):
    import torch

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")

    k = t["key"]
    if kind == "gguf":
        enc = {2: d.ENC_Q4_0, 3: d.ENC_Q4_1, 8: d.ENC_Q8_0, 14: d.ENC_Q6_K}[t["type_code"]]
        return d.QWeight(enc, t["rows"], t["cols"], dev(arrays[k + ".data"]))
    return d.QWeight(d.ENC_MLX_U4, t["rows"], t["cols"], dev(arrays[k + ".packed"]), dev(arrays[k + ".scales"]),
                     dev(arrays[k + ".biases"]), group_size=t["group_size"], scale_dtype=d.DTYPE_F32)


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["gguf", "mlx"])
def test_gpu_dequant_matches_golden(ctx, golden, kind):
    import dyninfer_amd as d
    arrays, manifest = golden
    for t in manifest[kind]:
        w = _gpu_weight(d, arrays, t, kind)
        got = ctx.dequant(w).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), arrays[t["key"] + ".w"].view(np.uint32)), t["name"]


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["gguf", "mlx"])
@pytest.mark.parametrize("batch", [1, 2])
def test_gpu_qlinear_matches_golden(ctx, golden, kind, batch):
    import torch
    import dyninfer_amd as d
    arrays, manifest = golden
    for t in manifest[kind]:
        k = t["key"]
        w = _gpu_weight(d, arrays, t, kind)
        x = torch.from_numpy(arrays[k + ".x"][:batch].copy()).to("cuda")
        y = ctx.qlinear(w, x).cpu().numpy()
        err = oracle.normalized_error(y, arrays[k + ".y64"][:batch], arrays[k + ".absdot"][:batch])
        assert err <= XF16, (t["name"], err)
