"""SafeTensors container index and the MLX affine convention through the C ABI
(dyninfer_mi355x_safetensors_*).

CPU tests restate the reference's own tests of
crates/dyninfer-checkpoint-safetensors: `indexes_dense_tensor`
(container.rs), `groups_real_mlx_weight_scale_bias_topology` and
`rejects_partial_compound_weight` (mlx.rs); write the reference's tiny MLX
checkpoint (fixture.rs:208-260) with a restatement of its writer
(`write_mixed_safetensors`, fixture.rs:11-55) from the committed golden
tensors and check every byte range; and cover the indexer's and the
convention's error cases (container.rs:82-300, mlx.rs:53-261) and the sibling
config.json (config_json.rs:129-143).  The GPU test uploads the fixture's
three components per weight and multiplies them against the golden f64
outputs.
"""
import json
import os
import struct

import numpy as np
import pytest

import dyninfer_amd as d
import oracle

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FAKE = 0x100000  # an aligned stand-in device address: descriptors are checked, never dereferenced
ERR_UNSUPPORTED = 2


def write_st(tensors, metadata=None, raw_header=None):
    """tensors: {name: (dtype, shape, bytes)} -> SafeTensors bytes, keys sorted as the
    reference's serde_json map writes them; data in key order."""
    header, data = {}, b""
    if metadata is not None:
        header["__metadata__"] = metadata
    for name in sorted(tensors):
        dt, shape, blob = tensors[name]
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [len(data), len(data) + len(blob)]}
        data += blob
    h = raw_header if raw_header is not None else json.dumps(dict(sorted(header.items())), separators=(",", ":")).encode()
    return struct.pack("<Q", len(h)) + h + data


def mixed():
    """mlx.rs `mixed_index`: one packed weight [2, 8] u32 with bf16 scales/biases [2, 1], one norm."""
    return {
        "layer.weight": ("U32", (2, 8), bytes(64)),
        "layer.scales": ("BF16", (2, 1), bytes(4)),
        "layer.biases": ("BF16", (2, 1), bytes(4)),
        "layer_norm.weight": ("BF16", (64,), bytes(128)),
    }


MLX_META = {"format": "mlx", "mlx.quantization.bits": 4, "mlx.quantization.group_size": 64}


def status_of(fn):
    with pytest.raises(d.DyninferError) as e:
        fn()
    return e.value


def test_indexes_dense_tensor():
    blob = write_st({"w.weight": ("F32", (2,), bytes(8))})
    st = d.SafeTensorsFile.from_bytes(blob)
    (t,) = st.tensors
    assert (t.name, t.dtype, t.shape, t.nbytes) == ("w.weight", "F32", (2,), 8)
    assert t.offset == 8 + struct.unpack("<Q", blob[:8])[0]  # offsets count from the header's end


def test_mlx_weight_scale_bias_topology():
    st = d.SafeTensorsFile.from_bytes(write_st(mixed(), MLX_META))
    assert [t.name for t in st.tensors] == sorted(mixed())
    w = st.mlx_qweight("layer.weight", FAKE, FAKE, FAKE)
    assert (w.encoding, w.rows, w.cols, w.group_size, w.scale_dtype) == (d.ENC_MLX_U4, 2, 64, 64, d.DTYPE_BF16)
    assert (w.data_bytes, w.scales_bytes, w.biases_bytes) == (64, 4, 4)
    assert st.metadata["format"] == "mlx" and st.metadata["mlx.quantization.bits"] == 4


def test_rejects_partial_compound_weight():
    t = mixed()
    del t["layer.biases"]
    st = d.SafeTensorsFile.from_bytes(write_st(t, MLX_META))
    e = status_of(lambda: st.mlx_qweight("layer.weight", FAKE, FAKE, FAKE))
    assert e.code == ERR_UNSUPPORTED and "both .scales and .biases" in str(e)


@pytest.fixture(scope="module")
def golden():
    with np.load(os.path.join(HERE, "tiny_llama_quant.npz"), allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    with open(os.path.join(HERE, "tiny_llama_quant.json")) as fh:
        manifest = json.load(fh)
    return arrays, manifest


def tiny_mlx_checkpoint(arrays, manifest):
    """fixture.rs:208-260 `tiny_llama_mlx_affine_u4`, written as write_mixed_safetensors does:
    every rank-2 weight as U32 words [rows, cols/8] with F32 scales and biases
    [rows, cols/64], the norms as dense F32, metadata numbers in __metadata__."""
    t = {}
    for e in manifest["mlx"]:
        base = e["name"][: -len(".weight")]
        r, c, g = e["rows"], e["cols"], e["group_size"]
        t[e["name"]] = ("U32", (r, c // 8), arrays[e["key"] + ".packed"].astype("<u4").tobytes())
        t[base + ".scales"] = ("F32", (r, c // g), arrays[e["key"] + ".scales"].astype("<f4").tobytes())
        t[base + ".biases"] = ("F32", (r, c // g), arrays[e["key"] + ".biases"].astype("<f4").tobytes())
    for name in ("blk.0.attn_norm.weight", "blk.0.ffn_norm.weight", "output_norm.weight"):
        t[name] = ("F32", (64,), np.ones(64, "<f4").tobytes())
    meta = {"format": "mlx", "mlx.quantization.bits": 4, "mlx.quantization.group_size": 64, "num_layers": 1,
            "hidden_size": 64, "intermediate_size": 128, "vocab_size": 32}
    return t, write_st(t, meta)


def test_tiny_mlx_checkpoint_exact_byte_ranges(golden):
    arrays, manifest = golden
    tensors, blob = tiny_mlx_checkpoint(arrays, manifest)
    st = d.SafeTensorsFile.from_bytes(blob)
    got = {t.name: t for t in st.tensors}
    assert sorted(got) == sorted(tensors)
    for name, (dt, shape, data) in tensors.items():
        t = got[name]
        assert (t.dtype, t.shape, t.nbytes) == (dt, shape, len(data))
        assert blob[t.offset:t.offset + t.nbytes] == data, name
    for e in manifest["mlx"]:
        w = st.mlx_qweight(e["name"], FAKE, FAKE, FAKE)
        assert (w.rows, w.cols, w.group_size, w.scale_dtype) == (e["rows"], e["cols"], 64, d.DTYPE_F32)


def _bad_cases():
    cases = {
        "short file": b"\x01\x00\x00",
        "zero header length": struct.pack("<Q", 0) + b"{}",
        "header length over 64 MiB": struct.pack("<Q", (64 << 20) + 1) + b"{}",
        "header past end of file": struct.pack("<Q", 100) + b"{}",
        "header not JSON": write_st({}, raw_header=b"{not json"),
        "header not an object": write_st({}, raw_header=b"[1,2]"),
        "header with a NUL": write_st({}, raw_header=b'{"a":1}\x00'),
        "unsupported dtype": write_st({"x": ("F8_E4M3", (4,), bytes(4))}),
        "byte length != numel x elem": write_st({"x": ("F32", (3,), bytes(8))}),
        "rank over 16": write_st({"x": ("U8", (1,) * 17, bytes(1))}),
        "dimension over 2^40": write_st({"x": ("U8", (2 ** 40 + 1, 0), b"")}),
        "key over 16 KiB": write_st({"k" * (16 * 1024 + 1): ("U8", (1,), bytes(1))}),
    }
    # hand-edited headers: offsets reversed, past the file, overlapping, duplicate key
    def with_header(obj, data):
        hb = json.dumps(obj).encode()
        return struct.pack("<Q", len(hb)) + hb + data
    cases["data_offsets end < start"] = with_header({"x": {"dtype": "U8", "shape": [0], "data_offsets": [4, 0]}}, bytes(4))
    cases["data past end of file"] = with_header({"x": {"dtype": "U8", "shape": [8], "data_offsets": [0, 8]}}, bytes(4))
    cases["overlapping ranges"] = with_header({"a": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]},
                                               "b": {"dtype": "U8", "shape": [4], "data_offsets": [2, 6]}}, bytes(8))
    dup = b'{"x":{"dtype":"U8","shape":[2],"data_offsets":[0,2]},"x":{"dtype":"U8","shape":[2],"data_offsets":[2,4]}}'
    cases["duplicate tensor name"] = struct.pack("<Q", len(dup)) + dup + bytes(4)
    cases["float shape"] = with_header({"x": {"dtype": "U8", "shape": [2.0], "data_offsets": [0, 2]}}, bytes(2))
    cases["missing data_offsets"] = with_header({"x": {"dtype": "U8", "shape": [2]}}, bytes(2))
    return cases


@pytest.mark.parametrize("case", sorted(_bad_cases()))
def test_invalid_files_are_rejected(case):
    blob = _bad_cases()[case]
    e = status_of(lambda: d.SafeTensorsFile.from_bytes(blob))
    assert e.code == ERR_UNSUPPORTED and "invalid SafeTensors" in str(e), str(e)


MLX_BAD = {
    # (edit of the mixed index, metadata, expected message fragment)
    "format not mlx": (None, {"mlx.quantization.bits": 4, "mlx.quantization.group_size": 64}, "format"),
    "bits missing": (None, {"format": "mlx", "mlx.quantization.group_size": 64}, "mlx.quantization.bits"),
    "group missing": (None, {"format": "mlx", "mlx.quantization.bits": 4}, "mlx.quantization.group_size"),
    "bits as a string": (None, {"format": "mlx", "mlx.quantization.bits": "4", "mlx.quantization.group_size": 64},
                         "mlx.quantization.bits"),
    "bits 5": (None, {**MLX_META, "mlx.quantization.bits": 5}, "unsupported MLX affine configuration"),
    "bits 8 (valid MLX, not this library)": ({"layer.weight": ("U32", (2, 16), bytes(128))},
                                             {**MLX_META, "mlx.quantization.bits": 8}, "mlx.affine.u4 only"),
    "packed not u32": ({"layer.weight": ("I32", (2, 8), bytes(64))}, MLX_META, "must be u32"),
    "scale/bias types differ": ({"layer.biases": ("F16", (2, 1), bytes(4))}, MLX_META, "same floating-point type"),
    "integer scales": ({"layer.scales": ("U16", (2, 1), bytes(4)), "layer.biases": ("U16", (2, 1), bytes(4))},
                       MLX_META, "same floating-point type"),
    "scales shape": ({"layer.scales": ("BF16", (2, 2), bytes(8))}, MLX_META, "does not match logical groups"),
    "not group divisible": ({"layer.weight": ("U32", (2, 4), bytes(32))}, MLX_META, "not group divisible"),
    "rank 3": ({"layer.weight": ("U32", (1, 2, 8), bytes(64)), "layer.scales": ("BF16", (1, 2, 1), bytes(4)),
                "layer.biases": ("BF16", (1, 2, 1), bytes(4))}, MLX_META, "not rank 2"),
}


@pytest.mark.parametrize("case", sorted(MLX_BAD))
def test_mlx_convention_errors(case):
    edit, meta, frag = MLX_BAD[case]
    t = mixed()
    t.update(edit or {})
    st = d.SafeTensorsFile.from_bytes(write_st(t, meta))
    e = status_of(lambda: st.mlx_qweight("layer.weight", FAKE, FAKE, FAKE))
    assert e.code == ERR_UNSUPPORTED and frag in str(e), str(e)


def test_non_weight_name_is_rejected():
    st = d.SafeTensorsFile.from_bytes(write_st(mixed(), MLX_META))
    e = status_of(lambda: st.mlx_qweight("layer.scales", FAKE, FAKE, FAKE))
    assert ".weight" in str(e)


def test_sibling_config_json_supplies_quantization(tmp_path):
    """config_json.rs:129-143: quantization(_config).bits / group_size map to
    mlx.quantization.*; header metadata wins where both are set."""
    (tmp_path / "model.safetensors").write_bytes(write_st(mixed(), {"format": "mlx"}))
    (tmp_path / "config.json").write_text(json.dumps({"quantization": {"bits": 4, "group_size": 64}, "hidden_size": 64}))
    st = d.SafeTensorsFile(str(tmp_path / "model.safetensors"))
    assert st.metadata["mlx.quantization.bits"] == 4 and st.metadata["mlx.quantization.group_size"] == 64
    w = st.mlx_qweight("layer.weight", FAKE, FAKE, FAKE)
    assert (w.cols, w.group_size) == (64, 64)
    # the header's group size wins over config.json's
    (tmp_path / "b.safetensors").write_bytes(write_st({**mixed(), "layer.scales": ("BF16", (2, 2), bytes(8)),
                                                       "layer.biases": ("BF16", (2, 2), bytes(8))},
                                                      {"format": "mlx", "mlx.quantization.group_size": 32}))
    st = d.SafeTensorsFile(str(tmp_path / "b.safetensors"))
    assert st.mlx_qweight("layer.weight", FAKE, FAKE, FAKE).group_size == 32
    # quantization_config is read too; a missing config.json leaves the keys absent
    (tmp_path / "config.json").write_text(json.dumps({"quantization_config": {"bits": 4, "group_size": 64}}))
    assert d.SafeTensorsFile(str(tmp_path / "model.safetensors")).metadata["mlx.quantization.bits"] == 4
    os.remove(tmp_path / "config.json")
    st = d.SafeTensorsFile(str(tmp_path / "model.safetensors"))
    assert "missing required MLX metadata" in str(status_of(lambda: st.mlx_qweight("layer.weight", FAKE, FAKE, FAKE)))


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [1, 2, 20])
def test_gpu_upload_then_qlinear_matches_golden(ctx, golden, tmp_path, batch):
    """Every MLX weight of the tiny checkpoint: its three components uploaded
    from the mapped file, described by mlx_qweight, multiplied (decode GEMV at
    1-2 rows, prefill GEMM at 20) against the f64 contraction of the fixture's
    exactly dequantised weights."""
    import torch
    arrays, manifest = golden
    _, blob = tiny_mlx_checkpoint(arrays, manifest)
    path = tmp_path / "tiny_mlx.safetensors"
    path.write_bytes(blob)
    st = d.SafeTensorsFile(str(path))
    for e in manifest["mlx"]:
        base = e["name"][: -len(".weight")]
        comps = [st.upload(n) for n in (e["name"], base + ".scales", base + ".biases")]
        for n, c in zip((".packed", ".scales", ".biases"), comps):
            assert c.cpu().numpy().tobytes() == arrays[e["key"] + n].tobytes()
        w = st.mlx_qweight(e["name"], *comps)
        x = oracle.randn(batch * e["cols"], seed=batch + e["seed"]).reshape(batch, e["cols"])
        y = ctx.qlinear(w, torch.from_numpy(x).to("cuda")).cpu().numpy()
        y64, absdot = oracle.linear_f64(x, arrays[e["key"] + ".w"])
        err = oracle.normalized_error(y, y64, absdot)
        assert err <= 2.0 ** -10 + 1e-4, (e["name"], err)
