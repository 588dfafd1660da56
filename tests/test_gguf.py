"""GGUF container indexing (dyninfer_mi355x_gguf_*), host only, plus one GPU
upload test.

The file under test is the reference's tiny mixed-quant checkpoint
(q4.rs:226-293) written by a restatement of its own writer `write_gguf`
(q4.rs:139-193: version 3, metadata, tensor infos with dims reversed and
32-byte-aligned relative offsets, data section aligned to 32); the quantized
tensors' bytes are the committed golden fixtures.  Checks: every tensor's name,
row-major shape, type code and exact byte range (the bytes at [offset,
offset + nbytes) equal what was written), metadata values, and the reference
indexer's error cases (container.rs:179-340).
"""
import json
import struct

import numpy as np
import pytest

import dyninfer_amd as d
import oracle
from tests.golden import make_golden

F32, Q4_0, Q4_1, Q8_0 = 0, 2, 3, 8


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(tensors: dict, meta: dict, alignment: int = 32, version: int = 3, extra_meta=b"") -> bytes:
    """write_gguf (q4.rs:139-193); meta values: ('u32', v) / ('f32', v) / ('str', v) / ('u64', v)."""
    body = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta) + (1 if extra_meta else 0))
    for k, (kind, v) in sorted(meta.items()):
        body += _s(k) + {"u32": lambda: struct.pack("<II", 4, v), "u64": lambda: struct.pack("<IQ", 10, v),
                         "f32": lambda: struct.pack("<If", 6, v), "str": lambda: struct.pack("<I", 8) + _s(v)}[kind]()
    body += extra_meta
    data = b""
    for name, (shape, code, raw) in sorted(tensors.items()):
        body += _s(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", x) for x in reversed(shape))
        body += struct.pack("<I", code)
        data += b"\0" * ((alignment - len(data) % alignment) % alignment)
        body += struct.pack("<Q", len(data))
        data += raw
    body += b"\0" * ((alignment - len(body) % alignment) % alignment)
    return body + data


def tiny_llama_q4():
    """tiny_llama_q4_0 (q4.rs:226-293): tensors {name: (shape, type, bytes)} and metadata."""
    arrays, manifest = make_golden.build()
    vocab, hidden = 32, 64
    tensors = {"token_embd.weight": ((vocab, hidden), F32, oracle.fill_f32(vocab * hidden, 1).tobytes())}
    ones = np.ones(hidden, np.float32).tobytes()
    for n in ("blk.0.attn_norm.weight", "blk.0.ffn_norm.weight", "output_norm.weight"):
        tensors[n] = ((hidden,), F32, ones)
    for t in manifest["gguf"]:
        if t["encoding"] != "q6_k":
            tensors[t["name"]] = ((t["rows"], t["cols"]), t["type_code"], arrays[t["key"] + ".data"].tobytes())
    meta = {"general.architecture": ("str", "llama"), "llama.block_count": ("u32", 1),
            "llama.embedding_length": ("u32", hidden), "llama.feed_forward_length": ("u32", 128),
            "llama.attention.head_count": ("u32", 4), "llama.attention.head_count_kv": ("u32", 4),
            "llama.vocab_size": ("u32", vocab), "llama.context_length": ("u32", 128),
            "llama.rope.dimension_count": ("u32", 16), "llama.attention.layer_norm_rms_epsilon": ("f32", 1e-5)}
    return tensors, meta


def test_index_tiny_llama_exact_byte_ranges(tmp_path):
    tensors, meta = tiny_llama_q4()
    blob = write_gguf(tensors, meta)
    path = tmp_path / "tiny.gguf"
    path.write_bytes(blob)
    for g in (d.GgufFile(str(path)), d.GgufFile.from_bytes(blob)):
        got = g.tensors
        assert [t.name for t in got] == sorted(tensors)
        for t in got:
            shape, code, raw = tensors[t.name]
            assert t.shape == tuple(shape) and t.type_code == code and t.nbytes == len(raw)
            assert t.offset % 32 == 0
            assert blob[t.offset:t.offset + t.nbytes] == raw
        assert g.find("blk.0.attn_q.weight").type_code == Q4_1
        m = g.metadata
        assert m["general.architecture"] == "llama" and m["llama.vocab_size"] == 32
        assert m["llama.attention.layer_norm_rms_epsilon"] == pytest.approx(1e-5, rel=1e-7)
        assert list(m) == sorted(m)
        w = g.qweight("blk.0.ffn_down.weight", 0x1000)
        assert (w.encoding, w.rows, w.cols) == (d.ENC_Q4_0, 64, 128)
        with pytest.raises(d.DyninferError) as e:
            g.qweight("token_embd.weight", 0x1000)
        assert e.value.code == d.ERR_UNSUPPORTED
        with pytest.raises(d.DyninferError):
            g.find("missing.weight")
        g.close()


def test_general_alignment_and_metadata_types():
    tensors = {"w": ((4, 32), Q4_0, bytes(range(72)))}
    arr = _s("tokens") + struct.pack("<IIQ", 9, 8, 2) + _s("a") + _s("bc")
    flt = _s("nan") + struct.pack("<If", 6, float("nan"))
    blob = write_gguf(tensors, {"general.alignment": ("u32", 64)}, alignment=64, extra_meta=arr)
    g = d.GgufFile.from_bytes(blob)
    t = g.find("w")
    assert t.offset % 64 == 0 and blob[t.offset:t.offset + 72] == bytes(range(72))
    assert g.metadata["tokens"] == ["a", "bc"]
    g2 = d.GgufFile.from_bytes(write_gguf(tensors, {}, extra_meta=flt))
    assert g2.metadata["nan"] is None  # serde_json: non-finite f32 -> null


@pytest.mark.parametrize("case", ["magic", "version", "truncated", "past_end", "block", "type", "value_type", "dup",
                                  "utf8_key", "utf8_value", "utf8_surrogate", "utf8_overlong", "align_overflow"])
def test_invalid_files_are_rejected(case):
    good = {"w": ((2, 32), Q4_0, bytes(36))}
    if case == "magic":
        blob = b"GGUX" + write_gguf(good, {})[4:]
    elif case == "version":
        blob = write_gguf(good, {}, version=4)
    elif case == "truncated":
        blob = write_gguf(good, {"k": ("str", "v")})[:30]
    elif case == "past_end":
        blob = write_gguf(good, {})[:-1]
    elif case == "block":
        blob = write_gguf({"w": ((2, 33), Q4_0, bytes(40))}, {})
    elif case == "type":
        blob = write_gguf({"w": ((2, 32), 99, bytes(36))}, {})
    elif case == "value_type":
        blob = write_gguf(good, {}, extra_meta=_s("k") + struct.pack("<I", 13))
    elif case.startswith("utf8"):
        # container.rs read_string: String::from_utf8 rejects the bytes
        bad = {"utf8_key": b"\xff", "utf8_value": b"\xc3\x28", "utf8_surrogate": b"\xed\xa0\x80",
               "utf8_overlong": b"\xc0\xaf"}[case]
        raw = struct.pack("<Q", len(bad)) + bad
        extra = raw + struct.pack("<I", 4) + struct.pack("<I", 1) if case == "utf8_key" else \
            _s("k") + struct.pack("<I", 8) + raw
        blob = write_gguf(good, {}, extra_meta=extra)
    elif case == "align_overflow":
        # align_up(pos, 2^64 - 1) = 2^64 - 1: the data section lies past the end of the file
        blob = write_gguf(good, {"general.alignment": ("u64", (1 << 64) - 1)}, alignment=32)
    else:
        blob = write_gguf({"wa": ((2, 32), Q4_0, bytes(36)), "wb": ((2, 32), Q4_0, bytes(36))}, {})
        blob = blob.replace(_s("wb"), _s("wa"), 1)
    msg = {"magic": "bad magic", "version": "version 4", "truncated": "truncated", "past_end": "past end",
           "block": "not divisible", "type": "unknown GGUF tensor type", "value_type": "value type 13",
           "dup": "duplicate", "utf8_key": "not UTF-8", "utf8_value": "not UTF-8", "utf8_surrogate": "not UTF-8",
           "utf8_overlong": "not UTF-8", "align_overflow": "past end"}[case]
    with pytest.raises(d.DyninferError) as e:
        d.GgufFile.from_bytes(blob)
    assert e.value.code == d.ERR_UNSUPPORTED and msg in e.value.message


def test_valid_utf8_metadata_is_kept():
    txt = "Größe ✓ \U0001F600"
    g = d.GgufFile.from_bytes(write_gguf({"w": ((2, 32), Q4_0, bytes(36))}, {"name": ("str", txt)}))
    assert g.metadata["name"] == txt


def test_invalid_file_opened_by_path_is_unmapped(tmp_path):
    """A file that fails indexing is reported and its mapping released (no
    mapping of it is left in the process after repeated failed opens)."""
    path = tmp_path / "bad_version.gguf"
    path.write_bytes(write_gguf({"w": ((2, 32), Q4_0, bytes(36))}, {}, version=4))
    for _ in range(20):
        with pytest.raises(d.DyninferError) as e:
            d.GgufFile(str(path))
        assert e.value.code == d.ERR_UNSUPPORTED and "version 4" in e.value.message
    maps = open("/proc/self/maps").read()
    assert str(path) not in maps


@pytest.mark.gpu
def test_gpu_upload_then_qlinear_matches_golden(ctx, tmp_path):
    """Upload exact byte ranges from the mapped file and run each linear of the
    tiny checkpoint against the golden fixture's f64 outputs."""
    import torch
    tensors, meta = tiny_llama_q4()
    path = tmp_path / "tiny.gguf"
    path.write_bytes(write_gguf(tensors, meta))
    g = d.GgufFile(str(path))
    arrays, manifest = make_golden.build()
    for t in manifest["gguf"]:
        if t["encoding"] == "q6_k":
            continue
        dev = g.upload(t["name"])
        assert torch.equal(dev.cpu(), torch.from_numpy(arrays[t["key"] + ".data"]))
        w = g.qweight(t["name"], dev)
        x = torch.from_numpy(arrays[t["key"] + ".x"]).to("cuda")
        y = ctx.qlinear(w, x).cpu().numpy()
        err = oracle.normalized_error(y, arrays[t["key"] + ".y64"], arrays[t["key"] + ".absdot"])
        assert err <= 2.0 ** -11 + 2e-5, (t["name"], err)
    with pytest.raises(d.DyninferError) as e:
        g.upload("blk.0.attn_k.weight", torch.empty(8, dtype=torch.uint8, device="cuda"))
    assert e.value.code == d.ERR_BUFFER_TOO_SMALL
