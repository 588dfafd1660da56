"""Kernel-registry restatement (C ABI) against the reference's selection rules.

The first five tests restate crates/dyninfer-kernel-registry/src/lib.rs:626-740
case for case; the rest check this library's gfx950 candidates against the
reference's own GGUF/MLX IREE candidates (generated here the way
gguf_codegen.rs:50-113 and mlx_affine.rs:157-238 generate them).
Host-only: no GPU is touched.
"""
import copy
import json

import pytest

import dyninfer_amd as d


# ---------------------------------------------------------------- serde helpers (reference shapes)
def target_any():
    return {"backends": ["any"]}


def candidate(cid, readiness="production"):
    """lib.rs:604-624 `candidate()`."""
    return {
        "id": cid, "operation": "linear", "encoding": {"id": "plain.f16", "version": 1},
        "input_types": ["f32"], "output_types": ["f32"], "accumulator_types": ["f32"],
        "shape": {"logical_rank": 2}, "orientations": ["native"], "target": target_any(),
        "modes": ["prefill", "decode"], "lowering": "dense.matmul.linalg", "deterministic_score": 100,
        "readiness": readiness, "notes": "",
    }


def request(op="linear", enc=("plain.f16", 1), shape=(64, 64), mode="decode", op_id="blk.0.attn_q"):
    """lib.rs:626-638 `request()`."""
    r = {
        "operation_id": op_id, "operation": op, "logical_shape": list(shape), "orientation": "native", "mode": mode,
        "precision_policy": {"id": "conservative_sensitive_ops", "version": 1, "sensitive_internal_type": "f32"},
        "parameter_slots": ["blk.0.attn_q.weight"], "checkpoint_component_keys": ["weights::blk.0.attn_q.weight::data"],
    }
    if enc is not None:
        r["encoding"] = {"id": enc[0], "version": enc[1]}
    return r


def cpu_host(features=("sse4.2", "avx", "avx2", "fma", "f16c")):
    """TargetProfile::llvm_cpu_host (crates/dyninfer-core/src/types.rs:274-296)."""
    return {"driver": "local-task", "device_id": 0, "triple": "x86_64-unknown-linux-gnu", "features": list(features)}


def hip(chip):
    """TargetProfile::hip_rocm (types.rs:299-329): driver hip, features rocm-target=<chip>."""
    return {"driver": "hip", "device_id": 0, "architecture": chip, "features": [f"rocm-target={chip}"]}


def cuda(arch):
    """TargetProfile::cuda (types.rs:331-377)."""
    sm = int(arch.replace("sm_", ""))
    f = [f"cuda-target={arch}"]
    f += ["native_f16"] if sm >= 53 else []
    f += ["integer_dot_product"] if sm >= 61 else []
    f += ["tensor_cores"] if sm >= 70 else []
    f += ["native_bf16"] if sm >= 80 else []
    f += ["nvfp4"] if sm >= 100 else []
    return {"driver": "cuda", "device_id": 0, "architecture": arch, "features": f}


def iree_gguf_candidates(codec, block):
    """The reference's GGUF candidates (gguf_codegen.rs:50-113)."""
    out = []
    for op, suffix in [("embedding", "gather"), ("linear", "matmul"), ("output_projection", "output")]:
        for backend, target in [("cpu", {"backends": ["local-task", "local-sync"], "required_features": ["avx2"]}),
                                ("hip", {"backends": ["hip", "rocm"]})]:
            out.append({
                "id": f"{codec}.{suffix}.iree_block_{backend}", "operation": op,
                "encoding": {"id": codec, "version": 1}, "input_types": ["f32"], "output_types": ["f32"],
                "accumulator_types": ["f32"],
                "shape": {"logical_rank": 2, "axis_multiples": [{"axis": 1, "multiple_of": block}]},
                "orientations": ["native"], "target": target, "modes": ["prefill", "decode"],
                "lowering": f"{codec}.{suffix}.iree_block", "deterministic_score": 300, "readiness": "production",
                "notes": "",
            })
    return out


def iree_mlx_candidates():
    """The reference's MLX U4 candidates (mlx_affine.rs:157-238)."""
    out = []
    for op, suffix, lowering in [("embedding", "embedding", "mlx.affine.u4.gather.iree_grouped"),
                                 ("linear", "matmul", "mlx.affine.u4.matmul.iree_grouped"),
                                 ("output_projection", "output", "mlx.affine.u4.matmul.iree_grouped")]:
        for backend, target in [("cpu", {"backends": ["local-task", "local-sync"], "required_features": ["avx2"]}),
                                ("hip", {"backends": ["hip", "rocm"]})]:
            out.append({
                "id": f"mlx.affine.u4.{suffix}.iree_grouped_{backend}", "operation": op,
                "encoding": {"id": "mlx.affine.u4", "version": 1}, "input_types": ["f32"], "output_types": ["f32"],
                "accumulator_types": ["f32"],
                "shape": {"logical_rank": 2, "axis_multiples": [{"axis": 1, "multiple_of": 32}]},
                "orientations": ["native"], "target": target, "modes": ["prefill", "decode"],
                "lowering": lowering if backend == "cpu" else lowering + "_gpu", "deterministic_score": 300,
                "readiness": "production", "notes": "",
            })
    return out


def full_registry():
    cands = []
    for codec, block in [("gguf.q4_0", 32), ("gguf.q4_1", 32), ("gguf.q8_0", 32), ("gguf.q6_k", 256)]:
        cands += iree_gguf_candidates(codec, block)
    cands += iree_mlx_candidates()
    return cands + d.candidates()


# ---------------------------------------------------------------- reference tests (lib.rs:640-740)
def test_only_production_candidates_can_be_selected():
    cands = [candidate("prototype", "prototype"), candidate("production")]
    rep = d.registry_select(request(), cpu_host(), cands)
    assert rep["selected"]["descriptor"]["id"] == "production"
    assert rep["rejected"][0]["reasons"] == [{"reason": "not_production_ready"}]


def test_tie_breaking_is_stable_by_kernel_id():
    sel = d.registry_require(request(), cpu_host(), [candidate("z.kernel"), candidate("a.kernel")])
    assert sel["descriptor"]["id"] == "a.kernel"


def test_unsupported_encoding_returns_structured_coverage_error():
    with pytest.raises(d.DyninferError) as e:
        d.registry_require(request(enc=("gguf.q8_0", 1)), cpu_host(), [candidate("dense")])
    assert e.value.code == d.ERR_UNSUPPORTED
    assert e.value.message.startswith("E_KERNEL_COVERAGE")
    assert "blk.0.attn_q" in e.value.message


def test_sensitive_operation_rejects_candidate_below_precision_floor():
    low = candidate("rms.f16")
    low["operation"] = "rms_norm"
    low["shape"]["logical_rank"] = 1
    low["accumulator_types"] = ["f16"]
    rep = d.registry_select(request(op="rms_norm", shape=(64,)), cpu_host(), [low])
    assert "selected" not in rep
    assert rep["rejected"][0]["reasons"] == [{"reason": "precision_floor", "required": "f32", "supported": ["f16"]}]


def test_exact_gpu_architecture_matches_architecture_not_cpu_triple():
    exact = candidate("cuda.sm100")
    exact["target"] = {"backends": ["cuda"], "exact_architectures": ["sm_100"], "required_features": ["nvfp4"]}
    rep = d.registry_select(request(), cuda("sm_100"), [exact])
    assert rep["selected"]["descriptor"]["id"] == "cuda.sm100"


# ---------------------------------------------------------------- gfx950 candidates
def gguf_request(codec, n, k, op="linear", mode="decode"):
    return request(op=op, enc=(codec, 1), shape=(n, k), mode=mode)


@pytest.mark.parametrize("codec,block", [("gguf.q4_0", 32), ("gguf.q4_1", 32), ("gguf.q8_0", 32), ("gguf.q6_k", 256),
                                         ("gguf.q4_k", 256), ("gguf.q5_k", 256), ("gguf.iq4_xs", 256),
                                         ("mlx.affine.u4", 32)])
@pytest.mark.parametrize("op,suffix", [("linear", "matmul"), ("output_projection", "output")])
@pytest.mark.parametrize("mode", ["decode", "prefill"])
def test_mi355x_entry_wins_on_gfx950(codec, block, op, suffix, mode):
    sel = d.registry_require(gguf_request(codec, 1024, 4 * block, op, mode), hip("gfx950"), full_registry())
    assert sel["descriptor"]["id"] == f"{codec}.{suffix}.mi355x_hip"
    assert sel["descriptor"]["lowering"].endswith(".mi355x_hip")
    assert sel["score"] == 1400  # 400 + exact-backend bonus, above IREE's 1300
    assert (sel["input_type"], sel["output_type"], sel["accumulator_type"]) == ("f32", "f32", "f32")


@pytest.mark.parametrize("codec", ["gguf.q4_0", "gguf.q6_k", "mlx.affine.u4"])
def test_mi355x_entry_rejected_off_gfx950(codec):
    block = 256 if codec == "gguf.q6_k" else 32
    rep = d.registry_select(gguf_request(codec, 512, 2 * block), hip("gfx1151"), full_registry())
    assert rep["selected"]["descriptor"]["id"].endswith("iree_block_hip") or \
        rep["selected"]["descriptor"]["id"].endswith("iree_grouped_hip")
    ours = [r for r in rep["rejected"] if r["candidate_id"] == f"{codec}.matmul.mi355x_hip"][0]
    assert ours["reasons"] == [{"reason": "architecture_mismatch", "selected": "gfx1151"}]


def test_q4_k_is_covered_only_on_gfx950():
    """gguf.q4_k is declared without kernels in the reference (gguf_block.rs:183-316):
    on gfx950 this library's entry is selected, elsewhere the request stays a
    coverage error (E_KERNEL_COVERAGE, lib.rs:350-399)."""
    req = gguf_request("gguf.q4_k", 4096, 4096)
    assert d.registry_require(req, hip("gfx950"), full_registry())["descriptor"]["id"] == "gguf.q4_k.matmul.mi355x_hip"
    with pytest.raises(d.DyninferError) as e:
        d.registry_require(req, hip("gfx1151"), full_registry())
    assert e.value.code == d.ERR_UNSUPPORTED


def test_cpu_target_keeps_iree_cpu_kernel_and_missing_avx2_is_coverage_error():
    sel = d.registry_require(gguf_request("gguf.q4_0", 64, 64), cpu_host(), full_registry())
    assert sel["descriptor"]["id"] == "gguf.q4_0.matmul.iree_block_cpu"
    assert sel["score"] == 1300
    rep = d.registry_select(gguf_request("gguf.q4_0", 64, 64), cpu_host(("sse4.2",)), full_registry())
    assert "selected" not in rep
    cpu = [r for r in rep["rejected"] if r["candidate_id"] == "gguf.q4_0.matmul.iree_block_cpu"][0]
    assert cpu["reasons"] == [{"reason": "missing_target_feature", "feature": "avx2"}]
    ours = [r for r in rep["rejected"] if r["candidate_id"] == "gguf.q4_0.matmul.mi355x_hip"][0]
    assert ours["reasons"] == [{"reason": "backend_mismatch", "selected": "local-task"},
                               {"reason": "architecture_mismatch", "selected": None}]


def test_axis_not_divisible_rejects():
    rep = d.registry_select(gguf_request("gguf.q6_k", 64, 300), hip("gfx950"), d.candidates())
    assert "selected" not in rep
    ours = [r for r in rep["rejected"] if r["candidate_id"] == "gguf.q6_k.matmul.mi355x_hip"][0]
    assert ours["reasons"] == [{"reason": "axis_not_divisible", "axis": 1, "dimension": 300, "multiple_of": 256}]


@pytest.mark.parametrize("codec,block,suffix", [("gguf.q4_0", 32, "gather"), ("gguf.q4_1", 32, "gather"),
                                                ("gguf.q8_0", 32, "gather"), ("gguf.q6_k", 256, "gather"),
                                                ("gguf.q4_k", 256, "gather"), ("gguf.q5_k", 256, "gather"),
                                                ("gguf.iq4_xs", 256, "gather"),
                                                ("mlx.affine.u4", 32, "embedding")])
def test_embedding_selects_mi355x_gather_on_gfx950(codec, block, suffix):
    req = gguf_request(codec, 151936, 4 * block, op="embedding", mode="prefill")
    sel = d.registry_require(req, hip("gfx950"), full_registry())
    assert sel["descriptor"]["id"] == f"{codec}.{suffix}.mi355x_hip" and sel["score"] == 1400
    rep = d.registry_select(req, hip("gfx1151"), full_registry())
    if codec in ("gguf.q4_k", "gguf.q5_k", "gguf.iq4_xs"):  # schema-only in the reference: no other kernel
        assert "selected" not in rep
    else:
        assert rep["selected"]["descriptor"]["id"] in (f"{codec}.gather.iree_block_hip",
                                                       "mlx.affine.u4.embedding.iree_grouped_hip")


def test_duplicate_candidate_ids_are_rejected():
    c = d.candidates()
    with pytest.raises(d.DyninferError) as e:
        d.registry_select(gguf_request("gguf.q4_0", 64, 64), hip("gfx950"), c + [copy.deepcopy(c[0])])
    assert e.value.code == d.ERR_INVALID_ARGUMENT and "duplicate kernel candidate" in e.value.message


def test_candidates_match_the_serde_schema():
    """Field names and enum spellings of KernelCandidateDescriptor (lib.rs:132-149)."""
    keys = {"id", "operation", "encoding", "input_types", "output_types", "accumulator_types", "shape",
            "orientations", "target", "modes", "lowering", "deterministic_score", "readiness", "notes"}
    cands = d.candidates()
    assert len(cands) == 40 and len({c["id"] for c in cands}) == 40
    for c in cands:
        assert set(c) == keys
        assert c["operation"] in ("embedding", "linear", "output_projection")
        assert c["readiness"] == "production"
        assert c["orientations"] == ["native"]
        assert set(c["modes"]) == {"prefill", "decode"}
        assert c["target"]["exact_architectures"] == ["gfx950"]
        assert c["target"]["backends"] == ["hip", "rocm"]
        assert c["encoding"]["version"] == 1
        assert c["shape"]["logical_rank"] == 2
        assert c["id"] == c["lowering"] and c["id"].endswith(".mi355x_hip")
        assert c["accumulator_types"] == ["f32"]
        bf16 = c["id"].split(".")[-2].endswith("_bf16")
        assert c["input_types"] == c["output_types"] == (["bf16"] if bf16 else ["f32"])
        assert c["deterministic_score"] == (390 if bf16 else 400)
    json.dumps(cands)


# ---------------------------------------------------------------- bf16 activations (compiler precision gate)
CODECS = [("gguf.q4_0", 32), ("gguf.q4_1", 32), ("gguf.q8_0", 32), ("gguf.q6_k", 256), ("mlx.affine.u4", 32)]


@pytest.mark.parametrize("codec,block", CODECS)
@pytest.mark.parametrize("op,suffix", [("linear", "matmul"), ("output_projection", "output")])
def test_request_without_activation_type_selects_as_the_reference(codec, block, op, suffix):
    """The bf16 entries score below the f32 ones, so the reference's own select
    (which ignores activation types) keeps the f32 entry, and the reference's
    all-f32 precision gate (lib.rs:289-306) accepts it."""
    sel = d.registry_require(gguf_request(codec, 1024, 4 * block, op), hip("gfx950"), full_registry())
    assert sel["descriptor"]["id"] == f"{codec}.{suffix}.mi355x_hip" and sel["input_type"] == "f32"
    d.precision_check(sel)
    d.precision_check(sel, "bf16")


@pytest.mark.parametrize("codec,block", CODECS)
@pytest.mark.parametrize("op,suffix", [("linear", "matmul_bf16"), ("output_projection", "output_bf16")])
def test_bf16_activations_select_the_bf16_entry(codec, block, op, suffix):
    req = dict(gguf_request(codec, 1024, 4 * block, op), activation_type="bf16")
    sel = d.registry_require(req, hip("gfx950"), full_registry())
    assert sel["descriptor"]["id"] == f"{codec}.{suffix}.mi355x_hip"
    assert (sel["input_type"], sel["output_type"], sel["activation_type"], sel["accumulator_type"]) == \
        ("bf16", "bf16", "bf16", "f32")
    assert sel["score"] == 1390
    # the f32-only gate of the reference rejects it; the relaxed gate accepts it
    with pytest.raises(d.DyninferError) as e:
        d.precision_check(sel)
    assert e.value.code == d.ERR_UNSUPPORTED
    assert f"selected kernel `{codec}.{suffix}.mi355x_hip` requires Bf16/Bf16/Bf16/F32" in e.value.message
    assert "qualified only for f32 compute" in e.value.message
    d.precision_check(sel, "bf16")
    # the f32 entry is rejected for a bf16 request, with the extension's reason
    rep = d.registry_select(req, hip("gfx950"), full_registry())
    f32 = [r for r in rep["rejected"] if r["candidate_id"] == f"{codec}.{suffix.replace('_bf16', '')}.mi355x_hip"][0]
    assert f32["reasons"] == [{"reason": "activation_type_mismatch", "required": "bf16", "supported": ["f32"]}]


def test_activation_type_leaves_embeddings_alone_and_unknown_types_uncovered():
    req = dict(gguf_request("gguf.q4_0", 151936, 1024, op="embedding"), activation_type="bf16")
    assert d.registry_require(req, hip("gfx950"), full_registry())["descriptor"]["id"] == "gguf.q4_0.gather.mi355x_hip"
    req = dict(gguf_request("gguf.q4_0", 1024, 1024), activation_type="f16")
    with pytest.raises(d.DyninferError) as e:
        d.registry_require(req, hip("gfx950"), d.candidates())
    assert e.value.code == d.ERR_UNSUPPORTED and e.value.message.startswith("E_KERNEL_COVERAGE")


def test_precision_gate_cases():
    sel = d.registry_require(dict(gguf_request("gguf.q4_0", 64, 64), activation_type="bf16"), hip("gfx950"),
                             d.candidates())
    # a bf16 kernel that is not this library's (an IREE lowering) stays rejected
    other = copy.deepcopy(sel)
    other["descriptor"]["id"] = other["descriptor"]["lowering"] = "gguf.q4_0.matmul.iree_block_hip"
    with pytest.raises(d.DyninferError):
        d.precision_check(other, "bf16")
    # bf16 accumulation stays rejected
    acc = copy.deepcopy(sel)
    acc["accumulator_type"] = "bf16"
    with pytest.raises(d.DyninferError) as e:
        d.precision_check(acc, "bf16")
    assert "requires Bf16/Bf16/Bf16/Bf16" in e.value.message
    # i64 inputs (token ids) pass, as in the reference
    ids = copy.deepcopy(sel)
    ids["input_type"] = "i64"
    d.precision_check(ids)
    with pytest.raises(d.DyninferError) as e:
        d.precision_check(sel, "f16")
    assert e.value.code == d.ERR_INVALID_ARGUMENT
