"""Writes tests/golden/tiny_llama_quant.npz and tiny_llama_quant.json.

The fixtures are the two tiny quantized Llama checkpoints the reference builds
for its end-to-end tests, restated tensor for tensor:
  * GGUF (crates/dyninfer-checkpoint-gguf/src/q4.rs:226-293): every linear
    filled by the LCG `fill_f32` with seeds 2..9 and packed by
    pack_q4_0 / pack_q4_1 / pack_q8_0 (q4.rs:16-96); attn_q is Q4_1,
    attn_v Q8_0, the rest Q4_0;
  * MLX affine U4 (crates/dyninfer-checkpoint-safetensors/src/fixture.rs:208-260):
    every rank-2 weight (embedding included, seeds 1..9) through
    quantize_affine_u4 (fixture.rs:287-317) with group 64 and f32 scales/biases.
The reference has no Q6_K packer and pins no Q6_K value, so one Q6_K tensor
(64 x 512, seeded synthetic super-blocks in the BASELINE distribution) is
added and labelled as such.

Per tensor the file holds the on-disk bytes, the exact dequantised f32 weights
(emit_dequant, gguf_codegen.rs:350-526; mlx_affine.rs:593-598), an activation
batch x [2, K] (fill_f32 seed 100 + tensor index) and the f64 contraction
y64 = x . W^T with sum |x||w| per output (the 2e-3 tolerance's normaliser).
The JSON manifest records shapes, encodings, seeds and the SHA-256 of each
byte stream.  Regenerate with `python tests/golden/make_golden.py`; the CPU
tests check that the oracle still reproduces every array bit for bit.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle  # noqa: E402

VOCAB, HIDDEN, INTER = 32, 64, 128

GGUF_SPECS = [  # (name, seed, rows, cols, encoding)  q4.rs:274-291
    ("blk.0.attn_q.weight", 2, HIDDEN, HIDDEN, oracle.Q4_1),
    ("blk.0.attn_k.weight", 3, HIDDEN, HIDDEN, oracle.Q4_0),
    ("blk.0.attn_v.weight", 4, HIDDEN, HIDDEN, oracle.Q8_0),
    ("blk.0.attn_output.weight", 5, HIDDEN, HIDDEN, oracle.Q4_0),
    ("blk.0.ffn_gate.weight", 6, INTER, HIDDEN, oracle.Q4_0),
    ("blk.0.ffn_up.weight", 7, INTER, HIDDEN, oracle.Q4_0),
    ("blk.0.ffn_down.weight", 8, HIDDEN, INTER, oracle.Q4_0),
    ("output.weight", 9, VOCAB, HIDDEN, oracle.Q4_0),
]
Q6K_SPEC = ("synthetic.q6_k.weight", 77, 64, 512, oracle.Q6_K)
MLX_SPECS = [  # (name, seed, rows, cols)  fixture.rs:236-246
    ("token_embd.weight", 1, VOCAB, HIDDEN),
    ("blk.0.attn_q.weight", 2, HIDDEN, HIDDEN),
    ("blk.0.attn_k.weight", 3, HIDDEN, HIDDEN),
    ("blk.0.attn_v.weight", 4, HIDDEN, HIDDEN),
    ("blk.0.attn_output.weight", 5, HIDDEN, HIDDEN),
    ("blk.0.ffn_gate.weight", 6, INTER, HIDDEN),
    ("blk.0.ffn_up.weight", 7, INTER, HIDDEN),
    ("blk.0.ffn_down.weight", 8, HIDDEN, INTER),
    ("output.weight", 9, VOCAB, HIDDEN),
]
MLX_GROUP = 64
BATCH = 2


def gguf_bytes(seed, rows, cols, enc):
    if enc == oracle.Q6_K:
        return oracle.synth_gguf(enc, rows, cols, seed)
    return oracle.pack(enc, oracle.fill_f32(rows * cols, seed))


def activations(index, cols):
    return oracle.fill_f32(BATCH * cols, 100 + index).reshape(BATCH, cols)


def build():
    arrays, manifest = {}, {"batch": BATCH, "gguf": [], "mlx": []}
    for i, (name, seed, rows, cols, enc) in enumerate(GGUF_SPECS + [Q6K_SPEC]):
        data = gguf_bytes(seed, rows, cols, enc)
        w = oracle.dequant_gguf(enc, data, rows, cols)
        x = activations(i, cols)
        y64, absdot = oracle.linear_f64(x, w)
        key = f"gguf{i}"
        arrays.update({f"{key}.data": data, f"{key}.w": w, f"{key}.x": x, f"{key}.y64": y64, f"{key}.absdot": absdot})
        manifest["gguf"].append({"key": key, "name": name, "seed": seed, "rows": rows, "cols": cols,
                                 "encoding": oracle.NAMES[enc], "type_code": enc,
                                 "source": "synthetic (oracle synth_gguf)" if enc == oracle.Q6_K else "q4.rs:274-291",
                                 "sha256": hashlib.sha256(data.tobytes()).hexdigest()})
    for i, (name, seed, rows, cols) in enumerate(MLX_SPECS):
        packed, scales, biases = oracle.quantize_affine_u4(oracle.fill_f32(rows * cols, seed), rows, cols, MLX_GROUP)
        w = oracle.dequant_mlx_u4(packed, scales, biases, oracle.D_F32, rows, cols, MLX_GROUP)
        x = activations(50 + i, cols)
        y64, absdot = oracle.linear_f64(x, w)
        key = f"mlx{i}"
        arrays.update({f"{key}.packed": packed, f"{key}.scales": scales, f"{key}.biases": biases, f"{key}.w": w,
                       f"{key}.x": x, f"{key}.y64": y64, f"{key}.absdot": absdot})
        blob = packed.tobytes() + scales.tobytes() + biases.tobytes()
        manifest["mlx"].append({"key": key, "name": name, "seed": seed, "rows": rows, "cols": cols,
                                "group_size": MLX_GROUP, "scale_dtype": "f32", "source": "fixture.rs:236-260",
                                "sha256": hashlib.sha256(blob).hexdigest()})
    return arrays, manifest


def main():
    arrays, manifest = build()
    np.savez_compressed(os.path.join(HERE, "tiny_llama_quant.npz"), **arrays)
    with open(os.path.join(HERE, "tiny_llama_quant.json"), "w") as fh:
        json.dump(manifest, fh, indent=1)
        fh.write("\n")


if __name__ == "__main__":
    main()
