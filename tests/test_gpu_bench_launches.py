"""Every distinct launch that bench.py times in its decode steps, at every batch
it times, against the CPU oracle through the C ABI.

The cases come from bench.step_layout, the table bench.py builds its steps
from: BASELINE config 4 (Qwen3-8B GGUF, batch 1/4/16), config 1 (Qwen3-0.6B
mixed Q4_0/Q4_1/Q8_0/Q6_K, batch 1/4), config 2 (Qwen3-0.6B MLX U4 g64, bf16
in and out, batch 1/8/16) and the Qwen3-8B Q4_K_M step (batch 1/4/16).  The
library picks the kernel, launch mode and tile from N, K, the batch and the
grouping (latency mode, persistent pipeline, streaming, MFMA GEMV with split or
whole tiles, K segments), so each launch is checked at its own exact shape and
grouping: the grouped weights share one activation through qlinear_multi, as
the step issues them, and each output is checked on up to 512 sampled rows
(gguf_codegen.rs:268-314, mlx_affine.rs:557-626 contraction; dequantisation as
the oracle restates gguf_codegen.rs:382-526 and mlx_affine.rs:593-598).

Bound per output (plus 2e-5·Σ|w||x| of f32 accumulation), the one
include/dyninfer_mi355x.h states: 2^-10·Σ|w||x| (one f16 rounding of each
activation and each weight), (2^-10 + 2^-11)·Σ|w||x| for Q6_K,
(2^-10 + 2^-11)·Σ|w||x| + 2^-10·Σ|dmin·m||x| for Q4_K; bf16 outputs add
2^-8·|y|.
"""
import functools

import numpy as np
import pytest
import torch

import bench
import dyninfer_amd as d
import oracle

pytestmark = pytest.mark.gpu

GTYPE = {"q4_0": oracle.Q4_0, "q4_1": oracle.Q4_1, "q8_0": oracle.Q8_0, "q6_k": oracle.Q6_K, "q4_k": oracle.Q4_K}
ENC = {"q4_0": d.ENC_Q4_0, "q4_1": d.ENC_Q4_1, "q8_0": d.ENC_Q8_0, "q6_k": d.ENC_Q6_K, "q4_k": d.ENC_Q4_K}


def _cases():
    seen, out = set(), []
    for name in ("config4", "config1", "config2", "q4_k_m"):
        xdt, ydt = bench.STEP_DTYPES[name]
        layout = {}
        for label, enc, shapes, _, _ in bench.step_layout(name):
            layout.setdefault((enc, tuple(shapes)), label)
        for (enc, shapes), label in layout.items():
            for b in bench.STEP_BATCHES[name]:
                key = (enc, shapes, b, xdt, ydt)
                if key not in seen:
                    seen.add(key)
                    out.append(pytest.param(enc, shapes, b, xdt, ydt, id=f"{name}-{label}-b{b}"))
    return out


CASES = _cases()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


@functools.lru_cache(maxsize=3)
def _weight(enc, n, k, seed):
    """(QWeight on the device, host bytes) of one synthetic weight; the last few stay cached so
    that the batches of one launch share them."""
    if enc == "mlx_u4":
        packed, sc, bi = oracle.synth_mlx_u4(n, k, 64, oracle.D_BF16, seed=seed)
        return d.QWeight(d.ENC_MLX_U4, n, k, dev(packed), dev(sc), dev(bi), 64, d.DTYPE_BF16), (packed, sc, bi)
    data = oracle.synth_gguf(GTYPE[enc], n, k, seed)
    return d.QWeight(ENC[enc], n, k, dev(data)), data


def _rows_dequant(enc, host, n, k, rows):
    """Exact f32 dequantisation of the sampled rows, and |dmin·m| per weight for Q4_K."""
    if enc == "mlx_u4":
        packed, sc, bi = host
        g = k // 64
        return oracle.dequant_mlx_u4(packed.reshape(n, -1)[rows], sc.reshape(n, g)[rows], bi.reshape(n, g)[rows],
                                     oracle.D_BF16, len(rows), k, 64), None
    gt = GTYPE[enc]
    bw, bb = oracle.BLOCK[gt]
    sub = host.reshape(n, (k // bw) * bb)[rows]
    wf = oracle.dequant_gguf(gt, sub.ravel(), len(rows), k)
    if enc != "q4_k":
        return wf, None
    z = sub.reshape(-1, bb).copy()
    z[:, 0:2] = 0  # d = 0 leaves -dmin·m
    return wf, np.abs(oracle.dequant_gguf(gt, z.ravel(), len(rows), k))


@pytest.mark.parametrize("enc,shapes,batch,xdt,ydt", CASES)
def test_bench_launch(ctx, enc, shapes, batch, xdt, ydt):
    k = shapes[0][1]
    ws, hosts = [], []
    for i, (n, kk) in enumerate(shapes):
        w, host = _weight(enc, n, kk, seed=1000 * i + n // 7 + kk)
        ws.append(w)
        hosts.append(host)
    x = oracle.randn(batch * k, seed=batch * 31 + k).reshape(batch, k)
    if xdt == "bf16":
        xb = oracle.f32_to_bf16_bits(x.reshape(-1)).reshape(batch, k)
        xd, x = dev(xb).view(torch.bfloat16), oracle.bf16_bits_to_f32(xb).reshape(batch, k)
    else:
        xd = dev(x)
    ytorch = torch.bfloat16 if ydt == "bf16" else torch.float32
    ys = [torch.full((batch, n), float("nan"), dtype=ytorch, device="cuda") for n, _ in shapes]
    if len(ws) == 1:
        ctx.qlinear(ws[0], xd, ys[0])
    else:
        ctx.qlinear_multi(ws, xd, ys)
    torch.cuda.synchronize()
    rel = {"q6_k": 2.0 ** -10 + 2.0 ** -11, "q4_k": 2.0 ** -10 + 2.0 ** -11}.get(enc, 2.0 ** -10) + 2e-5
    for (n, _), y, host in zip(shapes, ys, hosts):
        rows = np.sort(np.random.default_rng(n + batch).choice(n, size=min(512, n), replace=False))
        wf, offs = _rows_dequant(enc, host, n, k, rows)
        y64, absdot = oracle.linear_f64(x, wf)
        got = y.float().cpu().numpy()[:, rows].astype(np.float64)
        bound = rel * absdot
        if offs is not None:
            bound = bound + 2.0 ** -10 * (np.abs(x.astype(np.float64)) @ offs.astype(np.float64).T)
        if ydt == "bf16":
            bound = bound + 2.0 ** -8 * np.abs(y64)
        err = np.abs(got - y64)
        assert np.all(np.isfinite(got)), (n, batch)
        assert np.all(err <= bound), (n, batch, float((err / bound).max()))
        assert oracle.normalized_error(got, y64, absdot) <= 2e-3 + (2.0 ** -8 if ydt == "bf16" else 0.0)
