#!/usr/bin/env python3
"""Benchmark of the MI355X quantized weight-matmul path (one JSON line on stdout).

Metric: "quant GEMV weight HBM GB/s (% of 8 TB/s); Q4_0 prefill
GEMM TFLOP/s".  `value` is measured on BASELINE config 4, the largest
single-GPU configuration: one Qwen3-8B decode step's quantized matmuls at
batch 1 — 36 layers of q/k/v/o/gate/up (Q4_0) and down (Q6_K) plus the
lm_head (Q6_K), 4,884,639,744 weight bytes per step.  One step = every one of
those GEMVs once, in layer order, launched as a decode step would be: q/k/v
as one launch (shared activation), o, gate/up as one launch, down, then
lm_head; the step is captured once in a HIP graph and replayed.  Weights are
seeded synthetic bytes in the BASELINE distributions, resident in HBM before
timing.

value = weight bytes per step x steps / timed seconds (GB/s).  The other
configurations (0: rotating-pool single GEMV, 1: Qwen3-0.6B mixed GGUF step,
2: MLX U4 step, 3: Q4_0 prefill GEMM, 4 at batch 4 and 16) are reported under
"extra".
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA, TFLOP/s
METRIC = "quant GEMV weight HBM GB/s (% of 8 TB/s); Q4_0 prefill GEMM TFLOP/s"

# Qwen3-0.6B (hidden 1024, 28 layers, 16 q heads / 8 kv heads x 128, ffn 3072, vocab 151936)
QWEN06 = dict(layers=28, hidden=1024, q=2048, kv=1024, ffn=3072, vocab=151936)
# Qwen3-8B (hidden 4096, 36 layers, GQA 32/8 x 128, ffn 12288, vocab 151936)
QWEN8 = dict(layers=36, hidden=4096, q=4096, kv=1024, ffn=12288, vocab=151936)


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ synthetic weights (on the GPU)
def gguf_tensor(torch, d, enc: int, n: int, k: int, gen):
    """Seeded GGUF blocks in the BASELINE distributions, built on the device."""
    bw, bb = d.block_geometry(enc)
    nblk = n * (k // bw)
    dev = "cuda"
    blocks = torch.randint(0, 256, (nblk, bb), dtype=torch.uint8, device=dev, generator=gen)
    scale = (torch.randn(nblk, device=dev, generator=gen).abs() * 0.01).half().view(torch.uint8).view(nblk, 2)
    if enc == d.ENC_Q6_K:
        sc = torch.randint(-32, 32, (nblk, 16), dtype=torch.int8, device=dev, generator=gen).view(torch.uint8)
        blocks[:, 192:208] = sc
        blocks[:, 208:210] = scale
    else:
        blocks[:, 0:2] = scale
        if enc == d.ENC_Q4_1:
            m = (torch.randn(nblk, device=dev, generator=gen) * 0.01).half().view(torch.uint8).view(nblk, 2)
            blocks[:, 2:4] = m
        elif enc in (d.ENC_Q4_K, d.ENC_Q5_K):  # dmin = |N(0,1)|*0.005; scale bytes, high bits, codes uniform
            m = (torch.randn(nblk, device=dev, generator=gen).abs() * 0.005).half().view(torch.uint8).view(nblk, 2)
            blocks[:, 2:4] = m
        elif enc == d.ENC_Q8_0:
            q = torch.randint(-127, 128, (nblk, 32), dtype=torch.int16, device=dev, generator=gen)
            blocks[:, 2:34] = q.to(torch.int8).view(torch.uint8)
    return d.QWeight(enc, n, k, blocks.view(-1))


def mlx_tensor(torch, d, n: int, k: int, group: int, gen):
    dev = "cuda"
    packed = torch.randint(0, 2**31 - 1, (n * k // 8,), dtype=torch.int32, device=dev, generator=gen)
    packed ^= torch.randint(0, 2, (n * k // 8,), dtype=torch.int32, device=dev, generator=gen) << 31
    g = n * (k // group)
    scales = (torch.randn(g, device=dev, generator=gen).abs() * 0.02).bfloat16()
    biases = (torch.randn(g, device=dev, generator=gen) * 0.01).bfloat16()
    return d.QWeight(d.ENC_MLX_U4, n, k, packed, scales, biases, group, d.DTYPE_BF16)


# ------------------------------------------------------------------ decode step sets
class StepSet:
    """The matmuls of one decode step, grouped into launches as a decode step issues them."""

    def __init__(self, name: str):
        self.name = name
        self.launches = []  # (label, [QWeight], input key, [output keys])
        self.weight_bytes = 0

    def add(self, label, ws, xin, outs):
        self.launches.append((label, ws, xin, outs))
        self.weight_bytes += sum(w.nbytes for w in ws)


# The launches of each decode step, in step order, per layer then the lm_head:
# (label, encoding, [(N, K) of each weight sharing the launch's activation],
# activation key, [output keys]).  Encodings: GGUF type names or "mlx_u4"
# (group 64, bf16 scales and biases).  tests/test_gpu_bench_launches.py checks
# every distinct launch of these layouts against the oracle.
def step_layout(name: str):
    c = QWEN8 if name in ("config4", "q4_k_m") else QWEN06
    h, q, kv, f = c["hidden"], c["q"], c["kv"], c["ffn"]
    out = []
    for layer in range(c["layers"]):
        if name == "config4":
            e = ["q4_0"] * 4 + ["q6_k"]
        elif name == "config1":
            e = ["q4_0" if layer % 2 == 0 else "q4_1"] * 4 + ["q8_0"]
        elif name == "config2":
            e = ["mlx_u4"] * 5
        elif name == "q4_k_m":  # llama.cpp's Q4_K_M: Q6_K for attn_v, every other ffn_down and the lm_head
            out.append(("qk.gguf.q4_k", "q4_k", [(q, h), (kv, h)], "h", ["q", "k"]))
            out.append(("v.gguf.q6_k", "q6_k", [(kv, h)], "h", ["v"]))
            out.append(("o.gguf.q4_k", "q4_k", [(h, q)], "attn", ["o"]))
            out.append(("gate_up.gguf.q4_k", "q4_k", [(f, h), (f, h)], "h", ["gate", "up"]))
            dn = "q6_k" if layer % 2 == 0 else "q4_k"
            out.append((f"down.gguf.{dn}", dn, [(h, f)], "act", ["down"]))
            continue
        else:
            raise ValueError(name)
        tag = lambda enc: "mlx.u4" if enc == "mlx_u4" else f"gguf.{enc}"
        out.append((f"qkv.{tag(e[0])}", e[0], [(q, h), (kv, h), (kv, h)], "h", ["q", "k", "v"]))
        out.append((f"o.{tag(e[1])}", e[1], [(h, q)], "attn", ["o"]))
        out.append((f"gate_up.{tag(e[2])}", e[2], [(f, h), (f, h)], "h", ["gate", "up"]))
        out.append((f"down.{tag(e[4])}", e[4], [(h, f)], "act", ["down"]))
    head = "mlx_u4" if name == "config2" else "q6_k"
    out.append((f"lm_head.{'mlx.u4' if head == 'mlx_u4' else 'gguf.q6_k'}", head, [(c["vocab"], h)], "h", ["logits"]))
    return out


# activation rows of each layout's timed batches, and its activation / output dtypes
STEP_BATCHES = {"config4": (1, 4, 16), "config1": (1, 4), "config2": (1, 8, 16), "q4_k_m": (1, 4, 16)}
STEP_DTYPES = {"config4": ("f32", "f32"), "config1": ("f32", "f32"), "config2": ("bf16", "bf16"),
               "q4_k_m": ("f32", "f32")}
STEP_NAMES = {"config4": "qwen3-8b gguf", "config1": "qwen3-0.6b mixed gguf",
              "config2": "qwen3-0.6b mlx affine u4 g64", "q4_k_m": "qwen3-8b gguf q4_k_m"}


def build_step(torch, d, name: str, gen) -> StepSet:
    """Seeded synthetic weights for every launch of step_layout(name), on the device."""
    s = StepSet(STEP_NAMES[name])
    for label, enc, shapes, xin, outs in step_layout(name):
        if enc == "mlx_u4":
            ws = [mlx_tensor(torch, d, n, k, 64, gen) for n, k in shapes]
        else:
            e = getattr(d, "ENC_" + enc.upper())
            ws = [gguf_tensor(torch, d, e, n, k, gen) for n, k in shapes]
        s.add(label, ws, xin, outs)
    return s


class StepRunner:
    """Activations/outputs for one StepSet at a batch size, and the step itself."""

    def __init__(self, torch, d, ctx, steps: StepSet, batch: int, xdtype, ydtype):
        self.torch, self.d, self.ctx, self.set, self.batch = torch, d, ctx, steps, batch
        dims = {}
        for _, ws, xin, outs in steps.launches:
            dims[xin] = ws[0].cols
            for o, w in zip(outs, ws):
                dims[o] = w.rows
        gen = torch.Generator(device="cuda")
        gen.manual_seed(1234)
        self.bufs = {}
        for key, n in dims.items():
            dt = xdtype if key in ("h", "attn", "act") else ydtype
            self.bufs[key] = (torch.randn(batch, n, device="cuda", generator=gen)).to(dt)
        self.stream = torch.cuda.Stream()
        # one workspace for every launch of the step (they run in stream order):
        # the MFMA GEMV stages its activations in it once per call
        code = {torch.float32: d.DTYPE_F32, torch.bfloat16: d.DTYPE_BF16}
        need = max(d.prefill_workspace_bytes(ws, batch, code[self.bufs[xin].dtype], code[self.bufs[outs[0]].dtype])
                   for _, ws, xin, outs in steps.launches)
        self.work = torch.empty(need, dtype=torch.uint8, device="cuda") if need else None

    def launch(self, i: int, stream) -> None:
        _, ws, xin, outs = self.set.launches[i]
        x = self.bufs[xin]
        ys = [self.bufs[o] for o in outs]
        if len(ws) == 1:
            self.ctx.qlinear(ws[0], x, ys[0], stream=stream, workspace=self.work)
        else:
            self.ctx.qlinear_multi(ws, x, ys, stream=stream, workspace=self.work)

    def step(self, stream) -> None:
        for i in range(len(self.set.launches)):
            self.launch(i, stream)

    def capture(self):
        torch = self.torch
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(self.stream):
            self.step(self.stream)  # load code objects / occupancy queries outside the capture
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=self.stream):
                self.step(self.stream)
        torch.cuda.synchronize()
        return g

    def time_graph(self, g, steps: int, warmup: int) -> float:
        """ms per replay; replays and events both on the runner's stream."""
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for _ in range(warmup):
                g.replay()
            torch.cuda.synchronize()
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record(self.stream)
            for _ in range(steps):
                g.replay()
            t1.record(self.stream)
            torch.cuda.synchronize()
        return t0.elapsed_time(t1) / steps

    def label_times(self, reps: int = 20):
        """Per launch label: one graph holding all of the step's launches of that
        label in step order (distinct weights, so every launch streams from
        HBM), replayed between HIP events on the launch stream.
        {label: (launches per step, us per launch, weight bytes per launch)}.
        The time per launch includes the GPU's own gap between two dependent
        dispatches (about 1.5 us on MI355X), not host launch overhead."""
        torch = self.torch
        groups = {}
        for i, (label, _, _, _) in enumerate(self.set.launches):
            groups.setdefault(label, []).append(i)
        out = {}
        for label, idx in groups.items():
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(self.stream):
                with torch.cuda.graph(g, stream=self.stream):
                    for i in idx:
                        self.launch(i, self.stream)
            torch.cuda.synchronize()
            ms = self.time_graph(g, reps, 3)
            nbytes = sum(w.nbytes for i in idx for w in self.set.launches[i][1]) / len(idx)
            out[label] = (len(idx), ms * 1e3 / len(idx), nbytes)
            del g
        return out


# ------------------------------------------------------------------ other configurations
def bench_rotating_gemv(torch, d, ctx, enc, n, k, batch, pool_bytes=1.2e9, iters=200):
    """Config 0: one GEMV timed over a rotating pool of distinct weight copies (> MALL)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    w0 = gguf_tensor(torch, d, enc, n, k, gen)
    copies = max(2, int(pool_bytes // w0.nbytes))
    ws = [w0] + [gguf_tensor(torch, d, enc, n, k, gen) for _ in range(copies - 1)]
    x = torch.randn(batch, k, device="cuda", generator=gen)
    y = torch.empty(batch, n, device="cuda")
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        for w in ws[:4]:
            ctx.qlinear(w, x, y, stream=st)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            for i in range(copies):
                ctx.qlinear(ws[i], x, y, stream=st)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = max(1, iters // copies)
        a.record(st)
        for _ in range(reps):
            g.replay()
        b.record(st)
        torch.cuda.synchronize()
    ms = a.elapsed_time(b) / (reps * copies)
    del ws
    return {"us_per_gemv": ms * 1e3, "weight_GBps": w0.nbytes / ms / 1e6, "copies": copies,
            "hbm_frac": w0.nbytes / ms / 1e6 / HBM_PEAK_GBS}


def bench_gemm(torch, d, ctx, m, n, k, xdtype, calls=20, reps=10, enc=None):
    """Config 3: one prefill call (f16 MFMA, f32 accumulate, bf16 Y; Q4_0 unless
    `enc`), x f32 or bf16: the activation staging kernel (x to f16 operand
    fragments with a per-row power-of-two scale) plus the GEMM, into a
    workspace allocated once up front and sized by the library's query.
    `calls` back-to-back calls (one weight, one activation) are captured in a
    HIP graph and replayed between HIP events on the launch stream, so the
    time per call is GPU time plus the graph's dispatch gaps, without host
    launch overhead.  `eager_us` is the same call issued from Python."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    w = gguf_tensor(torch, d, d.ENC_Q4_0 if enc is None else enc, n, k, gen)
    x = torch.randn(m, k, device="cuda", generator=gen).to(xdtype)
    y = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    wsb = d.prefill_workspace_bytes([w], m, d.DTYPE_BF16 if xdtype == torch.bfloat16 else d.DTYPE_F32, d.DTYPE_BF16)
    work = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
    st = torch.cuda.Stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(st):
        for _ in range(3):
            ctx.qlinear(w, x, y, stream=st, workspace=work)
        torch.cuda.synchronize()
        a.record(st)
        for _ in range(reps * 5):
            ctx.qlinear(w, x, y, stream=st, workspace=work)
        b.record(st)
        torch.cuda.synchronize()
        eager_ms = a.elapsed_time(b) / (reps * 5)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            for _ in range(calls):
                ctx.qlinear(w, x, y, stream=st, workspace=work)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        a.record(st)
        for _ in range(reps):
            g.replay()
        b.record(st)
        torch.cuda.synchronize()
    ms = a.elapsed_time(b) / (reps * calls)
    del g
    tflops = 2.0 * m * n * k / ms / 1e9
    return {"us": ms * 1e3, "TFLOPs": tflops, "mfma_frac": tflops / MFMA_F16_PEAK_TFLOPS, "eager_us": eager_ms * 1e3,
            "workspace_bytes": wsb}


def bench_dense_gemm(torch, m, n, k, calls=20, reps=10):
    """The dense counterpart of config 3 on the same box: Y = X·Wᵀ with bf16 X
    [M, K] and a dense bf16 W (torch.matmul, i.e. hipBLASLt), bf16 Y, timed as
    bench_gemm (a graph of `calls` products, replayed between HIP events).
    The right operand is materialised as a contiguous [K, N] tensor."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    x = torch.randn(m, k, device="cuda", generator=gen).bfloat16()
    wt = torch.randn(n, k, device="cuda", generator=gen).bfloat16().t().contiguous()
    y = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    st = torch.cuda.Stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(st):
        for _ in range(3):
            torch.matmul(x, wt, out=y)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            for _ in range(calls):
                torch.matmul(x, wt, out=y)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        a.record(st)
        for _ in range(reps):
            g.replay()
        b.record(st)
        torch.cuda.synchronize()
    ms = a.elapsed_time(b) / (reps * calls)
    del g
    tflops = 2.0 * m * n * k / ms / 1e9
    return {"us": ms * 1e3, "TFLOPs": tflops, "mfma_frac": tflops / MFMA_F16_PEAK_TFLOPS}


# ------------------------------------------------------------------ CPU baseline
def bench_embedding(torch, d, ctx, enc, vocab, k, n, iters=50):
    """Embedding gather of n token rows from a [vocab, k] weight (the tied Qwen3
    embedding).  Algorithmic HBM bytes per launch: the n gathered rows' on-disk
    bytes plus their f32 output (4 k bytes each) plus the ids."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    w = gguf_tensor(torch, d, enc, vocab, k, gen)
    ids = torch.randint(0, vocab, (n,), device="cuda", generator=gen, dtype=torch.int64)
    out = torch.empty(n, k, device="cuda")
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        for _ in range(3):
            ctx.embedding(w, ids, out, stream=st)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st)
        for _ in range(iters):
            ctx.embedding(w, ids, out, stream=st)
        b.record(st)
        torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / iters
    nbytes = n * (w.nbytes // vocab + 4 * k + 8)
    return {"us": round(us, 3), "bytes_per_launch": nbytes, "GBps": round(nbytes / us / 1e3, 1),
            "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}


def cpu_baseline(threads_all: int | None = None, runs: int = 5):
    """The oracle's CPU contraction (dequantisation adjacent to an f32 dot, the
    reference's CPU semantics) timed on this host, as the baseline rules ask
    (1-thread and all-thread rates, median of several runs): a
    bounded sample of config 4 with the step's byte mix — one Qwen3-8B layer's
    matmuls (q/k/v/o/gate/up Q4_0, down Q6_K) plus 1/36 of the Q6_K lm_head rows
    — at 1 thread and at all threads of this box's CPU share, median of
    `runs` runs after a warm-up.  tokens/s = GB/s / the step's 4.88 GB."""
    import numpy as np
    import oracle
    if threads_all is None:  # the CPUs this process may run on (its share of the box), not the host's count
        threads_all = len(os.sched_getaffinity(0))
    c = QWEN8
    h, q, kv, f = c["hidden"], c["q"], c["kv"], c["ffn"]
    mats = [(oracle.Q4_0, q, h), (oracle.Q4_0, kv, h), (oracle.Q4_0, kv, h), (oracle.Q4_0, h, q),
            (oracle.Q4_0, f, h), (oracle.Q4_0, f, h), (oracle.Q6_K, h, f),
            (oracle.Q6_K, c["vocab"] // c["layers"], h)]
    data = [(t, n, k, oracle.synth_gguf(t, n, k, seed=i)) for i, (t, n, k) in enumerate(mats)]
    nbytes = sum(x[3].size for x in data)
    xs = {k: oracle.randn(k, seed=k).reshape(1, k) for k in {h, q, f}}
    step_bytes = 4884639744

    def one(threads):
        t0 = time.perf_counter()
        for t, n, k, w in data:
            oracle.qlinear_gguf_f32(t, w, xs[k], n, k, threads)
        return time.perf_counter() - t0

    out = {}
    for threads in (1, threads_all):
        one(threads)  # warm-up
        ts = sorted(one(threads) for _ in range(runs))
        med = ts[len(ts) // 2]
        out[threads] = {"GBps": round(nbytes / med / 1e9, 3), "median_s": round(med, 4),
                        "tokens_per_s": round(nbytes / med / step_bytes, 3)}
    allc = out[threads_all]
    return {"value": allc["GBps"], "unit": "GB/s", "cores": threads_all, "kind": "port",
            "nproc": os.cpu_count(), "one_thread": out[1], "all_threads": allc,
            "sample": f"config-4 byte mix: one Qwen3-8B layer's 7 matmuls + 1/36 of the Q6_K lm_head rows "
                      f"({nbytes} weight bytes) at batch 1, median of {runs} runs each at 1 and {threads_all} "
                      f"OpenMP threads (the CPUs in this process's affinity mask; the host has {os.cpu_count()}), "
                      f"oracle/oracle.c qlinear_gguf_f32 (C++ restatement of dyninfer CPU semantics)"}


# ------------------------------------------------------------------ main
def breakdown_of(stats):
    return {k: {"launches_per_step": n, "us_per_launch": round(us, 3), "GBps": round(nb / (us * 1e-6) / 1e9, 1)}
            for k, (n, us, nb) in sorted(stats.items())}


def us_per_label(stats):
    """{label: µs per launch} (the compact form of breakdown_of)."""
    return {k: round(us, 2) for k, (n, us, nb) in sorted(stats.items())}


def step_entry(nbytes, b, ms):
    return {"us_per_step": round(ms * 1e3, 1), "hbm_frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(b / (ms * 1e-3), 1)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--no-extra", action="store_true", help="skip configs 0/1/2/3 and config 4 at batch 4/16")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--gemm-probe", action="store_true",
                    help="for rocprofv3: 30 prefill calls (staging + GEMM, Q4_0, bf16 X and Y) at M512 N3072 K1024, "
                         "then 30 at M2048 N3072 K1024, then 30 each of Q4_1, Q8_0, Q6_K at M512 N3072 K1024")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="for rocprofv3 --pmc: one 64 MiB device copy (the counters' calibration), then one "
                         "eager decode step (--probe-config) and one M512 config-3 GEMM; prints the launch labels "
                         "in dispatch order")
    ap.add_argument("--probe-config", type=int, default=4, choices=(1, 2, 4),
                    help="the decode step --pmc-probe runs (at --batch rows): config 4 (Qwen3-8B), config 1 "
                         "(Qwen3-0.6B mixed GGUF) or config 2 (Qwen3-0.6B MLX, bf16 in/out)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path; run with --gpus 1)", file=sys.stderr)
        return 2

    import torch
    import dyninfer_amd as d

    ctx = d.Context(0)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)

    if args.gemm_probe:
        for enc, m in ((d.ENC_Q4_0, 512), (d.ENC_Q4_0, 2048), (d.ENC_Q4_1, 512), (d.ENC_Q8_0, 512), (d.ENC_Q6_K, 512)):
            wg = gguf_tensor(torch, d, enc, 3072, 1024, gen)
            xg = torch.randn(m, 1024, device="cuda", generator=gen).bfloat16()
            yg = torch.empty(m, 3072, device="cuda", dtype=torch.bfloat16)
            work = torch.empty(d.prefill_workspace_bytes([wg], m, d.DTYPE_BF16, d.DTYPE_BF16), dtype=torch.uint8,
                               device="cuda")
            torch.cuda.synchronize()
            for _ in range(30):
                ctx.qlinear(wg, xg, yg, workspace=work)
            torch.cuda.synchronize()
        print("gemm probe: Q4_0 M512, Q4_0 M2048, Q4_1, Q8_0, Q6_K M512 (N3072 K1024), 30 calls each", flush=True)
        return 0

    name = {1: "config1", 2: "config2", 4: "config4"}[args.probe_config] if args.pmc_probe else "config4"
    if name == "config4":
        log("building config 4 weights (Qwen3-8B GGUF, 4.88 GB) ...")
    s4 = build_step(torch, d, name, gen)
    dts = {"f32": torch.float32, "bf16": torch.bfloat16}
    r4 = StepRunner(torch, d, ctx, s4, args.batch, dts[STEP_DTYPES[name][0]], dts[STEP_DTYPES[name][1]])
    if args.pmc_probe:
        src = torch.ones(16 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)  # reads and writes 64 MiB: the counters' bytes-per-unit calibration
        torch.cuda.synchronize()
        with torch.cuda.stream(r4.stream):
            r4.step(r4.stream)
        torch.cuda.synchronize()
        wg = gguf_tensor(torch, d, d.ENC_Q4_0, 3072, 1024, gen)
        xg = torch.randn(512, 1024, device="cuda", generator=gen).bfloat16()
        yg = torch.empty(512, 3072, device="cuda", dtype=torch.bfloat16)
        torch.cuda.synchronize()
        ctx.qlinear(wg, xg, yg)
        torch.cuda.synchronize()
        print(json.dumps({"calibration_bytes": src.numel() * 4,
                          "launches": [[lab, sum(w.nbytes for w in ws)] for lab, ws, _, _ in s4.launches]
                          + [["gemm.q4_0.M512_N3072_K1024", wg.nbytes]]}))
        return 0
    g4 = r4.capture()
    ms = r4.time_graph(g4, args.steps, args.warmup)
    del g4
    step_bytes, step_launches = s4.weight_bytes, len(s4.launches)
    value = step_bytes / ms / 1e6
    log(f"config 4 batch {args.batch}: {ms * 1e3:.1f} us/step, {value:.1f} GB/s")

    # dominant kernel of the step: the launch label with the largest total time
    stats = r4.label_times(reps=10)
    dom_label, (dn, dom_us, dom_bytes) = max(stats.items(), key=lambda kv: kv[1][0] * kv[1][1])
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": dom_label, "bytes_per_launch": int(dom_bytes), "avg_launch_us": round(dom_us, 3),
                "timing": "HIP events on the launch stream around a graph of the step's launches of this label; "
                          "includes the dispatch gap"}
    tfile = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    if os.path.exists(tfile):
        with open(tfile) as fh:
            tj = json.load(fh)
        if dom_label in tj.get("bytes_per_launch", {}):
            roofline["traffic"] = tj["bytes_per_launch"][dom_label]
            roofline["traffic_source"] = tj.get("source")
    # `extra` (stdout) holds the compact figures; `detail` (one JSON line on
    # stderr) the per-label breakdowns in full
    c4 = {"weight_bytes_per_step": s4.weight_bytes, f"batch{args.batch}": step_entry(s4.weight_bytes, args.batch, ms),
          f"batch{args.batch}_us_per_launch": us_per_label(stats)}
    extra = {"config4": c4}
    detail = {"config4": {f"batch{args.batch}": breakdown_of(stats)}}
    del r4

    if not args.no_extra:
        for b in (4, 16):
            r = StepRunner(torch, d, ctx, s4, b, torch.float32, torch.float32)
            g = r.capture()
            ms8 = r.time_graph(g, max(5, args.steps // 5), 2)
            del g
            st8 = r.label_times(reps=5)
            c4[f"batch{b}"] = step_entry(s4.weight_bytes, b, ms8)
            c4[f"batch{b}_us_per_launch"] = us_per_label(st8)
            detail["config4"][f"batch{b}"] = breakdown_of(st8)
            del r
        del s4
        steps_extra = (("q4_k_m", "qwen3_8b_q4_k_m", torch.float32), ("config1", "config1", torch.float32),
                       ("config2", "config2", torch.bfloat16))
        for name, key, dt in steps_extra:
            log(f"{STEP_NAMES[name]} step ...")
            sx = build_step(torch, d, name, gen)
            cx = {"weight_bytes_per_step": sx.weight_bytes}
            detail[key] = {}
            for b in STEP_BATCHES[name]:
                r = StepRunner(torch, d, ctx, sx, b, dt, dt)
                g = r.capture()
                msx = r.time_graph(g, max(10, args.steps // 2), 3)
                del g
                cx[f"batch{b}"] = step_entry(sx.weight_bytes, b, msx)
                stx = r.label_times(reps=5)
                detail[key][f"batch{b}"] = breakdown_of(stx)
                if name == "config2" or b == 1:
                    cx[f"batch{b}_us_per_launch"] = us_per_label(stx)
                del r
            extra[key] = cx
            del sx
        log("config 0 (rotating pool) ...")
        extra["config0"] = {k: round(v, 4) for k, v in
                            bench_rotating_gemv(torch, d, ctx, d.ENC_Q4_0, 3072, 1024, 1).items()}
        log("config 3 (Q4_0 GEMM) and the dense bf16 GEMM ...")
        c3, c3f = {}, {}
        for m in (128, 512, 2048):
            for (n, k) in [(3072, 1024), (1024, 3072), (2048, 1024)]:
                r = bench_gemm(torch, d, ctx, m, n, k, torch.bfloat16)
                dn_ = bench_dense_gemm(torch, m, n, k)
                rf = bench_gemm(torch, d, ctx, m, n, k, torch.float32)
                c3[f"M{m}_N{n}_K{k}"] = {"us": round(r["us"], 2), "TFLOPs": round(r["TFLOPs"], 1),
                                         "mfma_frac": round(r["mfma_frac"], 4), "eager_us": round(r["eager_us"], 2),
                                         "xf32_us": round(rf["us"], 2), "workspace_bytes": r["workspace_bytes"],
                                         "dense_bf16_us": round(dn_["us"], 2),
                                         "dense_bf16_frac": round(dn_["mfma_frac"], 4)}
        extra["config3_q4_0"] = c3
        log("prefill GEMM, other encodings ...")
        extra["config3_other_encodings_us"] = {
            f"{name}_M512_N{n}_K{k}": round(bench_gemm(torch, d, ctx, 512, n, k, torch.bfloat16, enc=enc)["us"], 2)
            for name, enc in (("q4_1", d.ENC_Q4_1), ("q8_0", d.ENC_Q8_0), ("q6_k", d.ENC_Q6_K), ("q4_k", d.ENC_Q4_K),
                              ("q5_k", d.ENC_Q5_K), ("iq4_xs", d.ENC_IQ4_XS))
            for (n, k) in [(3072, 1024), (1024, 3072)]}
        g512 = c3["M512_N3072_K1024"]
        extra["config3_roofline"] = {"bound": "mfma", "kernel": "xprep + gemm (Q4_0), M512 N3072 K1024, bf16 X and Y",
                                     "achieved": g512["TFLOPs"], "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                     "frac": g512["mfma_frac"], "flops_per_launch": 2 * 512 * 3072 * 1024,
                                     "avg_call_us": g512["us"],
                                     "dense_bf16_same_shape_frac": g512["dense_bf16_frac"],
                                     "timing": "HIP events around graph replays of 20 calls (staging + GEMM, "
                                               "caller workspace); includes the dispatch gaps"}
        log("embedding gather (tied Qwen3 embeddings) ...")
        extra["embedding_gather_GBps"] = {
            f"{name}_n{n}": bench_embedding(torch, d, ctx, enc, 151936, k, n)["GBps"]
            for name, enc, k in (("q6_k_151936x1024", d.ENC_Q6_K, 1024), ("q4_0_151936x4096", d.ENC_Q4_0, 4096))
            for n in (1, 512, 4096)}

    cpu = None
    if not args.no_cpu:
        log("CPU baseline ...")
        cpu = cpu_baseline()

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 in/out, f16-rounded activations, f32 accumulate",
        "data": "synthetic (seeded GGUF blocks in the BASELINE distributions, resident in HBM)",
        "config": {"workload": "BASELINE config 4: Qwen3-8B GGUF decode-step GEMV set (Q4_0 q/k/v/o/gate/up, "
                               "Q6_K down and lm_head), graph-replayed",
                   "batch": args.batch, "weight_bytes_per_step": step_bytes,
                   "launches_per_step": step_launches, "hbm_frac": round(value / HBM_PEAK_GBS, 4),
                   "tokens_per_s": round(args.batch / (ms * 1e-3), 1)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    log("bench detail: " + json.dumps(detail))
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
