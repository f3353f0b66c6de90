"""Benchmark: Llama-3-8B per-layer fused chain on one MI355X.

One step = one decoder layer's hot-path chain on synthetic inputs already
resident in HBM:
    residual-add + RMSNorm        [T, 4096]
    fused RMSNorm + QKV + RoPE    [T, 4096] x [6144, 4096]^T, theta 5e5, bf16 out
    SiLU * mul (SwiGLU)           [T, 2 x 14336] -> [T, 14336]
(the GEMMs between them -- o_proj, gate_up, down -- are not part of this
path).  The headline line is the 8192-token prefill (the QKV projection is
matrix-core bound there); the batch-64 decode chain and the per-forward
embedding gather are reported in the same JSON line.

    python bench.py [--steps K] [--warmup W] [--tokens T] [--no-cpu]

Prints one JSON line.  `value` is microseconds per layer (lower is better):
K chain steps captured into one HIP graph and replayed between HIP events,
i.e. the GPU time of the three kernels back to back without Python launch
gaps; `eager_us_per_layer` is the same chain launched eagerly.  Per-kernel
rows are graph-replayed too.  `roofline` is for the dominant kernel (the QKV projection at
8192 tokens): its algorithmic FLOPs / its own average event-timed duration
against the 2.5 PFLOP/s dense-bf16 peak.  `cpu_baseline` times the oracle's
torch-CPU restatement of the same chain on a bounded token sample and scales
it linearly to T tokens.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from braidinfer_amd import _lib  # noqa: E402
from braidinfer_amd.kernels._qkv import fused_rmsnorm_qkv  # noqa: E402
from braidinfer_amd.layers import RMSNorm, SiluAndMul  # noqa: E402
from braidinfer_amd.layers.embed_head import embedding  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

# Llama-3-8B layer
H, HQ, HKV, D, INTER, VOCAB = 4096, 32, 8, 128, 14336, 128256
N = (HQ + 2 * HKV) * D
THETA, MAXPOS, EPS = 5e5, 8192, 1e-5


def rope_table(d, maxp, base):
    inv_freq = 1.0 / (base ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    t = torch.arange(maxp, dtype=torch.float32)
    freqs = torch.einsum("i,j -> ij", t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


class Chain:
    """Synthetic inputs of one layer at T tokens (seed 5, drawn on the CPU)."""

    def __init__(self, t: int, dev: torch.device, seed: int = 5):
        g = torch.Generator().manual_seed(seed)
        bf = torch.bfloat16

        def randn(*shape, std=1.0, mean=0.0):
            return (torch.randn(*shape, generator=g) * std + mean).to(bf).to(dev)

        self.t = t
        self.x = randn(t, H)
        self.residual = randn(t, H)
        self.norm = RMSNorm(H, eps=EPS).to(dev)
        with torch.no_grad():
            self.norm.weight.data = randn(H, std=0.1, mean=1.0)
        self.hidden = randn(t, H)
        self.ln_w = randn(H, std=0.1, mean=1.0)
        self.w_qkv = randn(N, H, std=0.02)
        self.positions = torch.randint(0, MAXPOS, (t,), generator=g).to(dev)
        self.cache = rope_table(D, MAXPOS, THETA).to(dev)
        self.gate_up = randn(t, 2 * INTER)
        self.silu = SiluAndMul()
        self.out_qkv = torch.empty(t, N, dtype=bf, device=dev)
        self.ids = torch.randint(0, VOCAB, (t,), generator=g).to(dev)

    def qkv(self):
        return fused_rmsnorm_qkv(self.hidden, self.ln_w, self.w_qkv, HQ, HKV, EPS,
                                 mixed_rounding=False, qkv_dtype=torch.float32,
                                 out_dtype=torch.bfloat16, positions=self.positions,
                                 cos_sin_cache=self.cache, out=self.out_qkv)

    def step(self):
        self.norm(self.x, self.residual)
        self.qkv()
        self.silu(self.gate_up)


class QkvStages:
    """Calls the two stages of the fused QKV op directly through the C ABI, so
    each kernel can be timed on its own: the RMSNorm operand pre-pass and the
    MFMA projection with the fused RoPE epilogue."""

    def __init__(self, c: Chain, dev):
        self.c = c
        self.dev = dev
        ws = _lib.call("bfa_fused_rmsnorm_qkv_workspace_size", c.t, H, N, D)
        self.op_bytes = (c.t * H * 2 + 255) // 256 * 256
        self.ws = torch.empty(max(ws, 16), dtype=torch.uint8, device=dev)
        self.status = _lib.status_word(dev)

    def operand(self):
        c = self.c
        _lib.call("bfa_rmsnorm_qkv_operand", _lib.ptr(c.hidden), _lib.BF16, c.t, H, H,
                  _lib.ptr(c.ln_w), _lib.BF16, 0, _lib.ptr(self.ws), _lib.BF16, EPS,
                  _lib.stream_of(self.dev))

    def projection(self):
        c = self.c
        part = self.ws.data_ptr() + self.op_bytes
        _lib.call("bfa_qkv_projection", _lib.ptr(self.ws), c.t, H, _lib.ptr(c.w_qkv), _lib.BF16, N, H,
                  None, 0, HQ, HKV, _lib.F32, None, None, 0, 0.0, _lib.BF16,
                  _lib.ptr(c.positions), _lib.I64, _lib.ptr(c.cache), MAXPOS,
                  _lib.ptr(c.out_qkv), _lib.BF16, N, _lib.c_void_p(part),
                  self.ws.numel() - self.op_bytes, _lib.ptr(self.status), _lib.stream_of(self.dev))


def time_fn(fn, iters: int, warmup: int = 3) -> float:
    """Average milliseconds per call, HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters


def kernel_table(c: Chain, dev, iters: int) -> dict:
    """Per-kernel event timing with algorithmic bytes / FLOPs and roofline fractions."""
    t = c.t
    st = QkvStages(c, dev)
    rows = {}

    def add(name, fn, nbytes, flops=0.0):
        rows[name] = _roof_row(time_graph(fn, iters), nbytes, flops)

    add("add_rms_norm", lambda: c.norm(c.x, c.residual), 4 * t * H * 2 + H * 2)
    add("qkv_operand_prepass", st.operand, 2 * t * H * 2 + H * 2)
    add("qkv_projection_rope", st.projection,
        t * H * 2 + N * H * 2 + t * N * 2 + t * 8 + t * D * 4, 2.0 * t * H * N)
    add("fused_rmsnorm_qkv_rope", c.qkv,
        t * H * 2 + H * 2 + N * H * 2 + t * N * 2 + t * 8 + t * D * 4, 2.0 * t * H * N)
    add("silu_and_mul", lambda: c.silu(c.gate_up), 3 * t * INTER * 2)
    table = torch.empty(VOCAB, H, dtype=torch.bfloat16, device=dev).normal_(0, 0.02)
    add("embedding_gather", lambda: embedding(c.ids, table), 2 * t * H * 2 + 8 * t)
    del table
    return rows


def _roof_row(ms: float, nbytes: float, flops: float = 0.0) -> dict:
    gbs = nbytes / (ms * 1e-3) / 1e9
    row = {"us": round(ms * 1e3, 3), "bytes": int(nbytes), "gbs": round(gbs, 1),
           "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    if flops:
        tf = flops / (ms * 1e-3) / 1e12
        row.update({"flops": flops, "tflops": round(tf, 1), "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4)})
    return row


def config_cases(dev) -> list:
    """The path's other workloads as (name, fn, algorithmic bytes, FLOPs), inputs
    drawn per configuration (seeds 1-4, CPU generator, fp32 then bf16):
      rmsnorm     TinyLlama RMSNorm, x [128, 2048], eps 1e-5
      tinyllama   fused RMSNorm+QKV(2048 -> 2560, 32/4 heads, D 64)+RoPE(theta 1e4), T 1/8/512
      qwen3       fused RMSNorm+QKV(1024 -> 4096, 16/8 heads, D 128)+q/k norm+RoPE(theta 1e6), T 1/2048
      rerotate    paged K [256 pages, 2, 8, 16, 128] in shuffled page order, 16 chunks of
                  16 pages, delta U[-4096, 4096], theta 1e6, rotated copy out
      swiglu      SiLU*mul [2048, 2 x 3072]
      kv_append   paged KV append, 8 kv heads x 128, page 16: 8192-token prefill,
                  and a 64-sequence decode batch in one launch
      cascade     paged cascade attention over 4096 cached Qwen3 tokens (16 moved
                  chunks, k_norm), 1 and 256 query tokens
      linear      gate_up+SiluAndMul, down_proj+residual, o_proj+residual at
                  Llama-3-8B shapes, T 8192 and 64"""
    from braidinfer_amd.layers import llama_attention_input, qwen3_attention_input, rerotate_paged_k
    bf = torch.bfloat16
    cases = []

    def gen(seed):
        g = torch.Generator().manual_seed(seed)

        def randn(*shape, std=1.0, mean=0.0):
            return (torch.randn(*shape, generator=g) * std + mean).to(bf).to(dev)
        return g, randn

    g, randn = gen(1)
    x = randn(128, 2048)
    norm = RMSNorm(2048, eps=1e-5).to(dev)
    with torch.no_grad():
        norm.weight.data = randn(2048, std=0.1, mean=1.0)
    cases.append(("rmsnorm_t128_h2048", lambda: norm(x), 2 * 128 * 2048 * 2 + 2048 * 2, 0.0))

    def tiny(t, h=2048, hq=32, hkv=4, d=64):
        n = (hq + 2 * hkv) * d
        xt, ln, w = randn(t, h), randn(h, std=0.1, mean=1.0), randn(n, h, std=0.02)
        pos = torch.randint(0, 2048, (t,), generator=g).to(dev)
        cache = rope_table(d, 2048, 1e4).to(dev)
        return (f"tinyllama_qkv_rope_t{t}", lambda: llama_attention_input(xt, ln, w, hq, hkv, 1e-5, pos, cache),
                t * h * 2 + h * 2 + n * h * 2 + t * n * 2 + t * 8 + t * d * 4, 2.0 * t * h * n)

    g, randn = gen(2)
    cases += [tiny(t) for t in (1, 8, 512)]

    def qwen(t, h=1024, hq=16, hkv=8, d=128):
        n = (hq + 2 * hkv) * d
        xt, w, ln = randn(t, h), randn(n, h, std=0.02), randn(h, std=0.1, mean=1.0)
        qn = randn(d, std=0.1, mean=1.0)
        kn = torch.exp(torch.empty(d).uniform_(-2.995732, 4.605170, generator=g)).to(bf).to(dev)
        pos = torch.randint(0, 2048, (t,), generator=g).to(dev)
        cache = rope_table(d, 40960, 1e6).to(dev)
        return (f"qwen3_qkv_qknorm_rope_t{t}",
                lambda: qwen3_attention_input(xt, ln, w, None, hq, hkv, 1e-6, pos, cache, qn, kn),
                t * h * 2 + h * 2 + n * h * 2 + t * n * 2 + t * 8 + t * d * 4 + 2 * d * 2, 2.0 * t * h * n)

    g, randn = gen(3)
    cases += [qwen(t) for t in (1, 2048)]

    g, randn = gen(4)
    pages, hkv, ps, d = 256, 8, 16, 128
    kv = randn(pages, 2, hkv, ps, d)
    page_idx = torch.randperm(pages, generator=g).to(torch.int32).to(dev)
    indptr = (torch.arange(17, dtype=torch.int32) * 16).to(dev)
    delta = torch.randint(-4096, 4097, (16,), generator=g).to(dev)
    last = torch.full((16,), ps, dtype=torch.int32, device=dev)
    rcache = rope_table(d, 40960, 1e6).to(dev)
    rout = torch.empty(pages, ps, hkv, d, dtype=bf, device=dev)
    cases.append(("rerotate_paged_k_4096tok",
                  lambda: rerotate_paged_k(kv, page_idx, indptr, delta, last, rcache, out=rout),
                  2 * pages * ps * hkv * d * 2, 0.0))
    gu = randn(2048, 2 * 3072)
    silu = SiluAndMul()
    cases.append(("swiglu_t2048_i3072", lambda: silu(gu), 3 * 2048 * 3072 * 2, 0.0))

    # paged KV append at Llama-3-8B kv geometry (8 heads x 128, page 16, HND):
    # an 8192-token prefill into 512 of 1024 shuffled pages, and a 64-sequence
    # decode batch (one new token each) in one batched launch
    cases += kv_append_cases(dev)
    cases += cascade_cases(dev)
    cases += linear_cases(dev)
    return cases


def linear_cases(dev) -> list:
    """GEMM-epilogue fusions at Llama-3-8B layer shapes (seed 8): gate_up_proj with
    SiluAndMul (4096 -> 2 x 14336 -> 14336), down_proj + residual (14336 -> 4096)
    and o_proj + residual (4096 -> 4096), for an 8192-token prefill and a 64-token
    decode batch.  Algorithmic bytes: operand, weight, residual and output once."""
    from braidinfer_amd.layers import gate_up_silu_and_mul, linear_add_residual
    g = torch.Generator().manual_seed(8)
    bf = torch.bfloat16
    h, inter = 4096, 14336

    def randn(*shape, std=1.0):
        return (torch.randn(*shape, generator=g) * std).to(bf).to(dev)

    w_gu, w_down, w_o = randn(2 * inter, h, std=0.02), randn(h, inter, std=0.01), randn(h, h, std=0.02)
    out = []
    for t in (8192, 64):
        x, xi, res = randn(t, h), randn(t, inter), randn(t, h)
        out += [
            (f"gate_up_silu_llama3_8b_t{t}", (lambda x=x: gate_up_silu_and_mul(x, w_gu)),
             (t * h + 2 * inter * h + t * inter) * 2, 2.0 * t * h * 2 * inter),
            (f"down_proj_residual_llama3_8b_t{t}", (lambda xi=xi, res=res: linear_add_residual(xi, w_down, res)),
             (t * inter + inter * h + 2 * t * h) * 2, 2.0 * t * inter * h),
            (f"o_proj_residual_llama3_8b_t{t}", (lambda x=x, res=res: linear_add_residual(x, w_o, res)),
             (2 * t * h + h * h + t * h) * 2, 2.0 * t * h * h),
        ]
    return out


def kv_append_cases(dev) -> list:
    """Paged KV append cases (seed 6), own scope so the lambdas bind their own tensors."""
    from braidinfer_amd.kernels import append_paged_kv_batch, append_to_paged_kv_cache_custom
    g = torch.Generator().manual_seed(6)
    bf = torch.bfloat16

    def randn(*shape):
        return torch.randn(*shape, generator=g).to(bf).to(dev)

    hkv, d, ps, pages = 8, 128, 16, 1024
    cache = randn(pages, 2, hkv, ps, d)
    table = torch.randperm(pages, generator=g)[:512].to(torch.int32).to(dev)
    kp, vp = randn(8192, hkv, d), randn(8192, hkv, d)
    pp = torch.arange(8192, dtype=torch.int32, device=dev)
    lens = torch.randint(0, 4000, (64,), generator=g)
    perm = torch.randperm(pages, generator=g)
    # sequence s: a table of lens[s] // 16 + 1 entries whose last (the one written) is a
    # page of its own
    per = lens // ps + 1
    ind = torch.cat([perm[s].repeat(int(per[s])) for s in range(64)]).to(torch.int32).to(dev)
    indptr = torch.cat([torch.zeros(1, dtype=torch.int64), per.cumsum(0)]).to(torch.int32).to(dev)
    bat = torch.arange(64, device=dev)
    pd = lens.to(dev)
    kd, vd = randn(64, hkv, d), randn(64, hkv, d)
    return [("kv_append_t8192", lambda: append_to_paged_kv_cache_custom(kp, vp, cache, table, pp, ps),
             4 * 8192 * hkv * d * 2 + 8192 * 4 + 512 * 4, 0.0),
            ("kv_append_batch_b64", lambda: append_paged_kv_batch(kd, vd, cache, ind, indptr, bat, pd, ps),
             4 * 64 * hkv * d * 2 + 64 * (8 + 8 + 4) + 65 * 4, 0.0)]


def cascade_cases(dev) -> list:
    """Cascade attention at Qwen3-0.6B shape (seed 7): 4096 cached tokens in 16 chunks of
    256, shuffled 16-token HND pages, each chunk moved by a delta in [-4096, 4096]
    (theta 1e6, rotary table 40960), k_norm with log-uniform weights; 16 query heads
    over 8 kv heads of 128.  A one-token decode step and a 256-token query chunk."""
    import math as _m
    from types import SimpleNamespace
    from braidinfer_amd.layers import CascadeAttention, RMSNorm, RotaryEmbedding
    g = torch.Generator().manual_seed(7)
    bf = torch.bfloat16
    hq, hkv, d, ps, pages = 16, 8, 128, 16, 512
    kv = torch.randn(pages, 2, hkv, ps, d, generator=g).to(bf).to(dev)
    perm = torch.randperm(pages, generator=g).tolist()
    deltas = torch.randint(-4096, 4097, (16,), generator=g).tolist()
    chunks = [SimpleNamespace(page_table=perm[16 * c:16 * c + 16], kv_length=256,
                              cached_position_start=8192 + 256 * c,
                              global_position_start=8192 + 256 * c + deltas[c],
                              chunk_type=SimpleNamespace(value="system_prompt" if c == 0 else "context"))
              for c in range(16)]
    rope = RotaryEmbedding(d, d, 40960, 1e6).to(dev)
    att = CascadeAttention(hq, d, d ** -0.5, hkv, ps, rotary_emb=rope)
    levels = att.create_cascade_levels(chunks)
    k_norm = RMSNorm(d, eps=1e-6).to(dev)
    with torch.no_grad():
        k_norm.weight.data = torch.exp(torch.empty(d).uniform_(_m.log(0.05), _m.log(100.0), generator=g)).to(bf).to(dev)
    kv_bytes = 4096 * hkv * d * 2 * 2
    out = []
    for t in (1, 256):
        q = torch.randn(t, hq, d, generator=g).to(bf).to(dev)
        qpos = torch.arange(4096 - t + 1, 4097, device=dev)
        out.append((f"cascade_attention_qwen3_4096kv_t{t}",
                    (lambda q=q, qpos=qpos: att.forward(q, qpos, kv, levels, 0, k_norm=k_norm)),
                    kv_bytes + 2 * t * hq * d * 2, 4.0 * t * hq * 4096 * d))
    return out


def config_table(dev, iters: int) -> dict:
    """Each case of config_cases graph-timed, with its roofline fractions."""
    return {name: _roof_row(time_graph(fn, iters), nbytes, flops)
            for name, fn, nbytes, flops in config_cases(dev)}


def _capture(fn, reps: int) -> torch.cuda.CUDAGraph:
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    return graph


def _settle(graph: torch.cuda.CUDAGraph, min_s: float) -> None:
    """Replays `graph` until `min_s` seconds have passed: the GPU clock ramps up
    over the first ~100 ms of sustained load, so a measurement that starts cold
    reads up to 30 % slow."""
    t0 = time.perf_counter()
    while True:
        graph.replay()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= min_s:
            return


def time_graph(fn, iters: int, reps: int = 20, settle_s: float = 0.2) -> float:
    """Average milliseconds per call of `fn` captured `reps` times into one HIP
    graph and replayed (after `settle_s` seconds of untimed replays): the GPU
    time of the kernels without Python launch gaps."""
    graph = _capture(fn, reps)
    _settle(graph, settle_s)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = max(1, iters // reps)
    s.record()
    for _ in range(n):
        graph.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / (n * reps)


def time_cold(fn, iters: int, flush: torch.Tensor) -> float:
    """Average milliseconds per call with the 256 MB Infinity Cache flushed
    before each call by reading a 512 MB buffer (a read leaves no dirty lines
    whose write-back would overlap the timed call); each call is bracketed by
    its own events."""
    fn()
    sink = torch.empty((), device=flush.device)
    pairs = []
    for _ in range(iters):
        torch.sum(flush, dim=0, out=sink)
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        pairs.append((s, e))
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in pairs) / iters


def cold_decode_table(dev, t: int, iters: int) -> dict:
    """Decode-shape kernels streaming their operands from HBM (cache flushed)."""
    c = Chain(t, dev)
    flush = torch.empty(512 * 2**20 // 4, dtype=torch.float32, device=dev)
    out = {}
    for name, fn, nbytes in (
        ("add_rms_norm", lambda: c.norm(c.x, c.residual), 4 * t * H * 2 + H * 2),
        ("fused_rmsnorm_qkv_rope", c.qkv,
         t * H * 2 + H * 2 + N * H * 2 + t * N * 2 + t * 8 + t * D * 4),
        ("silu_and_mul", lambda: c.silu(c.gate_up), 3 * t * INTER * 2),
    ):
        ms = time_cold(fn, iters, flush)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 3), "gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    del c, flush
    return out


def chain_graph_us(c: Chain, steps: int, warmup: int) -> float:
    """Microseconds per chain step: `steps` steps captured into one HIP graph;
    `warmup` untimed steps (whole replays of the graph, at least one), then
    exactly `steps` timed steps between HIP events."""
    graph = _capture(c.step, steps)
    done = 0
    while done < max(warmup, 1):
        graph.replay()
        done += steps
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    graph.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps * 1e3


def chain_us(c: Chain, steps: int, warmup: int) -> float:
    for _ in range(warmup):
        c.step()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        c.step()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps * 1e3


def cpu_baseline(t_full: int, budget_s: float = 12.0) -> dict:
    """The oracle's torch-CPU restatement of the same chain on a token sample,
    scaled linearly to t_full tokens (rows of every op are independent)."""
    from oracle import torch_ref as R
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    ts = 256
    g = torch.Generator().manual_seed(5)
    bf = torch.bfloat16
    x = torch.randn(ts, H, generator=g).to(bf)
    res = torch.randn(ts, H, generator=g).to(bf)
    w = (torch.randn(H, generator=g) * 0.1 + 1).to(bf)
    wq = (torch.randn(N, H, generator=g) * 0.02).to(bf)
    pos = torch.randint(0, MAXPOS, (ts,), generator=g)
    cache = rope_table(D, MAXPOS, THETA)
    gu = torch.randn(ts, 2 * INTER, generator=g).to(bf)

    def step():
        R.add_rms_forward(x, res, w, EPS)
        R.llama_attention_input(x, w, wq, HQ, HKV, EPS, pos, cache)
        R.silu_and_mul(gu)

    step()
    times = []
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s and len(times) < 30:
        s = time.perf_counter()
        step()
        times.append(time.perf_counter() - s)
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(med * 1e6 * t_full / ts, 1), "unit": "us/layer", "cores": threads,
            "kind": "port",
            "sample": f"oracle torch-CPU chain (add_rms_forward, llama attention input: minimal_f32 "
                      f"QKV + RoPE, silu_and_mul) at {ts} tokens, median of {len(times)} runs, "
                      f"scaled x{t_full / ts:g} to {t_full} tokens; torch {torch.__version__}"}


def read_traffic(name: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE),
    recorded in profiles/<name>.txt as a `traffic_bytes: N` line."""
    p = ROOT / "profiles" / f"{name}.txt"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("traffic_bytes:"):
            return int(float(line.split(":", 1)[1]))
    return None


def profile_one(kernel: str, tokens: int, steps: int, dev) -> int:
    """Runs one kernel `steps` times on the chain's inputs (or one case of
    config_cases by name); prints its event-timed average."""
    cases = {name: fn for name, fn, _, _ in config_cases(dev)} if kernel.startswith("case:") else {}
    if cases:
        ms = time_fn(cases[kernel[5:]], steps)
        print(json.dumps({"kernel": kernel, "calls": steps, "us": round(ms * 1e3, 3)}))
        return 0
    c = Chain(tokens, dev)
    st = QkvStages(c, dev)
    table = torch.empty(VOCAB, H, dtype=torch.bfloat16, device=dev) if kernel == "embedding" else None
    if kernel == "copy":
        # calibration for the HBM byte counters: a 512 MiB device-to-device copy
        # reads and writes exactly 512 MiB
        src = torch.empty(256 << 20, dtype=torch.bfloat16, device=dev).normal_()
        dst = torch.empty_like(src)
        ms = time_fn(lambda: dst.copy_(src), steps)
        print(json.dumps({"kernel": "copy", "bytes_read": src.numel() * 2, "bytes_written": dst.numel() * 2,
                          "calls": steps, "us": round(ms * 1e3, 3)}))
        return 0
    if kernel == "library_gemm":
        # the projection's product alone through torch.mm (hipBLASLt, bf16 out, no
        # epilogue): a reference point for qkv_projection's hardware counters
        wt, out = c.w_qkv.t(), torch.empty(tokens, N, dtype=torch.bfloat16, device=dev)
        ms = time_fn(lambda: torch.mm(c.hidden, wt, out=out), steps)
        print(json.dumps({"kernel": kernel, "tokens": tokens, "calls": steps, "us": round(ms * 1e3, 3)}))
        return 0
    fn = {"qkv_projection": st.projection, "qkv_operand": st.operand,
          "add_rms_norm": lambda: c.norm(c.x, c.residual), "silu_and_mul": lambda: c.silu(c.gate_up),
          "embedding": lambda: embedding(c.ids, table)}[kernel]
    ms = time_fn(fn, steps)
    print(json.dumps({"kernel": kernel, "tokens": tokens, "calls": steps, "us": round(ms * 1e3, 3)}))
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--tokens", type=int, default=8192)
    ap.add_argument("--decode-tokens", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-cold", action="store_true", help="skip the cold-cache decode table")
    ap.add_argument("--kernel", help="only run this kernel --steps times at --tokens (for "
                    "profilers): qkv_projection, qkv_operand, add_rms_norm, silu_and_mul, "
                    "embedding, copy, library_gemm (the projection's product through torch.mm), or "
                    "case:<name> for a case of the configuration table")
    args = ap.parse_args(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print("bench.py: this path is measured on one GPU only (the fused per-layer kernels "
              "shard by tokens or heads with no exchange); --gpus > 1 is not supported",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _lib.load()
    if args.kernel:
        return profile_one(args.kernel, args.tokens, args.steps, dev)

    def progress(stage: str) -> None:
        print(f"bench: {stage}", file=sys.stderr, flush=True)

    progress(f"prefill chain, {args.tokens} tokens")
    prefill = Chain(args.tokens, dev)
    us_eager = chain_us(prefill, args.steps, args.warmup)
    us = chain_graph_us(prefill, args.steps, args.warmup)
    kp = kernel_table(prefill, dev, max(10, args.steps))
    proj = kp["qkv_projection_rope"]
    del prefill
    torch.cuda.empty_cache()

    progress(f"decode chain, {args.decode_tokens} tokens")
    decode = Chain(args.decode_tokens, dev)
    us_dec_eager = chain_us(decode, max(args.steps, 100), args.warmup)
    us_dec = chain_graph_us(decode, max(args.steps, 100), max(args.warmup, 1000))
    kd = kernel_table(decode, dev, max(50, args.steps))
    del decode
    torch.cuda.empty_cache()
    cold = None if args.no_cold else cold_decode_table(dev, args.decode_tokens, 48)
    progress("other configurations")
    configs = config_table(dev, max(40, args.steps))
    _lib.check_device_status(dev)

    line = {
        "metric": "us/layer + % HBM / % MFMA peak, fused norm+QKV+RoPE+SwiGLU, 1 MI355X",
        "value": round(us, 2),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights, Llama-3-8B shapes)",
        "config": {"workload": f"Llama-3-8B layer chain, {args.tokens}-token prefill: add+RMSNorm "
                               f"[{args.tokens},4096] -> fused RMSNorm+QKV(4096->6144)+RoPE(theta 5e5) "
                               f"-> SiLU*mul [{args.tokens},2x14336]",
                   "tokens": args.tokens, "hidden": H, "q_heads": HQ, "kv_heads": HKV,
                   "head_dim": D, "intermediate": INTER},
        "roofline": {"bound": "mfma", "kernel": "qkv_projection_rope",
                     "achieved": proj["tflops"], "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": proj["mfma_frac"],
                     "traffic": read_traffic(f"traffic_qkv_projection_llama3_8b_t{args.tokens}")},
        "kernels_prefill": kp,
        "eager_us_per_layer": round(us_eager, 2),
        "decode": {"tokens": args.decode_tokens, "us_per_layer": round(us_dec, 2),
                   "eager_us_per_layer": round(us_dec_eager, 2),
                   "kernels_warm": kd, "kernels_cold": cold},
        "configs": configs,
    }
    if not args.no_cpu:
        progress("CPU baseline")
        line["cpu_baseline"] = cpu_baseline(args.tokens)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
