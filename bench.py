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
K chain steps captured into one HIP graph and replayed between HIP events
after the clock has settled, i.e. the GPU time of the three kernels back to
back without Python launch gaps; `eager_us_per_layer` is the same chain
launched eagerly; `rotating_weights_us_per_layer` is the graph-replayed chain
with the QKV weight taken from four copies in turn, as a model's consecutive
layers would (the repeated chain keeps its one weight in the Infinity Cache).  Every (kernel, workload) row -- kernels_prefill,
decode.kernels, configs -- carries:
    us, gbs / tflops, hbm_frac / mfma_frac   warm, graph-replayed
    us_cold, hbm_frac_cold                   Infinity Cache flushed before each call
    cpu_us, cpu_reps                         the oracle's torch-CPU restatement of the
                                             reference at the row's full size, median
    vs_oracle                                bit-exact, or max_abs / max_rel_normwise /
                                             allclose / beyond_tol_elements against the
                                             oracle (the reference's own rounding points)
    vs_fp32, oracle_vs_fp32                  float rows: the same figures against the fp32
                                             mode of the oracle (every op chain in fp32,
                                             one rounding: the "fp32 reference after bf16
                                             rounding" of the accuracy target), for the GPU
                                             result and for the reference's own rounding
`roofline` is for the dominant kernel (the QKV projection at 8192 tokens):
its algorithmic FLOPs / its own average event-timed duration against the
2.5 PFLOP/s dense-bf16 peak.  `cpu_baseline` is the sum of the three chain
ops' CPU times at the full token count; `cpu` records the host's CPU model,
threads and torch's parallel_info.
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
        self.cpu = {}

        def randn(name, *shape, std=1.0, mean=0.0):
            v = (torch.randn(*shape, generator=g) * std + mean).to(bf)
            self.cpu[name] = v
            return v.to(dev)

        self.t = t
        self.x = randn("x", t, H)
        self.residual = randn("residual", t, H)
        self.norm = RMSNorm(H, eps=EPS).to(dev)
        with torch.no_grad():
            self.norm.weight.data = randn("norm_w", H, std=0.1, mean=1.0)
        self.hidden = randn("hidden", t, H)
        self.ln_w = randn("ln_w", H, std=0.1, mean=1.0)
        self.w_qkv = randn("w_qkv", N, H, std=0.02)
        self.cpu["positions"] = torch.randint(0, MAXPOS, (t,), generator=g)
        self.positions = self.cpu["positions"].to(dev)
        self.cpu["cache"] = rope_table(D, MAXPOS, THETA)
        self.cache = self.cpu["cache"].to(dev)
        self.gate_up = randn("gate_up", t, 2 * INTER)
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
    """Calls the stages of the fused QKV op directly through the C ABI, so each
    kernel can be timed on its own: the row statistic (the first stage of the
    Llama chain's fused op, whose projection reads x with the norm weight folded
    into W), the RMSNorm operand pre-pass (the first stage of the mixed-rounding
    variants) and the MFMA projection with the fused RoPE epilogue, the same
    kernel as the fused op's, timed on the pre-pass operand (filled here once,
    so that it multiplies real data: on an operand of zeros the power-limited
    kernel runs much faster)."""

    def __init__(self, c: Chain, dev):
        self.c = c
        self.dev = dev
        ws = _lib.call("bfa_fused_rmsnorm_qkv_workspace_size", c.t, H, N, D)
        self.op_bytes = (c.t * H * 2 + 255) // 256 * 256
        self.ws = torch.empty(max(ws, 16), dtype=torch.uint8, device=dev)
        self.rs = torch.empty(c.t, dtype=torch.float32, device=dev)
        self.status = _lib.status_word(dev)
        self.operand()

    def operand(self):
        c = self.c
        _lib.call("bfa_rmsnorm_qkv_operand", _lib.ptr(c.hidden), _lib.BF16, c.t, H, H,
                  _lib.ptr(c.ln_w), _lib.BF16, 0, _lib.ptr(self.ws), _lib.BF16, EPS,
                  _lib.stream_of(self.dev))

    def row_statistic(self):
        c = self.c
        _lib.call("bfa_rmsnorm_row_scale", _lib.ptr(c.hidden), _lib.BF16, c.t, H, H, _lib.ptr(self.rs), EPS,
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


class Row:
    """One (kernel, workload) measurement.  `fn` runs the op on device inputs and
    returns what it produced; `ref` (optional) computes the oracle's result for
    the same inputs on the CPU, and `got` maps fn's output to the tensor(s)
    compared with it.  exact: integer/byte ops compared bit for bit."""

    def __init__(self, name, fn, nbytes, flops=0.0, ref=None, got=None, exact=False, note=None, ref32=None):
        self.name, self.fn, self.nbytes, self.flops = name, fn, nbytes, flops
        self.ref, self.got, self.exact, self.note = ref, got, exact, note
        self.ref32 = ref32  # the fp32 mode of the oracle (float rows)


def chain_rows(c: Chain, dev, stages: bool) -> list:
    """The chain's kernels at c.t tokens; `stages` adds the stages of the fused
    QKV op (row statistic, projection) as rows of their own."""
    t = c.t
    rows = [Row("add_rms_norm", lambda: c.norm(c.x, c.residual)[0], 4 * t * H * 2 + H * 2,
                ref=lambda: _oracle().add_rms_forward(c.cpu["x"], c.cpu["residual"], c.cpu["norm_w"], EPS)[0],
                ref32=lambda: _oracle32().add_rms_forward(c.cpu["x"], c.cpu["residual"], c.cpu["norm_w"], EPS)[0])]
    if stages:
        st = QkvStages(c, dev)
        rows += [Row("qkv_row_statistic", st.row_statistic, t * H * 2 + t * 4,
                     note="stage of the fused op (1 / rms per row)"),
                 Row("qkv_projection_rope", st.projection,
                     t * H * 2 + N * H * 2 + t * N * 2 + t * 8 + t * D * 4, 2.0 * t * H * N,
                     note="the fused op's projection kernel, timed on the pre-pass operand (in the fused "
                          "op it reads x, with the norm weight folded into W and a scale per row)")]

    def llama_ref(o=_oracle):
        q, k, v = o().llama_attention_input(c.cpu["hidden"], c.cpu["ln_w"], c.cpu["w_qkv"], HQ, HKV, EPS,
                                            c.cpu["positions"], c.cpu["cache"])
        return torch.cat([q, k, v], 1)
    rows += [Row("fused_rmsnorm_qkv_rope", c.qkv, t * H * 2 + H * 2 + N * H * 2 + t * N * 2 + t * 8 + t * D * 4,
                 2.0 * t * H * N, ref=llama_ref, ref32=lambda: llama_ref(_oracle32)),
             Row("silu_and_mul", lambda: c.silu(c.gate_up), 3 * t * INTER * 2,
                 ref=lambda: _oracle().silu_and_mul(c.cpu["gate_up"]),
                 ref32=lambda: _oracle32().silu_and_mul(c.cpu["gate_up"]))]
    table = torch.empty(VOCAB, H, dtype=torch.bfloat16, device=dev).normal_(0, 0.02)
    host = {}

    def gather_ref():
        if not host:  # one host copy of the table and ids, in the untimed first run
            host["table"], host["ids"] = table.cpu(), c.ids.cpu()
        return _oracle().embedding(host["ids"], host["table"])
    rows.append(Row("embedding_gather", lambda: embedding(c.ids, table), 2 * t * H * 2 + 8 * t,
                    ref=gather_ref, exact=True))
    return rows


def _roof_row(ms: float, nbytes: float, flops: float = 0.0) -> dict:
    gbs = nbytes / (ms * 1e-3) / 1e9
    row = {"us": round(ms * 1e3, 3), "bytes": int(nbytes), "gbs": round(gbs, 1),
           "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    if flops:
        tf = flops / (ms * 1e-3) / 1e12
        row.update({"flops": flops, "tflops": round(tf, 1), "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4)})
    return row


def _oracle():
    """The CPU restatement of the reference (oracle/): imported only by the CPU
    leg, which times it and checks the GPU results against it."""
    from oracle import torch_ref
    return torch_ref


def _oracle32():
    """The fp32 mode of the oracle (oracle/fp32_ref.py), for the vs_fp32 figures."""
    from oracle import fp32_ref
    return fp32_ref


class _Gen:
    """Seeded CPU generator: draws fp32, rounds to bf16, keeps the CPU copy."""

    def __init__(self, seed, dev):
        self.g = torch.Generator().manual_seed(seed)
        self.dev = dev

    def randn(self, *shape, std=1.0, mean=0.0):
        v = (torch.randn(*shape, generator=self.g) * std + mean).to(torch.bfloat16)
        return v, v.to(self.dev)


def config_cases(dev) -> list:
    """The path's other workloads, inputs drawn per configuration (seeds 1-4,
    CPU generator, fp32 then bf16):
      rmsnorm     TinyLlama RMSNorm, x [128, 2048], eps 1e-5
      tinyllama   fused RMSNorm+QKV(2048 -> 2560, 32/4 heads, D 64)+RoPE(theta 1e4), T 1/8/512
      qwen3       fused RMSNorm+QKV(1024 -> 4096, 16/8 heads, D 128)+q/k norm+RoPE(theta 1e6), T 1/2048
      rerotate    paged K [256 pages, 2, 8, 16, 128] in shuffled page order, 16 chunks of
                  16 pages, delta U[-4096, 4096], theta 1e6, rotated copy out
      swiglu      SiLU*mul [2048, 2 x 3072]
      kv_append   paged KV append, 8 kv heads x 128, page 16: 8192-token prefill,
                  and a 64-sequence decode batch in one launch
      cascade     paged cascade attention over 4096 cached Qwen3 tokens (16 moved
                  chunks, k_norm) and 2048 cached TinyLlama tokens (head_dim 64),
                  1 and 256 query tokens
      linear      gate_up+SiluAndMul, down_proj+residual, o_proj+residual at
                  Llama-3-8B shapes, T 8192 and 64"""
    from braidinfer_amd.layers import llama_attention_input, qwen3_attention_input, rerotate_paged_k
    bf = torch.bfloat16
    rows = []

    r = _Gen(1, dev)
    xc, x = r.randn(128, 2048)
    wc, w = r.randn(2048, std=0.1, mean=1.0)
    norm = RMSNorm(2048, eps=1e-5).to(dev)
    with torch.no_grad():
        norm.weight.data = w
    rows.append(Row("rmsnorm_t128_h2048", lambda: norm(x), 2 * 128 * 2048 * 2 + 2048 * 2,
                    ref=lambda: _oracle().rms_forward(xc, wc, 1e-5),
                    ref32=lambda: _oracle32().rms_forward(xc, wc, 1e-5)))

    def cat3(qkv):
        return torch.cat([t.reshape(t.shape[0], -1) for t in qkv], 1)

    def tiny(r, t, h=2048, hq=32, hkv=4, d=64):
        n = (hq + 2 * hkv) * d
        (xc, xt), (lc, ln), (wc, w) = r.randn(t, h), r.randn(h, std=0.1, mean=1.0), r.randn(n, h, std=0.02)
        pc = torch.randint(0, 2048, (t,), generator=r.g)
        cc = rope_table(d, 2048, 1e4)
        pos, cache = pc.to(dev), cc.to(dev)
        return Row(f"tinyllama_qkv_rope_t{t}", lambda: llama_attention_input(xt, ln, w, hq, hkv, 1e-5, pos, cache),
                   t * h * 2 + h * 2 + n * h * 2 + t * n * 2 + t * 8 + t * d * 4, 2.0 * t * h * n,
                   ref=lambda: cat3(_oracle().llama_attention_input(xc, lc, wc, hq, hkv, 1e-5, pc, cc)), got=cat3,
                   ref32=lambda: cat3(_oracle32().llama_attention_input(xc, lc, wc, hq, hkv, 1e-5, pc, cc)))

    r = _Gen(2, dev)
    rows += [tiny(r, t) for t in (1, 8, 512)]

    def qwen(r, t, h=1024, hq=16, hkv=8, d=128):
        n = (hq + 2 * hkv) * d
        (xc, xt), (wc, w), (lc, ln) = r.randn(t, h), r.randn(n, h, std=0.02), r.randn(h, std=0.1, mean=1.0)
        qc, qn = r.randn(d, std=0.1, mean=1.0)
        kc = torch.exp(torch.empty(d).uniform_(-2.995732, 4.605170, generator=r.g)).to(bf)
        kn = kc.to(dev)
        pc = torch.randint(0, 2048, (t,), generator=r.g)
        cc = rope_table(d, 40960, 1e6)
        pos, cache = pc.to(dev), cc.to(dev)
        return Row(f"qwen3_qkv_qknorm_rope_t{t}",
                   lambda: qwen3_attention_input(xt, ln, w, None, hq, hkv, 1e-6, pos, cache, qn, kn),
                   t * h * 2 + h * 2 + n * h * 2 + t * n * 2 + t * 8 + t * d * 4 + 2 * d * 2, 2.0 * t * h * n,
                   ref=lambda: cat3(_oracle().qwen3_attention_input(xc, lc, wc, None, hq, hkv, 1e-6, pc, cc, qc, kc)),
                   got=cat3,
                   ref32=lambda: cat3(_oracle32().qwen3_attention_input(xc, lc, wc, None, hq, hkv, 1e-6, pc, cc,
                                                                        qc, kc)))

    r = _Gen(3, dev)
    rows += [qwen(r, t) for t in (1, 2048)]

    r = _Gen(4, dev)
    pages, hkv, ps, d = 256, 8, 16, 128
    kvc, kv = r.randn(pages, 2, hkv, ps, d)
    pic = torch.randperm(pages, generator=r.g).to(torch.int32)
    ipc = torch.arange(17, dtype=torch.int32) * 16
    dc = torch.randint(-4096, 4097, (16,), generator=r.g)
    lpc = torch.full((16,), ps, dtype=torch.int32)
    rcc = rope_table(d, 40960, 1e6)
    page_idx, indptr, delta, last, rcache = (v.to(dev) for v in (pic, ipc, dc, lpc, rcc))
    rout = torch.empty(pages, ps, hkv, d, dtype=bf, device=dev)
    rows.append(Row("rerotate_paged_k_4096tok",
                    lambda: rerotate_paged_k(kv, page_idx, indptr, delta, last, rcache, out=rout),
                    2 * pages * ps * hkv * d * 2,
                    ref=lambda: _oracle().rerotate_paged_k(kvc, pic, ipc, dc, lpc, rcc), exact=True))
    guc, gu = r.randn(2048, 2 * 3072)
    silu = SiluAndMul()
    rows.append(Row("swiglu_t2048_i3072", lambda: silu(gu), 3 * 2048 * 3072 * 2,
                    ref=lambda: _oracle().silu_and_mul(guc), ref32=lambda: _oracle32().silu_and_mul(guc)))

    rows += kv_append_cases(dev)
    rows += fused_append_cases(dev)
    rows += cascade_cases(dev)
    rows += linear_cases(dev)
    return rows


def linear_cases(dev) -> list:
    """GEMM-epilogue fusions at Llama-3-8B layer shapes (seed 8): gate_up_proj with
    SiluAndMul (4096 -> 2 x 14336 -> 14336), down_proj + residual (14336 -> 4096)
    and o_proj + residual (4096 -> 4096), for an 8192-token prefill and a 64-token
    decode batch.  Algorithmic bytes: operand, weight, residual and output once."""
    from braidinfer_amd.layers import gate_up_silu_and_mul, linear_add_residual
    r = _Gen(8, dev)
    h, inter = 4096, 14336
    (guc, w_gu), (dnc, w_down), (oc, w_o) = r.randn(2 * inter, h, std=0.02), r.randn(h, inter, std=0.01), \
        r.randn(h, h, std=0.02)
    out = []
    for t in (8192, 64):
        (xc, x), (xic, xi), (rc, res) = r.randn(t, h), r.randn(t, inter), r.randn(t, h)
        out += [
            Row(f"gate_up_silu_llama3_8b_t{t}", (lambda x=x: gate_up_silu_and_mul(x, w_gu)),
                (t * h + 2 * inter * h + t * inter) * 2, 2.0 * t * h * 2 * inter,
                ref=lambda xc=xc: _oracle().gate_up_silu_and_mul(xc, guc),
                ref32=lambda xc=xc: _oracle32().gate_up_silu_and_mul(xc, guc)),
            Row(f"down_proj_residual_llama3_8b_t{t}", (lambda xi=xi, res=res: linear_add_residual(xi, w_down, res)),
                (t * inter + inter * h + 2 * t * h) * 2, 2.0 * t * inter * h,
                ref=lambda xic=xic, rc=rc: _oracle().linear_add_residual(xic, dnc, rc),
                ref32=lambda xic=xic, rc=rc: _oracle32().linear(xic, dnc, residual=rc)),
            Row(f"o_proj_residual_llama3_8b_t{t}", (lambda x=x, res=res: linear_add_residual(x, w_o, res)),
                (2 * t * h + h * h + t * h) * 2, 2.0 * t * h * h,
                ref=lambda xc=xc, rc=rc: _oracle().linear_add_residual(xc, oc, rc),
                ref32=lambda xc=xc, rc=rc: _oracle32().linear(xc, oc, residual=rc)),
        ]
    return out


def kv_append_cases(dev) -> list:
    """Paged KV append at Llama-3-8B kv geometry (8 heads x 128, page 16, HND;
    seed 6): an 8192-token prefill into 512 of 1024 shuffled pages, and a
    64-sequence decode batch (one new token each) in one batched launch.  The
    whole cache is compared bit for bit with the oracle's."""
    from braidinfer_amd.kernels import append_paged_kv_batch, append_to_paged_kv_cache_custom
    r = _Gen(6, dev)
    hkv, d, ps, pages = 8, 128, 16, 1024
    cc, cache = r.randn(pages, 2, hkv, ps, d)
    tc = torch.randperm(pages, generator=r.g)[:512].to(torch.int32)
    table = tc.to(dev)
    (kpc, kp), (vpc, vp) = r.randn(8192, hkv, d), r.randn(8192, hkv, d)
    ppc = torch.arange(8192, dtype=torch.int32)
    pp = ppc.to(dev)
    lens = torch.randint(0, 4000, (64,), generator=r.g)
    perm = torch.randperm(pages, generator=r.g)
    # sequence s: a table of lens[s] // 16 + 1 entries whose last (the one written) is a
    # page of its own
    per = lens // ps + 1
    indc = torch.cat([perm[s].repeat(int(per[s])) for s in range(64)]).to(torch.int32)
    iptc = torch.cat([torch.zeros(1, dtype=torch.int64), per.cumsum(0)]).to(torch.int32)
    batc = torch.arange(64)
    ind, indptr, bat, pd = indc.to(dev), iptc.to(dev), batc.to(dev), lens.to(dev)
    (kdc, kd), (vdc, vd) = r.randn(64, hkv, d), r.randn(64, hkv, d)

    cache_b = cache.clone()  # the batched append writes a cache of its own

    def prefill():
        append_to_paged_kv_cache_custom(kp, vp, cache, table, pp, ps)
        return cache

    def batch():
        append_paged_kv_batch(kd, vd, cache_b, ind, indptr, bat, pd, ps)
        return cache_b
    # each append writes the same values on every call, so the cache after the
    # timed repeats equals the oracle's single append into the initial cache
    return [Row("kv_append_t8192", prefill, 4 * 8192 * hkv * d * 2 + 8192 * 4 + 512 * 4,
                ref=lambda: _oracle().append_to_paged_kv_cache(kpc, vpc, cc, tc, ppc, ps)[0], exact=True,
                note="whole cache compared"),
            Row("kv_append_batch_b64", batch, 4 * 64 * hkv * d * 2 + 64 * (8 + 8 + 4) + 65 * 4,
                ref=lambda: _oracle().append_paged_kv_batch(kdc, vdc, cc, indc, iptc, batc, lens, ps)[0],
                exact=True, note="whole cache compared")]


def fused_append_cases(dev) -> list:
    """Fused RMSNorm+QKV+RoPE with the paged KV append in its epilogue
    (bfa_fused_rmsnorm_qkv_append) at Llama-3-8B shapes (seed 7), next to the two
    separate calls it replaces (fused QKV, then append_to_paged_kv_cache_custom
    or the batched append): an 8192-token prefill into 512 shuffled pages of a
    1024-page HND cache (page 16), with and without the k/v columns in the QKV
    output, and a 64-sequence decode batch (one token each, CSR page table).
    Every row returns the cache, compared with the oracle's QKV + append."""
    from braidinfer_amd.kernels import PagedKVAppend, append_paged_kv_batch, append_to_paged_kv_cache_custom
    from braidinfer_amd.layers import llama_attention_input
    r = _Gen(7, dev)
    hkv, d, ps, pages = HKV, D, 16, 1024
    kvb = 2 * HKV * D * 2  # k and v bytes per token
    rows = []
    for t in (8192, 64):
        (xc, x), (lc, ln), (wc, w) = r.randn(t, H), r.randn(H, std=0.1, mean=1.0), r.randn(N, H, std=0.02)
        pc = torch.randint(0, MAXPOS, (t,), generator=r.g)
        pos, rope = pc.to(dev), rope_table(D, MAXPOS, THETA).to(dev)
        rc_ = rope.cpu()
        cc, cache = r.randn(pages, 2, hkv, ps, d)
        if t == 8192:
            tc = torch.randperm(pages, generator=r.g)[:512].to(torch.int32)
            cpc = torch.arange(t, dtype=torch.int64)
            extra = dict(kv_indptr=None, batch_indices=None)
            ic = bc = None
        else:
            lens = torch.randint(0, 4000, (t,), generator=r.g)
            perm = torch.randperm(pages, generator=r.g)
            per = lens // ps + 1
            tc = torch.cat([perm[s].repeat(int(per[s])) for s in range(t)]).to(torch.int32)
            ic = torch.cat([torch.zeros(1, dtype=torch.int64), per.cumsum(0)]).to(torch.int32)
            bc = torch.arange(t)
            cpc = lens
            extra = dict(kv_indptr=ic.to(dev), batch_indices=bc.to(dev))
        table, cpos = tc.to(dev), cpc.to(dev)
        caches = {k: cache.clone() for k in ("fused", "qonly", "sep")}
        out = torch.empty(t, N, dtype=torch.bfloat16, device=dev)

        def fused(kind, t=t, x=x, ln=ln, w=w, pos=pos, rope=rope, table=table, cpos=cpos, extra=extra,
                  caches=caches, out=out):
            pkv = PagedKVAppend(caches[kind], table, cpos, ps, write_kv_out=kind == "fused", **extra)
            llama_attention_input(x, ln, w, HQ, HKV, EPS, pos, rope, paged_kv=pkv)
            return caches[kind]

        def separate(t=t, x=x, ln=ln, w=w, pos=pos, rope=rope, table=table, cpos=cpos, extra=extra,
                     caches=caches):
            _, k, v = llama_attention_input(x, ln, w, HQ, HKV, EPS, pos, rope)
            k, v = k.view(t, HKV, D), v.view(t, HKV, D)
            if extra["kv_indptr"] is None:
                append_to_paged_kv_cache_custom(k, v, caches["sep"], table, cpos, ps)
            else:
                append_paged_kv_batch(k, v, caches["sep"], table, extra["kv_indptr"], extra["batch_indices"],
                                      cpos, ps)
            return caches["sep"]

        def ref(t=t, xc=xc, lc=lc, wc=wc, pc=pc, rc_=rc_, cc=cc, tc=tc, cpc=cpc, ic=ic, bc=bc, qkv=_oracle):
            _, k, v = qkv().llama_attention_input(xc, lc, wc, HQ, HKV, EPS, pc, rc_)
            k, v = k.reshape(t, HKV, D), v.reshape(t, HKV, D)
            if ic is None:
                return _oracle().append_to_paged_kv_cache(k, v, cc, tc, cpc, ps)[0]
            return _oracle().append_paged_kv_batch(k, v, cc, tc, ic, bc, cpc, ps)[0]

        qkv_bytes = t * H * 2 + H * 2 + N * H * 2 + t * N * 2 + t * 8 + t * D * 4
        meta = t * (8 + 8 + 4)  # cache positions, slot offsets, page entries
        tag = "t8192" if t == 8192 else "b64"
        ref32 = (lambda ref=ref: ref(qkv=_oracle32))
        rows += [Row(f"qkv_rope_append_llama3_8b_{tag}", lambda fused=fused: fused("fused"),
                     qkv_bytes + t * kvb + meta, 2.0 * t * H * N, ref=ref, ref32=ref32,
                     note="fused QKV + RoPE + paged KV append, one call; cache compared"),
                 Row(f"qkv_rope_then_append_llama3_8b_{tag}", separate,
                     qkv_bytes + 2 * t * kvb + meta, 2.0 * t * H * N, ref=ref, ref32=ref32,
                     note="the two separate calls it replaces; cache compared")]
        if t == 8192:
            rows.append(Row(f"qkv_rope_append_q_only_llama3_8b_{tag}", lambda fused=fused: fused("qonly"),
                            qkv_bytes - t * kvb + t * kvb + meta, 2.0 * t * H * N, ref=ref, ref32=ref32,
                            note="write_kv_out=False: k/v only into the cache; cache compared"))
    return rows


def cascade_cases(dev) -> list:
    """Cascade attention at Qwen3-0.6B shape (seed 7): 4096 cached tokens in 16 chunks of
    256, shuffled 16-token HND pages, each chunk moved by a delta in [-4096, 4096]
    (theta 1e6, rotary table 40960), k_norm with log-uniform weights; 16 query heads
    over 8 kv heads of 128.  A one-token decode step and a 256-token query chunk.
    The same at TinyLlama-1.1B shape (seed 9): 32 query heads over 4 kv heads of 64,
    theta 1e4 (rotary table 4096), no k_norm, 2048 cached tokens in 8 chunks moved
    by up to +-1024."""
    return (_cascade_rows(dev, "qwen3", 7, 16, 8, 128, 4096, 1e6, 40960, True)
            + _cascade_rows(dev, "tinyllama", 9, 32, 4, 64, 2048, 1e4, 4096, False))


def _cascade_rows(dev, label, seed, hq, hkv, d, keys, theta, max_pos, knorm) -> list:
    import math as _m
    from types import SimpleNamespace
    from braidinfer_amd.layers import CascadeAttention, RMSNorm, RotaryEmbedding
    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16
    ps = 16
    nch = keys // 256
    pages = 2 * keys // ps
    kvc = torch.randn(pages, 2, hkv, ps, d, generator=g).to(bf)
    kv = kvc.to(dev)
    perm = torch.randperm(pages, generator=g).tolist()
    span = min(4096, max_pos // 4)
    deltas = torch.randint(-span, span + 1, (nch,), generator=g).tolist()
    start = 8192 if max_pos > 8192 else 0  # cached position of the first chunk
    chunks = [SimpleNamespace(page_table=perm[16 * c:16 * c + 16], kv_length=256,
                              cached_position_start=start + 256 * c,
                              global_position_start=start + 256 * c + deltas[c],
                              chunk_type=SimpleNamespace(value="system_prompt" if c == 0 else "context"))
              for c in range(nch)]
    rope = RotaryEmbedding(d, d, max_pos, theta).to(dev)
    att = CascadeAttention(hq, d, d ** -0.5, hkv, ps, rotary_emb=rope)
    levels = att.create_cascade_levels(chunks)
    cpu_levels = [SimpleNamespace(chunks=lv.chunks, kv_page_indices=lv.kv_page_indices.cpu(),
                                  kv_page_indptr=lv.kv_page_indptr.cpu(),
                                  kv_last_page_len=lv.kv_last_page_len.cpu()) for lv in levels]
    knc, k_norm = None, None
    if knorm:
        knc = torch.exp(torch.empty(d).uniform_(_m.log(0.05), _m.log(100.0), generator=g)).to(bf)
        k_norm = RMSNorm(d, eps=1e-6).to(dev)
        with torch.no_grad():
            k_norm.weight.data = knc.to(dev)
    csc = rope.cos_sin_cache.cpu()
    kv_bytes = keys * hkv * d * 2 * 2
    out = []
    for t in (1, 256):
        qc = torch.randn(t, hq, d, generator=g).to(bf)
        q = qc.to(dev)
        qpc = torch.arange(keys - t + 1, keys + 1)
        qpos = qpc.to(dev)
        out.append(Row(f"cascade_attention_{label}_{keys}kv_t{t}",
                       (lambda q=q, qpos=qpos: att.forward(q, qpos, kv, levels, 0, k_norm=k_norm)),
                       kv_bytes + 2 * t * hq * d * 2, 4.0 * t * hq * keys * d,
                       ref=lambda qc=qc, qpc=qpc: _oracle().cascade_attention(
                           qc, qpc, kvc, cpu_levels, hq, hkv, d ** -0.5, ps, cos_sin_cache=csc,
                           k_norm_weight=knc, k_norm_eps=1e-6),
                       # fp32 mode: the same op chain on fp32 copies of the bf16 inputs
                       # (no intermediate rounding), rounded once to bf16
                       ref32=lambda qc=qc, qpc=qpc: _oracle().cascade_attention(
                           qc.float(), qpc, kvc.float(), cpu_levels, hq, hkv, d ** -0.5, ps, cos_sin_cache=csc,
                           k_norm_weight=None if knc is None else knc.float(), k_norm_eps=1e-6).to(bf)))
    return out


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


def chain_graph_us(c: Chain, steps: int, warmup: int, step=None) -> float:
    """Microseconds per chain step: `steps` steps captured into one HIP graph;
    `warmup` untimed steps (whole replays of the graph, at least one) and 0.3 s
    of untimed replays for the clock to settle, then exactly `steps` timed steps
    between HIP events."""
    graph = _capture(step or c.step, steps)
    done = 0
    while done < max(warmup, 1):
        graph.replay()
        done += steps
    torch.cuda.synchronize()
    _settle(graph, 0.3)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    graph.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps * 1e3


def chain_graph_rotating_us(c: Chain, steps: int, warmup: int, nw: int = 4) -> float:
    """As chain_graph_us, with the QKV weight taken from `nw` copies in turn (one
    per captured step), as consecutive layers of a model use different weights:
    the repeated chain otherwise finds its 50 MB weight in the Infinity Cache."""
    ws = [c.w_qkv] + [c.w_qkv.clone() for _ in range(nw - 1)]
    turn = [0]

    def step():
        c.w_qkv = ws[turn[0] % nw]
        turn[0] += 1
        c.step()
    try:
        # one eager step per copy first, as a model's warm-up forward would: each
        # weight gets its folded copy before the capture (a fold is never captured)
        for _ in range(nw):
            step()
        torch.cuda.synchronize()
        return chain_graph_us(c, -(-steps // nw) * nw, warmup, step)
    finally:
        c.w_qkv = ws[0]


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


def measure_rows(rows: list, iters: int, flush: torch.Tensor, cold_iters: int) -> dict:
    """Warm (graph-replayed, settled clock, operands left in the caches by the
    previous call) and cold (Infinity Cache flushed before each call) GPU time of
    every row, with its roofline fractions."""
    out = {}
    for r in rows:
        d = _roof_row(time_graph(r.fn, iters), r.nbytes, r.flops)
        if cold_iters > 0:
            cold_ms = time_cold(r.fn, cold_iters, flush)
            d["us_cold"] = round(cold_ms * 1e3, 3)
            d["hbm_frac_cold"] = round(r.nbytes / (cold_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        if r.note:
            d["note"] = r.note
        out[r.name] = d
    return out


def _bits(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t.view({2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()])


def compare(got: torch.Tensor, exp: torch.Tensor, exact: bool, brief: bool = False) -> dict:
    """Error figures of a GPU result against the oracle's: bit-exact for the
    integer/byte ops; otherwise max-abs, normwise relative error and the
    elements outside |d| <= 2e-2 + 1e-2 |r| (the float tolerance; those are
    the elements a documented rounding allowance of the parity tests covers).
    brief: without allclose and numel (the vs_fp32 figures)."""
    got = got.detach().cpu()
    if exact:
        mism = int((_bits(got) != _bits(exp)).sum())
        return {"bit_exact": mism == 0, "mismatches": mism, "numel": exp.numel()}
    a, e = got.float(), exp.float()
    fin = torch.isfinite(e)
    same_pattern = bool(torch.equal(torch.isfinite(a), fin))
    d = (a - e).abs()[fin]
    ef = e[fin]
    outside = int((d > 2e-2 + 1e-2 * ef.abs()).sum())
    out = {"max_abs": float(f"{d.max().item():.4g}") if d.numel() else 0.0,
           "max_rel_normwise": float(f"{(d.norm() / ef.norm().clamp_min(1e-30)).item():.4g}"),
           "beyond_tol_elements": outside}
    if not brief:
        out.update({"allclose": same_pattern and outside == 0, "numel": exp.numel()})
    return out


def time_cpu(fn, min_reps: int = 3, max_reps: int = 10, budget_s: float = 3.0):
    """Median seconds of `fn` on the CPU over at least `min_reps` runs (more, up
    to `max_reps`, while within `budget_s`), after one untimed run whose result
    is returned."""
    result = fn()
    times = []
    t0 = time.perf_counter()
    while len(times) < max_reps and (len(times) < min_reps or time.perf_counter() - t0 < budget_s):
        s = time.perf_counter()
        fn()
        times.append(time.perf_counter() - s)
    times.sort()
    return times[len(times) // 2], len(times), result


def cpu_info() -> dict:
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"model": model, "threads": len(os.sched_getaffinity(0)),
            "parallel_info": torch.__config__.parallel_info()}


def cpu_leg(groups: dict, tables: dict) -> None:
    """The CPU baseline and check: each row's oracle (the torch-CPU restatement of
    the reference) runs at the row's full size on the host cores -- timed,
    median of >= 3 runs -- and the GPU result is compared with it.  Adds cpu_us,
    cpu_reps and the error figures to the rows of `tables`."""
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    for gname, rows in groups.items():
        for r in rows:
            if r.ref is None:
                continue
            got = r.fn()
            if r.got is not None:
                got = r.got(got)
            torch.cuda.synchronize()
            sec, reps, exp = time_cpu(r.ref)
            row = tables[gname][r.name]
            row["cpu_us"] = round(sec * 1e6, 1)
            row["cpu_reps"] = reps
            row["vs_oracle"] = compare(got, exp, r.exact)
            if r.ref32 is not None:
                exp32 = r.ref32()
                row["vs_fp32"] = compare(got, exp32, False, brief=True)
                row["oracle_vs_fp32"] = compare(exp, exp32, False, brief=True)


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
    cases = {r.name: r.fn for r in config_cases(dev)} if kernel.startswith("case:") else {}
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
    fn = {"qkv_projection": st.projection, "qkv_operand": st.operand, "qkv_row_statistic": st.row_statistic,
          "fused_qkv": c.qkv,
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
    ap.add_argument("--no-cold", action="store_true", help="skip the cold-cache timings")
    ap.add_argument("--kernel", help="only run this kernel --steps times at --tokens (for "
                    "profilers): qkv_projection, qkv_operand, qkv_row_statistic, fused_qkv (the whole fused "
                    "RMSNorm+QKV+RoPE op), add_rms_norm, silu_and_mul, "
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
    flush = torch.empty(512 * 2**20 // 4, dtype=torch.float32, device=dev)
    prefill = Chain(args.tokens, dev)
    us_eager = chain_us(prefill, args.steps, args.warmup)
    us = chain_graph_us(prefill, args.steps, args.warmup)
    rows_p = chain_rows(prefill, dev, stages=True)
    nc = 0 if args.no_cold else 1
    kp = measure_rows(rows_p, max(10, args.steps), flush, 10 * nc)
    proj = kp["qkv_projection_rope"]

    progress(f"decode chain, {args.decode_tokens} tokens")
    decode = Chain(args.decode_tokens, dev)
    us_dec_eager = chain_us(decode, max(args.steps, 100), args.warmup)
    us_dec = chain_graph_us(decode, max(args.steps, 100), max(args.warmup, 1000))
    rows_d = chain_rows(decode, dev, stages=False)
    kd = measure_rows(rows_d, max(50, args.steps), flush, 48 * nc)
    progress("other configurations")
    rows_c = config_cases(dev)
    configs = measure_rows(rows_c, max(40, args.steps), flush, 24 * nc)
    # after every per-kernel row, so that its heat does not reach them
    progress("prefill chain with rotating QKV weights")
    us_rot = chain_graph_rotating_us(prefill, args.steps, args.warmup)
    _lib.check_device_status(dev)
    tables = {"prefill": kp, "decode": kd, "configs": configs}
    cpu = None
    if not args.no_cpu:
        progress("CPU baseline and checks against the oracle")
        cpu_leg({"prefill": rows_p, "decode": rows_d, "configs": rows_c}, tables)
        chain = ("add_rms_norm", "fused_rmsnorm_qkv_rope", "silu_and_mul")
        cpu = {"value": round(sum(kp[k]["cpu_us"] for k in chain), 1), "unit": "us/layer",
               "cores": len(os.sched_getaffinity(0)), "kind": "port",
               "sample": f"the full {args.tokens}-token chain, not a sample: the oracle's torch-CPU "
                         f"add_rms_forward, llama attention input (minimal_f32 QKV + RoPE) and "
                         f"silu_and_mul at [{args.tokens}, 4096] / [{args.tokens}, 2x14336], each the "
                         f"median of >= 3 runs (kernels_prefill.*.cpu_us); torch {torch.__version__}"}
    del prefill, decode, flush
    torch.cuda.empty_cache()

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
        "configs": configs,
        "timing": "us: graph-replayed HIP-event average after >= 0.2 s of settling replays (warm: "
                  "operands in the caches from the previous call); us_cold: each call after a 512 MB "
                  "read that flushes the 256 MB Infinity Cache",
        "cpu": cpu_info() if not args.no_cpu else None,
        "kernels_prefill": kp,
        "decode": {"tokens": args.decode_tokens, "us_per_layer": round(us_dec, 2),
                   "eager_us_per_layer": round(us_dec_eager, 2), "kernels": kd},
        "eager_us_per_layer": round(us_eager, 2),
        "rotating_weights_us_per_layer": round(us_rot, 2),
        "roofline": {"bound": "mfma", "kernel": "qkv_projection_rope",
                     "achieved": proj["tflops"], "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": proj["mfma_frac"],
                     "traffic": read_traffic(f"traffic_qkv_projection_llama3_8b_t{args.tokens}"),
                     "traffic_source": f"profiles/traffic_qkv_projection_llama3_8b_t{args.tokens}.txt "
                                       "(rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, calibrated on a device "
                                       "copy; read from the file, not measured in this run)"},
    }
    if cpu is not None:
        line["cpu_baseline"] = cpu
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
