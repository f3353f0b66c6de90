"""GPU path against the fp32 mode of the oracle (oracle/fp32_ref.py): each op
chain computed in fp32 from the bf16 inputs and rounded once.

The accuracy target is stated against that fp32 reference: |d| <= 2e-2 +
1e-2 |r| elementwise, with the max-abs and normwise relative errors reported.
The reference's own rounding points already move some results away from it:
for the Qwen3 k heads after k_norm weights up to 100 (values near 100, where a
bf16 ulp is 0.5) the reference itself leaves about 4 % of elements outside
that bound.  So every case asserts:

* where the reference's rounding keeps every element inside the bound (the
  norms, SiLU*mul, the Llama chains, the v heads, the linear fusions), the GPU
  path keeps every element inside it too -- the bound itself, outright;
* elsewhere (the Qwen3 q/k heads after the extreme k_norm weights), that the
  GPU path is no further from the fp32 reference than the reference's rounding
  is: at most 1e-4 of the elements more outside the bound (the count is
  recorded as a rounding allowance in the session summary);
* in both cases a normwise relative error below 5e-3 (half the relative bound)
  or within 1.5x of the reference's own where that is larger.

The fp32 variants (minimal_f32,
with_bias) round their operand to bf16 for the matrix cores where the
reference's fp32 dot product runs at TF32 on its GPUs; their normwise error
(about 2e-3) comes from that and stays inside the bound.
"""
from __future__ import annotations

import math

import pytest
import torch

from braidinfer_amd.kernels import FusedRMSNormQKV, FusedRMSNormQKVMinimalF32, FusedRMSNormQKVMixedPrecision
from braidinfer_amd.layers import RMSNorm, SiluAndMul, llama_attention_input, qwen3_attention_input
from braidinfer_amd.layers.linear import gate_up_silu_and_mul, linear_add_residual
from oracle import fp32_ref as F
from oracle import torch_ref as R
from tests.helpers import ATOL, RTOL, gen, randn, record_allowance

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _figures(a, e):
    a, e = a.detach().float().cpu(), e.detach().float().cpu()
    d = (a - e).abs()
    outside = int((d > ATOL + RTOL * e.abs()).sum())
    return d.max().item(), (d.norm() / e.norm().clamp_min(1e-30)).item(), outside


def check_vs_fp32(gpu, ref_mode, fp32_mode, what):
    g_abs, g_nw, g_out = _figures(gpu, fp32_mode)
    r_abs, r_nw, r_out = _figures(ref_mode, fp32_mode)
    n = fp32_mode.numel()
    slack = math.ceil(1e-4 * n)
    print(f"{what}: vs fp32 mode max_abs {g_abs:.3e} normwise {g_nw:.3e} outside {g_out}/{n}; "
          f"reference rounding: max_abs {r_abs:.3e} normwise {r_nw:.3e} outside {r_out}", flush=True)
    assert torch.isfinite(gpu).all(), f"{what}: non-finite output"
    if r_out == 0:
        assert g_out == 0, f"{what}: {g_out} elements outside the bound where the reference has none"
    else:
        record_allowance(f"{what} (vs fp32; reference itself {r_out} outside)", max(0, g_out - r_out), n)
        assert g_out <= r_out + slack, f"{what}: {g_out} elements outside the bound (reference {r_out})"
    assert g_nw <= max(1.5 * r_nw, 5e-3) + 1e-4, f"{what}: normwise {g_nw:.3e} against the reference's {r_nw:.3e}"


def test_rms_norm_c1():
    g = gen(1)
    x, w = randn(g, 128, 2048), randn(g, 2048, mean=1.0, std=0.1)
    norm = RMSNorm(2048, eps=1e-5).to(DEV)
    with torch.no_grad():
        norm.weight.data = w.to(DEV)
    check_vs_fp32(norm(x.to(DEV)), R.rms_forward(x, w, 1e-5), F.rms_forward(x, w, 1e-5), "rms [128, 2048]")


def test_add_rms_norm():
    g = gen(2)
    x, r = randn(g, 1024, 4096), randn(g, 1024, 4096)
    w = randn(g, 4096, mean=1.0, std=0.1)
    norm = RMSNorm(4096, eps=1e-5).to(DEV)
    with torch.no_grad():
        norm.weight.data = w.to(DEV)
    y, _ = norm(x.to(DEV), r.to(DEV))
    check_vs_fp32(y, R.add_rms_forward(x, r, w, 1e-5)[0], F.add_rms_forward(x, r, w, 1e-5)[0],
                  "add_rms [1024, 4096]")


def test_silu_and_mul():
    g = gen(4)
    x = randn(g, 2048, 2 * 3072)
    check_vs_fp32(SiluAndMul()(x.to(DEV)), R.silu_and_mul(x), F.silu_and_mul(x), "silu_and_mul [2048, 6144]")


@pytest.mark.parametrize("t,h,hq,hkv,d", [(1, 2048, 32, 4, 64), (512, 2048, 32, 4, 64), (64, 4096, 32, 8, 128)])
def test_qkv_variants(t, h, hq, hkv, d):
    g = gen(5)
    x, ln = randn(g, t, h), randn(g, h, mean=1.0, std=0.1)
    w = randn(g, (hq + 2 * hkv) * d, h, std=0.02)
    xd, lnd, wd = x.to(DEV), ln.to(DEV), w.to(DEV)
    got = torch.cat([v.reshape(t, -1) for v in FusedRMSNormQKVMixedPrecision.forward(xd, lnd, wd, None, hq, hkv)], 1)
    check_vs_fp32(got, R.qkv_mixed_precision(x, ln, w, None, 1e-6), F.qkv(x, ln, w, None, 1e-6, torch.bfloat16),
                  f"mixed t={t}")
    got = torch.cat([v.reshape(t, -1) for v in FusedRMSNormQKV.forward(xd, lnd, wd, hq, hkv)], 1)
    check_vs_fp32(got, R.qkv_production(x, ln, w, 1e-6), F.qkv(x, ln, w, None, 1e-6, torch.bfloat16),
                  f"production t={t}")
    got = torch.cat([v.reshape(t, -1) for v in FusedRMSNormQKVMinimalF32.forward(xd, lnd, wd, hq, hkv)], 1)
    check_vs_fp32(got, R.qkv_minimal_f32(x, ln, w, 1e-6), F.qkv(x, ln, w, None, 1e-6, torch.float32),
                  f"minimal_f32 t={t}")


@pytest.mark.parametrize("t", [1, 64, 2048])
def test_qwen3_chain_extreme_k_norm(t):
    """Qwen3-0.6B shape with k_norm weights log-uniform in [0.05, 100]."""
    g = gen(3)
    h, hq, hkv, d = 1024, 16, 8, 128
    x, ln = randn(g, t, h), randn(g, h, mean=1.0, std=0.1)
    w = randn(g, (hq + 2 * hkv) * d, h, std=0.02)
    qn = randn(g, d, mean=1.0, std=0.1)
    kn = torch.exp(torch.empty(d).uniform_(math.log(0.05), math.log(100.0), generator=g)).bfloat16()
    pos = torch.randint(0, 2048, (t,), generator=g)
    cache = R.cos_sin_cache(d, 40960, 1e6)
    got = qwen3_attention_input(x.to(DEV), ln.to(DEV), w.to(DEV), None, hq, hkv, 1e-6, pos.to(DEV), cache.to(DEV),
                                qn.to(DEV), kn.to(DEV))
    ref = R.qwen3_attention_input(x, ln, w, None, hq, hkv, 1e-6, pos, cache, qn, kn)
    f32 = F.qwen3_attention_input(x, ln, w, None, hq, hkv, 1e-6, pos, cache, qn, kn)
    for name, a, b, c in zip("qkv", got, ref, f32):
        check_vs_fp32(a, b, c, f"qwen3 t={t} {name}")


@pytest.mark.parametrize("t", [64, 512])
def test_llama_chain(t):
    g = gen(6)
    h, hq, hkv, d = 4096, 32, 8, 128
    x, ln = randn(g, t, h), randn(g, h, mean=1.0, std=0.1)
    w = randn(g, (hq + 2 * hkv) * d, h, std=0.02)
    pos = torch.randint(0, 8192, (t,), generator=g)
    cache = R.cos_sin_cache(d, 8192, 5e5)
    got = llama_attention_input(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, 1e-5, pos.to(DEV), cache.to(DEV))
    ref = R.llama_attention_input(x, ln, w, hq, hkv, 1e-5, pos, cache)
    f32 = F.llama_attention_input(x, ln, w, hq, hkv, 1e-5, pos, cache)
    for name, a, b, c in zip("qkv", got, ref, f32):
        check_vs_fp32(a, b, c, f"llama t={t} {name}")


def test_linear_fusions():
    g = gen(7)
    t, h, i = 64, 4096, 14336
    x = randn(g, t, h)
    wgu = randn(g, 2 * i, h, std=0.02)
    check_vs_fp32(gate_up_silu_and_mul(x.to(DEV), wgu.to(DEV)), R.gate_up_silu_and_mul(x, wgu),
                  F.gate_up_silu_and_mul(x, wgu), "gate_up + silu_and_mul t=64")
    xo, wo, res = randn(g, 300, 4096), randn(g, 4096, 4096, std=0.02), randn(g, 300, 4096)
    check_vs_fp32(linear_add_residual(xo.to(DEV), wo.to(DEV), res.to(DEV)), R.linear_add_residual(xo, wo, res),
                  F.linear(xo, wo, residual=res), "o_proj + residual t=300")
