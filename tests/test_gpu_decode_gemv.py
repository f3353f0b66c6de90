"""GPU parity of the one-launch decode kernel (qkv_gemv.hip): the fused
RMSNorm+QKV(+bias, RoPE, KV append) of 1-8 tokens without q/k norm, in one
launch (a workgroup per 16 output columns, the whole of K), against the
oracle's restatement of each reference variant (kernels/fused_rmsnorm_qkv_*.py,
models/llama.py:169-205).

The planner takes the kernel up to 4 tokens, and up to 8 when the grid is at
most 192 workgroups, without q/k norm; the DECODE_GEMV override = 0 keeps the
split-K kernels and their reduction.  Every case runs both ways, each against
the oracle within |d| <= 2e-2 + 1e-2 |r| (tests/helpers.py)."""
from __future__ import annotations

import pytest
import torch

import braidinfer_amd
from braidinfer_amd.kernels import (FusedRMSNormQKV, FusedRMSNormQKVMinimalF32,
                                    FusedRMSNormQKVMixedPrecision, FusedRMSNormQKVWithBias)
from braidinfer_amd.layers import llama_attention_input
from oracle import torch_ref as R
from tests.helpers import assert_close, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = [
    # t, hidden, hq, hkv, d
    (1, 2048, 32, 4, 64),     # TinyLlama decode, one token
    (2, 2048, 32, 4, 64),     # two tokens
    (3, 2048, 32, 4, 64),     # three (4-token capacity, a padded row)
    (8, 2048, 32, 4, 64),     # TinyLlama decode batch 8
    (4, 1024, 16, 8, 128),    # four, Qwen3-0.6B geometry without q/k norm
    (6, 1024, 8, 4, 128),     # six (8-token capacity, 128 workgroups)
    (1, 4096, 32, 8, 128),    # Llama-3-8B, one token (two weight batches per wave)
    (5, 512, 4, 2, 96),       # head_dim 96 (six column groups per head), hidden 512
]


def make(seed, t, h, hq, hkv, d):
    g = gen(seed)
    n = (hq + 2 * hkv) * d
    return (g, randn(g, t, h), randn(g, h, mean=1.0, std=0.1), randn(g, n, h, std=0.02),
            randn(g, n, std=0.05))


def both_ways(tuning, fn):
    """fn() with the one-launch kernel and with the split-K kernels."""
    out = []
    for mode in (None, 0):
        tuning("DECODE_GEMV", mode)
        out.append(fn())
        torch.cuda.synchronize()
        braidinfer_amd.check_device_status()
    return out


@pytest.mark.parametrize("t,h,hq,hkv,d", SHAPES)
def test_gemv_mixed_precision_bias(tuning, t, h, hq, hkv, d):
    _, x, ln, w, b = make(401, t, h, hq, hkv, d)
    ref = R.split_qkv(R.qkv_mixed_precision(x, ln, w, b, 1e-6), hq, hkv)
    for got in both_ways(tuning, lambda: FusedRMSNormQKVMixedPrecision.forward(
            x.to(DEV), ln.to(DEV), w.to(DEV), b.to(DEV), hq, hkv, eps=1e-6)):
        for g_, e_, name in zip(got, ref, "qkv"):
            assert_close(g_, e_, what=f"gemv mixed+bias {name} t={t}")


@pytest.mark.parametrize("t,h,hq,hkv,d", SHAPES)
def test_gemv_production_and_minimal_f32(tuning, t, h, hq, hkv, d):
    _, x, ln, w, _ = make(402, t, h, hq, hkv, d)
    ref = R.split_qkv(R.qkv_production(x, ln, w, 1e-6), hq, hkv)
    for got in both_ways(tuning, lambda: FusedRMSNormQKV.forward(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv,
                                                                 eps=1e-6)):
        for g_, e_ in zip(got, ref):
            assert_close(g_, e_, what=f"gemv production t={t}")
    ref = R.split_qkv(R.qkv_minimal_f32(x, ln, w, 1e-5), hq, hkv)
    for got in both_ways(tuning, lambda: FusedRMSNormQKVMinimalF32.forward(x.to(DEV), ln.to(DEV), w.to(DEV),
                                                                           hq, hkv, eps=1e-5)):
        for g_, e_ in zip(got, ref):
            assert g_.dtype == torch.float32
            assert_close(g_, e_, what=f"gemv minimal_f32 t={t}")


@pytest.mark.parametrize("t,h,hq,hkv,d", SHAPES)
def test_gemv_with_bias_variant(tuning, t, h, hq, hkv, d):
    _, x, ln, w, b = make(403, t, h, hq, hkv, d)
    ref = R.split_qkv(R.qkv_with_bias(x, ln, w, b, 1e-6), hq, hkv)
    for got in both_ways(tuning, lambda: FusedRMSNormQKVWithBias.forward(x.to(DEV), ln.to(DEV), w.to(DEV),
                                                                         b.to(DEV), hq, hkv, eps=1e-6)):
        for g_, e_ in zip(got, ref):
            assert_close(g_, e_, what=f"gemv with_bias t={t}")


@pytest.mark.parametrize("t,h,hq,hkv,d", SHAPES)
def test_gemv_llama_chain(tuning, t, h, hq, hkv, d):
    """minimal_f32 projection, RoPE (theta 5e5) on q and k, bf16 out; one position
    outside the table raises."""
    g, x, ln, w, _ = make(404, t, h, hq, hkv, d)
    cache = R.cos_sin_cache(d, 8192, 5e5)
    pos = torch.randint(0, 8192, (t,), generator=g)
    ref = R.llama_attention_input(x, ln, w, hq, hkv, 1e-5, pos, cache)
    for got in both_ways(tuning, lambda: llama_attention_input(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, 1e-5,
                                                               pos.to(DEV), cache.to(DEV))):
        for g_, e_, name in zip(got, ref, "qkv"):
            assert_close(g_, e_, what=f"gemv llama {name} t={t}")
    bad = pos.clone()
    bad[-1] = 9000
    tuning("DECODE_GEMV", None)
    llama_attention_input(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, 1e-5, bad.to(DEV), cache.to(DEV))
    torch.cuda.synchronize()
    with pytest.raises(IndexError):
        braidinfer_amd.check_device_status()
