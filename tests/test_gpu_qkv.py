"""GPU parity of the fused RMSNorm+QKV kernels (all four reference variants and
the fused Qwen3 / Llama attention-input chains) against the oracle.

Tolerance: |d| <= 2e-2 + 1e-2 |r| elementwise (tests/helpers.py) against the
oracle's restatement of each variant.  The fp32 variants round the normalised
operand once to bf16 for the MFMA units (the reference's fp32 tl.dot rounds it
to TF32); the tolerance covers that.  At the 8192-token prefill the oracle is
evaluated on a sample of rows (rows of a GEMM are independent).
"""
from __future__ import annotations

import math

import pytest
import torch

import braidinfer_amd
from braidinfer_amd.kernels import (FusedRMSNormQKV, FusedRMSNormQKVMinimalF32,
                                    FusedRMSNormQKVMixedPrecision, FusedRMSNormQKVWithBias)
from braidinfer_amd.layers import llama_attention_input, qwen3_attention_input
from oracle import torch_ref as R
from tests.helpers import assert_close, gen, randn, rope_flip_slack

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make(seed, t, h, hq, hkv, d, dtype=torch.bfloat16, wstd=0.02):
    g = gen(seed)
    n = (hq + 2 * hkv) * d
    x = randn(g, t, h, dtype=dtype)
    ln = randn(g, h, mean=1.0, std=0.1, dtype=dtype)
    w = randn(g, n, h, std=wstd, dtype=dtype)
    b = randn(g, n, std=0.05, dtype=dtype)
    return g, x, ln, w, b


SHAPES = [
    # t, h, hq, hkv, d
    (1, 2048, 32, 4, 64),      # TinyLlama decode batch 1
    (8, 2048, 32, 4, 64),      # TinyLlama decode batch 8
    (64, 1024, 16, 8, 128),    # Qwen3 shape, decode batch 64
    (100, 256, 8, 4, 32),      # prefill path, head_dim 32
    (300, 512, 6, 2, 80),      # head_dim 80: raw projection + row epilogue
    (512, 2048, 32, 4, 64),    # TinyLlama 512-token prefill
]


@pytest.mark.parametrize("t,h,hq,hkv,d", SHAPES)
def test_mixed_precision(t, h, hq, hkv, d):
    _, x, ln, w, b = make(201, t, h, hq, hkv, d)
    for bias in (None, b):
        q, k, v = FusedRMSNormQKVMixedPrecision.forward(x.to(DEV), ln.to(DEV), w.to(DEV),
                                                        None if bias is None else bias.to(DEV),
                                                        hq, hkv, eps=1e-6)
        ref = R.split_qkv(R.qkv_mixed_precision(x, ln, w, bias, 1e-6), hq, hkv)
        for got, exp, name in zip((q, k, v), ref, "qkv"):
            assert got.shape == exp.shape and got.dtype == x.dtype
            assert_close(got, exp, what=f"mixed {name}")
        assert q.data_ptr() + hq * d * 2 == k.data_ptr(), "q, k, v are views of one buffer"


@pytest.mark.parametrize("t,h,hq,hkv,d", SHAPES)
def test_production(t, h, hq, hkv, d):
    _, x, ln, w, _ = make(202, t, h, hq, hkv, d)
    q, k, v = FusedRMSNormQKV.forward(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, eps=1e-6)
    ref = R.split_qkv(R.qkv_production(x, ln, w, 1e-6), hq, hkv)
    for got, exp in zip((q, k, v), ref):
        assert got.dtype == torch.bfloat16
        assert_close(got, exp, what="production")


@pytest.mark.parametrize("t,h,hq,hkv,d", SHAPES)
def test_minimal_f32(t, h, hq, hkv, d):
    _, x, ln, w, _ = make(203, t, h, hq, hkv, d)
    q, k, v = FusedRMSNormQKVMinimalF32.forward(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, eps=1e-5)
    ref = R.split_qkv(R.qkv_minimal_f32(x, ln, w, 1e-5), hq, hkv)
    for got, exp in zip((q, k, v), ref):
        assert got.dtype == torch.float32
        assert_close(got, exp, what="minimal_f32")


@pytest.mark.parametrize("t,heads,h", [
    (1, 3, 64),        # one 64-deep segment per split
    (20, 4, 8192),     # 2 segments per split
    (37, 8, 6144),     # 3
    (64, 8, 8192),     # 4
    (5, 16, 5120),     # 5
    (20, 16, 6144),    # 6
    (37, 16, 7168),    # 7
    (64, 16, 8192),    # 8
])
def test_decode_split_depths(t, heads, h):
    """Decode (T <= 64) weight-streaming path: the K slice per split is chosen from
    k / 64 and the column-tile count; these shapes give every slice depth 1..8 and
    every 16-token block count 1..4.  From 17 tokens up, (20, 16, 6144),
    (37, 16, 7168) and (64, 16, 8192) take the deep-K form (two chunks of 256 per
    split, two to four token blocks)."""
    hq, hkv, d = heads - 2, 1, 128
    _, x, ln, w, _ = make(209, t, h, hq, hkv, d)
    q, k, v = FusedRMSNormQKV.forward(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, eps=1e-6)
    ref = R.split_qkv(R.qkv_production(x, ln, w, 1e-6), hq, hkv)
    for got, exp, name in zip((q, k, v), ref, "qkv"):
        assert_close(got, exp, what=f"decode {name} t={t} h={h}")


@pytest.mark.parametrize("t,heads,h,gdtype", [
    (17, 48, 4096, torch.bfloat16),   # Llama-3-8B shape, two 16-token blocks
    (33, 48, 4096, torch.bfloat16),   # three blocks
    (64, 48, 4096, torch.bfloat16),   # four blocks, four splits of four chunks
    (64, 16, 8192, torch.bfloat16),   # eight chunks per split
    (64, 48, 4096, torch.float32),    # fp32 gamma: the operand pre-pass path instead
])
def test_decode_scale_after(t, heads, h, gdtype):
    """The fp32 variants from 17 to 64 tokens (bf16 x, W and gamma) project
    bf16(x * gamma) and multiply the split sum by 1 / rms in the reduction; the
    result stays within the tolerance of the oracle's (x / rms) * gamma operand,
    for FusedRMSNormQKVMinimalF32 and for FusedRMSNormQKVWithBias."""
    hq, hkv, d = heads - 16, 8, 128
    if heads == 16:
        hq, hkv = 8, 4
    _, x, ln, w, b = make(215, t, h, hq, hkv, d)
    ln = ln.to(gdtype)
    q, k, v = FusedRMSNormQKVMinimalF32.forward(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, eps=1e-5)
    ref = R.split_qkv(R.qkv_minimal_f32(x, ln, w, 1e-5), hq, hkv)
    for got, exp, name in zip((q, k, v), ref, "qkv"):
        assert got.dtype == torch.float32
        assert_close(got, exp, what=f"scale-after minimal_f32 {name} t={t}")
    q, k, v = FusedRMSNormQKVWithBias.forward(x.to(DEV), ln.to(DEV), w.to(DEV), b.to(DEV), hq, hkv, eps=1e-5)
    ref = R.split_qkv(R.qkv_with_bias(x, ln, w, b, 1e-5), hq, hkv)
    for got, exp, name in zip((q, k, v), ref, "qkv"):
        assert_close(got, exp, what=f"scale-after with_bias {name} t={t}")


@pytest.mark.parametrize("t,h,hq,hkv,d,strided,gdtype,sample", [
    (65, 4096, 32, 8, 128, False, torch.bfloat16, 1),     # 128x128 tiles (32-deep stage ring)
    (300, 2048, 32, 4, 64, True, torch.bfloat16, 1),      # head_dim 64, ragged rows, rows 2112 apart
    (100, 256, 8, 4, 32, False, torch.bfloat16, 1),       # head_dim 32, four stages
    (2048, 4096, 32, 8, 128, False, torch.bfloat16, 7),   # 128x256 tiles (64-deep stages)
    (4096, 4096, 32, 8, 128, False, torch.bfloat16, 13),  # 256x256 tiles
    (1024, 8192, 32, 8, 128, False, torch.bfloat16, 5),   # hidden 8192
    (300, 2048, 32, 4, 64, False, torch.float32, 1),      # fp32 gamma
])
def test_prefill_fp32_variants(t, h, hq, hkv, d, strided, gdtype, sample):
    """FusedRMSNormQKVMinimalF32 and FusedRMSNormQKVWithBias over the prefill
    tile forms (the row statistic, then the GEMM of x on the weight with the norm
    weight folded in, and the fp32 epilogue scaling each row): within
    the tolerance of the oracle's (x / rms) * gamma operand in fp32, with
    strided and ragged inputs; every `sample`-th row is checked at the large
    sizes (rows of a GEMM are independent)."""
    _, x, ln, w, b = make(217, t, h, hq, hkv, d)
    ln = ln.to(gdtype)
    xd = x.to(DEV)
    if strided:
        wide = torch.zeros(t, h + 64, dtype=x.dtype, device=DEV)
        wide[:, :h] = xd
        xd = wide[:, :h]
    rows = torch.arange(0, t, sample)
    got = FusedRMSNormQKVMinimalF32.forward(xd, ln.to(DEV), w.to(DEV), hq, hkv, eps=1e-5)
    ref = R.split_qkv(R.qkv_minimal_f32(x[rows], ln, w, 1e-5), hq, hkv)
    for g_, exp, name in zip(got, ref, "qkv"):
        assert g_.dtype == torch.float32
        assert_close(g_[rows.to(DEV)], exp, what=f"prefill minimal_f32 {name} t={t}")
    got = FusedRMSNormQKVWithBias.forward(xd, ln.to(DEV), w.to(DEV), b.to(DEV), hq, hkv, eps=1e-5)
    ref = R.split_qkv(R.qkv_with_bias(x[rows], ln, w, b, 1e-5), hq, hkv)
    for g_, exp, name in zip(got, ref, "qkv"):
        assert_close(g_[rows.to(DEV)], exp, what=f"prefill with_bias {name} t={t}")


@pytest.mark.parametrize("t,h,dtype,strided", [
    (1, 4096, torch.bfloat16, False),   # Llama-3-8B batch-1 decode: eight 16-byte chunks per lane
    (3, 4096, torch.bfloat16, True),    # rows 4160 elements apart
    (4, 1024, torch.float16, False),    # largest folded batch, fp16
    (2, 64, torch.bfloat16, False),     # one 64-deep segment, a partial chunk row
    (8, 2048, torch.bfloat16, False),   # two rows per wave: TinyLlama batch 8
    (6, 1024, torch.float16, True),     # two rows per wave, the second row of waves 2-3 absent
    (16, 1024, torch.bfloat16, False),  # four rows per wave: Qwen3 batch 16
    (13, 1024, torch.float16, True),    # four rows per wave, ragged last row group
])
def test_decode_operand_fold(t, h, dtype, strided):
    """Up to 16 decode tokens with x in the weight dtype: the weight-streaming
    kernel computes the row statistics and normalises its own K slice (no
    pre-pass launch; one row per wave up to 4 tokens, two up to 8, four up to
    16).  Mixed and production rounding, with the RMSNorm weight in the input
    dtype and in fp32."""
    hq, hkv, d = 6, 1, 64
    g, x, ln, w, _ = make(211, t, h, hq, hkv, d, dtype=dtype)
    xd = x.to(DEV)
    if strided:
        wide = torch.zeros(t, h + 64, dtype=dtype, device=DEV)
        wide[:, :h] = xd
        xd = wide[:, :h]
        assert xd.stride(0) == h + 64
    for lnw in (ln, ln.float()):
        q, k, v = FusedRMSNormQKVMixedPrecision.forward(xd, lnw.to(DEV), w.to(DEV), None, hq, hkv, eps=1e-6)
        ref = R.split_qkv(R.qkv_mixed_precision(x, lnw, w, None, 1e-6), hq, hkv)
        for got, exp, name in zip((q, k, v), ref, "qkv"):
            assert_close(got, exp, what=f"fold mixed {name} t={t} h={h} ln {lnw.dtype}")
        q, k, v = FusedRMSNormQKV.forward(xd, lnw.to(DEV), w.to(DEV), hq, hkv, eps=1e-6)
        ref = R.split_qkv(R.qkv_production(x, lnw, w, 1e-6), hq, hkv)
        for got, exp, name in zip((q, k, v), ref, "qkv"):
            assert_close(got, exp, what=f"fold production {name} t={t} h={h} ln {lnw.dtype}")


def test_with_bias_reference_cases():
    """tests/test_qwen3_bias_handling.py and test_numerical_stability.py:237-294 on the HIP path."""
    g = gen(204)
    t, h, hq, hkv, d = 8, 256, 8, 2, 32
    n = (hq + 2 * hkv) * d
    x = randn(g, t, h).to(DEV)
    ln = torch.ones(h, dtype=torch.bfloat16, device=DEV)
    w = (torch.randn(n, h, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    q1, k1, v1 = FusedRMSNormQKVWithBias.forward(x, ln, w, None, hq, hkv, eps=1e-6)
    q2, k2, v2 = FusedRMSNormQKVWithBias.forward(x, ln, w, torch.zeros(n, dtype=torch.bfloat16, device=DEV),
                                                 hq, hkv, eps=1e-6)
    for a, b in ((q1, q2), (k1, k2), (v1, v2)):
        assert a.is_contiguous() and a.dtype == torch.float32 and torch.allclose(a, b, atol=1e-6)
    assert q1.shape == (t, hq, d)
    for name, bias in (("normal", torch.randn(n, generator=g) * 0.01),
                       ("extreme", torch.full((n,), 1e30)), ("inf", torch.full((n,), float("inf"))),
                       ("nan", torch.full((n,), float("nan")))):
        bb = bias.to(torch.bfloat16)
        q, k, v = FusedRMSNormQKVWithBias.forward(x, ln, w, bb.to(DEV), hq, hkv, eps=1e-6)
        ref = R.split_qkv(R.qkv_with_bias(x.cpu(), ln.cpu(), w.cpu(), bb, 1e-6), hq, hkv)
        for got, exp in zip((q, k, v), ref):
            assert_close(got, exp, what=f"with_bias {name}")
    # extreme K weights (x96.5) stay finite with fp32 accumulation
    w2 = w.clone()
    w2[hq * d:(hq + hkv) * d] *= 96.5
    q, k, v = FusedRMSNormQKVWithBias.forward((x.float() * 0.01).to(torch.bfloat16), ln, w2, None,
                                              hq, hkv, eps=1e-6)
    assert all(torch.isfinite(z).all() for z in (q, k, v))


def test_fp16_inputs():
    _, x, ln, w, _ = make(205, 40, 256, 8, 4, 32, dtype=torch.float16, wstd=0.1)
    q, k, v = FusedRMSNormQKVWithBias.forward(x.to(DEV), ln.to(DEV), w.to(DEV), None, 8, 4)
    ref = R.split_qkv(R.qkv_with_bias(x, ln, w, None, 1e-6), 8, 4)
    for got, exp in zip((q, k, v), ref):
        assert_close(got, exp, what="fp16 with_bias")
    q, k, v = FusedRMSNormQKVMixedPrecision.forward(x.to(DEV), ln.to(DEV), w.to(DEV), None, 8, 4)
    assert q.dtype == torch.float16
    ref = R.split_qkv(R.qkv_mixed_precision(x, ln, w, None, 1e-6), 8, 4)
    for got, exp in zip((q, k, v), ref):
        assert_close(got, exp, what="fp16 mixed")


# ---------------------------------------------------- fused model chains
def _qwen3_case(seed, t, h=1024, hq=16, hkv=8, d=128):
    g, x, ln, w, _ = make(seed, t, h, hq, hkv, d)
    qn = randn(g, d, mean=1.0, std=0.1)
    kn = torch.exp(torch.empty(d).uniform_(math.log(0.05), math.log(100), generator=g)).to(torch.bfloat16)
    pos = torch.randint(0, 2048, (t,), generator=g)
    return x, ln, w, qn, kn, pos


def _qwen3_rope_inputs(x, ln, w, qn, kn, hq=16, hkv=8, eps=1e-6):
    """The oracle's normalised q and k (the RoPE inputs), for rope_flip_slack."""
    q, k, _ = R.split_qkv(R.qkv_mixed_precision(x, ln, w, None, eps), hq, hkv)
    return (R.rms_forward(q.float(), qn, eps).to(x.dtype),
            R.rms_forward(k.float(), kn, eps).to(x.dtype))


@pytest.mark.parametrize("t", [1, 7, 64, 300, 2048])
def test_qwen3_chain(t):
    """Qwen3-0.6B: fused QKV + per-head q/k RMSNorm (extreme k_norm weights) + RoPE.

    q and k carry, on top of the path tolerance, two bf16 ulps of each RoPE input
    (rope_flip_slack) for at most 1e-4 of their elements: with k_norm weights up
    to 100 the normalised k reaches ~100 (ulp 0.5), and a projection summed in
    another order than the oracle's can round one element an ulp away; where the
    rotation cancels, that reaches the output.  At 2048 tokens 15 of 2.1 M k
    elements need it; v has no allowance."""
    x, ln, w, qn, kn, pos = _qwen3_case(206, t)
    cache = R.cos_sin_cache(128, 40960, 1e6)
    q, k, v = qwen3_attention_input(x.to(DEV), ln.to(DEV), w.to(DEV), None, 16, 8, 1e-6,
                                    pos.to(DEV), cache.to(DEV), qn.to(DEV), kn.to(DEV))
    rq, rk, rv = R.qwen3_attention_input(x, ln, w, None, 16, 8, 1e-6, pos, cache, qn, kn)
    pq, pk = _qwen3_rope_inputs(x, ln, w, qn, kn)
    assert_close(q, rq, what="qwen3 q", slack=rope_flip_slack(pq).reshape(rq.shape))
    assert_close(k, rk, what="qwen3 k", slack=rope_flip_slack(pk).reshape(rk.shape))
    assert_close(v, rv, what="qwen3 v")
    # extreme k_norm weights: fp32-accumulated k stays finite and inside bf16 / fp16 range
    assert torch.isfinite(k).all() and k.abs().max().item() < 65504.0
    braidinfer_amd.check_device_status()


@pytest.mark.parametrize("t,h,hq,hkv,d,base,maxp", [
    (1, 2048, 32, 4, 64, 1e4, 2048),       # TinyLlama decode
    (8, 2048, 32, 4, 64, 1e4, 2048),
    (512, 2048, 32, 4, 64, 1e4, 2048),     # TinyLlama prefill
    (64, 4096, 32, 8, 128, 5e5, 8192),     # Llama-3-8B decode batch 64
])
def test_llama_chain(t, h, hq, hkv, d, base, maxp):
    g, x, ln, w, _ = make(207, t, h, hq, hkv, d)
    pos = torch.randint(0, maxp, (t,), generator=g)
    cache = R.cos_sin_cache(d, maxp, base)
    q, k, v = llama_attention_input(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, 1e-5, pos.to(DEV),
                                    cache.to(DEV))
    rq, rk, rv = R.llama_attention_input(x, ln, w, hq, hkv, 1e-5, pos, cache)
    assert_close(q, rq, what="llama q")
    assert_close(k, rk, what="llama k")
    assert_close(v, rv, what="llama v")


def test_prefill_raw_epilogue_256_tiles():
    """head_dim 80 at 8192 tokens: 256x256 tiles with the raw fp32 store and the
    row epilogue kernel (the fused epilogue covers head_dim 32/64/128 only)."""
    t, h, hq, hkv, d = 8192, 256, 48, 4, 80
    g, x, ln, w, _ = make(210, t, h, hq, hkv, d)
    rows = torch.cat([torch.arange(0, 4), torch.randint(0, t, (60,), generator=g), torch.arange(t - 4, t)])
    q, k, v = FusedRMSNormQKV.forward(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, eps=1e-6)
    ref = R.split_qkv(R.qkv_production(x[rows], ln, w, 1e-6), hq, hkv)
    rd = rows.to(DEV)
    for got, exp, name in zip((q, k, v), ref, "qkv"):
        assert_close(got[rd], exp, what=f"raw 256-tile {name}")


@pytest.mark.parametrize("tile", [2, 3])
@pytest.mark.parametrize("h", [64, 192, 320, 448])
@pytest.mark.parametrize("d,hq,hkv", [(128, 4, 2), (80, 6, 2)])
def test_prefill_16x16_stage_counts(tuning, tile, h, d, hq, hkv):
    """The 64-deep DMA loop of the 256x256 (tile 2) and 128x256 8-wave (tile 3)
    tiles, which multiplies 16x16x32 blocks: 1, 3, 5 and 7 stages (the odd tail
    after the two-stage loop), ragged rows and column tiles, through the fused
    epilogue (head_dim 128, with RoPE) and the raw fp32 store plus the row
    epilogue (head_dim 80), each against the oracle."""
    tuning("QKV_TILE", tile)
    t = 300
    g, x, ln, w, _ = make(260 + h + d, t, h, hq, hkv, d)
    q, k, v = FusedRMSNormQKV.forward(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, eps=1e-6)
    for got, exp, name in zip((q, k, v), R.split_qkv(R.qkv_production(x, ln, w, 1e-6), hq, hkv), "qkv"):
        assert_close(got, exp, what=f"16x16 production {name} tile={tile} h={h} d={d}")
    if d == 128:
        pos = torch.randint(0, 4096, (t,), generator=g)
        cache = R.cos_sin_cache(d, 4096, 1e4)
        q, k, v = llama_attention_input(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, 1e-5, pos.to(DEV),
                                        cache.to(DEV))
        for got, exp, name in zip((q, k, v), R.llama_attention_input(x, ln, w, hq, hkv, 1e-5, pos, cache), "qkv"):
            assert_close(got, exp, what=f"16x16 llama {name} tile={tile} h={h}")


@pytest.mark.parametrize("chain", ["llama", "qwen3"])
def test_prefill_8192_sampled_rows(chain):
    """Llama-3-8B / Qwen3 prefill shapes at full size; the oracle checks a row sample."""
    t = 8192
    if chain == "llama":
        h, hq, hkv, d, base, maxp = 4096, 32, 8, 128, 5e5, 8192
    else:
        h, hq, hkv, d, base, maxp = 1024, 16, 8, 128, 1e6, 40960
    g, x, ln, w, _ = make(208, t, h, hq, hkv, d)
    pos = torch.randint(0, 8192, (t,), generator=g)
    cache = R.cos_sin_cache(d, maxp, base)
    rows = torch.cat([torch.arange(0, 4), torch.randint(0, t, (60,), generator=g), torch.arange(t - 4, t)])
    if chain == "llama":
        q, k, v = llama_attention_input(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, 1e-5, pos.to(DEV),
                                        cache.to(DEV))
        ref = R.llama_attention_input(x[rows], ln, w, hq, hkv, 1e-5, pos[rows], cache)
    else:
        qn = randn(g, d, mean=1.0, std=0.1)
        kn = torch.exp(torch.empty(d).uniform_(math.log(0.05), math.log(100), generator=g)).to(torch.bfloat16)
        q, k, v = qwen3_attention_input(x.to(DEV), ln.to(DEV), w.to(DEV), None, hq, hkv, 1e-6,
                                        pos.to(DEV), cache.to(DEV), qn.to(DEV), kn.to(DEV))
        ref = R.qwen3_attention_input(x[rows], ln, w, None, hq, hkv, 1e-6, pos[rows], cache, qn, kn)
    rd = rows.to(DEV)
    slack = [None, None, None]
    if chain == "qwen3":  # see test_qwen3_chain
        pq, pk = _qwen3_rope_inputs(x[rows], ln, w, qn, kn, hq, hkv)
        slack[0], slack[1] = rope_flip_slack(pq), rope_flip_slack(pk)
    for got, exp, name, sl in zip((q, k, v), ref, "qkv", slack):
        assert_close(got[rd], exp, what=f"{chain} 8192 {name}",
                     slack=None if sl is None else sl.reshape(exp.shape))


@pytest.mark.parametrize("tile", [None, 128, 64])
@pytest.mark.parametrize("t,h,hq,hkv,d", [
    (512, 2048, 32, 4, 64),   # TinyLlama prefill: the planner takes 128x64 (160 tiles)
    (300, 512, 8, 2, 32),     # head_dim 32 (two heads per 64-column wave), ragged rows
    (1100, 1024, 8, 4, 64),   # nine row tiles, the last one ragged
])
def test_prefill_narrow_tile(tuning, tile, t, h, hq, hkv, d):
    """The 128x64 tile (head_dim <= 64 under 128 tiles of 128x128; 8 lanes per
    row in the fused epilogue) and the 128x128 form it replaces, each against
    the oracle: the Llama chain, a q/k-norm chain with extreme k_norm weights
    (rope_flip_slack as in test_qwen3_chain) and the mixed variant with bias."""
    tuning("QKV_TILE", tile)
    g, x, ln, w, b = make(230 + d, t, h, hq, hkv, d)
    pos = torch.randint(0, 4096, (t,), generator=g)
    cache = R.cos_sin_cache(d, 4096, 1e4)
    q, k, v = llama_attention_input(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, 1e-5, pos.to(DEV), cache.to(DEV))
    for got, exp, name in zip((q, k, v), R.llama_attention_input(x, ln, w, hq, hkv, 1e-5, pos, cache), "qkv"):
        assert_close(got, exp, what=f"narrow llama {name} t={t} tile={tile}")
    qn = randn(g, d, mean=1.0, std=0.1)
    kn = torch.exp(torch.empty(d).uniform_(math.log(0.05), math.log(100), generator=g)).to(torch.bfloat16)
    q, k, v = qwen3_attention_input(x.to(DEV), ln.to(DEV), w.to(DEV), None, hq, hkv, 1e-6, pos.to(DEV),
                                    cache.to(DEV), qn.to(DEV), kn.to(DEV))
    ref = R.qwen3_attention_input(x, ln, w, None, hq, hkv, 1e-6, pos, cache, qn, kn)
    pq, pk = _qwen3_rope_inputs(x, ln, w, qn, kn, hq, hkv)
    assert_close(q, ref[0], what=f"narrow q/k-norm q t={t}", slack=rope_flip_slack(pq).reshape(ref[0].shape))
    assert_close(k, ref[1], what=f"narrow q/k-norm k t={t}", slack=rope_flip_slack(pk).reshape(ref[1].shape))
    assert_close(v, ref[2], what=f"narrow q/k-norm v t={t}")
    got = FusedRMSNormQKVMixedPrecision.forward(x.to(DEV), ln.to(DEV), w.to(DEV), b.to(DEV), hq, hkv, eps=1e-6)
    for g_, exp, name in zip(got, R.split_qkv(R.qkv_mixed_precision(x, ln, w, b, 1e-6), hq, hkv), "qkv"):
        assert_close(g_, exp, what=f"narrow mixed+bias {name} t={t}")
    braidinfer_amd.check_device_status()
