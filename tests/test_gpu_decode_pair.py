"""GPU parity of the whole-K column-pair decode kernel (qkv_decode_pair_kernel):
17-64 tokens, head_dim a multiple of 32, no q/k norm.  A workgroup owns 16 RoPE
pairs of one head for every token and the whole of K, so the projection, the
RMSNorm row scale of the fp32 variants (gamma on the weight rows, the rows' sums
of squares from the operand fragments), bias, RoPE and the KV append all run in
one launch (models/llama.py:169-205, kernels/fused_rmsnorm_qkv_minimal_f32.py,
kernels/fused_rmsnorm_qkv_production.py, kernels/kv_cache_utils.py:9-78).

The library takes this kernel by itself from 128 column tiles up (Llama-3-8B at
64 tokens, test_gpu_qkv.py's llama chain and scale-after cases); here
The DECODE_PAIR planner override forces it on smaller shapes, so that every token-block count
(2-4), head_dim 64 and 128, bias, RoPE with in- and out-of-range positions, the
bf16 variants (operand from the pre-pass) and the fp32 ones (scale-after) and
the fused KV append each run it.  Tolerance as the other QKV tests
(|d| <= 2e-2 + 1e-2 |r| against the oracle); the KV append is bit-exact against
the oracle's append of the kernel's own k/v output."""
from __future__ import annotations

import pytest
import torch

import braidinfer_amd
from braidinfer_amd.kernels import (FusedRMSNormQKV, FusedRMSNormQKVMinimalF32,
                                    FusedRMSNormQKVMixedPrecision, FusedRMSNormQKVWithBias)
from braidinfer_amd.layers import llama_attention_input
from oracle import torch_ref as R
from tests.helpers import assert_close, gen, randn
from tests.test_gpu_fused_append import check as append_check
from tests.test_gpu_fused_append import make_case as append_case

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def force_pair(tuning):
    tuning("DECODE_PAIR", 1)


def make(seed, t, h, hq, hkv, d):
    g = gen(seed)
    n = (hq + 2 * hkv) * d
    return (g, randn(g, t, h), randn(g, h, mean=1.0, std=0.1), randn(g, n, h, std=0.02),
            randn(g, n, std=0.05))


SHAPES = [
    # t, h, hq, hkv, d
    (17, 1024, 8, 4, 128),    # two 16-token blocks, one row of the second
    (33, 1024, 8, 4, 128),    # three
    (48, 2048, 16, 4, 64),    # three, full; head_dim 64 (two pair tiles per head)
    (64, 1024, 8, 4, 128),    # four
    (64, 3072, 4, 2, 64),     # twelve 256-deep chunks per wave ring
]


@pytest.mark.parametrize("t,h,hq,hkv,d", SHAPES)
def test_pair_fp32_variants_scale_after(t, h, hq, hkv, d):
    """minimal_f32 and with_bias with bf16 x, W and gamma: x projected onto
    bf16(W * gamma), the row scale 1/rms from the in-kernel sums of squares."""
    _, x, ln, w, b = make(301 + t, t, h, hq, hkv, d)
    q, k, v = FusedRMSNormQKVMinimalF32.forward(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, eps=1e-5)
    ref = R.split_qkv(R.qkv_minimal_f32(x, ln, w, 1e-5), hq, hkv)
    for got, exp, name in zip((q, k, v), ref, "qkv"):
        assert got.dtype == torch.float32
        assert_close(got, exp, what=f"pair minimal_f32 {name} t={t} d={d}")
    q, k, v = FusedRMSNormQKVWithBias.forward(x.to(DEV), ln.to(DEV), w.to(DEV), b.to(DEV), hq, hkv, eps=1e-5)
    ref = R.split_qkv(R.qkv_with_bias(x, ln, w, b, 1e-5), hq, hkv)
    for got, exp, name in zip((q, k, v), ref, "qkv"):
        assert_close(got, exp, what=f"pair with_bias {name} t={t} d={d}")


@pytest.mark.parametrize("t,h,hq,hkv,d", [SHAPES[0], SHAPES[2], SHAPES[3]])
def test_pair_bf16_variants(t, h, hq, hkv, d):
    """production and mixed precision (bf16 output, operand from the pre-pass),
    with and without bias; fp32 gamma takes the pre-pass for minimal_f32 too."""
    _, x, ln, w, b = make(311 + t, t, h, hq, hkv, d)
    q, k, v = FusedRMSNormQKV.forward(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, eps=1e-6)
    ref = R.split_qkv(R.qkv_production(x, ln, w, 1e-6), hq, hkv)
    for got, exp, name in zip((q, k, v), ref, "qkv"):
        assert got.dtype == torch.bfloat16
        assert_close(got, exp, what=f"pair production {name} t={t}")
    for bias in (None, b):
        q, k, v = FusedRMSNormQKVMixedPrecision.forward(x.to(DEV), ln.to(DEV), w.to(DEV),
                                                        None if bias is None else bias.to(DEV),
                                                        hq, hkv, eps=1e-6)
        ref = R.split_qkv(R.qkv_mixed_precision(x, ln, w, bias, 1e-6), hq, hkv)
        for got, exp, name in zip((q, k, v), ref, "qkv"):
            assert_close(got, exp, what=f"pair mixed {name} t={t} bias={bias is not None}")
    lnf = ln.float()
    q, k, v = FusedRMSNormQKVMinimalF32.forward(x.to(DEV), lnf.to(DEV), w.to(DEV), hq, hkv, eps=1e-5)
    ref = R.split_qkv(R.qkv_minimal_f32(x, lnf, w, 1e-5), hq, hkv)
    for got, exp, name in zip((q, k, v), ref, "qkv"):
        assert_close(got, exp, what=f"pair minimal_f32 fp32 gamma {name} t={t}")


@pytest.mark.parametrize("t,h,hq,hkv,d,base,maxp", [
    (17, 2048, 32, 4, 64, 1e4, 2048),    # TinyLlama-shaped
    (40, 1024, 8, 4, 128, 5e5, 8192),
    (64, 2048, 16, 8, 128, 5e5, 8192),
])
def test_pair_llama_chain(t, h, hq, hkv, d, base, maxp):
    """RMSNorm + QKV + RoPE of the Llama attention input (fp32 projection, RoPE in
    fp32, bf16 store) in the one launch."""
    g, x, ln, w, _ = make(321 + t, t, h, hq, hkv, d)
    pos = torch.randint(0, maxp, (t,), generator=g)
    pos[0] = -1  # negative positions wrap like a torch index
    cache = R.cos_sin_cache(d, maxp, base)
    q, k, v = llama_attention_input(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, 1e-5, pos.to(DEV), cache.to(DEV))
    rq, rk, rv = R.llama_attention_input(x, ln, w, hq, hkv, 1e-5, pos, cache)
    assert_close(q, rq, what=f"pair llama q t={t}")
    assert_close(k, rk, what=f"pair llama k t={t}")
    assert_close(v, rv, what=f"pair llama v t={t}")
    braidinfer_amd.check_device_status()


def test_pair_position_out_of_range():
    """A position past the table is reported (IndexError, as torch indexing would
    raise) and its q/k rows are zero; v and the other rows are unaffected."""
    t, h, hq, hkv, d, maxp = 24, 1024, 8, 4, 128, 512
    g, x, ln, w, _ = make(331, t, h, hq, hkv, d)
    pos = torch.randint(0, maxp, (t,), generator=g)
    pos[5] = maxp + 3
    cache = R.cos_sin_cache(d, maxp, 5e5)
    braidinfer_amd.check_device_status()
    q, k, v = llama_attention_input(x.to(DEV), ln.to(DEV), w.to(DEV), hq, hkv, 1e-5, pos.to(DEV), cache.to(DEV))
    torch.cuda.synchronize()
    with pytest.raises(IndexError):
        braidinfer_amd.check_device_status()
    assert bool((q[5] == 0).all()) and bool((k[5] == 0).all())
    ok = torch.ones(t, dtype=torch.bool)
    ok[5] = False
    pos_ok = pos.clone()
    pos_ok[5] = 0
    rq, rk, rv = R.llama_attention_input(x, ln, w, hq, hkv, 1e-5, pos_ok, cache)
    assert_close(q[ok.to(DEV)], rq[ok], what="pair oob q")
    assert_close(k[ok.to(DEV)], rk[ok], what="pair oob k")
    assert_close(v, rv, what="pair oob v")


LLAMA = dict(hidden=1024, hq=8, hkv=2, d=128, qwen=False)


@pytest.mark.parametrize("tokens", [17, 40, 64])
def test_pair_fused_append(tokens):
    """bfa_fused_rmsnorm_qkv_append through the pair kernel: output bit-exact
    against the plain call, cache bit-exact against the oracle's append."""
    c = append_case(400 + tokens, tokens, **LLAMA)
    assert append_check(c, f"pair append T={tokens}") == []
    braidinfer_amd.check_device_status()


def test_pair_fused_append_nhd_q_only():
    c = append_case(450, 33, hidden=2048, hq=8, hkv=2, d=64, qwen=False, ps=8, layout="NHD")
    append_check(c, "pair append NHD D=64 q-only", write_kv_out=False)
    braidinfer_amd.check_device_status()
