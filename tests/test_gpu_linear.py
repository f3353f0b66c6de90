"""GPU parity of the linear-layer fusions (bfa_linear) against the oracle:
F.linear with and without bias, residual + F.linear, SiluAndMul of the packed
gate_up projection, and FusedAttentionOutput's fp16-stored projection.

Shapes cover the split-K decode path (1..64 tokens, both partial layouts, and
the deep-K form with 2, 8 and 16 chunks of 256 per split), the
DMA prefill tiles (256x256, 128x256, 128x128) and the register-staged path (K
not a multiple of 64, strided rows), with output widths that are not multiples
of the tile or of 8 (masked stores).  Tolerance: |d| <= 2e-2 + 1e-2 |r|
elementwise (tests/helpers.py), with fp32 sums in another order than the
oracle's allowed to move a result by the bf16 ulps the tolerance covers.
"""
from __future__ import annotations

import pytest
import torch

from braidinfer_amd.kernels import FusedAttentionOutput, attention_output, attention_output_gemv
from braidinfer_amd.layers import (MergedColumnParallelLinear, RowParallelLinear, gate_up_silu_and_mul,
                                   linear, linear_add_residual)
from oracle import torch_ref as R
from tests.helpers import assert_close, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = [
    # tokens, k, n
    (1, 1024, 1024),      # Qwen3-0.6B o_proj decode
    (7, 4096, 1000),      # odd token count, n not a multiple of 8
    (33, 2048, 5632),     # three 16-token blocks (register-order partials)
    (64, 4096, 4096),     # largest decode batch (deep-K form: 2 chunks of 256 per split)
    (20, 4096, 12288),    # two 16-token blocks, 8 chunks per split
    (40, 2048, 8192),     # three 16-token blocks, 2 chunks per split
    (65, 1024, 3072),     # smallest prefill
    (300, 4096, 1000),    # ragged prefill tile, masked columns
    (1024, 2048, 2048),   # 128x256 tiles
    (2048, 4096, 4096),   # 256x256 tiles
    (200, 1040, 768),     # K % 64 != 0: register-staged path
]


def _ids(s):
    return "t{}_k{}_n{}".format(*s)


@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
@pytest.mark.parametrize("bias", [False, True])
def test_linear(shape, bias):
    t, k, n = shape
    g = gen(t * 7 + k + n + int(bias))
    x, w = randn(g, t, k), randn(g, n, k, std=0.03)
    b = randn(g, n, std=0.5) if bias else None
    got = linear(x.to(DEV), w.to(DEV), None if b is None else b.to(DEV))
    assert got.dtype == torch.bfloat16 and got.shape == (t, n)
    assert_close(got, R.linear(x, w, b), what=f"linear {shape}")


@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
def test_linear_add_residual(shape):
    t, k, n = shape
    g = gen(t * 11 + k + n)
    x, w, r = randn(g, t, k), randn(g, n, k, std=0.03), randn(g, t, n, std=2.0)
    got = linear_add_residual(x.to(DEV), w.to(DEV), r.to(DEV))
    # The projection is rounded before the residual is added: where a sum in
    # another order lands on the other side of that rounding, the result moves
    # by one bf16 ulp of the projection, which the residual may then cancel
    # down to a small value -- allowed for at most 1e-3 of the elements.
    slack = 2.0 ** -7 * R.linear(x, w).float().abs()
    assert_close(got, R.linear_add_residual(x, w, r), what=f"linear+residual {shape}", slack=slack,
                 max_slack_frac=1e-3)
    layer = RowParallelLinear(k, n).to(DEV).to(torch.bfloat16)
    with torch.no_grad():
        layer.weight.copy_(w.to(DEV))
    assert torch.equal(layer.forward_add_residual(x.to(DEV), r.to(DEV)), got)


@pytest.mark.parametrize("splits,t", [("4", 64), ("1", 48), ("2", 20), ("3", 33)])
def test_deep_k_chunk_counts(tuning, splits, t):
    """The deep-K decode form with the split count forced (K = 3072: 12 chunks of
    256): 3, 12, 6 and 4 chunks per split, two to four 16-token blocks, against
    the oracle."""
    tuning("DECODE_SPLITS", int(splits))
    g = gen(900 + t)
    k, n = 3072, 2048
    x, w, b = randn(g, t, k), randn(g, n, k, std=0.03), randn(g, n, std=0.5)
    assert_close(linear(x.to(DEV), w.to(DEV), b.to(DEV)), R.linear(x, w, b), what=f"deep-K splits={splits} t={t}")


@pytest.mark.parametrize("shape", [(1, 1024, 3072), (16, 2048, 5632), (64, 4096, 1000), (64, 4096, 14336),
                                   (65, 1024, 3072), (500, 2048, 1000), (2048, 4096, 3584),
                                   (96, 1040, 512)], ids=_ids)
def test_gate_up_silu_and_mul(shape):
    t, k, inter = shape
    g = gen(t * 13 + k + inter)
    x, w = randn(g, t, k), randn(g, 2 * inter, k, std=0.05)
    got = gate_up_silu_and_mul(x.to(DEV), w.to(DEV))
    assert got.shape == (t, inter)
    # silu(g) and u are each rounded to bf16 before their product is: a sum in
    # another order can flip either rounding, one ulp each, so up to two more
    # ulps of the result than the plain tolerance covers -- allowed for at most
    # 1e-4 of the elements.
    exp = R.gate_up_silu_and_mul(x, w)
    assert_close(got, exp, what=f"gate_up silu {shape}", slack=2.0 ** -6 * exp.float().abs(),
                 max_slack_frac=1e-4)
    layer = MergedColumnParallelLinear(k, [inter, inter]).to(DEV).to(torch.bfloat16)
    with torch.no_grad():
        layer.weight.copy_(w.to(DEV))
    assert torch.equal(layer.forward_silu_and_mul(x.to(DEV)), got)


def test_gate_up_silu_and_mul_8192_tokens_sampled_rows():
    """Llama-3-8B gate_up_proj + SiluAndMul at the 8192-token prefill (4096 ->
    2 x 14336, 256x256 tiles over the full grid): the rows of a GEMM are
    independent, so 128 rows sampled across the whole range (both ends, every
    row tile's neighbourhood) are checked against the oracle, with the same
    one-ulp flip allowance as above, and against the fp32 mode of the oracle."""
    from oracle import fp32_ref as F
    g = gen(8192)
    t, k, inter = 8192, 4096, 14336
    x = randn(g, t, k)
    w = randn(g, 2 * inter, k, std=0.02)
    got = gate_up_silu_and_mul(x.to(DEV), w.to(DEV))
    rows = torch.cat([torch.tensor([0, 1, 255, 256, t - 2, t - 1]),
                      torch.randperm(t, generator=g)[:122]]).sort().values
    sub = got[rows.to(DEV)].cpu()
    exp = R.gate_up_silu_and_mul(x[rows], w)
    assert_close(sub, exp, what="gate_up silu t=8192 (128 sampled rows)", slack=2.0 ** -6 * exp.float().abs(),
                 max_slack_frac=1e-4)
    f32 = F.gate_up_silu_and_mul(x[rows], w)
    d = (sub.float() - f32.float()).abs()
    assert ((d - (2e-2 + 1e-2 * f32.float().abs())) > 0).sum().item() <= 1e-4 * d.numel()
    assert (d.norm() / f32.float().norm()).item() < 5e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("t", [1, 40, 300])
def test_attention_output(dtype, t):
    g = gen(17 + t)
    h = 1024
    x, w, r = randn(g, t, h, dtype=dtype), randn(g, h, h, std=0.03, dtype=dtype), randn(g, t, h, dtype=dtype)
    got = attention_output(x.to(DEV), w.to(DEV), r.to(DEV))
    assert got.dtype == dtype
    assert_close(got, R.fused_attention_output(x, w, r), what=f"attention output t={t} {dtype}")
    assert_close(attention_output_gemv(x.to(DEV), w.to(DEV)), R.fused_attention_output(x, w),
                 what=f"attention output gemv t={t}")


def test_fused_attention_output_class_keeps_reference_shapes():
    g = gen(3)
    h = 896
    x, w, r = randn(g, 1, 1, h), randn(g, h, h, std=0.03), randn(g, 1, 1, h)
    got = FusedAttentionOutput.forward(x.to(DEV), w.to(DEV), r.to(DEV))
    assert got.shape == (1, 1, h)
    assert_close(got, R.fused_attention_output(x.view(1, h), w, r.view(1, h)).view(1, 1, h),
                 what="FusedAttentionOutput.forward")
    y = FusedAttentionOutput.gemv(x.view(1, h).to(DEV), w.to(DEV))
    assert_close(y, R.fused_attention_output(x.view(1, h), w), what="FusedAttentionOutput.gemv")
    with pytest.raises(AssertionError):
        FusedAttentionOutput.forward(torch.zeros(1, 2, h, dtype=torch.bfloat16, device=DEV), w.to(DEV),
                                     torch.zeros(1, 2, h, dtype=torch.bfloat16, device=DEV))


def test_fp16_overflow_is_inf_like_the_reference():
    # 300 * 250 = 75000 > fp16 max: the reference's fp16 store makes it inf
    x = torch.zeros(1, 64, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(64, 64, dtype=torch.bfloat16, device=DEV)
    x[0, 0] = 300.0
    w[:, 0] = 250.0
    assert torch.isinf(attention_output_gemv(x, w)).all()
    assert torch.isfinite(linear(x, w)).all()


def test_strided_rows_and_empty():
    g = gen(5)
    base = randn(g, 70, 2048 + 64)
    x = base[:, :2048]  # row stride 2112
    w = randn(g, 512, 2048, std=0.03)
    assert_close(linear(x.to(DEV), w.to(DEV)), R.linear(x, w), what="strided x, prefill")
    assert_close(linear(x[:5].to(DEV), w.to(DEV)), R.linear(x[:5], w), what="strided x, decode")
    xd = base.to(DEV)[:, :2048]
    assert xd.stride(0) == 2112
    assert_close(linear(xd, w.to(DEV)), R.linear(x, w), what="strided device view")
    empty = linear(torch.empty(0, 2048, dtype=torch.bfloat16, device=DEV), w.to(DEV))
    assert empty.shape == (0, 512)


def test_mismatched_dtypes_raise():
    x = torch.zeros(4, 64, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(32, 64, dtype=torch.float16, device=DEV)
    with pytest.raises(TypeError):
        linear(x, w)
    with pytest.raises(ValueError):
        linear(torch.zeros(4, 60, dtype=torch.bfloat16, device=DEV), torch.zeros(8, 60, dtype=torch.bfloat16,
                                                                                 device=DEV))
