"""GPU parity of the memory-bound kernels against the oracle.

Every test runs the HIP path through the C ABI (braidinfer_amd.*) on seeded
inputs and compares with oracle/torch_ref.py on CPU: bit-exact for the gather
(and for RoPE, whose fp32 op sequence is reproduced exactly), otherwise
|d| <= 2e-2 + 1e-2 |r| elementwise (tests/helpers.py).
"""
from __future__ import annotations

import math

import pytest
import torch

import braidinfer_amd
from braidinfer_amd.kernels import RMSNormF32
from braidinfer_amd.layers import (RMSNorm, RotaryEmbedding, SiluAndMul, VocabParallelEmbedding,
                                   apply_rotary_emb, get_rope, rerotate_paged_k)
from braidinfer_amd.layers.embed_head import embedding
from oracle import torch_ref as R
from tests.helpers import assert_close, bits, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def cuda(*ts):
    return [t.to(DEV) for t in ts]


def exact_fraction(a, b):
    return (bits(a) == bits(b)).float().mean().item()


# --------------------------------------------------------------------- norms
@pytest.mark.parametrize("shape,dtype,wdtype", [
    ((128, 2048), torch.bfloat16, torch.bfloat16),     # TinyLlama RMSNorm [128, 2048]
    ((64, 4096), torch.bfloat16, torch.bfloat16),
    ((1, 1024), torch.bfloat16, torch.float32),
    ((3, 7, 896), torch.float16, torch.float16),
    ((1500, 4096), torch.bfloat16, torch.bfloat16),
    ((5, 100), torch.bfloat16, torch.bfloat16),         # unaligned hidden: scalar path
    ((2, 40000), torch.bfloat16, torch.bfloat16),       # beyond the register-resident sizes
])
def test_rms_forward(shape, dtype, wdtype):
    g = gen(101)
    x = randn(g, *shape, dtype=dtype)
    w = randn(g, shape[-1], mean=1.0, std=0.1, dtype=wdtype)
    norm = RMSNorm(shape[-1], eps=1e-5).to(DEV)
    with torch.no_grad():
        norm.weight.data = w.to(DEV)
    y = norm(x.to(DEV))
    ref = R.rms_forward(x, w, 1e-5)
    assert y.dtype == ref.dtype and y.shape == ref.shape
    assert_close(y, ref, what="rms_forward")
    assert exact_fraction(y, ref) > 0.99


def test_rms_forward_fp32_mutates_and_returns_input():
    g = gen(102)
    x = randn(g, 32, 1024, dtype=torch.float32).to(DEV)
    keep = x.clone()
    norm = RMSNorm(1024, eps=1e-6).to(DEV)
    y = norm(x)
    assert y is x, "fp32 rms_forward returns the (mutated) input tensor"
    assert_close(y, R.rms_forward(keep.cpu(), norm.weight.detach().cpu(), 1e-6), atol=1e-5, rtol=1e-5)


def test_per_head_norm_on_strided_view():
    """q/k norm on [T, heads, D] views of a packed qkv buffer (models/qwen3.py:258)."""
    g = gen(103)
    t, hq, hkv, d = 37, 16, 8, 128
    buf = randn(g, t, (hq + 2 * hkv) * d).to(DEV)
    k = buf[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    w = torch.exp(torch.empty(d).uniform_(math.log(0.05), math.log(100), generator=g)).to(torch.bfloat16)
    norm = RMSNorm(d, eps=1e-6).to(DEV)
    with torch.no_grad():
        norm.weight.data = w.to(DEV)
    y = norm(k)
    assert_close(y, R.rms_forward(k.cpu(), w, 1e-6), what="k_norm view")
    yf = norm(k.float())  # q.float() path of the Qwen3 glue
    assert_close(yf, R.rms_forward(k.cpu().float(), w, 1e-6), atol=1e-4, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_add_rms_forward(dtype):
    g = gen(104)
    x, r = randn(g, 64, 4096, dtype=dtype), randn(g, 64, 4096, dtype=dtype)
    w = randn(g, 4096, mean=1.0, std=0.1, dtype=dtype)
    norm = RMSNorm(4096, eps=1e-5).to(DEV)
    with torch.no_grad():
        norm.weight.data = w.to(DEV)
    y, res = norm(x.to(DEV), r.to(DEV))
    ry, rres = R.add_rms_forward(x, r, w, 1e-5)
    assert torch.equal(bits(res), bits(rres)), "residual_out = to(dtype)(x + r) is exact"
    assert_close(y, ry, what="add_rms y")


def test_add_rms_forward_fp32_aliases():
    g = gen(105)
    x, r = randn(g, 16, 512, dtype=torch.float32), randn(g, 16, 512, dtype=torch.float32)
    norm = RMSNorm(512).to(DEV)
    xd = x.to(DEV)
    a, b = norm(xd, r.to(DEV))
    assert a is xd and b is xd
    ry, _ = R.add_rms_forward(x, r, torch.ones(512), 1e-6)
    assert_close(a, ry, atol=1e-5, rtol=1e-5)


def test_add_rms_forward_unsupported_dtype_raises_type_error():
    """float64 (which no kernel takes) raises the library's dtype error, not a
    bare KeyError from the 16-bit fast path."""
    norm = RMSNorm(64).to(DEV)
    x = torch.randn(4, 64, dtype=torch.float64, device=DEV)
    with pytest.raises(TypeError, match="unsupported dtype"):
        norm(x, torch.randn_like(x))


def test_rmsnorm_f32_reference_tests():
    """The checks of tests/test_rmsnorm_f32.py, run on the HIP kernel."""
    g = gen(106)

    def pytorch_rmsnorm(x, weight, eps=1e-6):
        x_f32 = x.float()
        var = x_f32.pow(2).mean(dim=-1, keepdim=True)
        return x_f32 / torch.sqrt(var + eps) * weight.float()

    x, w = cuda(randn(g, 4, 8), randn(g, 8))
    out = RMSNormF32.forward(x, w, 1e-6)
    assert out.dtype == torch.float32 and out.shape == x.shape
    assert (pytorch_rmsnorm(x, w) - out).abs().max().item() < 1e-5
    x, w = cuda(randn(g, 512, 1024), randn(g, 1024))
    ref = pytorch_rmsnorm(x, w)
    assert ((ref - RMSNormF32.forward(x, w, 1e-6)) / (ref + 1e-8)).abs().max().item() < 1e-4
    w[0] = 96.5
    w[100:110] = 50.0
    ref = pytorch_rmsnorm(x[:128], w)
    out = RMSNormF32.forward(x[:128], w, 1e-6)
    assert torch.isfinite(out).all() and ((ref - out) / (ref + 1e-8)).abs().max().item() < 1e-3
    buf = torch.empty(64, 256, dtype=torch.float32, device=DEV)
    xi, wi = cuda(randn(g, 64, 256), randn(g, 256))
    res = RMSNormF32.forward(xi, wi, 1e-6, output=buf)
    assert res.data_ptr() == buf.data_ptr()
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        xd, wd = cuda(randn(g, 32, 128, dtype=dtype), randn(g, 128, dtype=dtype))
        out = RMSNormF32.forward(xd, wd, 1e-6)
        ref = pytorch_rmsnorm(xd, wd)
        assert out.dtype == torch.float32 and ((ref - out) / (ref + 1e-8)).abs().max().item() < 1e-4
    # column-strided input (the reference kernel takes both strides)
    xt = randn(g, 256, 64).to(DEV).t()
    out = RMSNormF32.forward(xt, wi, 1e-6)
    assert_close(out, R.rmsnorm_f32(xt.cpu(), wi.cpu(), 1e-6), atol=1e-5, rtol=1e-5)
    xs = (torch.ones(16, 64) + torch.randn(16, 64, generator=g) * 1e-4).to(torch.bfloat16).to(DEV)
    out = RMSNormF32.forward(xs, torch.ones(64, dtype=torch.bfloat16, device=DEV), 1e-6)
    assert torch.isfinite(out).all() and out.abs().max() < 10


# ---------------------------------------------------------------- gather
@pytest.mark.parametrize("v,h,ids_shape,idt", [
    (128256, 4096, (64,), torch.int64),   # Llama-3-8B table, batch-64 decode
    (5000, 4096, (2, 600), torch.int64),
    (1000, 1024, (7,), torch.int32),
    (333, 13, (50,), torch.int64),       # row bytes not a multiple of 16: element path
])
def test_embedding_bit_exact(v, h, ids_shape, idt):
    g = gen(107)
    table = randn(g, v, h, std=0.02)
    ids = torch.randint(0, v, ids_shape, generator=g, dtype=idt)
    emb = VocabParallelEmbedding(v, h).to(DEV)
    with torch.no_grad():
        emb.weight.data = table.to(DEV)
    out = emb(ids.to(DEV))
    ref = R.embedding(ids.long(), table)
    assert out.shape == ref.shape and torch.equal(bits(out), bits(ref))
    braidinfer_amd.check_device_status()


@pytest.mark.parametrize("idt", [torch.int32, torch.int64])
def test_embedding_many_ids_four_rows_per_workgroup(idt):
    """From 4096 ids, rows of up to 8 KiB are gathered four per workgroup: a
    count that leaves a partial last block, out-of-range ids (zero rows and
    IndexError) inside a block, and the scaled (Qwen3) form."""
    g = gen(123)
    v, h, t = 3000, 2048, 4099
    table = randn(g, v, h, std=0.02)
    ids = torch.randint(0, v, (t,), generator=g, dtype=idt)
    out = embedding(ids.to(DEV), table.to(DEV))
    assert torch.equal(bits(out), bits(R.embedding(ids.long(), table)))
    braidinfer_amd.check_device_status()
    outs = embedding(ids.to(DEV), table.to(DEV), scale=1.0 / (h ** 0.5))
    assert torch.equal(bits(outs), bits(R.embedding_scaled(ids.long(), table, h)))
    bad = ids.clone()
    bad[4097] = v          # in the partial last block
    bad[5] = -1
    out = embedding(bad.to(DEV), table.to(DEV))
    with pytest.raises(IndexError):
        braidinfer_amd.check_device_status()
    keep = torch.ones(t, dtype=torch.bool)
    keep[[5, 4097]] = False
    assert out[5].eq(0).all() and out[4097].eq(0).all()
    assert torch.equal(bits(out[keep.to(DEV)]), bits(R.embedding(ids.long(), table)[keep]))
    braidinfer_amd.check_device_status()  # cleared


def test_embedding_scaled_matches_qwen3_glue():
    g = gen(108)
    table = randn(g, 4000, 2048, std=0.02)
    ids = torch.randint(0, 4000, (33,), generator=g)
    out = embedding(ids.to(DEV), table.to(DEV), scale=1.0 / (2048 ** 0.5))
    assert torch.equal(bits(out), bits(R.embedding_scaled(ids, table, 2048)))


def test_embedding_out_of_range():
    table = torch.zeros(10, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(IndexError):
        embedding(torch.tensor([3, 10]), table)          # host ids: checked before launch
    out = embedding(torch.tensor([3, 11, -1], device=DEV), table + 1)
    with pytest.raises(IndexError):
        braidinfer_amd.check_device_status()
    assert out[0].eq(1).all() and out[1:].eq(0).all()
    braidinfer_amd.check_device_status()  # cleared


# ---------------------------------------------------------------- SwiGLU
@pytest.mark.parametrize("shape,dtype", [
    ((2048, 2 * 3072), torch.bfloat16),   # Qwen3-0.6B SwiGLU shape
    ((64, 2 * 14336), torch.bfloat16),    # Llama-3-8B decode
    ((3, 5, 2 * 512), torch.float16),
    ((17, 2 * 100), torch.float32),
    ((9, 2 * 13), torch.bfloat16),        # odd intermediate size: element path
])
def test_silu_and_mul(shape, dtype):
    g = gen(109)
    x = randn(g, *shape, dtype=dtype)
    y = SiluAndMul()(x.to(DEV))
    ref = R.silu_and_mul(x)
    assert y.shape == ref.shape and y.dtype == ref.dtype
    assert_close(y, ref, what="silu_and_mul")
    if dtype != torch.float32:
        assert exact_fraction(y, ref) > 0.99


# ------------------------------------------------------------------ RoPE
@pytest.mark.parametrize("d,base,maxp,hq,hkv,dtype", [
    (64, 1e4, 2048, 32, 4, torch.bfloat16),    # TinyLlama
    (128, 1e6, 40960, 16, 8, torch.bfloat16),  # Qwen3-0.6B
    (128, 5e5, 8192, 32, 8, torch.float32),    # Llama-3-8B (fp32 q/k from minimal_f32)
    (96, 1e4, 512, 3, 1, torch.float16),
    (10, 1e4, 64, 2, 2, torch.bfloat16),       # head_dim not a multiple of 16: element path
])
def test_rotary_embedding_matches_exactly(d, base, maxp, hq, hkv, dtype):
    g = gen(110)
    t = 41
    rope = RotaryEmbedding(d, d, maxp, base).to(DEV)
    cache = R.cos_sin_cache(d, maxp, base)
    assert torch.equal(rope.cos_sin_cache.cpu(), cache)
    buf = randn(g, t, (hq + 2 * hkv) * d, dtype=dtype)
    q = buf[:, : hq * d]                    # strided views, as split() returns them
    k = buf[:, hq * d:(hq + hkv) * d]
    pos = torch.randint(-maxp, maxp, (t,), generator=g)
    bd = buf.to(DEV)
    qo, ko = rope(pos.to(DEV), bd[:, : hq * d], bd[:, hq * d:(hq + hkv) * d])
    rq, rk = R.rotary_forward(cache, d, pos, q, k)
    assert qo.shape == q.shape and ko.dtype == dtype
    # same fp32 op sequence and rounding: bit-exact
    assert torch.equal(bits(qo), bits(rq)) and torch.equal(bits(ko), bits(rk))


def test_rotary_key_regrouped_by_positions():
    """attention.py:200: k_full with more rows than positions is viewed as
    [num_tokens, -1, head_size] (the reference's view semantics)."""
    g = gen(111)
    rope = get_rope(64, 64, 2048, 10000.0).to(DEV)
    k_full = randn(g, 12, 4, 64)
    pos = torch.randint(0, 2048, (6,), generator=g)
    _, ko = rope(pos.to(DEV), torch.empty(6, 64, device=DEV, dtype=torch.bfloat16), k_full.to(DEV))
    _, rk = R.rotary_forward(R.cos_sin_cache(64, 2048, 10000.0), 64, pos,
                             torch.empty(6, 64, dtype=torch.bfloat16), k_full)
    assert torch.equal(bits(ko), bits(rk))


def test_apply_rotary_emb():
    g = gen(112)
    x = randn(g, 9, 5, 128)
    cache = R.cos_sin_cache(128, 4096, 1e6)
    pos = torch.randint(0, 4096, (9,), generator=g)
    cos, sin = cache[pos].chunk(2, dim=-1)
    y = apply_rotary_emb(x.to(DEV), cos.to(DEV), sin.to(DEV))
    assert torch.equal(bits(y), bits(R.apply_rotary_emb(x, cos, sin)))


def test_rotary_out_of_range_position():
    rope = RotaryEmbedding(64, 64, 128, 1e4).to(DEV)
    q = torch.ones(2, 64, device=DEV, dtype=torch.bfloat16)
    rope(torch.tensor([5, 128], device=DEV), q, q)
    with pytest.raises(IndexError):
        braidinfer_amd.check_device_status()


# ------------------------------------------------------ paged diff-RoPE
def _paged(seed, pages, hkv, ps, d, chunk_pages, last_lens):
    g = gen(seed)
    kv = randn(g, pages, 2, hkv, ps, d)
    perm = torch.randperm(pages, generator=g)
    indptr = torch.tensor([0] + list(torch.tensor(chunk_pages).cumsum(0)), dtype=torch.int32)
    return kv, perm[: int(indptr[-1])].to(torch.int32), indptr, torch.tensor(last_lens, dtype=torch.int32)


@pytest.mark.parametrize("hkv,d", [(8, 128), (4, 64), (2, 256), (4, 32), (1, 16), (2, 96), (1, 1024)])
def test_rerotate_paged_k(hkv, d):
    """Every row-group width of the one-workgroup-per-entry kernel (head_dim 16 ..
    1024, 96 with idle lanes in each row group)."""
    maxp = 40960
    cache = R.cos_sin_cache(d, maxp, 1e6)
    kv, idx, indptr, last = _paged(113, 64, hkv, 16, d, [16, 1, 20, 7, 0, 4], [16, 9, 3, 16, 0, 1])
    delta = torch.tensor([1234, -4096, 0, 4096, 7, -1], dtype=torch.int64)
    w = torch.exp(torch.empty(d).uniform_(math.log(0.05), math.log(100), generator=gen(5))).to(torch.bfloat16)
    args = [t.to(DEV) for t in (idx, indptr, delta, last)]
    kvd = kv.to(DEV)
    out = rerotate_paged_k(kvd, args[0], args[1], args[2], args[3], cache.to(DEV))
    ref = R.rerotate_paged_k(kv, idx, indptr, delta, last, cache)
    assert torch.equal(bits(out), bits(ref)), "same fp32 op sequence: bit-exact"
    assert torch.equal(bits(kvd), bits(kv)), "out-of-place mode leaves the cache untouched"
    outn = rerotate_paged_k(kvd, *args, cache.to(DEV), k_norm_weight=w.to(DEV), k_norm_eps=1e-6)
    refn = R.rerotate_paged_k(kv, idx, indptr, delta, last, cache, w, 1e-6)
    assert_close(outn, refn, what="rerotate + k_norm")
    # in place: rotated pages land back in the HND cache
    rerotate_paged_k(kvd, *args, cache.to(DEV), inplace=True)
    for e in range(idx.numel()):
        c = int(torch.searchsorted(indptr, torch.tensor(e, dtype=torch.int32), right=True)) - 1
        n = int(last[c]) if e == int(indptr[c + 1]) - 1 else 16
        got = kvd[int(idx[e]), 0, :, :n].transpose(0, 1).cpu()
        assert torch.equal(bits(got), bits(ref[e, :n]))
    braidinfer_amd.check_device_status()


def test_rerotate_paged_k_wide_heads():
    """head_dim above 1024 takes the per-(entry, kv head) kernel; the fused k_norm
    is refused there."""
    maxp, d = 4096, 2048
    cache = R.cos_sin_cache(d, maxp, 1e4)
    kv, idx, indptr, last = _paged(31, 6, 2, 4, d, [2, 3], [4, 2])
    delta = torch.tensor([-17, 300], dtype=torch.int64)
    args = [t.to(DEV) for t in (idx, indptr, delta, last)]
    out = rerotate_paged_k(kv.to(DEV), *args, cache.to(DEV))
    ref = R.rerotate_paged_k(kv, idx, indptr, delta, last, cache)
    assert torch.equal(bits(out), bits(ref))
    with pytest.raises(ValueError):
        rerotate_paged_k(kv.to(DEV), *args, cache.to(DEV), k_norm_weight=torch.ones(d, device=DEV))
    braidinfer_amd.check_device_status()


def test_rerotate_paged_k_many_chunks():
    """More than 64 chunks (the chunk search walks several 64-chunk blocks), empty
    chunks among them, and a final chunk whose last page is partly filled."""
    g = gen(21)
    hkv, ps, d, maxp = 2, 16, 128, 40960
    cache = R.cos_sin_cache(d, maxp, 1e6)
    counts = [int(x) for x in torch.randint(0, 3, (150,), generator=g)]
    pages = sum(counts) + 3
    lasts = [int(x) for x in torch.randint(1, ps + 1, (150,), generator=g)]
    kv, idx, indptr, last = _paged(22, pages, hkv, ps, d, counts, lasts)
    delta = torch.randint(-4096, 4097, (150,), generator=g)
    args = [t.to(DEV) for t in (idx, indptr, delta, last)]
    out = rerotate_paged_k(kv.to(DEV), *args, cache.to(DEV))
    ref = R.rerotate_paged_k(kv, idx, indptr, delta, last, cache)
    assert torch.equal(bits(out), bits(ref))
    braidinfer_amd.check_device_status()


def test_rerotate_paged_k_full_config():
    """The configured workload at full size: 4096 cached tokens x 8 kv heads x 128
    in 256 pages of 16 (HND), pages in shuffled order, 16 chunks of 16 pages,
    one delta per chunk from U[-4096, 4096], theta 1e6, table of 40960 positions
    (negative deltas wrap): bit-exact against the oracle."""
    g = gen(4)
    pages, hkv, ps, d, maxp = 256, 8, 16, 128, 40960
    kv = randn(g, pages, 2, hkv, ps, d)
    idx = torch.randperm(pages, generator=g).to(torch.int32)
    indptr = (torch.arange(17, dtype=torch.int32) * 16)
    delta = torch.randint(-4096, 4097, (16,), generator=g)
    last = torch.full((16,), ps, dtype=torch.int32)
    cache = R.cos_sin_cache(d, maxp, 1e6)
    out = rerotate_paged_k(kv.to(DEV), idx.to(DEV), indptr.to(DEV), delta.to(DEV), last.to(DEV), cache.to(DEV))
    ref = R.rerotate_paged_k(kv, idx, indptr, delta, last, cache)
    assert torch.equal(bits(out), bits(ref))
    braidinfer_amd.check_device_status()


def test_rerotate_delta_out_of_table():
    cache = R.cos_sin_cache(64, 128, 1e4).to(DEV)
    kv = torch.zeros(2, 2, 1, 16, 64, device=DEV, dtype=torch.bfloat16)
    one = lambda v: torch.tensor(v, dtype=torch.int32, device=DEV)
    rerotate_paged_k(kv, one([0]), one([0, 1]), torch.tensor([-129], device=DEV), one([16]), cache)
    with pytest.raises(IndexError):
        braidinfer_amd.check_device_status()


# ------------------------------------------- Llama-3-8B 8192-token prefill sizes
# The memory-bound ops at the 8192-token configuration.  Rows are independent,
# so the oracle runs on a seeded sample of rows (and the integer parts -- the
# gather and the residual sum -- on every row).
def _sample_rows(g, n, k=384):
    return torch.randperm(n, generator=g)[:k].sort().values


def test_add_rms_forward_8192_tokens():
    g = gen(120)
    t, h = 8192, 4096
    x, r = randn(g, t, h), randn(g, t, h)
    w = randn(g, h, mean=1.0, std=0.1)
    norm = RMSNorm(h, eps=1e-5).to(DEV)
    with torch.no_grad():
        norm.weight.data = w.to(DEV)
    y, res = norm(x.to(DEV), r.to(DEV))
    y, res = y.cpu(), res.cpu()
    assert torch.equal(bits(res), bits((x.float() + r.float()).bfloat16())), "residual_out exact on every row"
    rows = _sample_rows(g, t)
    ry, _ = R.add_rms_forward(x[rows], r[rows], w, 1e-5)
    assert_close(y[rows], ry, what="add_rms y, 8192 tokens (sampled rows)")


def test_silu_and_mul_8192_tokens():
    g = gen(121)
    t, i = 8192, 14336
    xd = torch.randn(t, 2 * i, device=DEV, dtype=torch.float32,
                     generator=torch.Generator(device=DEV).manual_seed(121)).bfloat16()
    y = SiluAndMul()(xd)
    rows = _sample_rows(g, t)
    xs = xd[rows.to(DEV)].cpu()
    assert_close(y[rows.to(DEV)], R.silu_and_mul(xs), what="silu_and_mul, 8192 x 2*14336 (sampled rows)")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_streamed_outputs_equal_cached_stores(dtype):
    """Outputs of 64 MiB and more are stored with the nontemporal hint, smaller
    ones plainly; the hint must not change a value.  A call whose output is just
    over 64 MiB and a call on its first rows (well under it) agree bit for bit on
    those rows: SiLU*mul, and add+RMSNorm's y and residual."""
    esz = torch.tensor([], dtype=dtype).element_size()
    dg = torch.Generator(device=DEV).manual_seed(131)
    inter = 4096
    rows = (64 << 20) // (inter * esz) + 8
    xd = torch.randn(rows, 2 * inter, device=DEV, generator=dg).to(dtype)
    y_full = SiluAndMul()(xd)
    for lo in (0, rows - 64):
        y_part = SiluAndMul()(xd[lo:lo + 64].contiguous())
        assert torch.equal(bits(y_full[lo:lo + 64]), bits(y_part)), f"silu_and_mul rows {lo}.."
    h = 4096
    rows = (64 << 20) // (h * esz) + 8
    x = torch.randn(rows, h, device=DEV, generator=dg).to(dtype)
    r = torch.randn(rows, h, device=DEV, generator=dg).to(dtype)
    w = (torch.randn(h, device=DEV, generator=dg) * 0.1 + 1.0).to(dtype)
    norm = RMSNorm(h, eps=1e-5).to(DEV)
    with torch.no_grad():
        norm.weight.data = w
    y_full, r_full = norm(x.clone(), r.clone())  # fp32 normalises in place: work on copies
    y_full, r_full = y_full.clone(), r_full.clone()
    for lo in (0, rows - 64):
        y_part, r_part = norm(x[lo:lo + 64].clone(), r[lo:lo + 64].clone())
        assert torch.equal(bits(y_full[lo:lo + 64]), bits(y_part)), f"add_rms y rows {lo}.."
        assert torch.equal(bits(r_full[lo:lo + 64]), bits(r_part)), f"add_rms residual rows {lo}.."


def test_embedding_full_llama3_table_8192_ids():
    """The gather over the whole [128256, 4096] table with 8192 ids (about a
    quarter of them repeated), bit for bit against indexing a host copy."""
    v, h, t = 128256, 4096, 8192
    gd = torch.Generator(device=DEV).manual_seed(122)
    table = (torch.randn(v, h, device=DEV, generator=gd) * 0.02).bfloat16()
    ids = torch.randint(0, v, (t,), device=DEV, generator=gd)
    ids[::4] = ids[1::4]
    emb = VocabParallelEmbedding(v, h).to(DEV)
    with torch.no_grad():
        emb.weight.data = table
    out = emb(ids)
    ref = R.embedding(ids.cpu(), table.cpu())
    assert torch.equal(bits(out), bits(ref))
    braidinfer_amd.check_device_status()
