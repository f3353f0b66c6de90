"""GPU parity of the fused QKV + paged KV append (bfa_fused_rmsnorm_qkv_append):
one call that does what the reference's attention layer does with two -- the
fused RMSNorm+QKV(+q/k norm)+RoPE projection (kernels/fused_rmsnorm_qkv_*.py,
models/llama.py:169-205, models/qwen3.py:236-309) and the append of its k and v
heads to the layer's paged cache (kernels/kv_cache_utils.py:9-78).

Each case runs the fused call and checks
  * its output against the plain fused QKV call on the same inputs: bit for bit
    (the k/v columns too, unless write_kv_out=False, when they must be left as
    they were);
  * the whole cache against the oracle's append (oracle/torch_ref.py) of the
    k and v heads that output holds: bit for bit.
The token counts reach every epilogue that writes the cache: 1-16 tokens (the
one-launch kernel's epilogue where the planner takes it, without q/k norm;
else the row epilogue after the weight-streaming kernel), 17-64 (the split-K decode
epilogue), more (the prefill GEMM's fused epilogue, every tile form), and
head_dim 80 (the raw projection + row epilogue)."""
from __future__ import annotations

import pytest
import torch

import braidinfer_amd
from braidinfer_amd.kernels import PagedKVAppend
from braidinfer_amd.kernels._qkv import fused_rmsnorm_qkv
from oracle import torch_ref as R
from tests.helpers import bits, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make_case(seed, tokens, hidden, hq, hkv, d, qwen, ps=16, pages=None, start=3, layout="HND",
              cache_dtype=torch.bfloat16):
    g = gen(seed)
    n = (hq + 2 * hkv) * d
    c = dict(x=randn(g, tokens, hidden), ln=randn(g, hidden, mean=1.0, std=0.1),
             w=randn(g, n, hidden, std=0.02), hq=hq, hkv=hkv, d=d, qwen=qwen)
    if qwen:
        c["qn"] = randn(g, d, mean=1.0, std=0.1)
        c["kn"] = randn(g, d, mean=1.0, std=0.3)
    c["pos"] = torch.randint(0, 4096, (tokens,), generator=g)
    c["table"] = R.cos_sin_cache(d, 4096, 1e6 if qwen else 5e5)
    need = (start + tokens + ps - 1) // ps
    pages = pages or need + 7
    c["kv_indices"] = torch.randperm(pages, generator=g)[:need].to(torch.int32)
    shape = (pages, 2, hkv, ps, d) if layout == "HND" else (pages, 2, ps, hkv, d)
    c["cache"] = randn(g, *shape, dtype=cache_dtype)
    c["cache_pos"] = torch.arange(start, start + tokens, dtype=torch.int64)
    c["ps"], c["layout"] = ps, layout
    return c


def call(c, paged_kv=None, out=None):
    kw = dict(positions=c["pos_d"], cos_sin_cache=c["table_d"], out=out, paged_kv=paged_kv)
    if c["qwen"]:
        return fused_rmsnorm_qkv(c["x_d"], c["ln_d"], c["w_d"], c["hq"], c["hkv"], 1e-6,
                                 mixed_rounding=True, qkv_dtype=torch.bfloat16, out_dtype=torch.bfloat16,
                                 q_norm_weight=c["qn_d"], k_norm_weight=c["kn_d"], qk_norm_eps=1e-6,
                                 qk_norm_out_dtype=torch.bfloat16, **kw)
    return fused_rmsnorm_qkv(c["x_d"], c["ln_d"], c["w_d"], c["hq"], c["hkv"], 1e-5,
                             mixed_rounding=False, qkv_dtype=torch.float32, out_dtype=torch.bfloat16, **kw)


def to_dev(c):
    for k in ("x", "ln", "w", "qn", "kn", "pos", "table"):
        if k in c:
            c[k + "_d"] = c[k].to(DEV)


def run_case(c, write_kv_out=True):
    """Returns (fused output, plain output, fused cache, oracle cache, skipped)."""
    to_dev(c)
    braidinfer_amd.check_device_status()
    plain = call(c)
    cache_d = c["cache"].to(DEV)
    pkv = PagedKVAppend(cache_d, c["kv_indices"].to(DEV), c["cache_pos"].to(DEV), c["ps"], c["layout"],
                        write_kv_out=write_kv_out)
    out = torch.full_like(plain, 7.0)
    fused = call(c, pkv, out=out)
    torch.cuda.synchronize()
    t, hq, hkv, d = plain.shape[0], c["hq"], c["hkv"], c["d"]
    p = plain.cpu()
    k = p[:, hq * d:(hq + hkv) * d].reshape(t, hkv, d)
    v = p[:, (hq + hkv) * d:].reshape(t, hkv, d)
    exp, skipped = R.append_to_paged_kv_cache(k.to(c["cache"].dtype), v.to(c["cache"].dtype), c["cache"],
                                              c["kv_indices"], c["cache_pos"], c["ps"], c["layout"])
    return fused.cpu(), p, cache_d.cpu(), exp, skipped


def check(c, what, write_kv_out=True):
    fused, plain, got, exp, skipped = run_case(c, write_kv_out)
    hq, d = c["hq"], c["d"]
    if write_kv_out:
        assert torch.equal(bits(fused), bits(plain)), f"{what}: output differs from the plain fused call"
    else:
        assert torch.equal(bits(fused[:, :hq * d]), bits(plain[:, :hq * d])), f"{what}: q columns differ"
        assert bool((fused[:, hq * d:] == 7.0).all()), f"{what}: k/v columns were written"
    assert torch.equal(bits(got), bits(exp)), f"{what}: cache differs from the oracle's append"
    return skipped


LLAMA = dict(hidden=1024, hq=8, hkv=2, d=128, qwen=False)
QWEN = dict(hidden=1024, hq=8, hkv=4, d=128, qwen=True)


@pytest.mark.parametrize("tokens", [1, 5, 16, 17, 40, 64, 100, 700])
@pytest.mark.parametrize("model", ["llama", "qwen3"])
def test_fused_append_every_epilogue(model, tokens):
    cfg = LLAMA if model == "llama" else QWEN
    c = make_case(tokens * 7 + (model == "qwen3"), tokens, **cfg)
    assert check(c, f"{model} T={tokens}") == []
    braidinfer_amd.check_device_status()


@pytest.mark.parametrize("tile", ["2", "3", "1", "128"])
def test_fused_append_tile_forms(tuning, tile):
    tuning("QKV_TILE", int(tile))
    c = make_case(50 + int(tile), 300, **LLAMA)
    check(c, f"tile {tile}")
    c = make_case(60 + int(tile), 300, **QWEN)
    check(c, f"qwen3 tile {tile}")


@pytest.mark.parametrize("tokens", [3, 33, 257])
def test_fused_append_nhd_fp32_cache_head_dim_64(tokens):
    c = make_case(90 + tokens, tokens, hidden=512, hq=8, hkv=2, d=64, qwen=False, ps=8, layout="NHD",
                  cache_dtype=torch.float32)
    check(c, f"NHD fp32 D=64 T={tokens}")


@pytest.mark.parametrize("tokens", [9, 130])
def test_fused_append_head_dim_80(tokens):
    # head_dim 80: raw projection (or decode partials) + the row epilogue
    c = make_case(110 + tokens, tokens, hidden=256, hq=4, hkv=2, d=80, qwen=False)
    check(c, f"D=80 T={tokens}")


@pytest.mark.parametrize("tokens", [12, 48, 400])
def test_fused_append_q_only_output(tokens):
    c = make_case(130 + tokens, tokens, **LLAMA)
    check(c, f"write_kv_out=False T={tokens}", write_kv_out=False)


def test_fused_append_skips_tokens_past_the_table():
    c = make_case(150, 80, **LLAMA, start=0)
    c["kv_indices"] = c["kv_indices"][:3]  # 48 slots for 80 tokens
    skipped = check(c, "skips")
    assert skipped == list(range(48, 80))
    with pytest.warns(RuntimeWarning, match="skipped"):
        braidinfer_amd.check_device_status()


def test_fused_append_batched_sequences():
    """Three sequences in one call (CSR page table, a sequence id per token)."""
    g = gen(170)
    c = make_case(171, 90, **LLAMA)
    lens, starts = [30, 20, 40], [5, 0, 17]
    tables = [torch.randperm(64, generator=g)[:(s + n + 15) // 16].to(torch.int32) for s, n in zip(starts, lens)]
    indices = torch.cat(tables)
    indptr = torch.tensor([0] + list(torch.cumsum(torch.tensor([len(t) for t in tables]), 0)), dtype=torch.int32)
    batch = torch.cat([torch.full((n,), i, dtype=torch.int32) for i, n in enumerate(lens)])
    cpos = torch.cat([torch.arange(s, s + n) for s, n in zip(starts, lens)])
    cache = randn(g, 64, 2, 2, 16, 128)
    to_dev(c)
    plain = call(c)
    cache_d = cache.to(DEV)
    pkv = PagedKVAppend(cache_d, indices.to(DEV), cpos.to(DEV), 16, kv_indptr=indptr.to(DEV),
                        batch_indices=batch.to(DEV))
    fused = call(c, pkv)
    torch.cuda.synchronize()
    assert torch.equal(bits(fused.cpu()), bits(plain.cpu()))
    p = plain.cpu()
    k = p[:, 8 * 128:10 * 128].reshape(90, 2, 128)
    v = p[:, 10 * 128:].reshape(90, 2, 128)
    exp = R.append_paged_kv_batch(k, v, cache, indices, indptr, batch, cpos, 16)
    exp = exp[0] if isinstance(exp, tuple) else exp
    assert torch.equal(bits(cache_d.cpu()), bits(exp))
    braidinfer_amd.check_device_status()
