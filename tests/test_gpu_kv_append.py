"""GPU parity of the paged KV append (append_to_paged_kv_cache_custom,
kernels/kv_cache_utils.py:9-78) against the oracle: the whole cache must match
oracle/torch_ref.py's restatement bit for bit (the kernel moves values; a dtype
change rounds to nearest even, as the tensor assignment does)."""
from __future__ import annotations

import warnings

import pytest
import torch

import braidinfer_amd
from braidinfer_amd.kernels import (append_paged_kv_batch, append_to_paged_kv_cache_custom,
                                    build_paged_kv_indices)
from oracle import torch_ref as R
from tests.helpers import bits, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def run_both(k, v, cache, table, pos, ps, layout="HND"):
    """Device append on copies of the inputs, then the oracle; returns (device cache on CPU,
    oracle cache, oracle skipped list)."""
    braidinfer_amd.check_device_status()
    dc = cache.to(DEV)
    append_to_paged_kv_cache_custom(k.to(DEV), v.to(DEV), dc, table.to(DEV), pos.to(DEV), ps, layout)
    torch.cuda.synchronize()
    exp, skipped = R.append_to_paged_kv_cache(k, v, cache, table, pos, ps, layout)
    return dc.cpu(), exp, skipped


def assert_bits(got, exp, what):
    assert got.dtype == exp.dtype and got.shape == exp.shape, what
    assert torch.equal(bits(got), bits(exp)), f"{what}: caches differ"


def sequence_case(seed, tokens, pages, hkv, ps, d, start=0, dtype=torch.bfloat16):
    g = gen(seed)
    need = (start + tokens + ps - 1) // ps
    table = torch.randperm(pages, generator=g)[:need].to(torch.int32)
    k, v = randn(g, tokens, hkv, d, dtype=dtype), randn(g, tokens, hkv, d, dtype=dtype)
    cache = randn(g, pages, 2, hkv, ps, d, dtype=dtype)
    pos = torch.arange(start, start + tokens, dtype=torch.int32)
    return k, v, cache, table, pos


@pytest.mark.parametrize("tokens,pages,hkv,ps,d,start", [
    (64, 80, 8, 16, 128, 1000),     # Llama-3-8B decode-sized batch of one sequence, mid-page start
    (8192, 600, 8, 16, 128, 0),     # Llama-3-8B 8192-token prefill into 512 shuffled pages
    (4096, 300, 8, 16, 128, 5),     # Qwen3-0.6B chunk, unaligned start
    (1, 4, 4, 16, 64, 17),          # TinyLlama single decode token
    (37, 20, 2, 8, 80, 3),          # head_dim 80
])
def test_append_hnd_bit_exact(tokens, pages, hkv, ps, d, start):
    k, v, cache, table, pos = sequence_case(tokens + d, tokens, pages, hkv, ps, d, start)
    got, exp, skipped = run_both(k, v, cache, table, pos, ps)
    assert skipped == []
    assert_bits(got, exp, f"HND T={tokens}")
    braidinfer_amd.check_device_status()


def test_append_nhd_int64_indices():
    k, v, cache, table, pos = sequence_case(7, 300, 64, 4, 16, 64, start=9)
    cache = cache.transpose(2, 3).contiguous()
    got, exp, _ = run_both(k, v, cache, table.long(), pos.long(), 16, "NHD")
    assert_bits(got, exp, "NHD")


def test_append_strided_views_of_qkv_output():
    """k and v as the views the QKV split hands out: rows of a [T, (Hq+2Hkv)D] buffer."""
    g = gen(8)
    t, hq, hkv, d, ps, pages = 200, 32, 8, 128, 16, 40
    out = randn(g, t, (hq + 2 * hkv) * d)
    k = out[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    v = out[:, (hq + hkv) * d:].view(t, hkv, d)
    table = torch.randperm(pages, generator=g)[:13].to(torch.int32)
    cache = torch.zeros(pages, 2, hkv, ps, d, dtype=torch.bfloat16)
    dout = out.to(DEV)
    dk = dout[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    dv = dout[:, (hq + hkv) * d:].view(t, hkv, d)
    assert dk.stride() == (dout.shape[1], d, 1)
    dc = cache.to(DEV)
    pos = torch.arange(t)
    append_to_paged_kv_cache_custom(dk, dv, dc, table.to(DEV), pos.to(DEV), ps)
    exp, _ = R.append_to_paged_kv_cache(k, v, cache, table, pos, ps)
    assert_bits(dc.cpu(), exp, "strided views")


@pytest.mark.parametrize("src,dst", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32),
                                     (torch.float16, torch.float16), (torch.float32, torch.float16)])
def test_append_dtype_conversion(src, dst):
    g = gen(9)
    k, v = randn(g, 50, 2, 32, dtype=src), randn(g, 50, 2, 32, dtype=src)
    cache = randn(g, 10, 2, 2, 8, 32, dtype=dst)
    table = torch.randperm(10, generator=g)[:7].to(torch.int32)
    got, exp, _ = run_both(k, v, cache, table, torch.arange(50), 8)
    assert_bits(got, exp, f"{src}->{dst}")


def test_append_scalar_path_odd_head_dim():
    g = gen(10)
    k, v = randn(g, 23, 3, 36), randn(g, 23, 3, 36)
    cache = randn(g, 9, 2, 3, 4, 36)
    table = torch.randperm(9, generator=g)[:6].to(torch.int32)
    got, exp, _ = run_both(k, v, cache, table, torch.arange(23), 4)
    assert_bits(got, exp, "head_dim 36")


def test_append_negative_positions_and_skipped_tokens():
    g = gen(11)
    ps = 4
    k, v = randn(g, 5, 2, 16), randn(g, 5, 2, 16)
    cache = randn(g, 8, 2, 2, ps, 16)
    table = torch.tensor([3, 7, 1], dtype=torch.int32)
    pos = torch.tensor([-1, -5, 2, 12, 40])  # last entry / slot 3, second-last, in range, two past
    braidinfer_amd.check_device_status()
    dc = cache.to(DEV)
    append_to_paged_kv_cache_custom(k.to(DEV), v.to(DEV), dc, table.to(DEV), pos.to(DEV), ps)
    with pytest.warns(RuntimeWarning, match="skipped"):
        braidinfer_amd.check_device_status()
    exp, skipped = R.append_to_paged_kv_cache(k, v, cache, table, pos, ps)
    assert skipped == [3, 4]
    assert_bits(dc.cpu(), exp, "negative / skipped")


def test_append_out_of_range_indices_raise():
    g = gen(12)
    k, v = randn(g, 2, 2, 16), randn(g, 2, 2, 16)
    cache = randn(g, 4, 2, 2, 4, 16).to(DEV)
    for table, pos in ((torch.tensor([9], dtype=torch.int32), torch.tensor([0, 1])),   # page id >= pages
                       (torch.tensor([1, 2], dtype=torch.int32), torch.tensor([-9, 0]))):  # offset < -len
        braidinfer_amd.check_device_status()
        with pytest.raises(IndexError):
            R.append_to_paged_kv_cache(k, v, cache.cpu(), table, pos, 4)
        append_to_paged_kv_cache_custom(k.to(DEV), v.to(DEV), cache, table.to(DEV), pos.to(DEV), 4)
        with pytest.raises(IndexError):
            braidinfer_amd.check_device_status()
    # negative page ids wrap like a torch index
    cache0 = cache.cpu()
    got, exp, _ = run_both(k, v, cache0, torch.tensor([-1], dtype=torch.int32), torch.tensor([0, 3]), 4)
    assert_bits(got, exp, "negative page id")


def test_append_host_checks_and_empty():
    cache = torch.zeros(2, 2, 2, 4, 8, dtype=torch.bfloat16, device=DEV)
    k = torch.zeros(0, 2, 8, dtype=torch.bfloat16, device=DEV)
    append_to_paged_kv_cache_custom(k, k, cache, torch.zeros(1, dtype=torch.int32, device=DEV),
                                    torch.zeros(0, dtype=torch.int32, device=DEV), 4)
    with pytest.raises(ValueError, match="Unknown kv_layout"):
        append_to_paged_kv_cache_custom(k, k, cache, torch.zeros(1, device=DEV), k, 4, "HDN")
    with pytest.raises(RuntimeError):
        bad = torch.zeros(3, 4, 8, dtype=torch.bfloat16, device=DEV)  # 4 heads for a 2-head cache
        append_to_paged_kv_cache_custom(bad, bad, cache, torch.zeros(1, device=DEV),
                                        torch.zeros(3, dtype=torch.int32, device=DEV), 4)


def test_build_paged_kv_indices_matches_reference_rule():
    idx, indptr, last = build_paged_kv_indices([[4, 1], [0], [], [2, 3, 5]], [20, 16, 0, 33], 16)
    assert idx.cpu().tolist() == [4, 1, 0, 2, 3, 5]
    assert indptr.cpu().tolist() == [0, 2, 3, 3, 6]
    assert last.cpu().tolist() == [4, 16, 0, 1]
    assert idx.dtype == indptr.dtype == last.dtype == torch.int32 and idx.is_cuda


def test_append_then_rerotate_round_trip():
    """The appended K, re-rotated by delta 0 through the cascade path, reads back unchanged."""
    from braidinfer_amd.layers import rerotate_paged_k
    k, v, cache, table, pos = sequence_case(13, 70, 16, 2, 16, 64)
    dc = cache.to(DEV)
    append_to_paged_kv_cache_custom(k.to(DEV), v.to(DEV), dc, table.to(DEV), pos.to(DEV), 16)
    indptr = torch.tensor([0, len(table)], dtype=torch.int32, device=DEV)
    last = torch.tensor([70 - 16 * (len(table) - 1)], dtype=torch.int32, device=DEV)
    cs = R.cos_sin_cache(64, 128, 1e4).to(DEV)
    out = rerotate_paged_k(dc, table.to(DEV), indptr, torch.zeros(1, dtype=torch.int64, device=DEV),
                           last, cs)
    flat = out.reshape(-1, 2, 64)[:70].cpu()
    assert torch.equal(bits(flat), bits(k))
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        braidinfer_amd.check_device_status()


@pytest.mark.parametrize("seqs,new_tokens", [(64, 1), (8, 300), (3, 1)])
def test_append_batch_bit_exact(seqs, new_tokens):
    """A decode batch (64 sequences, one new token each, Llama-3-8B kv heads) and a
    batched prefill, in one launch, against one reference call per sequence."""
    g = gen(20 + seqs)
    hkv, d, ps, pages = 8, 128, 16, 2048
    lens = torch.randint(0, 900, (seqs,), generator=g).tolist()
    perm = torch.randperm(pages, generator=g).tolist()
    tables, used = [], 0
    for n in lens:
        need = (n + new_tokens + ps - 1) // ps
        tables.append(perm[used:used + need])
        used += need
    kv_indices, kv_indptr, _ = build_paged_kv_indices(tables, [n + new_tokens for n in lens], ps)
    batch = torch.repeat_interleave(torch.arange(seqs), new_tokens)
    pos = torch.cat([torch.arange(n, n + new_tokens) for n in lens])
    tok = seqs * new_tokens
    k, v = randn(g, tok, hkv, d), randn(g, tok, hkv, d)
    cache = randn(g, pages, 2, hkv, ps, d)
    braidinfer_amd.check_device_status()
    dc = cache.to(DEV)
    append_paged_kv_batch(k.to(DEV), v.to(DEV), dc, kv_indices, kv_indptr, batch.to(DEV),
                          pos.to(DEV), ps)
    exp, skipped = R.append_paged_kv_batch(k, v, cache, kv_indices.cpu(), kv_indptr.cpu(), batch, pos, ps)
    assert skipped == []
    assert_bits(dc.cpu(), exp, f"batch {seqs}x{new_tokens}")
    braidinfer_amd.check_device_status()


def test_append_batch_bad_sequence_id_raises():
    g = gen(30)
    cache = randn(g, 6, 2, 2, 4, 16).to(DEV)
    k = randn(g, 2, 2, 16).to(DEV)
    idx = torch.tensor([1, 2, 3], dtype=torch.int32, device=DEV)
    indptr = torch.tensor([0, 2, 3], dtype=torch.int32, device=DEV)
    braidinfer_amd.check_device_status()
    append_paged_kv_batch(k, k, cache, idx, indptr, torch.tensor([0, 5], device=DEV),
                          torch.tensor([1, 1], device=DEV), 4)
    with pytest.raises(IndexError):
        braidinfer_amd.check_device_status()
