"""GPU parity of the paged cascade attention (CascadeAttention.forward,
layers/cascade_attention.py:50-231) and of online_softmax_update
(kernels/online_softmax.py:214-297) against the oracle's page-by-page restatement.

online_softmax_update: fp32 state within 1e-5, the reference test's bound
(tests/test_online_softmax_kernel.py:95-103).  Cascade attention: the output
within |d| <= 2e-2 + 1e-2 |r| (tests/helpers.py); the kernel computes scores in
fp32 from bf16 q and k like the reference, and rounds the softmax weights to
bf16 for the P.V matrix product (a relative error of at most 2^-9 per weight).
Three kernel forms serve a call: the decode form (up to 4 query rows per kv
head), the fused kernel, and from 97 rows the flat form (K rotated and
normalised once by a pre-pass, DMA'd tiles); the oracle cases run through the
fused kernel and, forced by the CASCADE_FLAT planner override, through the flat form."""
from __future__ import annotations

import math
import zlib
from types import SimpleNamespace

import pytest
import torch

import braidinfer_amd
from braidinfer_amd.kernels import online_softmax_update
from braidinfer_amd.layers import CascadeAttention, RMSNorm, RotaryEmbedding
from oracle import torch_ref as R
from tests.helpers import assert_close, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype,d,causal", [(torch.float32, 64, False), (torch.float32, 64, True),
                                            (torch.bfloat16, 128, True), (torch.float16, 96, False)])
def test_online_softmax_update(dtype, d, causal):
    g = gen(60)
    h, b, n = 8, 4, 16
    q = randn(g, h, b, d, dtype=dtype)
    k, v = randn(g, h, n, d, dtype=dtype), randn(g, h, n, d, dtype=dtype)
    m0 = torch.full((h, b), float("-inf"))
    l0, a0 = torch.zeros(h, b), torch.zeros(h, b, d)
    qpos, kpos = torch.tensor([0, 5, 8, 30]), torch.arange(n)
    em, el, ea = R.online_softmax_update(q, k, v, m0, l0, a0, qpos, kpos, d ** -0.5, causal)
    m, l, acc = m0.to(DEV), l0.to(DEV), a0.to(DEV)
    online_softmax_update(q.to(DEV), k.to(DEV), v.to(DEV), m, l, acc, qpos.to(DEV), kpos.to(DEV),
                          d ** -0.5, causal)
    # a second block continues from the state (the per-page use in cascade attention)
    k2, v2 = randn(g, h, 5, d, dtype=dtype), randn(g, h, 5, d, dtype=dtype)
    kpos2 = torch.arange(n, n + 5)
    em, el, ea = R.online_softmax_update(q, k2, v2, em, el, ea, qpos, kpos2, d ** -0.5, causal)
    online_softmax_update(q.to(DEV), k2.to(DEV), v2.to(DEV), m, l, acc, qpos.to(DEV), kpos2.to(DEV),
                          d ** -0.5, causal)
    torch.cuda.synchronize()
    for got, exp, name in ((m, em, "m"), (l, el, "l"), (acc, ea, "acc")):
        fin = torch.isfinite(exp)
        assert torch.equal(torch.isfinite(got.cpu()), fin), name
        assert (got.cpu()[fin] - exp[fin]).abs().max().item() < 1e-5 * max(1.0, exp[fin].abs().max().item()), name


def make_levels(att, chunks_per_level, dev):
    return [att._create_level(chunks, position_offset=0) for chunks in chunks_per_level]


def cpu_levels(levels):
    return [SimpleNamespace(chunks=lv.chunks, kv_page_indices=lv.kv_page_indices.cpu(),
                            kv_page_indptr=lv.kv_page_indptr.cpu(), kv_last_page_len=lv.kv_last_page_len.cpu())
            for lv in levels]


def chunk(page_table, kv_length, cached=0, glob=0, kind="context"):
    return SimpleNamespace(page_table=page_table, kv_length=kv_length, cached_position_start=cached,
                           global_position_start=glob, chunk_type=SimpleNamespace(value=kind))


def build_case(seed, hq, hkv, lengths, deltas, pages, ps=16, dtype=torch.bfloat16, d=128):
    """A system chunk and context chunks of the given token counts in shuffled pages,
    each moved by its delta; plus an empty chunk and one with pages but no tokens."""
    g = gen(seed)
    perm = torch.randperm(pages, generator=g).tolist()
    chunks, used, pos = [], 0, 0
    for i, (n, dl) in enumerate(zip(lengths, deltas)):
        npg = max(1, (n + ps - 1) // ps)
        chunks.append(chunk(perm[used:used + npg], n, 1000 + pos, 1000 + pos + dl,
                            "system_prompt" if i == 0 else "context"))
        used += npg
        pos += n
    chunks.insert(2, chunk([], 0))
    chunks.insert(3, chunk(perm[used:used + 1], 0))
    kv = randn(g, pages, 2, hkv, ps, d, dtype=dtype)
    return chunks, kv, sum(lengths)


CASES = [
    ("llama decode", 1, 32, 8, [100, 37, 516], [0, 4000, -77], True, False),
    ("llama decode batch", 4, 32, 8, [64, 300, 5], [0, 0, 12], True, False),
    ("qwen3 decode k-norm", 1, 16, 8, [200, 17, 1000], [0, -4096, 3000], True, True),
    ("qwen3 prefill chunk", 37, 16, 8, [48, 130, 64], [0, 77, -5], True, True),
    ("llama prefill", 300, 32, 8, [128, 700, 300], [0, 2048, 0], True, False),
    ("non-causal", 9, 16, 8, [33, 16, 1], [0, 5, 0], False, True),
]


# head_dim 64 (TinyLlama-1.1B: 32 query / 4 kv heads, theta 1e4), through the
# decode form (up to 4 query rows per kv head: GQA 4 at one token, GQA 2 at
# two), the fused kernel and the flat form (natural from 97 rows, forced below)
CASES_D64 = [
    ("tinyllama decode", 1, 32, 4, [100, 37, 516], [0, 4000, -77], True, False),
    ("d64 decode form gqa4 k-norm", 1, 8, 2, [200, 17, 1000], [0, -4096, 3000], True, True),
    ("d64 decode form gqa2 two tokens", 2, 16, 8, [64, 300, 5], [0, 0, 12], True, False),
    ("tinyllama prefill chunk k-norm", 37, 32, 4, [48, 130, 64], [0, 77, -5], True, True),
    ("tinyllama prefill", 300, 32, 4, [128, 700, 300], [0, 2048, 0], True, False),
    ("d64 non-causal", 9, 16, 8, [33, 16, 1], [0, 5, 0], False, True),
]


@pytest.mark.parametrize("name,tokens,hq,hkv,lengths,deltas,causal,knorm", CASES)
def test_cascade_attention(name, tokens, hq, hkv, lengths, deltas, causal, knorm):
    _check_case(name, tokens, hq, hkv, lengths, deltas, causal, knorm)


@pytest.mark.parametrize("name,tokens,hq,hkv,lengths,deltas,causal,knorm",
                         [c for c in CASES if c[1] * c[2] // c[3] > 4])
def test_cascade_attention_flat_form(tuning, name, tokens, hq, hkv, lengths, deltas, causal, knorm):
    """The same oracle cases through the flat form (K rotated / normalised once
    by a pre-pass, DMA'd tiles), which runs by itself only from 97 rows per kv
    head: forced here for every case above 4 rows."""
    tuning("CASCADE_FLAT", 1)
    _check_case(name, tokens, hq, hkv, lengths, deltas, causal, knorm)


@pytest.mark.parametrize("name,tokens,hq,hkv,lengths,deltas,causal,knorm", CASES_D64)
def test_cascade_attention_head_dim_64(tuning, name, tokens, hq, hkv, lengths, deltas, causal, knorm):
    tuning("CASCADE_FLAT", 0)  # the fused kernel (or the decode form) for every case
    _check_case(name, tokens, hq, hkv, lengths, deltas, causal, knorm, d=64, base=1e4)


@pytest.mark.parametrize("name,tokens,hq,hkv,lengths,deltas,causal,knorm",
                         [c for c in CASES_D64 if c[1] * c[2] // c[3] > 4])
def test_cascade_attention_head_dim_64_flat_form(tuning, name, tokens, hq, hkv, lengths, deltas, causal,
                                                 knorm):
    tuning("CASCADE_FLAT", 1)
    _check_case(name, tokens, hq, hkv, lengths, deltas, causal, knorm, d=64, base=1e4)


# head dims other than 64 and 128 (a wave per query row walks the pages: the
# same rounding points, scores on the VALU): decode, a prefill chunk and a
# non-causal case, with k_norm, GQA 2 and 4, moved chunks
CASES_OTHER_D = [
    ("d32 decode k-norm", 32, 1, 8, 2, [200, 17, 1000], [0, -4096, 3000], True, True),
    ("d96 decode", 96, 1, 16, 8, [100, 37, 516], [0, 4000, -77], True, False),
    ("d96 prefill chunk k-norm", 96, 37, 16, 8, [48, 130, 64], [0, 77, -5], True, True),
    ("d80 non-causal k-norm", 80, 9, 16, 4, [33, 16, 1], [0, 5, 0], False, True),
    ("d256 decode batch", 256, 4, 8, 4, [64, 300, 5], [0, 0, 12], True, False),
    ("d256 prefill k-norm", 256, 20, 8, 2, [128, 70, 30], [0, 2048, 0], True, True),
]


@pytest.mark.parametrize("name,d,tokens,hq,hkv,lengths,deltas,causal,knorm", CASES_OTHER_D)
def test_cascade_attention_other_head_dims(name, d, tokens, hq, hkv, lengths, deltas, causal, knorm):
    _check_case(name, tokens, hq, hkv, lengths, deltas, causal, knorm, d=d, base=1e4)


def _check_case(name, tokens, hq, hkv, lengths, deltas, causal, knorm, d=128, base=1e6):
    seed = zlib.crc32(name.encode()) % 1000
    g = gen(seed)
    ps, max_pos = 16, 40960
    chunks, kv, total = build_case(seed + 1, hq, hkv, lengths, deltas, pages=300, d=d)
    rope = RotaryEmbedding(d, d, max_pos, base).to(DEV)
    att = CascadeAttention(hq, d, d ** -0.5, hkv, ps, rotary_emb=rope)
    levels = att.create_cascade_levels(chunks)
    q = randn(g, tokens, hq, d)
    qpos = torch.arange(total - tokens + 1, total + 1) if causal else torch.full((tokens,), 5)
    k_norm, kn_w = None, None
    if knorm:
        k_norm = RMSNorm(d, eps=1e-6).to(DEV)
        kn_w = torch.exp(torch.empty(d).uniform_(math.log(0.05), math.log(100.0), generator=g)).to(torch.bfloat16)
        with torch.no_grad():
            k_norm.weight.data = kn_w.to(DEV)
    braidinfer_amd.check_device_status()
    out = att.forward(q.to(DEV), qpos.to(DEV), kv.to(DEV), levels, 0, causal_mask=causal, k_norm=k_norm)
    torch.cuda.synchronize()
    braidinfer_amd.check_device_status()
    exp = R.cascade_attention(q, qpos, kv, cpu_levels(levels), hq, hkv, d ** -0.5, ps,
                              rope.cos_sin_cache.cpu(), kn_w, 1e-6, causal)
    assert out.shape == (tokens, hq * d) and out.dtype == q.dtype
    assert_close(out, exp, what=name)


@pytest.mark.parametrize("ps,tokens,dtype,d", [(8, 1, torch.bfloat16, 128), (32, 2, torch.bfloat16, 128),
                                               (16, 2, torch.float16, 128), (32, 1, torch.float16, 128),
                                               (8, 2, torch.bfloat16, 64), (32, 1, torch.float16, 64)])
def test_cascade_decode_form_page_sizes(ps, tokens, dtype, d):
    """Up to 4 query rows per kv head run in the decode kernel, which walks
    (entry, 16-slot block) items: page size 8 leaves half the lane groups idle,
    32 takes two blocks per page.  Qwen3 geometry (16 / 8 heads), k_norm, moved
    chunks, a partial last page; head_dim 128 and 64."""
    g = gen(90 + ps + tokens + d)
    hq, hkv, max_pos = 16, 8, 40960
    chunks, kv, total = build_case(91 + ps, hq, hkv, [45, 130, 77], [0, 300, -41], pages=64, ps=ps, dtype=dtype,
                                   d=d)
    rope = RotaryEmbedding(d, d, max_pos, 1e6).to(DEV)
    att = CascadeAttention(hq, d, d ** -0.5, hkv, ps, rotary_emb=rope)
    levels = att.create_cascade_levels(chunks)
    q = randn(g, tokens, hq, d, dtype=dtype)
    qpos = torch.arange(total - tokens + 1, total + 1)
    kn_w = torch.exp(torch.empty(d).uniform_(math.log(0.05), math.log(100.0), generator=g)).to(dtype)
    k_norm = RMSNorm(d, eps=1e-6).to(DEV)
    with torch.no_grad():
        k_norm.weight.data = kn_w.to(DEV)
    out = att.forward(q.to(DEV), qpos.to(DEV), kv.to(DEV), levels, 0, k_norm=k_norm)
    torch.cuda.synchronize()
    braidinfer_amd.check_device_status()
    exp = R.cascade_attention(q, qpos, kv, cpu_levels(levels), hq, hkv, d ** -0.5, ps,
                              rope.cos_sin_cache.cpu(), kn_w, 1e-6, True)
    assert_close(out, exp, what=f"decode form ps={ps} t={tokens} {dtype} d={d}")


@pytest.mark.parametrize("target", [8, 32, 64, 96, 256, 1024, 8192])
def test_cascade_decode_split_merges(tuning, target):
    """The decode kernel's split count follows the workgroup target; every
    combination form is taken over about 3000 keys (about 190 pages) at 8 kv
    heads: one split (no merge), 4, 8 and 12 (a wave per row, sized for 4, 8
    and 16 splits), 32 (one round trip, 16 splits per wave), about 95 and
    about 190 (the looped merge)."""
    tuning("CASCADE_DECODE_WG", target)
    g = gen(120 + target)
    hq, hkv, d, ps, max_pos = 32, 8, 128, 16, 40960
    chunks, kv, total = build_case(121, hq, hkv, [1500, 900, 601], [0, 2000, -700], pages=200, ps=ps, d=d)
    rope = RotaryEmbedding(d, d, max_pos, 1e6).to(DEV)
    att = CascadeAttention(hq, d, d ** -0.5, hkv, ps, rotary_emb=rope)
    levels = att.create_cascade_levels(chunks)
    q = randn(g, 1, hq, d)
    qpos = torch.tensor([total])
    out = att.forward(q.to(DEV), qpos.to(DEV), kv.to(DEV), levels, 0)
    torch.cuda.synchronize()
    braidinfer_amd.check_device_status()
    exp = R.cascade_attention(q, qpos, kv, cpu_levels(levels), hq, hkv, d ** -0.5, ps,
                              rope.cos_sin_cache.cpu(), None, 1e-6, True)
    assert_close(out, exp, what=f"decode splits, target {target}")


@pytest.mark.parametrize("ps,dtype,d", [(8, torch.bfloat16, 128), (32, torch.float16, 128), (8, torch.float16, 64)])
def test_cascade_flat_form_page_sizes(tuning, ps, dtype, d):
    """Flat form with pages of 8 (8 pages per 64-key tile) and 32 slots, a
    partial last page and moved chunks, Qwen3 geometry with k_norm."""
    tuning("CASCADE_FLAT", 1)
    g = gen(95 + ps + d)
    hq, hkv, max_pos, tokens = 16, 8, 40960, 8
    chunks, kv, total = build_case(96 + ps, hq, hkv, [45, 130, 77], [0, 300, -41], pages=64, ps=ps, dtype=dtype,
                                   d=d)
    rope = RotaryEmbedding(d, d, max_pos, 1e6).to(DEV)
    att = CascadeAttention(hq, d, d ** -0.5, hkv, ps, rotary_emb=rope)
    levels = att.create_cascade_levels(chunks)
    q = randn(g, tokens, hq, d, dtype=dtype)
    qpos = torch.arange(total - tokens + 1, total + 1)
    kn_w = torch.exp(torch.empty(d).uniform_(math.log(0.05), math.log(100.0), generator=g)).to(dtype)
    k_norm = RMSNorm(d, eps=1e-6).to(DEV)
    with torch.no_grad():
        k_norm.weight.data = kn_w.to(DEV)
    out = att.forward(q.to(DEV), qpos.to(DEV), kv.to(DEV), levels, 0, k_norm=k_norm)
    torch.cuda.synchronize()
    braidinfer_amd.check_device_status()
    exp = R.cascade_attention(q, qpos, kv, cpu_levels(levels), hq, hkv, d ** -0.5, ps,
                              rope.cos_sin_cache.cpu(), kn_w, 1e-6, True)
    assert_close(out, exp, what=f"flat form ps={ps} {dtype} d={d}")


@pytest.mark.parametrize("flat", ["0", "1"])
def test_cascade_attention_fp16_query_before_keys_and_empty(tuning, flat):
    tuning("CASCADE_FLAT", int(flat))
    g = gen(70)
    hq, hkv, d, ps = 16, 8, 128, 16
    chunks, kv, total = build_case(71, hq, hkv, [20, 40], [0, 3], pages=20, dtype=torch.float16)
    att = CascadeAttention(hq, d, d ** -0.5, hkv, ps)
    levels = att.create_cascade_levels(chunks)
    q = randn(g, 3, hq, d, dtype=torch.float16)
    qpos = torch.tensor([-1, 10, 70])  # the first query precedes every key: zeros
    out = att.forward(q.to(DEV), qpos.to(DEV), kv.to(DEV), levels, 0)
    exp = R.cascade_attention(q, qpos, kv, cpu_levels(levels), hq, hkv, d ** -0.5, ps, None, None, 1e-6, True)
    assert torch.count_nonzero(out[0]) == 0
    assert_close(out, exp, what="fp16")
    # no levels at all: every query attends nothing
    out = att.forward(q.to(DEV), qpos.to(DEV), kv.to(DEV), [], 0)
    assert torch.count_nonzero(out) == 0
    # flat and 2-D query shapes are accepted as in the reference
    out2 = att.forward(q.reshape(-1).to(DEV), qpos.to(DEV), kv.to(DEV), levels, 0)
    out3 = att.forward(q.reshape(3, -1).to(DEV), qpos.to(DEV), kv.to(DEV), levels, 0)
    assert torch.equal(out2, out3)


def test_cascade_attention_delta_out_of_table_raises():
    hq, hkv, d, ps = 16, 8, 128, 16
    chunks, kv, total = build_case(72, hq, hkv, [20, 40], [0, -5000], pages=20)
    rope = RotaryEmbedding(d, d, 4096, 1e6).to(DEV)
    att = CascadeAttention(hq, d, d ** -0.5, hkv, ps, rotary_emb=rope)
    levels = att.create_cascade_levels(chunks)
    q = randn(gen(73), 2, hq, d)
    braidinfer_amd.check_device_status()
    att.forward(q.to(DEV), torch.tensor([60, 61], device=DEV), kv.to(DEV), levels, 0)
    with pytest.raises(IndexError):
        braidinfer_amd.check_device_status()


def test_cascade_flat_form_delta_out_of_table_raises(tuning):
    """The flat form's pre-pass reports a delta outside the rotary table the
    same way."""
    tuning("CASCADE_FLAT", 1)
    hq, hkv, d, ps = 16, 8, 128, 16
    chunks, kv, total = build_case(76, hq, hkv, [20, 40], [0, -5000], pages=20)
    rope = RotaryEmbedding(d, d, 4096, 1e6).to(DEV)
    att = CascadeAttention(hq, d, d ** -0.5, hkv, ps, rotary_emb=rope)
    levels = att.create_cascade_levels(chunks)
    q = randn(gen(77), 8, hq, d)
    braidinfer_amd.check_device_status()
    att.forward(q.to(DEV), torch.arange(60, 68, device=DEV), kv.to(DEV), levels, 0)
    with pytest.raises(IndexError):
        braidinfer_amd.check_device_status()


def test_cascade_flat_form_matches_fused_kernel(tuning):
    """The flat form (pre-pass + DMA'd tiles) and the fused kernel agree on a
    256-query Qwen3 call with k_norm and moved chunks (the oracle check of both
    is in test_cascade_attention)."""
    g = gen(78)
    hq, hkv, d, ps, max_pos = 16, 8, 128, 16, 40960
    chunks, kv, total = build_case(79, hq, hkv, [300, 1000, 700], [0, 513, -2000], pages=200)
    rope = RotaryEmbedding(d, d, max_pos, 1e6).to(DEV)
    att = CascadeAttention(hq, d, d ** -0.5, hkv, ps, rotary_emb=rope)
    levels = att.create_cascade_levels(chunks)
    q = randn(g, 256, hq, d).to(DEV)
    qpos = torch.arange(total - 255, total + 1, device=DEV)
    k_norm = RMSNorm(d, eps=1e-6).to(DEV)
    kv = kv.to(DEV)
    tuning("CASCADE_FLAT", 1)
    flat = att.forward(q, qpos, kv, levels, 0, k_norm=k_norm).clone()
    tuning("CASCADE_FLAT", 0)
    fused = att.forward(q, qpos, kv, levels, 0, k_norm=k_norm)
    torch.cuda.synchronize()
    braidinfer_amd.check_device_status()
    assert_close(flat, fused, what="flat form vs fused kernel")


def test_cascade_attention_graph_replays_match_eager():
    """After one eager call the forward makes no host-to-device copy, so it can be
    captured; every replay (with eager work in between) equals the eager result."""
    hq, hkv, d, ps = 16, 8, 128, 16
    chunks, kv, total = build_case(74, hq, hkv, [64, 300, 40], [0, 9, -3], pages=40)
    rope = RotaryEmbedding(d, d, 4096, 1e6).to(DEV)
    att = CascadeAttention(hq, d, d ** -0.5, hkv, ps, rotary_emb=rope)
    levels = att.create_cascade_levels(chunks)
    q = randn(gen(75), 1, hq, d).to(DEV)
    qpos = torch.tensor([total], device=DEV)
    kvd = kv.to(DEV)
    eager = att.forward(q, qpos, kvd, levels, 0).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        att.forward(q, qpos, kvd, levels, 0)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = att.forward(q, qpos, kvd, levels, 0)
    for i in range(4):
        torch.randn(1000, device=DEV).sum()  # unrelated eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
