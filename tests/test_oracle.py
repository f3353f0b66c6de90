"""Pins the oracle (oracle/torch_ref.py) before it is trusted as the checker.

Each oracle function is checked against at least one of: a closed form or
special case, an invariant, the reference tests' own formulas and tolerances,
brute force on tiny inputs, and the independent numpy restatement
(oracle/numpy_ref.py).  The checks are chosen so that plausible mistakes (a
dropped eps, a wrong RoPE sign, a transposed weight, a missing gamma) fail;
test_planted_mistakes_are_caught demonstrates that on mutated copies.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import numpy_ref as N
from oracle import torch_ref as R
from tests.helpers import gen, randn

BF16_REL_ULP = 2.0 ** -7  # one bf16 ulp, relative


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().double().cpu().numpy()


def check_bf16_agreement(a: torch.Tensor, b: np.ndarray, max_frac=1e-2, what=""):
    """a (torch bf16 result) vs b (numpy float64 already rounded to bf16): all
    within one bf16 ulp and at most `max_frac` of elements differing at all
    (the only differences allowed are float32-vs-float64 intermediates landing
    on the other side of a rounding boundary)."""
    x = _np(a)
    diff = np.abs(x - b)
    tol = BF16_REL_ULP * np.maximum(np.abs(b), 1e-30) + 1e-30
    assert np.all(diff <= tol), f"{what}: max diff {diff.max():.3e} beyond 1 bf16 ulp"
    frac = float(np.mean(diff > 0))
    assert frac <= max_frac, f"{what}: {frac:.4f} of elements differ"


# ------------------------------------------------------------------- norms
def pin_rms_forward(fn):
    g = gen(11)
    # constant rows, gamma = 1 -> +-1 exactly (the eps term is far below bf16 resolution)
    x = torch.tensor([[2.0] * 64, [-0.5] * 64], dtype=torch.bfloat16)
    y = fn(x, torch.ones(64, dtype=torch.bfloat16), 1e-6)
    assert torch.equal(y.float(), torch.sign(x.float())), "constant rows must normalise to +-1"
    # eps matters for small rows: x = 1e-3 -> 1e-3/sqrt(1e-6 + 1e-6) = 1/sqrt(2)
    xs = torch.full((1, 64), 1e-3, dtype=torch.float32)
    ys = fn(xs, torch.ones(64), 1e-6)
    assert abs(ys[0, 0].item() - 1e-3 / math.sqrt(float(torch.tensor(1e-3, dtype=torch.float32)) ** 2 + 1e-6)) < 1e-5
    # scale invariance by a power of two is exact with eps = 0
    x = randn(g, 16, 256)
    w = randn(g, 256, mean=1.0, std=0.1)
    assert torch.equal(fn(x, w, 0.0), fn((x.float() * 4).to(torch.bfloat16), w, 0.0))
    # gamma is applied per column
    y1 = fn(x, torch.ones(256, dtype=torch.bfloat16), 1e-6)
    y2 = fn(x, torch.full((256,), 2.0, dtype=torch.bfloat16), 1e-6)
    assert torch.equal(y2.float(), y1.float() * 2)
    # independent numpy restatement
    check_bf16_agreement(fn(x, w, 1e-5), N.rms_forward(_np(x), _np(w), 1e-5), what="rms_forward")


def test_rms_forward_pinned():
    pin_rms_forward(R.rms_forward)


def test_rms_forward_fp32_is_plain_fp32():
    g = gen(12)
    x = randn(g, 8, 128, dtype=torch.float32)
    w = randn(g, 128, mean=1.0, std=0.1, dtype=torch.float32)
    y = R.rms_forward(x, w, 1e-6)
    ref = N.rmsnorm_f32(_np(x), _np(w), 1e-6)  # x*rsqrt(mean+eps) == x/sqrt(mean+eps)
    np.testing.assert_allclose(_np(y), ref, rtol=2e-6, atol=1e-7)


def test_add_rms_forward_pinned():
    g = gen(13)
    x, r = randn(g, 32, 512), randn(g, 32, 512)
    w = randn(g, 512, mean=1.0, std=0.1)
    y, res = R.add_rms_forward(x, r, w, 1e-5)
    # residual = 0 reduces to rms_forward exactly
    y0, res0 = R.add_rms_forward(x, torch.zeros_like(x), w, 1e-5)
    assert torch.equal(y0, R.rms_forward(x, w, 1e-5)) and torch.equal(res0, x)
    ny, nres = N.add_rms_forward(_np(x), _np(r), _np(w), 1e-5)
    assert np.array_equal(_np(res), nres), "residual_out must be bf16(x + r) exactly"
    check_bf16_agreement(y, ny, what="add_rms_forward")
    # the statistic comes from the fp32 sum, not from the rounded residual: the
    # normalisation of the rounded residual moves some outputs by an ulp
    assert not torch.equal(y, R.rms_forward(res, w, 1e-5))
    # fp32: one tensor returned twice
    xf, rf = x.float(), r.float()
    a, b = R.add_rms_forward(xf, rf, w.float(), 1e-5)
    assert a is b


def test_rmsnorm_f32_reference_test_formulas():
    """Tolerances of tests/test_rmsnorm_f32.py:29-157 against its pytorch_rmsnorm (:22-27)."""
    g = gen(14)

    def pytorch_rmsnorm(x, weight, eps=1e-6):
        x_f32 = x.float()
        var = x_f32.pow(2).mean(dim=-1, keepdim=True)
        return x_f32 / torch.sqrt(var + eps) * weight.float()

    x, w = randn(g, 4, 8), randn(g, 8)
    assert (R.rmsnorm_f32(x, w, 1e-6) - pytorch_rmsnorm(x, w)).abs().max() < 1e-5
    x, w = randn(g, 512, 1024), randn(g, 1024)
    ref = pytorch_rmsnorm(x, w)
    assert ((R.rmsnorm_f32(x, w, 1e-6) - ref) / (ref + 1e-8)).abs().max() < 1e-4
    w = randn(g, 1024)
    w[0] = 96.5
    w[100:110] = 50.0
    ref = pytorch_rmsnorm(x[:128], w)
    out = R.rmsnorm_f32(x[:128], w, 1e-6)
    assert torch.isfinite(out).all() and ((out - ref) / (ref + 1e-8)).abs().max() < 1e-3
    np.testing.assert_allclose(_np(R.rmsnorm_f32(x, w, 1e-6)), N.rmsnorm_f32(_np(x), _np(w), 1e-6),
                               rtol=1e-5, atol=1e-6)
    # small variance stays bounded (test_rmsnorm_f32.py:142-157)
    xs = (torch.ones(16, 64) + torch.randn(16, 64, generator=g) * 1e-4).to(torch.bfloat16)
    out = R.rmsnorm_f32(xs, torch.ones(64, dtype=torch.bfloat16), 1e-6)
    assert torch.isfinite(out).all() and out.abs().max() < 10


# ---------------------------------------------------------------- gather
def test_embedding_brute_force():
    g = gen(15)
    table = randn(g, 37, 24, std=0.02)
    ids = torch.randint(0, 37, (3, 5), generator=g)
    out = R.embedding(ids, table)
    ref = N.embedding(ids.numpy(), table.view(torch.int16).numpy())
    assert np.array_equal(out.view(torch.int16).numpy(), ref), "gather must be a bit-exact copy"
    with pytest.raises(IndexError):
        R.embedding(torch.tensor([37]), table)


def test_embedding_scaled_closed_form():
    g = gen(16)
    table = randn(g, 50, 1024, std=0.02)
    ids = torch.randint(0, 50, (9,), generator=g)
    out = R.embedding_scaled(ids, table, 1024)
    # 1/sqrt(1024) = 2^-5: the scaling is exact in bf16
    assert torch.equal(out.float(), table[ids].float() / 32)
    out = R.embedding_scaled(ids, table, 2048)
    ref = N.round_bf16(_np(table[ids]) * float(np.float32(1.0 / 2048 ** 0.5)))
    assert np.array_equal(_np(out), ref)


# ---------------------------------------------------------------- SwiGLU
def test_silu_and_mul_pinned():
    g = gen(17)
    u = randn(g, 4, 64)
    for gate, expect in ((0.0, lambda u: torch.zeros_like(u.float())),
                         (-100.0, lambda u: torch.zeros_like(u.float()))):
        x = torch.cat([torch.full_like(u, gate), u], dim=-1)
        assert torch.equal(R.silu_and_mul(x).float().abs(), expect(u).abs())
    # large positive gate: silu(20) = 20 to within 5e-8, bf16(20) = 20
    x = torch.cat([torch.full_like(u, 20.0), u], dim=-1)
    assert torch.equal(R.silu_and_mul(x).float(), (u.float() * 20).to(torch.bfloat16).float())
    x = randn(g, 64, 2 * 384)
    check_bf16_agreement(R.silu_and_mul(x), N.silu_and_mul(_np(x)), what="silu_and_mul")


# ------------------------------------------------------------------ RoPE
def pin_rotary(rot_fn):
    """rot_fn(cache, head_size, positions, q, k) -> (q', k') like RotaryEmbedding.forward."""
    g = gen(18)
    d, maxp, base = 64, 2048, 10000.0
    cache = R.cos_sin_cache(d, maxp, base)
    q = randn(g, 8, 4 * d, dtype=torch.float32)
    k = randn(g, 8, 2 * d, dtype=torch.float32)
    # position 0 is the identity
    zq, zk = rot_fn(cache, d, torch.zeros(8, dtype=torch.int64), q, k)
    assert torch.equal(zq, q) and torch.equal(zk, k)
    # composition R(a) R(b) = R(a+b), and rotation preserves pair norms
    a, b = torch.randint(0, 900, (8,), generator=g), torch.randint(0, 900, (8,), generator=g)
    q1, _ = rot_fn(cache, d, b, q, k)
    q2, _ = rot_fn(cache, d, a, q1, k)
    q3, _ = rot_fn(cache, d, a + b, q, k)
    assert (q2 - q3).abs().max() < 2e-4
    h = d // 2
    qa, qb = q.view(8, 4, d), q1.view(8, 4, d)
    np.testing.assert_allclose(_np(qa[..., :h] ** 2 + qa[..., h:] ** 2),
                               _np(qb[..., :h] ** 2 + qb[..., h:] ** 2), rtol=1e-5, atol=1e-6)
    # negative positions index from the end of the table (torch semantics)
    n1, _ = rot_fn(cache, d, torch.full((8,), -3, dtype=torch.int64), q, k)
    n2, _ = rot_fn(cache, d, torch.full((8,), maxp - 3, dtype=torch.int64), q, k)
    assert torch.equal(n1, n2)
    # independent numpy restatement (same table), bf16 output
    qb16 = q.to(torch.bfloat16)
    pos = torch.randint(0, maxp, (8,), generator=g)
    rq, _ = rot_fn(cache, d, pos, qb16, k.to(torch.bfloat16))
    check_bf16_agreement(rq, N.rotary_forward(_np(cache), pos.numpy(), _np(qb16), d), what="rope")


def test_rotary_pinned():
    pin_rotary(R.rotary_forward)


def test_cos_sin_table_closed_form():
    d, maxp = 128, 40960
    cache = R.cos_sin_cache(d, maxp, 1e6)
    inv = (1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))).numpy()
    ang32 = (np.arange(maxp, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float64)
    np.testing.assert_allclose(_np(cache[:, : d // 2]), np.cos(ang32), atol=2e-6)
    np.testing.assert_allclose(_np(cache[:, d // 2:]), np.sin(ang32), atol=2e-6)
    # and the float64 closed form; fp32 angle rounding grows with the position
    # (|angle| <= 63 rad here -> <= 63 * 2^-24 rad)
    ref = N.cos_sin_table(d, 64, 1e6)
    np.testing.assert_allclose(_np(cache[:64]), ref, atol=1e-6 + 63 * 2.0 ** -24)


def test_differential_rope_reference_invariant():
    """tests/test_differential_rope.py:41-135: rotating a key cached at p by
    delta equals rotating the raw key at p + delta (fp16, tol 5e-3)."""
    g = gen(19)
    d = 64
    cache = R.cos_sin_cache(d, 2048, 10000.0)
    key = randn(g, 16, 8 * d, dtype=torch.float16)
    for cached0, global0 in ((0, 100), (0, 50), (10, 100), (100, 200)):
        cp = torch.arange(cached0, cached0 + 16)
        gp = torch.arange(global0, global0 + 16)
        _, kc = R.rotary_forward(cache, d, cp, torch.zeros_like(key), key)
        _, kd = R.rotary_forward(cache, d, gp - cp, torch.zeros_like(kc), kc)
        _, kg = R.rotary_forward(cache, d, gp, torch.zeros_like(key), key)
        assert (kd.float() - kg.float()).abs().max() < 5e-3
    _, k0 = R.rotary_forward(cache, d, torch.zeros(16, dtype=torch.int64), torch.zeros_like(key), key)
    assert (k0.float() - key.float()).abs().max() < 1e-5


def _paged_case(seed, pages=12, hkv=2, ps=16, d=64, chunks=3):
    g = gen(seed)
    kv = randn(g, pages, 2, hkv, ps, d)
    perm = torch.randperm(pages, generator=g)
    per = [4, 5, 3][:chunks]
    indptr = torch.tensor([0] + list(np.cumsum(per)), dtype=torch.int32)
    page_idx = perm[: int(indptr[-1])].to(torch.int32)
    last = torch.tensor([16, 7, 1][:chunks], dtype=torch.int32)
    return kv, page_idx, indptr, last


def test_rerotate_paged_k_pinned():
    d, maxp = 64, 2048
    cache = R.cos_sin_cache(d, maxp, 10000.0)
    kv, page_idx, indptr, last = _paged_case(20)
    delta = torch.tensor([0, 37, -5], dtype=torch.int64)
    out = R.rerotate_paged_k(kv, page_idx, indptr, delta, last, cache)
    ps = kv.shape[3]
    for c in range(3):
        for e in range(int(indptr[c]), int(indptr[c + 1])):
            n = int(last[c]) if e == int(indptr[c + 1]) - 1 else ps
            raw = kv[int(page_idx[e]), 0, :, :n].transpose(0, 1)  # [n, hkv, d]
            if int(delta[c]) == 0:
                assert torch.equal(out[e, :n], raw)
            else:
                p = int(delta[c]) % maxp
                ref = N.rope(_np(raw), _np(cache[p, : d // 2]), _np(cache[p, d // 2:]))
                check_bf16_agreement(out[e, :n], ref, what="rerotate")
            assert torch.count_nonzero(out[e, n:]) == 0
    # with k_norm: equals rms_forward of the rotated page
    w = randn(gen(21), d, mean=1.0, std=0.1)
    outn = R.rerotate_paged_k(kv, page_idx, indptr, delta, last, cache, w, 1e-6)
    e = int(indptr[1])
    assert torch.equal(outn[e], R.rms_forward(out[e], w, 1e-6))


# ----------------------------------------------------------- paged KV append
def pin_kv_append(fn):
    """fn(k, v, cache, kv_indices, positions, page_size, layout) -> (cache, skipped)."""
    g = gen(31)
    pages, hkv, ps, d = 12, 3, 4, 8
    # round trip: a sequence of L tokens at positions 0..L-1 through a shuffled
    # table of distinct pages is read back, token by token, from
    # (kv_indices[p // ps], p % ps); every other slot keeps its old value
    L = 29
    table = torch.randperm(pages, generator=g)[: (L + ps - 1) // ps].to(torch.int32)
    k, v = randn(g, L, hkv, d), randn(g, L, hkv, d)
    cache0 = randn(g, pages, 2, hkv, ps, d)
    pos = torch.arange(L)
    out, skipped = fn(k, v, cache0, table, pos, ps, "HND")
    assert skipped == []
    touched = torch.zeros(pages, ps, dtype=torch.bool)
    for t in range(L):
        page, slot = int(table[t // ps]), t % ps
        assert torch.equal(out[page, 0, :, slot], k[t]) and torch.equal(out[page, 1, :, slot], v[t])
        touched[page, slot] = True
    keep = ~touched
    assert torch.equal(out.permute(0, 3, 1, 2, 4)[keep], cache0.permute(0, 3, 1, 2, 4)[keep])
    # NHD holds the same values as HND with the head and slot axes swapped
    out_nhd, _ = fn(k, v, cache0.transpose(2, 3).contiguous(), table, pos, ps, "NHD")
    assert torch.equal(out_nhd, out.transpose(2, 3))
    # negative positions: Python floor division (-1 -> last entry of the table, slot ps-1),
    # and a page offset past the table skips the token
    pos2 = torch.tensor([-1, -ps - 1, len(table) * ps])
    k2, v2 = randn(g, 3, hkv, d), randn(g, 3, hkv, d)
    out2, skipped2 = fn(k2, v2, cache0, table, pos2, ps, "HND")
    assert skipped2 == [2]
    assert torch.equal(out2[int(table[-1]), 0, :, ps - 1], k2[0])
    assert torch.equal(out2[int(table[-2]), 1, :, ps - 1], v2[1])
    # independent numpy restatement, both layouts, int64 table
    for layout, c0 in (("HND", cache0), ("NHD", cache0.transpose(2, 3).contiguous())):
        allpos = torch.cat([pos, pos2])
        kk, vv = torch.cat([k, k2]), torch.cat([v, v2])
        got, sk = fn(kk, vv, c0, table.long(), allpos, ps, layout)
        exp, sk_np = N.append_paged_kv(_np(kk), _np(vv), _np(c0), table.numpy(), allpos.numpy(), ps, layout)
        assert sk == sk_np and np.array_equal(_np(got), exp), layout


def test_kv_append_pinned():
    pin_kv_append(R.append_to_paged_kv_cache)
    # the batched composition equals one per-sequence call for each sequence
    g = gen(32)
    pages, hkv, ps, d = 40, 2, 4, 8
    lens = [5, 0, 9, 3]
    tables = [torch.randperm(pages, generator=g)[:3].to(torch.int32) for _ in lens]
    indptr = torch.tensor([0, 3, 6, 9, 12], dtype=torch.int32)
    flat = torch.cat(tables)
    batch = torch.tensor([0, 2, 3, 2, 0, 3, 2], dtype=torch.int64)
    pos = torch.tensor([5, 9, 3, 10, 6, 4, 40])
    k, v = randn(g, 7, hkv, d), randn(g, 7, hkv, d)
    cache0 = randn(g, pages, 2, hkv, ps, d)
    got, skipped = R.append_paged_kv_batch(k, v, cache0, flat, indptr, batch, pos, ps)
    exp = cache0.clone()
    for s_ in range(4):
        toks = [t for t in range(7) if int(batch[t]) == s_]
        for t in toks:
            p = int(pos[t])
            if p // ps < 3:
                exp[int(tables[s_][p // ps]), 0, :, p % ps] = k[t]
                exp[int(tables[s_][p // ps]), 1, :, p % ps] = v[t]
    assert torch.equal(got, exp) and skipped == [6]
    with pytest.raises(ValueError):
        R.append_to_paged_kv_cache(torch.zeros(1, 1, 8), torch.zeros(1, 1, 8),
                                   torch.zeros(1, 2, 1, 4, 8), torch.zeros(1, dtype=torch.int32),
                                   torch.zeros(1, dtype=torch.int64), 4, "XYZ")


# --------------------------------------------------------- cascade attention
def pin_online_softmax(fn):
    g = gen(41)
    h, b, n, d = 4, 3, 20, 16
    q, k, v = (torch.randn(h, b, d, generator=g), torch.randn(h, n, d, generator=g),
               torch.randn(h, n, d, generator=g))
    scale = d ** -0.5
    m0, l0, a0 = torch.full((h, b), float("-inf")), torch.zeros(h, b), torch.zeros(h, b, d)
    qpos, kpos = torch.tensor([3, 11, 40]), torch.arange(n)
    for causal in (False, True):
        m, l, acc = fn(q, k, v, m0, l0, a0, qpos, kpos, scale, causal)
        exp = N.attention(q.transpose(0, 1).numpy(), k.transpose(0, 1).numpy(), v.transpose(0, 1).numpy(),
                          qpos.numpy(), kpos.numpy(), scale, 1, causal)
        np.testing.assert_allclose((acc / l.unsqueeze(-1)).transpose(0, 1).numpy(), exp, rtol=1e-5, atol=1e-5)
        # two blocks of keys in sequence give the state of one block
        m1, l1, a1 = fn(q, k[:, :7], v[:, :7], m0, l0, a0, qpos, kpos[:7], scale, causal)
        m2, l2, a2 = fn(q, k[:, 7:], v[:, 7:], m1, l1, a1, qpos, kpos[7:], scale, causal)
        np.testing.assert_allclose(a2.numpy(), acc.numpy(), rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(l2.numpy(), l.numpy(), rtol=1e-5, atol=1e-6)
    # causal: a query at position 3 sees keys 0..3 only
    m, l, acc = fn(q, k, v, m0, l0, a0, qpos, kpos, scale, True)
    exp = N.attention(q[:, :1].transpose(0, 1).numpy(), k[:, :4].transpose(0, 1).numpy(),
                      v[:, :4].transpose(0, 1).numpy(), qpos[:1].numpy(), kpos[:4].numpy(), scale, 1, False)
    np.testing.assert_allclose((acc[:, :1] / l[:, :1].unsqueeze(-1)).transpose(0, 1).numpy(), exp, rtol=1e-5, atol=1e-5)


class _Chunk:
    def __init__(self, page_table, kv_length, cached=0, glob=0):
        self.page_table, self.kv_length = page_table, kv_length
        self.cached_position_start, self.global_position_start = cached, glob


class _Level:
    def __init__(self, chunks, ps):
        idx, ptr, last = [], [0], []
        for c in chunks:
            if c.page_table:
                idx += c.page_table
                ptr.append(len(idx))
                n = c.kv_length if len(c.page_table) == 1 else (c.kv_length % ps or (ps if c.kv_length else 0))
                last.append(n)
            else:
                ptr.append(len(idx))
                last.append(0)
        self.chunks = chunks
        self.kv_page_indices = torch.tensor(idx, dtype=torch.int32)
        self.kv_page_indptr = torch.tensor(ptr, dtype=torch.int32)
        self.kv_last_page_len = torch.tensor(last, dtype=torch.int32)


def cascade_case(seed, hq=8, hkv=2, d=32, ps=4, t=5, pages=24, deltas=(0, 9, -3, 0)):
    """Two levels: a 6-token system chunk, then a context chunk of 11 tokens, an empty
    chunk, a chunk with pages but kv_length 0, and a 9-token chunk; shuffled pages."""
    g = gen(seed)
    perm = torch.randperm(pages, generator=g).tolist()
    c0 = _Chunk(perm[0:2], 6, 100, 100 + deltas[0])
    c1 = _Chunk(perm[2:5], 11, 7, 7 + deltas[1])
    c2 = _Chunk([], 0)
    c3 = _Chunk(perm[5:6], 0)
    c4 = _Chunk(perm[6:9], 9, 50, 50 + deltas[2])
    levels = [_Level([c0], ps), _Level([c1, c2, c3, c4], ps)]
    kv = randn(g, pages, 2, hkv, ps, d)
    q = randn(g, t, hq, d)
    return levels, kv, q


def flat_keys(levels, kv, ps, cache, hkv, d, k_norm_weight=None):
    """K (rotated by the re-rotation oracle, normalised) and V of every attended token,
    in the walk order, with their key positions."""
    ks, vs, pos, cum = [], [], [], 0
    for level in levels:
        for ci, ch in enumerate(level.chunks):
            if not ch.page_table or ch.kv_length == 0:
                continue
            s_, e_ = int(level.kv_page_indptr[ci]), int(level.kv_page_indptr[ci + 1])
            pidx = level.kv_page_indices[s_:e_]
            delta = torch.tensor([ch.global_position_start - ch.cached_position_start])
            rot = R.rerotate_paged_k(kv, pidx, torch.tensor([0, e_ - s_], dtype=torch.int32), delta,
                                     level.kv_last_page_len[ci:ci + 1], cache, k_norm_weight, 1e-6)
            for j in range(e_ - s_):
                n = int(level.kv_last_page_len[ci]) if j == e_ - s_ - 1 else ps
                ks.append(rot[j, :n])
                vs.append(kv[int(pidx[j]), 1, :, :n].transpose(0, 1))
                pos += list(range(cum + j * ps, cum + j * ps + n))
            cum += ch.kv_length
    return torch.cat(ks), torch.cat(vs), torch.tensor(pos)


def pin_cascade(fn):
    hq, hkv, d, ps = 8, 2, 32, 4
    cache = R.cos_sin_cache(d, 256, 1e4)
    for causal, kn in ((True, None), (False, randn(gen(43), d, mean=1.0, std=0.3))):
        levels, kv, q = cascade_case(42)
        qpos = torch.tensor([0, 5, 12, 17, 40])
        got = fn(q, qpos, kv, levels, hq, hkv, d ** -0.5, ps, cache, kn, 1e-6, causal)
        k, v, kpos = flat_keys(levels, kv, ps, cache, hkv, d, kn)
        exp = N.attention(_np(q), _np(k), _np(v), qpos.numpy(), kpos.numpy(), d ** -0.5, hq // hkv, causal)
        check_bf16_agreement(got.view(q.shape), N.round_bf16(exp), max_frac=0.05, what="cascade")
    # a query before every key attends nothing: zeros
    levels, kv, q = cascade_case(44)
    got = fn(q[:1], torch.tensor([-1]), kv, levels, hq, hkv, 1.0, ps, cache, None, 1e-6, True)
    assert torch.count_nonzero(got) == 0


def _cascade_oracle(q, qpos, kv, levels, hq, hkv, scale, ps, cache, kn, eps, causal):
    return R.cascade_attention(q, qpos, kv, levels, hq, hkv, scale, ps, cache, kn, eps, causal)


def test_cascade_attention_pinned():
    pin_online_softmax(R.online_softmax_update)
    pin_cascade(_cascade_oracle)


def test_planted_cascade_mistakes_are_caught():
    def no_scale(q, k, v, m, l, a, qp, kp, scale, causal):
        return R.online_softmax_update(q, k, v, m, l, a, qp, kp, 1.0, causal)

    with pytest.raises(AssertionError):
        pin_online_softmax(no_scale)

    def strict_causal(q, k, v, m, l, a, qp, kp, scale, causal):  # key_pos < query_pos
        return R.online_softmax_update(q, k, v, m, l, a, qp - 1, kp, scale, causal)

    with pytest.raises(AssertionError):
        pin_online_softmax(strict_causal)

    def gqa_modulo(q, qpos, kv, levels, hq, hkv, scale, ps, cache, kn, eps, causal):
        # query head h reads kv head h % Hkv instead of h // (Hq / Hkv)
        perm = torch.arange(hq).view(hkv, hq // hkv).t().reshape(-1)
        out = R.cascade_attention(q[:, perm], qpos, kv, levels, hq, hkv, scale, ps, cache, kn, eps, causal)
        inv = torch.argsort(perm)
        return out.view(q.shape)[:, inv].reshape(q.shape[0], -1)

    with pytest.raises(AssertionError):
        pin_cascade(gqa_modulo)

    def no_rotation(q, qpos, kv, levels, hq, hkv, scale, ps, cache, kn, eps, causal):
        return R.cascade_attention(q, qpos, kv, levels, hq, hkv, scale, ps, None, kn, eps, causal)

    with pytest.raises(AssertionError):
        pin_cascade(no_rotation)


# ------------------------------------------------------- fused RMSNorm+QKV
def _qkv_inputs(seed, t=24, h=256, hq=8, hkv=2, d=32):
    g = gen(seed)
    n = (hq + 2 * hkv) * d
    x = randn(g, t, h)
    ln = randn(g, h, mean=1.0, std=0.1)
    w = randn(g, n, h, std=0.02)
    b = randn(g, n, std=0.01)
    return x, ln, w, b, hq, hkv


def pin_qkv(fn_mixed, fn_prod, fn_f32):
    x, ln, w, b, hq, hkv = _qkv_inputs(22)
    check_bf16_agreement(fn_mixed(x, ln, w, b, 1e-6), N.qkv(_np(x), _np(ln), _np(w), _np(b), 1e-6, "mixed"),
                         max_frac=2e-2, what="qkv mixed")
    check_bf16_agreement(fn_prod(x, ln, w, 1e-6), N.qkv(_np(x), _np(ln), _np(w), None, 1e-6, "production"),
                         max_frac=2e-2, what="qkv production")
    np.testing.assert_allclose(_np(fn_f32(x, ln, w, 1e-6)), N.qkv(_np(x), _np(ln), _np(w), None, 1e-6, "f32"),
                               rtol=1e-4, atol=1e-5)
    # [q; k; v] row layout: a weight with only the k rows non-zero lights up
    # exactly the k columns (QKVParallelLinear, layers/linear.py:103-114)
    d = w.shape[0] // (hq + 2 * hkv)
    wk = torch.zeros_like(w)
    wk[hq * d:(hq + hkv) * d] = w[hq * d:(hq + hkv) * d]
    out = fn_f32(x, ln, wk, 1e-6)
    assert torch.count_nonzero(out[:, : hq * d]) == 0 and torch.count_nonzero(out[:, (hq + hkv) * d:]) == 0
    assert torch.count_nonzero(out[:, hq * d:(hq + hkv) * d]) > 0
    # known answer: W = scaled identity block -> output column j = n[:, j] * s
    h = x.shape[1]
    eye = torch.zeros(w.shape[0], h, dtype=torch.bfloat16)
    eye[:h, :h] = torch.eye(h) * 0.5
    out = fn_f32(x, ln, eye, 1e-6)
    nrm = R.rmsnorm_f32(x, ln, 1e-6)
    np.testing.assert_allclose(_np(out[:, :h]), _np(nrm) * 0.5, rtol=1e-6, atol=1e-7)


def test_qkv_variants_pinned():
    pin_qkv(R.qkv_mixed_precision, R.qkv_production, R.qkv_minimal_f32)


def test_qkv_reference_stability_checks():
    """tests/test_numerical_stability.py:180-235 and tests/test_qwen3_bias_handling.py:132-228."""
    g = gen(23)
    h, hq, hkv = 256, 8, 2
    n = (hq + 2 * hkv) * h // hq
    x = randn(g, 8, h)
    ln = torch.ones(h, dtype=torch.bfloat16)
    ln[0] = 96.5
    w = (torch.randn(n, h, generator=g) * 0.1).to(torch.bfloat16)
    fused = R.qkv_minimal_f32(x, ln, w, 1e-6)
    sep = R.rmsnorm_f32(x, ln, 1e-6) @ w.t().float()
    assert (fused - sep).abs().max() < 5e-2
    assert torch.equal(R.qkv_with_bias(x, ln, w, None, 1e-6),
                       R.qkv_with_bias(x, ln, w, torch.zeros(n, dtype=torch.bfloat16), 1e-6))
    w2 = w.clone()
    w2[hq * (h // hq):(hq + hkv) * (h // hq)] *= 96.5
    assert torch.isfinite(R.qkv_with_bias(x.float().mul(0.01).to(torch.bfloat16), ln, w2, None, 1e-6)).all()


def test_bias_sanitization():
    b = torch.tensor([float("nan"), float("inf"), -float("inf"), 1e30, -1e30, 0.5])
    s = R.sanitize_bias(b)
    assert s.tolist() == [0.0, 1e10, -1e10, 1e10, -1e10, 0.5]
    assert R.sanitize_bias(None) is None


def test_model_chains_pinned():
    g = gen(24)
    t, h, hq, hkv, d = 12, 256, 4, 2, 64
    n = (hq + 2 * hkv) * d
    x = randn(g, t, h)
    ln = randn(g, h, mean=1.0, std=0.1)
    w = randn(g, n, h, std=0.02)
    qn = randn(g, d, mean=1.0, std=0.1)
    kn = torch.exp(torch.empty(d).uniform_(math.log(0.05), math.log(100), generator=g)).to(torch.bfloat16)
    pos = torch.randint(0, 2048, (t,), generator=g)
    cache = R.cos_sin_cache(d, 2048, 1e6)
    q, k, v = R.qwen3_attention_input(x, ln, w, None, hq, hkv, 1e-6, pos, cache, qn, kn)
    base = N.qkv(_np(x), _np(ln), _np(w), None, 1e-6, "mixed")
    nq = N.head_norm(base[:, : hq * d].reshape(t, hq, d), _np(qn), 1e-6, "bf16")
    nk = N.head_norm(base[:, hq * d:(hq + hkv) * d].reshape(t, hkv, d), _np(kn), 1e-6, "bf16")
    c = _np(cache)
    rq = N.rotary_forward(c, pos.numpy(), nq.reshape(t, -1), d)
    rk = N.rotary_forward(c, pos.numpy(), nk.reshape(t, -1), d)
    # a one-ulp flip in the projection can move the head norm, so compare in tolerance
    np.testing.assert_allclose(_np(q), rq, rtol=2e-2, atol=2e-2)
    np.testing.assert_allclose(_np(k), rk, rtol=2e-2, atol=2e-2 * float(_np(kn).max()))
    check_bf16_agreement(v, base[:, (hq + hkv) * d:], max_frac=2e-2, what="qwen3 v")
    q, k, v = R.llama_attention_input(x, ln, w, hq, hkv, 1e-5, pos, cache)
    base = N.qkv(_np(x), _np(ln), _np(w), None, 1e-5, "f32")
    rq = N.rotary_forward(c, pos.numpy(), base[:, : hq * d], d, dtype="f32")
    check_bf16_agreement(q, N.round_bf16(rq), max_frac=2e-2, what="llama q")


# --------------------------------------------------- planted mistakes fail
def test_planted_mistakes_are_caught():
    """Each pin above must reject a plausible mistake planted in a copy of the oracle."""

    def rope_wrong_sign(cache, d, positions, q, k):
        cos, sin = cache[positions].chunk(2, dim=-1)

        def app(x):
            x1, x2 = torch.chunk(x.float(), 2, dim=-1)
            c, s = cos.unsqueeze(-2), sin.unsqueeze(-2)
            return torch.cat((x1 * c + x2 * s, x2 * c - x1 * s), dim=-1).to(x.dtype)
        t = positions.size(0)
        return (app(q.reshape(t, -1, d)).view(q.shape), app(k.reshape(t, -1, d)).view(k.shape))

    with pytest.raises(AssertionError):
        pin_rotary(rope_wrong_sign)

    def rms_no_gamma(x, w, eps):
        return R.rms_forward(x, torch.ones_like(w), eps)

    with pytest.raises(AssertionError):
        pin_rms_forward(rms_no_gamma)

    def rms_no_eps(x, w, eps):
        return R.rms_forward(x, w, 0.0)

    with pytest.raises(AssertionError):
        pin_rms_forward(rms_no_eps)

    def f32_transposed_halves(x, ln, w, eps):  # columns of W read in the wrong order
        return R.qkv_minimal_f32(x, ln, w.flip(1), eps)

    with pytest.raises(AssertionError):
        pin_qkv(R.qkv_mixed_precision, R.qkv_production, f32_transposed_halves)

    def mixed_rounds_late(x, ln, w, b, eps):  # drops the bf16 rounding before gamma
        return R.qkv_production(x, ln, w, eps) if b is None else (
            R.qkv_minimal_f32(x, ln, w, eps) + b.float()).to(torch.bfloat16)

    with pytest.raises(AssertionError):
        pin_qkv(mixed_rounds_late, R.qkv_production, R.qkv_minimal_f32)


def test_planted_kv_append_mistakes_are_caught():
    def truncating(k, v, cache, idx, pos, ps, layout):  # C-style division for negatives
        cache, skipped = cache.clone(), []
        for t in range(k.shape[0]):
            p = int(pos[t])
            off = int(p / ps)  # rounds toward zero
            slot = p - off * ps  # then negative: wraps as a torch index
            if off < len(idx):
                page = int(idx[off])
                if layout == "HND":
                    cache[page, 0, :, slot], cache[page, 1, :, slot] = k[t], v[t]
                else:
                    cache[page, 0, slot], cache[page, 1, slot] = k[t], v[t]
            else:
                skipped.append(t)
        return cache, skipped

    with pytest.raises(AssertionError):
        pin_kv_append(truncating)

    def kv_swapped(k, v, cache, idx, pos, ps, layout):
        return R.append_to_paged_kv_cache(v, k, cache, idx, pos, ps, layout)

    with pytest.raises(AssertionError):
        pin_kv_append(kv_swapped)

    def slot_as_page(k, v, cache, idx, pos, ps, layout):  # table indexed by slot, not by page offset
        swapped = (pos % ps) * ps + pos // ps
        return R.append_to_paged_kv_cache(k, v, cache, idx, swapped, ps, layout)

    with pytest.raises(AssertionError):
        pin_kv_append(slot_as_page)


def test_rope_rounding_allowance_is_a_property_of_the_arithmetic():
    """The qwen3 chain with extreme k_norm weights, computed twice by the oracle:
    once as the reference does, once with the fp32 RMS statistic of the input
    norm one ulp larger (what another summation order of the same sum can give)
    and the projection accumulated in float64.  Every result is rounded where
    the reference rounds.  The statistic moves a few x/rms values of some tokens
    to the other bf16 neighbour, which shifts those tokens' projections; after
    the k_norm weights (up to 100) and a cancelling rotation, a few k elements
    differ beyond the strict path tolerance, all within rope_flip_slack -- the
    allowance the GPU test grants (its own misses come from the same place: the
    GPU sums the statistic in another order)."""
    from tests.helpers import ATOL, RTOL, rope_flip_slack
    g = gen(206)
    t, h, hq, hkv, d = 2048, 1024, 16, 8, 128
    n = (hq + 2 * hkv) * d
    x = randn(g, t, h)
    ln = randn(g, h, mean=1.0, std=0.1)
    w = randn(g, n, h, std=0.02)
    kn = torch.exp(torch.empty(d).uniform_(math.log(0.05), math.log(100), generator=g)).to(torch.bfloat16)
    pos = torch.randint(0, 2048, (t,), generator=g)
    cache = R.cos_sin_cache(d, 40960, 1e6)

    def chain_k(acc_dtype, rms_ulps=0):
        x32 = x.float()
        rms = torch.sqrt((x32 * x32).sum(-1, keepdim=True) / h + 1e-6)
        for _ in range(rms_ulps):
            rms = torch.nextafter(rms, torch.full_like(rms, math.inf))
        nrm = (x32 / rms).to(torch.bfloat16) * ln
        proj = (nrm.to(acc_dtype) @ w.to(acc_dtype).t()).to(torch.bfloat16)
        k = proj[:, hq * d:(hq + hkv) * d].reshape(t, hkv, d)
        pre = R.rms_forward(k.float(), kn, 1e-6).to(torch.bfloat16)
        _, kr = R.rotary_forward(cache, d, pos, pre.reshape(t, -1), pre.reshape(t, -1))
        return kr.float(), pre

    k32, pre32 = chain_k(torch.float32)
    k64, _ = chain_k(torch.float64, rms_ulps=1)
    diff = (k32 - k64).abs()
    strict = ATOL + RTOL * k64.abs()
    beyond = diff > strict
    assert 0 < int(beyond.sum()) <= 1e-4 * diff.numel()
    assert torch.all(diff <= strict + rope_flip_slack(pre32.reshape(t, -1)))


# ------------------------------------------------------- linear fusions
def pin_linear_family(lin, lin_res, gate_up, attn_out):
    """Pins of the four linear-layer restatements.
    * small-integer operands make every product and sum exact in fp32 and the
      result exact in bf16: x W^T + b must equal the integer matmul (a
      transposed or column-flipped W, or a dropped bias, fails);
    * a residual of 2^-8 on a projection of 1 + 2^-8: rounding the projection
      first gives 1.0 twice (ties to even), adding before rounding gives
      1 + 2^-7 -- the order of the two roundings is fixed;
    * SiluAndMul of the projection: gate rows first (a swapped [up; gate] fails);
    * the fp16 store of FusedAttentionOutput: 75000 is beyond fp16 and must
      come out inf even for a bf16 output (skipping the fp16 rounding fails);
    * random operands against the float64 numpy restatements."""
    rng = np.random.default_rng(5)
    bf = torch.bfloat16
    x = rng.integers(-2, 3, (5, 16))
    w = rng.integers(-2, 3, (24, 16))
    b = rng.integers(-8, 9, 24)
    t = lambda a: torch.tensor(a, dtype=torch.float32).to(bf)  # noqa: E731
    got = lin(t(x), t(w), t(b)).float().numpy()
    assert np.array_equal(got, (x @ w.T + b).astype(np.float64)), "linear != integer matmul"
    xs = torch.zeros(1, 16, dtype=bf)
    xs[0, 0], xs[0, 1] = 1.0, 2.0 ** -8
    ws = torch.zeros(3, 16, dtype=bf)
    ws[:, 0], ws[:, 1] = 1.0, 1.0
    r = torch.full((1, 3), 2.0 ** -8, dtype=bf)
    assert torch.equal(lin_res(xs, ws, r).float(), torch.ones(1, 3)), "residual rounding order"
    wg, wu = rng.integers(-2, 3, (8, 16)), rng.integers(-2, 3, (8, 16))
    gu = gate_up(t(x), t(np.concatenate([wg, wu]))).float().numpy()
    g_, u_ = (x @ wg.T).astype(np.float64), (x @ wu.T).astype(np.float64)
    expect = N.round_bf16(N.round_bf16(g_ / (1.0 + np.exp(-g_))) * u_)
    assert np.array_equal(gu, expect), "gate/up order or SiLU rounding"
    xb = torch.zeros(1, 16, dtype=bf)
    xb[0, 0] = 300.0
    wb = torch.zeros(2, 16, dtype=bf)
    wb[:, 0] = 250.0
    assert torch.isinf(attn_out(xb, wb, None).float()).all(), "fp16 store of the output"
    xr, wr, br, rr = randn(gen(31), 37, 256), randn(gen(32), 96, 256), randn(gen(33), 96), randn(gen(34), 37, 96)
    check_bf16_agreement(lin(xr, wr, br), N.linear(_np(xr), _np(wr), _np(br)), what="linear")
    check_bf16_agreement(lin_res(xr, wr, rr), N.linear(_np(xr), _np(wr), residual=_np(rr)), what="linear+res")
    check_bf16_agreement(gate_up(xr, wr), N.gate_up_silu_and_mul(_np(xr), _np(wr)), what="gate_up")
    a = attn_out(xr, wr, rr).float().numpy()
    e = N.linear(_np(xr), _np(wr), residual=_np(rr), proj="f32", mid="f16", out="bf16")
    assert np.all(np.abs(a - e) <= 2 * BF16_REL_ULP * np.abs(e) + 1e-30), "attention output"


def test_linear_family_pinned():
    pin_linear_family(R.linear, R.linear_add_residual, R.gate_up_silu_and_mul,
                      R.fused_attention_output)


def test_planted_linear_mistakes_are_caught():
    def lin_flipped(x, w, b=None):
        return R.linear(x, w.flip(1), b)

    def lin_no_bias(x, w, b=None):
        return R.linear(x, w)

    def res_adds_first(x, w, res, b=None):
        acc = x.float() @ w.float().t() + res.float()
        return acc.to(x.dtype)

    def gate_up_swapped(x, w):
        g, u = w.chunk(2, 0)
        return R.gate_up_silu_and_mul(x, torch.cat([u, g]))

    def attn_no_f16(x, w, res=None):
        acc = x.float() @ w.float().t()
        return (acc if res is None else acc + res.float()).to(x.dtype)

    ok = (R.linear, R.linear_add_residual, R.gate_up_silu_and_mul, R.fused_attention_output)
    for i, bad in ((0, lin_flipped), (0, lin_no_bias), (1, res_adds_first), (2, gate_up_swapped),
                   (3, attn_no_f16)):
        fns = list(ok)
        fns[i] = bad
        with pytest.raises(AssertionError):
            pin_linear_family(*fns)


# ------------------------------------------------------------ fp32 mode pins
def test_fp32_mode_closed_forms():
    """oracle/fp32_ref.py: the reference op chains in fp32 with one rounding,
    pinned by closed forms that a dropped term, a wrong sign or a transposed
    operand breaks."""
    from oracle import fp32_ref as F
    g = gen(40)
    w = randn(g, 64, mean=1.0, std=0.1)
    # constant rows c: x * rsqrt(c^2) = sign(c) exactly (powers of two), so y = sign * w
    x = torch.tensor([[2.0] * 64, [-4.0] * 64], dtype=torch.bfloat16)
    y = F.rms_forward(x, w, 0.0)
    assert torch.equal(y[0], w) and torch.equal(y[1], -w)
    # add_rms with a zero residual is rms_forward; residual_out is the rounded sum
    xs, rs = randn(g, 8, 64), randn(g, 8, 64)
    assert torch.equal(F.add_rms_forward(xs, torch.zeros_like(xs), w, 1e-5)[0], F.rms_forward(xs, w, 1e-5))
    assert torch.equal(F.add_rms_forward(xs, rs, w, 1e-5)[1], (xs.float() + rs.float()).bfloat16())
    # silu(0) * u = 0; silu(g) * u -> g * u for large g, -> 0 for large -g
    u = randn(g, 4, 16)
    assert F.silu_and_mul(torch.cat([torch.zeros_like(u), u], -1)).eq(0).all()
    big = torch.full_like(u, 60.0)
    assert torch.equal(F.silu_and_mul(torch.cat([big, u], -1)), (big.float() * u.float()).bfloat16())
    assert F.silu_and_mul(torch.cat([-big, u], -1)).abs().max() < 1e-20
    # qkv with an identity weight is the fp32 RMSNorm, plus the bias
    h = 32
    xq = randn(g, 5, h)
    gq = randn(g, h, mean=1.0, std=0.1)
    eye = torch.eye(h, dtype=torch.bfloat16)
    bias = randn(g, h)
    ref = xq.float() * torch.rsqrt(xq.float().pow(2).mean(-1, keepdim=True) + 1e-6) * gq.float()
    torch.testing.assert_close(F.qkv(xq, gq, eye, None, 1e-6, torch.float32), ref, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(F.qkv(xq, gq, eye, bias, 1e-6, torch.float32), ref + bias.float(),
                               rtol=1e-6, atol=1e-6)
    # permuted weight rows permute the output columns (W is [N, H], not [H, N])
    perm = torch.randperm(h, generator=g)
    torch.testing.assert_close(F.qkv(xq, gq, eye[perm], None, 1e-6, torch.float32), ref[:, perm],
                               rtol=1e-6, atol=1e-6)


def test_fp32_mode_linear_closed_forms():
    """fp32_ref.linear / gate_up_silu_and_mul pinned without restating them:
    integer-valued operands make every product and sum exact in fp32 and in
    float64, so a brute-force triple loop in float64 fixes the result bit for
    bit; identity and selection weights fix the operand order (W is [N, K])."""
    from oracle import fp32_ref as F
    g = gen(44)
    t, k, n = 3, 5, 4
    xi = torch.randint(-4, 5, (t, k), generator=g).to(torch.bfloat16)
    wi = torch.randint(-3, 4, (n, k), generator=g).to(torch.bfloat16)
    bi = torch.randint(-8, 9, (n,), generator=g).to(torch.bfloat16)
    ri = torch.randint(-8, 9, (t, n), generator=g).to(torch.bfloat16)
    brute = torch.zeros(t, n, dtype=torch.float64)
    for i in range(t):
        for j in range(n):
            acc = 0.0
            for c in range(k):
                acc += float(xi[i, c]) * float(wi[j, c])
            brute[i, j] = acc
    assert torch.equal(F.linear(xi, wi), brute.to(torch.bfloat16))
    assert torch.equal(F.linear(xi, wi, bi), (brute + bi.double()).to(torch.bfloat16))
    assert torch.equal(F.linear(xi, wi, bi, residual=ri), (brute + bi.double() + ri.double()).to(torch.bfloat16))
    # one rounding: x + b with both bf16 is formed in fp32 and rounded once
    x, b = randn(g, 6, 16), randn(g, 16)
    eye = torch.eye(16, dtype=torch.bfloat16)
    assert torch.equal(F.linear(x, eye), x)
    assert torch.equal(F.linear(x, eye, b), (x.float() + b.float()).bfloat16())
    # a selection weight picks input columns in its row order
    sel = eye[[3, 0, 7]]
    assert torch.equal(F.linear(x, sel), x[:, [3, 0, 7]])
    # gate_up: [gate rows; up rows].  W = [I; I]: silu(x) * x in fp32, one rounding
    xs = randn(g, 4, 16)
    xf = xs.double()
    want = (xf * torch.sigmoid(xf) * xf).to(torch.bfloat16)
    got = F.gate_up_silu_and_mul(xs, torch.cat([eye, eye]))
    assert (got.float() - want.float()).abs().le(want.float().abs() * 2.0 ** -8 + 1e-30).all()
    zero = torch.zeros_like(eye)
    assert F.gate_up_silu_and_mul(xs, torch.cat([eye, zero])).eq(0).all()  # up = 0
    assert F.gate_up_silu_and_mul(xs, torch.cat([zero, eye])).eq(0).all()  # silu(0) = 0
    # the gate is the first half: a large gate leaves silu(g) * u = g * u; with
    # the halves swapped the result is silu(u) * g, not the same
    big = torch.full((4, 16), 40.0, dtype=torch.bfloat16)
    gate_sel = torch.cat([eye, zero], 1)  # picks the first 16 of 32 input columns
    up_sel = torch.cat([zero, eye], 1)
    xin = torch.cat([big, xs], 1)
    y = F.gate_up_silu_and_mul(xin, torch.cat([gate_sel, up_sel]))
    assert torch.equal(y, (big.float() * xs.float()).bfloat16())
    y_swapped = F.gate_up_silu_and_mul(xin, torch.cat([up_sel, gate_sel]))
    assert not torch.equal(y_swapped, y)


def test_planted_fp32_linear_mistakes_are_caught():
    """Copies of fp32_ref.linear / gate_up_silu_and_mul with a planted mistake
    (transposed weight, bias dropped, halves swapped, silu on the up half, a
    bf16 rounding of the projection) fail the closed forms above."""
    g = gen(45)
    x = randn(g, 4, 16)
    eye = torch.eye(16, dtype=torch.bfloat16)
    sel = eye[[3, 0, 7]]
    b = randn(g, 16)

    def transposed(x, w):
        return (x.float() @ w.float()).bfloat16()
    with pytest.raises(RuntimeError):  # [4, 16] @ [3, 16] does not even compose
        transposed(x, sel)
    perm = torch.randperm(16, generator=g)
    assert not torch.equal(transposed(x, eye[perm]), x[:, perm])

    def no_bias(x, w, bias=None):
        return (x.float() @ w.float().t()).bfloat16()
    assert not torch.equal(no_bias(x, eye, b), (x.float() + b.float()).bfloat16())

    def two_roundings(x, w, bias):
        return ((x.float() @ w.float().t()).bfloat16().float() + bias.float()).bfloat16()
    # W = I + shift: out_j = x_j + x_(j+1), not representable in bf16 in general
    xr, br = randn(g, 64, 16), randn(g, 16, std=0.01)
    w2 = eye + eye.roll(1, 1)
    once = (xr.double() + xr.double().roll(-1, 1) + br.double()).to(torch.bfloat16)
    from oracle import fp32_ref as F
    assert torch.equal(F.linear(xr, w2, br), once)
    assert not torch.equal(two_roundings(xr, w2, br), once)

    def silu_on_up(x, w):
        gu = x.float() @ w.float().t()
        gg, u = gu.chunk(2, -1)
        return (gg * u * torch.sigmoid(u)).bfloat16()
    zero = torch.zeros_like(eye)
    big = torch.full((4, 16), 40.0, dtype=torch.bfloat16)
    xin = torch.cat([big, x], 1)
    w = torch.cat([torch.cat([eye, zero], 1), torch.cat([zero, eye], 1)])
    assert not torch.equal(silu_on_up(xin, w), (big.float() * x.float()).bfloat16())


def test_fp32_mode_chains_match_the_pinned_fp32_pieces():
    """The attention-input chains of fp32_ref equal their pieces composed from
    the ref-rounding oracle's fp32 forms: rotary_forward on fp32 q/k (it rounds
    to the input dtype, fp32 here) and rms_forward on fp32 heads (fp32 in, so
    no intermediate rounding) -- pinned above and in the RoPE tests."""
    from oracle import fp32_ref as F
    g = gen(41)
    t, h, hq, hkv, d = 6, 64, 4, 2, 16
    x = randn(g, t, h)
    ln = randn(g, h, mean=1.0, std=0.1)
    w = randn(g, (hq + 2 * hkv) * d, h, std=0.1)
    qn, kn = randn(g, d, mean=1.0, std=0.1), randn(g, d, mean=2.0, std=0.5)
    pos = torch.randint(0, 64, (t,), generator=g)
    cache = R.cos_sin_cache(d, 64, 1e4)
    acc = F.qkv(x, ln, w, None, 1e-6, torch.float32)
    q, k, v = acc.split([hq * d, hkv * d, hkv * d], dim=-1)
    qh = R.rms_forward(q.reshape(t, hq, d), qn.float(), 1e-6).reshape(t, -1)
    kh = R.rms_forward(k.reshape(t, hkv, d), kn.float(), 1e-6).reshape(t, -1)
    rq, rk = R.rotary_forward(cache, d, pos, qh, kh)
    got = F.qwen3_attention_input(x, ln, w, None, hq, hkv, 1e-6, pos, cache, qn, kn)
    for a, b in zip(got, (rq, rk, v)):
        torch.testing.assert_close(a.float(), b.bfloat16().float(), rtol=0, atol=0)
    rq, rk = R.rotary_forward(cache, d, pos, q, k)
    got = F.llama_attention_input(x, ln, w, hq, hkv, 1e-6, pos, cache)
    for a, b in zip(got, (rq, rk, v)):
        torch.testing.assert_close(a.float(), b.bfloat16().float(), rtol=0, atol=0)


def test_fp32_mode_is_within_the_reference_rounding_of_ref_mode():
    """Both modes compute the same function: on generic data they agree to the
    reference's own bf16 rounding (normwise relative difference of a few 1e-3)."""
    from oracle import fp32_ref as F
    g = gen(42)
    x = randn(g, 64, 512)
    w = randn(g, 512, mean=1.0, std=0.1)
    wq = randn(g, 384, 512, std=0.05)

    def nw(a, b):
        a, b = a.float(), b.float()
        return ((a - b).norm() / b.norm()).item()
    assert nw(R.rms_forward(x, w, 1e-5), F.rms_forward(x, w, 1e-5)) < 5e-3
    assert nw(R.silu_and_mul(x), F.silu_and_mul(x)) < 5e-3
    assert nw(R.qkv_mixed_precision(x, w, wq, None, 1e-5), F.qkv(x, w, wq, None, 1e-5, torch.bfloat16)) < 8e-3
    # minimal_f32 is fp32 in the reference too: the modes agree to fp32 rounding
    assert nw(R.qkv_minimal_f32(x, w, wq, 1e-5), F.qkv(x, w, wq, None, 1e-5, torch.float32)) < 1e-6


def test_planted_fp32_mode_mistakes_are_caught():
    """Copies of fp32_ref with a planted mistake fail the pins above."""
    from oracle import fp32_ref as F
    g = gen(43)
    h = 32
    xq, gq = randn(g, 5, h), randn(g, h, mean=1.0, std=0.1)
    eye = torch.eye(h, dtype=torch.bfloat16)
    ref = F.qkv(xq, gq, eye, None, 1e-6, torch.float32)

    def no_gamma(x, norm_weight, qkv_weight, qkv_bias, eps, out_dtype):
        x32 = x.float()
        return (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps) @ qkv_weight.float().t()).to(out_dtype)

    def transposed(x, norm_weight, qkv_weight, qkv_bias, eps, out_dtype):
        x32 = x.float()
        n = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps) * norm_weight.float()
        return (n @ qkv_weight.float()).to(out_dtype)
    perm = torch.randperm(h, generator=g)
    assert not torch.allclose(no_gamma(xq, gq, eye, None, 1e-6, torch.float32), ref, rtol=1e-4, atol=1e-4)
    assert not torch.allclose(transposed(xq, gq, eye[perm], None, 1e-6, torch.float32), ref[:, perm],
                              rtol=1e-4, atol=1e-4)
    # a RoPE with the sign of the sine flipped differs from the pinned rotary_forward
    d, t = 16, 4
    cache = R.cos_sin_cache(d, 32, 1e4)
    pos = torch.arange(1, t + 1)
    q = randn(g, t, d).float()
    cos, sin = cache[pos].chunk(2, -1)
    x1, x2 = q.chunk(2, -1)
    wrong = torch.cat((x1 * cos + x2 * sin, x2 * cos - x1 * sin), -1)
    assert not torch.allclose(wrong, R.rotary_forward(cache, d, pos, q, q)[0], atol=1e-3)
