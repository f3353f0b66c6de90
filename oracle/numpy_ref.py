"""numpy restatement of the reference hot-path ops (test infrastructure only).

Written independently of oracle.torch_ref: float64 arithmetic, with the
reference's bf16/fp16/fp32 rounding points emulated explicitly (bf16 by
round-to-nearest-even on the float32 bit pattern).  Used to pin the torch
restatement: the two agree up to the last-bit effects of float64 vs float32
intermediates.
"""
from __future__ import annotations

import numpy as np


def to_f32(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64).astype(np.float32)


def round_bf16(a) -> np.ndarray:
    """Rounds to the nearest bfloat16 (ties to even), returned as float64."""
    f = to_f32(a)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).astype(np.float64)
    return np.where(np.isnan(f), np.nan, out)


def round_f16(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64).astype(np.float16).astype(np.float64)


def round_to(a, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return round_bf16(a)
    if dtype == "f16":
        return round_f16(a)
    if dtype == "f32":
        return to_f32(a).astype(np.float64)
    raise ValueError(dtype)


# --------------------------------------------------------------------- norms
def rms_forward(x, w, eps, dtype="bf16"):
    """y = R(R(x / sqrt(mean(x^2) + eps)) * w), R = rounding to the input dtype
    (layers/layernorm.py:35-44)."""
    x = np.asarray(x, np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return round_to(round_to(x * r, dtype) * np.asarray(w, np.float64), dtype)


def add_rms_forward(x, res, w, eps, dtype="bf16"):
    """(y, residual_out) of layers/layernorm.py:46-57; statistics from the
    unrounded fp32 sum."""
    s = to_f32(np.asarray(x, np.float64) + np.asarray(res, np.float64)).astype(np.float64)
    y = rms_forward_unrounded_input(s, w, eps, dtype)
    return y, round_to(s, dtype)


def rms_forward_unrounded_input(s, w, eps, dtype):
    r = 1.0 / np.sqrt(np.mean(s * s, axis=-1, keepdims=True) + eps)
    return round_to(round_to(s * r, dtype) * np.asarray(w, np.float64), dtype)


def rmsnorm_f32(x, w, eps):
    """kernels/rmsnorm_f32.py:47-96 in float64."""
    x = np.asarray(x, np.float64)
    rms = np.sqrt(np.sum(x * x, axis=-1, keepdims=True) / x.shape[-1] + eps)
    return (x / rms) * np.asarray(w, np.float64)


# ---------------------------------------------------------------- elementwise
def embedding(ids, table):
    ids = np.asarray(ids)
    out = np.empty(ids.shape + table.shape[1:], dtype=table.dtype)
    for idx in np.ndindex(ids.shape):
        out[idx] = table[int(ids[idx])]
    return out


def silu_and_mul(x, dtype="bf16"):
    x = np.asarray(x, np.float64)
    i = x.shape[-1] // 2
    g, u = x[..., :i], x[..., i:]
    return round_to(round_to(g / (1.0 + np.exp(-g)), dtype) * u, dtype)


# ---------------------------------------------------------------------- RoPE
def cos_sin_table(head_size, max_position, base):
    """Closed form of the RoPE table in float64: angle(t, j) = t * base^(-2j/D)."""
    inv_freq = 1.0 / (base ** (np.arange(0, head_size, 2, dtype=np.float64) / head_size))
    ang = np.arange(max_position, dtype=np.float64)[:, None] * inv_freq[None, :]
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=-1)


def rope(x, cos, sin, dtype="bf16"):
    """Neox rotation of x [..., D] by cos/sin [..., D/2] (broadcast), rounded to dtype."""
    x = np.asarray(x, np.float64)
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    return round_to(np.concatenate([x1 * cos - x2 * sin, x2 * cos + x1 * sin], axis=-1), dtype)


def rotary_forward(table, positions, x, head_size, dtype="bf16"):
    """RotaryEmbedding.forward for x [T, H*D] / [T, H, D] with a table [P, D]."""
    t = len(positions)
    x3 = np.asarray(x, np.float64).reshape(t, -1, head_size)
    p = np.asarray(positions) % table.shape[0]  # torch negative-index wrap
    cs = table[p]
    cos, sin = cs[:, None, : head_size // 2], cs[:, None, head_size // 2:]
    return rope(x3, cos, sin, dtype).reshape(np.asarray(x).shape)


# ----------------------------------------------------------- fused RMSNorm+QKV
def qkv(x, norm_w, w, bias, eps, variant, in_dtype="bf16"):
    """Projection of the four variants; returns float64 values already rounded
    to the variant's output dtype ("mixed" -> bf16 then in_dtype,
    "production" -> bf16, "f32" -> fp32, "with_bias" -> fp32)."""
    x = np.asarray(x, np.float64)
    gw = np.asarray(norm_w, np.float64)
    rms = np.sqrt(np.sum(x * x, axis=-1, keepdims=True) / x.shape[-1] + eps)
    wt = np.asarray(w, np.float64)
    if variant == "mixed":
        n = round_bf16(round_bf16(x / rms) * gw)
        acc = n @ round_bf16(wt).T
        if bias is not None:
            acc = acc + np.asarray(bias, np.float64)
        return round_to(round_bf16(acc), in_dtype)
    if variant == "production":
        n = round_bf16((x / rms) * gw)
        return round_bf16(n @ round_bf16(wt).T)
    if variant in ("f32", "with_bias"):
        acc = ((x / rms) * gw) @ wt.T
        if bias is not None:
            acc = acc + np.asarray(bias, np.float64)
        return to_f32(acc).astype(np.float64)
    raise ValueError(variant)


def head_norm(x, w, eps, out_dtype):
    """RMSNorm over the last dim on fp32 values, cast to out_dtype
    (q_norm(q.float()).to(dtype), models/qwen3.py:257-281)."""
    x = np.asarray(x, np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return round_to((x * r) * np.asarray(w, np.float64), out_dtype)


def append_paged_kv(k, v, cache, kv_indices, positions, page_size, layout="HND"):
    """Paged KV append (kernels/kv_cache_utils.py:9-78) with the index arithmetic
    written out: offset = floor(pos / page_size), slot = pos - offset * page_size,
    Python-style wrap of negative offsets and page ids.  cache is copied; returns
    (cache, skipped token indices).  Values are moved, not converted."""
    out = np.array(cache, copy=True)
    n_idx, n_pages = len(kv_indices), out.shape[0]
    skipped = []
    for t in range(k.shape[0]):
        pos = int(positions[t])
        off = int(np.floor(pos / page_size))
        slot = pos - off * page_size
        if off >= n_idx:
            skipped.append(t)
            continue
        if off < -n_idx:
            raise IndexError("page offset out of range")
        page = int(kv_indices[off + n_idx if off < 0 else off])
        if page < -n_pages or page >= n_pages:
            raise IndexError("page id out of range")
        page = page + n_pages if page < 0 else page
        for kv, src in ((0, k), (1, v)):
            if layout == "HND":
                out[page, kv, :, slot, :] = src[t]
            else:
                out[page, kv, slot, :, :] = src[t]
    return out, skipped


def attention(q, k, v, qpos, kpos, scale, group, causal=True):
    """Softmax attention in float64, written directly: q [T, H, D], k/v [N, Hkv, D],
    query head h reads kv head h // group; keys whose position exceeds the query's
    are excluded when causal; a query with no key gets 0.  Returns [T, H, D]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    t_, h, d = q.shape
    out = np.zeros((t_, h, d))
    for hh in range(h):
        kh, vh = k[:, hh // group], v[:, hh // group]
        s = q[:, hh] @ kh.T * scale  # [T, N]
        if causal:
            s = np.where(np.asarray(kpos)[None, :] <= np.asarray(qpos)[:, None], s, -np.inf)
        mx = np.max(s, axis=1, keepdims=True)
        ok = np.isfinite(mx[:, 0])
        w = np.where(ok[:, None], np.exp(s - np.where(ok[:, None], mx, 0.0)), 0.0)
        den = w.sum(axis=1, keepdims=True)
        out[:, hh] = np.where(ok[:, None], (w @ vh) / np.where(den > 0, den, 1.0), 0.0)
    return out


def linear(x, w, bias=None, residual=None, proj="bf16", mid="f32", out="bf16"):
    """out(mid(proj(x W^T + bias) + residual)) in float64 arithmetic: F.linear
    (layers/linear.py:37-38) and its residual / FusedAttentionOutput
    (kernels/fused_attention_output.py:17-134) roundings."""
    acc = np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
    if bias is not None:
        acc = acc + np.asarray(bias, np.float64)
    acc = round_to(acc, proj)
    if residual is not None:
        acc = acc + np.asarray(residual, np.float64)
    return round_to(round_to(acc, mid), out)


def gate_up_silu_and_mul(x, w, dtype="bf16"):
    """SiluAndMul(F.linear(x, [Wg; Wu])) (models/qwen3.py:388-392)."""
    return silu_and_mul(linear(x, w, proj=dtype, out=dtype), dtype)
