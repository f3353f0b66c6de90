"""Rotary embedding on MI355X, mirroring braidinfer/layers/rotary_embedding.py:6-78.

The cos/sin table is built exactly as the reference builds it (fp32
inv_freq, t (x) inv_freq, cat(cos, sin); `:29-47`) so its values are the same
bits; the rotation itself runs in the HIP kernel (bfa_rotary_embedding).
`forward` keeps the reference's `.view(num_tokens, -1, head_size)` semantics,
so q/k may be strided views (e.g. slices of a packed qkv buffer) and a key
with a different number of rows than positions is regrouped the same way.
"""
from __future__ import annotations

from functools import lru_cache

import torch
from torch import nn

from .. import _lib


def _as_heads(x: torch.Tensor, num_tokens: int, head_size: int) -> torch.Tensor:
    v = x.view(num_tokens, -1, head_size)
    if v.stride(-1) != 1:
        v = v.contiguous()
    return v


def apply_rotary_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Neox rotation of x [T, heads, D] by per-token cos/sin [T, D/2]; fp32 math,
    result in x.dtype (rotary_embedding.py:6-24)."""
    if x.dim() != 3:
        raise NotImplementedError("apply_rotary_emb expects x as [num_tokens, heads, head_size]")
    t, heads, d = x.shape
    cos = cos.reshape(t, d // 2)
    sin = sin.reshape(t, d // 2)
    if cos.dtype != torch.float32:
        cos = cos.to(torch.float32)
    if sin.dtype != torch.float32:
        sin = sin.to(torch.float32)
    if cos.stride(-1) != 1 or sin.stride(-1) != 1 or cos.stride(0) != sin.stride(0):
        cos, sin = cos.contiguous(), sin.contiguous()
    if x.stride(-1) != 1:
        x = x.contiguous()
    dev = _lib.require_device(x, cos, sin)
    out = torch.empty((t, heads, d), dtype=x.dtype, device=dev)
    _lib.call("bfa_apply_rotary_emb", _lib.ptr(x), _lib.dtype_code(x), t, heads, d,
              x.stride(0), x.stride(1), _lib.ptr(cos), _lib.ptr(sin), cos.stride(0),
              _lib.ptr(out), _lib.stream_of(dev))
    return out


class RotaryEmbedding(nn.Module):

    def __init__(self, head_size: int, rotary_dim: int, max_position_embeddings: int,
                 base: float) -> None:
        super().__init__()
        self.head_size = head_size
        assert rotary_dim == head_size
        inv_freq = 1.0 / (base ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))
        t = torch.arange(max_position_embeddings, dtype=torch.float32)
        freqs = torch.einsum("i,j -> ij", t, inv_freq)
        cache = torch.cat((freqs.cos(), freqs.sin()), dim=-1)
        self.register_buffer("cos_sin_cache", cache.to(torch.float32), persistent=False)

    def forward(self, positions: torch.Tensor, query: torch.Tensor,
                key: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        num_tokens = positions.size(0)
        query_shape, key_shape = query.shape, key.shape
        q3 = _as_heads(query, num_tokens, self.head_size)
        k3 = _as_heads(key, num_tokens, self.head_size)
        cache = self.cos_sin_cache
        dev = _lib.require_device(positions, q3, k3, cache)
        if positions.dtype not in (torch.int64, torch.int32):
            positions = positions.long()
        positions = positions.contiguous()
        q_out = torch.empty(q3.shape, dtype=q3.dtype, device=dev)
        k_out = torch.empty(k3.shape, dtype=k3.dtype, device=dev)
        status = _lib.status_word(dev)
        if q3.dtype == k3.dtype:
            _lib.call("bfa_rotary_embedding", _lib.ptr(positions), _lib.dtype_code(positions),
                      num_tokens, _lib.ptr(cache), cache.shape[0], self.head_size,
                      _lib.dtype_code(q3), _lib.ptr(q3), q3.shape[1], q3.stride(0), q3.stride(1),
                      _lib.ptr(q_out), _lib.ptr(k3), k3.shape[1], k3.stride(0), k3.stride(1),
                      _lib.ptr(k_out), _lib.ptr(status), _lib.stream_of(dev))
        else:
            for src, dst in ((q3, q_out), (k3, k_out)):
                _lib.call("bfa_rotary_embedding", _lib.ptr(positions), _lib.dtype_code(positions),
                          num_tokens, _lib.ptr(cache), cache.shape[0], self.head_size,
                          _lib.dtype_code(src), _lib.ptr(src), src.shape[1], src.stride(0),
                          src.stride(1), _lib.ptr(dst), None, 0, 0, 0, None, _lib.ptr(status),
                          _lib.stream_of(dev))
        return q_out.view(query_shape), k_out.view(key_shape)


@lru_cache(1)
def get_rope(head_size: int, rotary_dim: int, max_position: int, base: float,
             rope_scaling: dict | None = None):
    assert rope_scaling is None
    return RotaryEmbedding(head_size, rotary_dim, max_position, base)
