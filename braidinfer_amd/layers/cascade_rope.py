"""Paged differential-RoPE re-rotation of cached chunk K on MI355X.

Replaces the per-page Python loop body of CascadeAttention.forward
(braidinfer/layers/cascade_attention.py:116-178): for every page of every
chunk, K[page, 0, :, :tokens, :] is rotated by the chunk's position delta
(global_position_start - cached_position_start) with
`rotary_emb(pos_diff, dummy_q, page_k)`, i.e. cos_sin_cache[delta] with torch
negative-index wrap, and then k_norm is applied.  One kernel launch covers all
pages of all chunks (the reference issues ~10 launches and a host sync per
16-token page).
"""
from __future__ import annotations

import torch

from .. import _lib


def rerotate_paged_k(kv_cache_layer: torch.Tensor, page_indices: torch.Tensor,
                     chunk_indptr: torch.Tensor, chunk_delta: torch.Tensor,
                     last_page_len: torch.Tensor, cos_sin_cache: torch.Tensor,
                     out: torch.Tensor | None = None, k_norm_weight: torch.Tensor | None = None,
                     k_norm_eps: float = 1e-6, inplace: bool = False) -> torch.Tensor:
    """Rotates the K half of one layer of the paged HND cache
    ([num_pages, 2, num_kv_heads, page_size, head_dim], page_manager.py:36-42).

    page_indices / chunk_indptr / last_page_len: int32 (as
    CascadeAttention._create_level builds them); chunk_delta: int64/int32 per chunk.

    inplace=True rotates the cache itself and returns it (no k_norm allowed).
    Otherwise returns out [num_entries, page_size, num_kv_heads, head_dim]
    (page-padded NHD; entry e, token t is page_indices[e]'s t-th token), with
    k_norm applied when k_norm_weight is given -- the page_k tensors the
    reference loop hands to online_softmax_update, concatenated.
    """
    if kv_cache_layer.dim() != 5 or kv_cache_layer.shape[1] != 2:
        raise ValueError("kv_cache_layer must be [num_pages, 2, num_kv_heads, page_size, head_dim]")
    if not kv_cache_layer.is_contiguous():
        raise ValueError("kv_cache_layer must be contiguous")
    num_pages, _, hkv, page_size, head_dim = kv_cache_layer.shape
    meta = []
    for name, t in (("page_indices", page_indices), ("chunk_indptr", chunk_indptr),
                    ("last_page_len", last_page_len)):
        if t.dtype != torch.int32:
            raise TypeError(f"{name} must be int32")
        meta.append(t.contiguous())
    page_indices, chunk_indptr, last_page_len = meta
    chunk_delta = chunk_delta.contiguous()
    num_chunks = chunk_delta.numel()
    if chunk_indptr.numel() != num_chunks + 1 or last_page_len.numel() != num_chunks:
        raise ValueError("chunk_indptr must have num_chunks+1 entries and last_page_len num_chunks")
    if cos_sin_cache.dtype != torch.float32:
        raise TypeError("cos_sin_cache must be float32")
    cos_sin_cache = cos_sin_cache.contiguous()
    dev = _lib.require_device(kv_cache_layer, page_indices, chunk_indptr, chunk_delta,
                              last_page_len, cos_sin_cache, k_norm_weight)
    num_entries = page_indices.numel()
    if inplace:
        if k_norm_weight is not None:
            raise ValueError("k_norm is applied to the rotated copy, not to the cache")
        out = None
    elif out is None:
        out = torch.empty((num_entries, page_size, hkv, head_dim), dtype=kv_cache_layer.dtype,
                          device=dev)
    if k_norm_weight is not None:
        k_norm_weight = k_norm_weight.contiguous()
    _lib.call("bfa_rerotate_paged_k", _lib.ptr(kv_cache_layer), _lib.dtype_code(kv_cache_layer),
              num_pages, hkv, page_size, head_dim, _lib.ptr(page_indices), num_entries,
              _lib.ptr(chunk_indptr), _lib.ptr(last_page_len), _lib.ptr(chunk_delta),
              _lib.dtype_code(chunk_delta), num_chunks, _lib.ptr(cos_sin_cache),
              cos_sin_cache.shape[0], _lib.ptr(k_norm_weight),
              _lib.dtype_code(k_norm_weight) if k_norm_weight is not None else 0,
              float(k_norm_eps), _lib.ptr(out), _lib.ptr(_lib.status_word(dev)),
              _lib.stream_of(dev))
    return kv_cache_layer if inplace else out
