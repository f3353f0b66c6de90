"""Paged KV-cache append on MI355X, under the names of braidinfer/kernels/kv_cache_utils.py.

``append_to_paged_kv_cache_custom`` replaces the reference's per-token Python
loop (two ``.item()`` host syncs and two slice assignments per token,
kernels/kv_cache_utils.py:9-78) with one launch of ``bfa_append_paged_kv``.
``build_paged_kv_indices`` is the reference's host-side CSR builder
(kernels/kv_cache_utils.py:81-118), restated.  ``PagedKVAppend`` names where a
fused RMSNorm+QKV call (``fused_rmsnorm_qkv(..., paged_kv=...)``) appends its k
and v heads itself, in the projection's epilogue.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch

from .. import _lib

_LAYOUT_DIMS = {"HND": (2, 3), "NHD": (3, 2)}  # (head dim, slot dim) of the 5-D layer cache


def append_to_paged_kv_cache_custom(
    k: torch.Tensor,
    v: torch.Tensor,
    layer_cache: torch.Tensor,
    kv_indices: torch.Tensor,
    positions: torch.Tensor,
    page_size: int,
    kv_layout: str = "HND",
) -> None:
    """Writes token t's K and V (``k[t]``, ``v[t]``: [num_heads, head_dim]) into
    ``layer_cache`` at page ``kv_indices[positions[t] // page_size]``, slot
    ``positions[t] % page_size``.

    layer_cache: HND [num_pages, 2, num_heads, page_size, head_dim] or
    NHD [num_pages, 2, page_size, num_heads, head_dim] (K at index 0, V at 1).
    As in the reference, a token whose page offset is past ``kv_indices`` is
    skipped (the reference prints an error; here the device status word records
    it and ``braidinfer_amd.check_device_status()`` warns), and other
    out-of-range indices raise IndexError at the next status check.  Runs
    asynchronously on the current stream; nothing is returned.
    """
    _append(k, v, layer_cache, kv_indices, None, None, positions, page_size, kv_layout)


def append_paged_kv_batch(
    k: torch.Tensor,
    v: torch.Tensor,
    layer_cache: torch.Tensor,
    kv_indices: torch.Tensor,
    kv_indptr: torch.Tensor,
    batch_indices: torch.Tensor,
    positions: torch.Tensor,
    page_size: int,
    kv_layout: str = "HND",
) -> None:
    """One launch for a batch of sequences (no single reference function: the
    reference's page manager calls append_to_paged_kv_cache_custom once per
    sequence, engine/page_manager.py:180-210).  Token t belongs to sequence
    ``batch_indices[t]``, whose page table is
    ``kv_indices[kv_indptr[s]:kv_indptr[s+1]]`` (the CSR form
    build_paged_kv_indices returns); within it the per-sequence rule applies."""
    if kv_indptr.dtype != torch.int32:
        kv_indptr = kv_indptr.to(torch.int32)
    if batch_indices.dtype not in (torch.int32, torch.int64):
        batch_indices = batch_indices.long()
    batch_indices = batch_indices.reshape(-1)
    if batch_indices.numel() < k.shape[0]:
        raise IndexError(f"{batch_indices.numel()} batch indices for {k.shape[0]} tokens")
    _append(k, v, layer_cache, kv_indices, kv_indptr.reshape(-1).contiguous(),
            batch_indices[: k.shape[0]].contiguous(), positions, page_size, kv_layout)


def _append(k, v, layer_cache, kv_indices, kv_indptr, batch_indices, positions, page_size,
            kv_layout):
    if kv_layout not in _LAYOUT_DIMS:
        raise ValueError(f"Unknown kv_layout: {kv_layout}")
    if layer_cache.dim() != 5 or layer_cache.shape[1] != 2:
        raise ValueError("layer_cache must be [num_pages, 2, ...] with 5 dimensions")
    hdim, sdim = _LAYOUT_DIMS[kv_layout]
    num_pages = layer_cache.shape[0]
    heads, slots, head_dim = layer_cache.shape[hdim], layer_cache.shape[sdim], layer_cache.shape[4]
    num_tokens = k.shape[0]
    for name, t in (("k", k), ("v", v)):
        if tuple(t.shape) != (num_tokens, heads, head_dim):
            raise RuntimeError(f"{name} of shape {tuple(t.shape)} does not match the cache's "
                               f"[tokens, {heads}, {head_dim}] rows")
    if v.dtype != k.dtype:
        v = v.to(k.dtype)
    if k.stride(-1) != 1:
        k = k.contiguous()
    if v.stride(-1) != 1:
        v = v.contiguous()
    if layer_cache.stride(-1) != 1:
        raise ValueError("layer_cache must have unit stride along head_dim")
    if num_tokens and page_size == 0:
        raise ZeroDivisionError("integer division or modulo by zero")
    if page_size < 0:
        raise ValueError("page_size must be positive")
    positions = positions.reshape(-1)
    if positions.numel() < num_tokens:  # the reference indexes positions[t] for every token
        raise IndexError(f"{positions.numel()} positions for {num_tokens} tokens")
    positions = positions[:num_tokens]
    if positions.dtype not in (torch.int32, torch.int64):
        positions = positions.long()
    if kv_indices.dim() > 1:
        raise ValueError("kv_indices must be one-dimensional")
    kv_indices = kv_indices.reshape(-1)
    if kv_indices.dtype not in (torch.int32, torch.int64):
        kv_indices = kv_indices.long()
    positions = positions.contiguous()
    kv_indices = kv_indices.contiguous()
    dev = _lib.require_device(k, v, layer_cache, kv_indices, positions, kv_indptr, batch_indices)
    if num_tokens == 0:
        return
    st = layer_cache.stride()
    _lib.call(
        "bfa_append_paged_kv",
        _lib.ptr(k), _lib.ptr(v), _lib.dtype_code(k), num_tokens, heads, head_dim,
        k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        _lib.ptr(layer_cache), _lib.dtype_code(layer_cache), num_pages, slots,
        st[0], st[1], st[hdim], st[sdim],
        _lib.ptr(kv_indices), _lib.dtype_code(kv_indices), kv_indices.numel(),
        _lib.ptr(kv_indptr), _lib.ptr(batch_indices),
        _lib.dtype_code(batch_indices) if batch_indices is not None else 0,
        kv_indptr.numel() - 1 if kv_indptr is not None else 0,
        _lib.ptr(positions), _lib.dtype_code(positions), int(page_size),
        _lib.ptr(_lib.status_word(dev)), _lib.stream_of(dev),
    )


@dataclass
class PagedKVAppend:
    """The cache side of append_to_paged_kv_cache_custom (or, with ``kv_indptr``
    and ``batch_indices``, of append_paged_kv_batch) for a fused QKV call that
    appends its own k and v heads: the appended rows are the call's k and v
    outputs ([tokens, num_kv_heads, head_dim] in its output dtype), at
    ``positions`` (the tokens' positions in their sequences).  With
    ``write_kv_out=False`` the call leaves the k/v columns of its output
    unwritten and only the cache receives them."""

    layer_cache: torch.Tensor
    kv_indices: torch.Tensor
    positions: torch.Tensor
    page_size: int
    kv_layout: str = "HND"
    kv_indptr: Optional[torch.Tensor] = None
    batch_indices: Optional[torch.Tensor] = None
    write_kv_out: bool = True

    def c_args(self, num_tokens: int, num_kv_heads: int, head_dim: int) -> tuple:
        """Checks the cache against the call's kv heads and returns the cache
        arguments of bfa_fused_rmsnorm_qkv_append (layer_cache .. write_kv_out)."""
        cache = self.layer_cache
        if self.kv_layout not in _LAYOUT_DIMS:
            raise ValueError(f"Unknown kv_layout: {self.kv_layout}")
        if cache.dim() != 5 or cache.shape[1] != 2:
            raise ValueError("layer_cache must be [num_pages, 2, ...] with 5 dimensions")
        hdim, sdim = _LAYOUT_DIMS[self.kv_layout]
        if cache.shape[hdim] != num_kv_heads or cache.shape[4] != head_dim:
            raise RuntimeError(f"layer_cache holds {cache.shape[hdim]} heads x {cache.shape[4]}, the "
                               f"call's k/v rows are {num_kv_heads} x {head_dim}")
        if cache.stride(-1) != 1:
            raise ValueError("layer_cache must have unit stride along head_dim")
        if num_tokens and self.page_size == 0:
            raise ZeroDivisionError("integer division or modulo by zero")
        if self.page_size < 0:
            raise ValueError("page_size must be positive")
        positions = self.positions.reshape(-1)
        if positions.numel() < num_tokens:
            raise IndexError(f"{positions.numel()} positions for {num_tokens} tokens")
        positions = positions[:num_tokens]
        if positions.dtype not in (torch.int32, torch.int64):
            positions = positions.long()
        if self.kv_indices.dim() > 1:
            raise ValueError("kv_indices must be one-dimensional")
        kv_indices = self.kv_indices.reshape(-1)
        if kv_indices.dtype not in (torch.int32, torch.int64):
            kv_indices = kv_indices.long()
        kv_indptr = batch_indices = None
        if self.kv_indptr is not None:
            if self.batch_indices is None:
                raise ValueError("a batched append needs batch_indices")
            kv_indptr = self.kv_indptr.reshape(-1).to(torch.int32).contiguous()
            batch_indices = self.batch_indices.reshape(-1)
            if batch_indices.dtype not in (torch.int32, torch.int64):
                batch_indices = batch_indices.long()
            if batch_indices.numel() < num_tokens:
                raise IndexError(f"{batch_indices.numel()} batch indices for {num_tokens} tokens")
            batch_indices = batch_indices[:num_tokens].contiguous()
        # keep the converted tensors alive until the call has been queued
        self._keep = (positions.contiguous(), kv_indices.contiguous(), kv_indptr, batch_indices)
        positions, kv_indices = self._keep[0], self._keep[1]
        _lib.require_device(cache, kv_indices, positions, kv_indptr, batch_indices)
        st = cache.stride()
        return (
            _lib.ptr(cache), _lib.dtype_code(cache), cache.shape[0], cache.shape[sdim],
            st[0], st[1], st[hdim], st[sdim],
            _lib.ptr(kv_indices), _lib.dtype_code(kv_indices), kv_indices.numel(),
            _lib.ptr(kv_indptr), _lib.ptr(batch_indices),
            _lib.dtype_code(batch_indices) if batch_indices is not None else 0,
            kv_indptr.numel() - 1 if kv_indptr is not None else 0,
            _lib.ptr(positions), _lib.dtype_code(positions), int(self.page_size),
            int(bool(self.write_kv_out)),
        )


def build_paged_kv_indices(
    page_tables: List[List[int]],
    seq_lens: List[int],
    page_size: int,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """CSR page indices for a batch of sequences: (kv_indices, kv_indptr,
    kv_last_page_len), int32 on the current ROCm device.  The last page of a
    sequence holds ``seq_len % page_size`` tokens, or a full page when that is 0
    and the sequence is not empty."""
    kv_indices: List[int] = []
    kv_indptr = [0]
    kv_last_page_len = []
    for page_table, seq_len in zip(page_tables, seq_lens):
        kv_indices.extend(page_table)
        kv_indptr.append(len(kv_indices))
        last = seq_len % page_size
        if last == 0 and seq_len > 0:
            last = page_size
        kv_last_page_len.append(last)
    dev = torch.device("cuda", torch.cuda.current_device())
    return (torch.tensor(kv_indices, dtype=torch.int32, device=dev),
            torch.tensor(kv_indptr, dtype=torch.int32, device=dev),
            torch.tensor(kv_last_page_len, dtype=torch.int32, device=dev))
