"""Paged cascade attention on MI355X, mirroring braidinfer/layers/cascade_attention.py.

``CascadeAttention.forward`` keeps the reference's signature and result: the
online-softmax attention of every query over the pages of every chunk of every
cascade level, with the per-chunk differential RoPE of the cached K and the
optional k_norm (cascade_attention.py:50-231).  The reference walks pages in a
Python loop with host syncs and about a dozen launches per 16-token page; here
the whole walk is one ``bfa_cascade_attention`` launch (two when the key range
is split for a small query count).  ``CascadeLevel``, ``create_cascade_levels``
and ``_create_level`` restate the reference's host-side level construction
(:19-25, :234-293).
"""
from __future__ import annotations

import weakref
from collections import OrderedDict
from dataclasses import dataclass, field
from typing import List

import numpy as np
import torch

from .. import _lib


@dataclass
class CascadeLevel:
    """One level of the cascade hierarchy (cascade_attention.py:19-25)."""
    chunks: list
    kv_page_indices: torch.Tensor  # [E] int32, the pages of every chunk in order
    kv_page_indptr: torch.Tensor   # [num_chunks + 1] int32
    kv_last_page_len: torch.Tensor  # [num_chunks] int32
    position_offset: int
    # host copies of the three tensors, with a stamp of the tensors they were
    # taken from (written by _create_level, or by the first forward that reads
    # the tensors); a stale stamp makes the next forward read the tensors again
    host_arrays: object = field(default=None, repr=False, compare=False)


def _stamp(level: CascadeLevel):
    """Identity of a level's three tensors: the objects, their storage and their
    version counters (an in-place write moves the counter, an assignment of
    another tensor changes the object)."""
    ts = (level.kv_page_indices, level.kv_page_indptr, level.kv_last_page_len)
    return tuple((weakref.ref(t), t.data_ptr(), t._version) for t in ts), ts


def _stamp_matches(stamp, ts) -> bool:
    return all(r() is t and p == t.data_ptr() and v == t._version for (r, p, v), t in zip(stamp, ts))


def _level_arrays(level: CascadeLevel):
    """(page indices, indptr, last page lengths) of a level as int64 numpy
    arrays, read from the device only when the host copy is missing or stale."""
    ts = (level.kv_page_indices, level.kv_page_indptr, level.kv_last_page_len)
    host = level.host_arrays
    if host is not None and _stamp_matches(host[3], ts):
        return host[:3]
    arrs = tuple(t.reshape(-1).cpu().numpy().astype(np.int64) for t in ts)
    level.host_arrays = arrs + (_stamp(level)[0],)
    return arrs


class CascadeAttention:
    """Cascade attention over the paged KV cache (cascade_attention.py:28-48)."""

    def __init__(self, num_heads: int, head_dim: int, scale: float, num_kv_heads: int,
                 page_size: int = 16, rotary_emb=None):
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.page_size = page_size
        self.heads_per_kv = num_heads // num_kv_heads
        self.rotary_emb = rotary_emb

    # Device plans shared by every CascadeAttention of the process, keyed by
    # content (device, page size, the levels' page arrays, the chunk metadata):
    # each layer of a forward pass builds its own levels from the same chunks,
    # and all of them find the first layer's plan.  Plans used while a HIP
    # graph is being captured are pinned (never evicted), since the graph reads
    # them on every replay; release_pinned_plans() drops them.
    _plans: "OrderedDict" = OrderedDict()
    _pinned: dict = {}
    _MAX_PLANS = 64

    @classmethod
    def release_pinned_plans(cls) -> None:
        """Forgets the plans pinned by graph captures (call once the graphs that
        captured cascade attention are destroyed)."""
        cls._pinned.clear()

    def forward(self, query: torch.Tensor, query_positions: torch.Tensor, kv_cache: torch.Tensor,
                cascade_levels: List[CascadeLevel], layer_idx: int, causal_mask: bool = True,
                k_norm=None) -> torch.Tensor:
        """Returns [num_tokens, num_heads * head_dim] in the query dtype.

        kv_cache: this layer's paged cache [num_pages, 2, num_kv_heads, page_size, head_dim]
        (K at index 0), as the reference indexes it.  layer_idx is accepted for
        signature parity (the reference does not use it either)."""
        hd = self.num_heads * self.head_dim
        if query.dim() == 1:
            if query.shape[0] % hd != 0:
                raise ValueError(f"Query size {query.shape[0]} not divisible by num_heads*head_dim={hd}")
            query = query.view(query.shape[0] // hd, self.num_heads, self.head_dim)
        elif query.dim() == 2:
            if query.shape[1] != hd:
                raise ValueError(f"query rows have {query.shape[1]} elements, num_heads*head_dim={hd}")
            query = query.view(query.shape[0], self.num_heads, self.head_dim)
        elif query.dim() != 3:
            raise ValueError(f"Unexpected query shape: {query.shape}")
        elif tuple(query.shape[1:]) != (self.num_heads, self.head_dim):
            raise ValueError(f"query of shape {tuple(query.shape)} does not match "
                             f"[tokens, {self.num_heads}, {self.head_dim}]")
        tokens = query.shape[0]
        if query.stride(-1) != 1 or query.stride(1) % 8 or query.stride(0) % 8 or query.data_ptr() % 16:
            query = query.contiguous()
        if kv_cache.dim() != 5 or kv_cache.shape[1] != 2:
            raise ValueError("kv_cache must be one layer [num_pages, 2, num_kv_heads, page_size, head_dim]")
        num_pages, _, hkv, cache_ps, d = kv_cache.shape
        if hkv != self.num_kv_heads or d != self.head_dim:
            raise ValueError("kv_cache heads / head_dim do not match the layer")
        if kv_cache.dtype != query.dtype:
            raise TypeError("query and kv_cache must share a dtype")
        dev = _lib.require_device(query, kv_cache, query_positions)
        out = torch.empty(tokens, hd, dtype=query.dtype, device=dev)
        if tokens == 0:
            return out

        if cache_ps < self.page_size:
            raise ValueError(f"kv_cache pages hold {cache_ps} slots, fewer than page_size={self.page_size}")
        meta = self._chunk_meta(cascade_levels)
        e_page, e_kstart, e_delta, e_info = self._plan(cascade_levels, meta, dev)
        entries = 0 if e_page is None else e_page.numel()

        cs = None
        max_pos = 0
        if entries and self.rotary_emb is not None and any(m[2] & 2 for m in meta):
            cs = self.rotary_emb.cos_sin_cache
            if cs.dtype != torch.float32 or cs.shape[-1] != d:
                raise ValueError("rotary_emb.cos_sin_cache must be float32 [max_position, head_dim]")
            cs = cs.contiguous()
            max_pos = cs.shape[0]
        kn_w, kn_dt, kn_eps = None, 0, 0.0
        if k_norm is not None:
            kn_w = k_norm.weight.detach()
            if kn_w.numel() != d:
                raise ValueError("k_norm weight must have head_dim elements")
            kn_w = kn_w.contiguous()
            kn_dt = _lib.dtype_code(kn_w)
            kn_eps = float(getattr(k_norm, "eps", getattr(k_norm, "variance_epsilon", 1e-6)))
        qpos = query_positions.reshape(-1)
        if qpos.numel() < tokens:
            raise IndexError(f"{qpos.numel()} query positions for {tokens} tokens")
        qpos = qpos[:tokens].contiguous()
        if qpos.dtype not in (torch.int32, torch.int64):
            qpos = qpos.long()
        ws_bytes = _lib.workspace_size("bfa_cascade_attention_workspace_size", tokens, self.num_heads, hkv, d,
                                       entries, self.page_size)
        ws = _lib.workspace(dev, ws_bytes)
        st = kv_cache.stride()
        _lib.call(
            "bfa_cascade_attention",
            _lib.ptr(query), _lib.dtype_code(query), tokens, self.num_heads,
            query.stride(0), query.stride(1), _lib.ptr(qpos), _lib.dtype_code(qpos),
            _lib.ptr(kv_cache), num_pages, hkv, self.page_size, d, st[0], st[1], st[2], st[3],
            entries, _lib.ptr(e_page), _lib.ptr(e_kstart), _lib.ptr(e_delta), _lib.ptr(e_info),
            _lib.ptr(cs), max_pos, _lib.ptr(kn_w), kn_dt, kn_eps,
            float(self.scale), int(bool(causal_mask)), _lib.ptr(out), out.stride(0),
            _lib.ptr(ws), ws.numel(), _lib.ptr(_lib.status_word(dev)), _lib.stream_of(dev),
        )
        return out

    __call__ = forward

    def _chunk_meta(self, cascade_levels):
        """(delta, first key position, flags) of every chunk in the reference's walk
        order (:119-224); attended chunks (pages and kv_length != 0) advance the key
        position by their kv_length.  flags bit 0: attended, bit 1: K is rotated
        (a rotary table, a global_position_start and a nonzero delta, :148-170)."""
        meta, cumulative = [], 0
        for level in cascade_levels:
            for chunk in level.chunks:
                attended = bool(chunk.page_table) and chunk.kv_length != 0
                cached = getattr(chunk, "cached_position_start", 0)
                glob = getattr(chunk, "global_position_start", cached)
                delta = glob - cached
                rotate = self.rotary_emb is not None and hasattr(chunk, "global_position_start") and delta != 0
                meta.append((delta, cumulative, int(attended) | (int(rotate) << 1)))
                if attended:
                    cumulative += chunk.kv_length
        return meta

    def _plan(self, cascade_levels, meta, dev):
        """Per-entry arrays of the attended pages, in the reference's walk order:
        page id (int32), key position of slot 0 (int64), the chunk's delta (int64)
        and tokens | rotate << 16 (int32).  Each chunk's pages are
        kv_page_indices[indptr[c]:indptr[c+1]], its last page holds
        kv_last_page_len[c] tokens and the others page_size (:124-137); pages with
        no tokens are dropped.  The level arrays come from their host copies
        (no device read when _create_level built the level or an earlier call
        read it), and the device arrays are shared by content across layers and
        instances, so only the first layer of a forward pass copies to the
        device, and a call with a cached plan can be captured in a HIP graph."""
        ps = self.page_size
        arrays = [_level_arrays(lv) if lv.chunks else None for lv in cascade_levels]
        key = (str(dev), ps, tuple(meta),
               tuple(None if a is None else (a[0].tobytes(), a[1].tobytes(), a[2].tobytes()) for a in arrays))
        cls = type(self)
        plan = cls._pinned.get(key)
        if plan is None:
            plan = cls._plans.get(key)
            if plan is not None:
                cls._plans.move_to_end(key)
        if plan is None:
            plan = self._build_plan(cascade_levels, arrays, meta, dev)
            cls._plans[key] = plan
            while len(cls._plans) > cls._MAX_PLANS:
                cls._plans.popitem(last=False)
        if dev.type == "cuda" and torch.cuda.is_current_stream_capturing():
            cls._pinned[key] = plan
        return plan

    def _build_plan(self, cascade_levels, arrays, meta, dev):
        ps = self.page_size
        pages, kstart, delta, info = [], [], [], []
        ci = 0
        for level, arrs in zip(cascade_levels, arrays):
            n = len(level.chunks)
            if n == 0:
                continue
            idx, ptr, last = arrs
            if ptr.shape[0] < n + 1 or last.shape[0] < n:
                raise ValueError(f"level with {n} chunks has {ptr.shape[0]} indptr entries and "
                                 f"{last.shape[0]} last-page lengths")
            for c in range(n):
                dlt, cum, flags = meta[ci + c]
                if not flags & 1:
                    continue
                chunk_pages = idx[int(ptr[c]):int(ptr[c + 1])]
                k = chunk_pages.shape[0]
                if k == 0:
                    continue
                tok = np.full(k, ps, dtype=np.int64)
                tok[-1] = last[c]
                if tok[-1] > ps:
                    raise ValueError(f"kv_last_page_len {int(tok[-1])} exceeds page_size={ps}")
                keep = tok > 0
                pages.append(chunk_pages[keep])
                kstart.append(cum + ps * np.arange(k, dtype=np.int64)[keep])
                delta.append(np.full(int(keep.sum()), dlt, dtype=np.int64))
                info.append(tok[keep] | ((flags >> 1) & 1) << 16)
            ci += n
        if pages and sum(p.shape[0] for p in pages):
            cat = np.concatenate
            return (torch.from_numpy(cat(pages).astype(np.int32)).to(dev),
                    torch.from_numpy(cat(kstart)).to(dev),
                    torch.from_numpy(cat(delta)).to(dev),
                    torch.from_numpy(cat(info).astype(np.int32)).to(dev))
        return (None,) * 4

    def create_cascade_levels(self, chunks, page_manager=None) -> List[CascadeLevel]:
        """Two levels: system-prompt chunks, then every other chunk
        (cascade_attention.py:234-261)."""
        levels = []
        system_chunks = [c for c in chunks if c.chunk_type.value == "system_prompt"]
        other_chunks = [c for c in chunks if c.chunk_type.value != "system_prompt"]
        if system_chunks:
            levels.append(self._create_level(system_chunks, position_offset=0))
        if other_chunks:
            prev_tokens = sum(c.kv_length for c in system_chunks)
            levels.append(self._create_level(other_chunks, position_offset=prev_tokens))
        return levels

    def _create_level(self, chunks, position_offset: int) -> CascadeLevel:
        """Page indices, CSR pointers and last-page lengths of a level's chunks
        (cascade_attention.py:263-293): a one-page chunk's last page holds
        kv_length tokens; otherwise kv_length % page_size, or a full page when that
        is 0 and the chunk is not empty."""
        all_page_indices, page_indptr, last_page_lens = [], [0], []
        for chunk in chunks:
            if chunk.page_table:
                all_page_indices.extend(chunk.page_table)
                page_indptr.append(len(all_page_indices))
                if len(chunk.page_table) == 1:
                    last_page_len = chunk.kv_length
                else:
                    last_page_len = chunk.kv_length % self.page_size
                    if last_page_len == 0 and chunk.kv_length > 0:
                        last_page_len = self.page_size
                last_page_lens.append(last_page_len)
            else:
                page_indptr.append(len(all_page_indices))
                last_page_lens.append(0)
        dev = torch.device("cuda", torch.cuda.current_device())
        level = CascadeLevel(
            chunks=chunks,
            kv_page_indices=torch.tensor(all_page_indices, dtype=torch.int32, device=dev),
            kv_page_indptr=torch.tensor(page_indptr, dtype=torch.int32, device=dev),
            kv_last_page_len=torch.tensor(last_page_lens, dtype=torch.int32, device=dev),
            position_offset=position_offset,
        )
        # the host lists are at hand: keep them so forward reads nothing back
        level.host_arrays = (np.asarray(all_page_indices, dtype=np.int64), np.asarray(page_indptr, dtype=np.int64),
                             np.asarray(last_page_lens, dtype=np.int64), _stamp(level)[0])
        return level
