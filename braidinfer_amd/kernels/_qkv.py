"""Shared launcher for the fused RMSNorm+QKV variants (bfa_fused_rmsnorm_qkv).

The four reference classes differ only in rounding points and output dtype
(braidinfer/kernels/fused_rmsnorm_qkv_{mixed_precision,production,minimal_f32,
with_bias}.py); each class module calls :func:`fused_rmsnorm_qkv` with its
own settings.  The optional q/k-norm and RoPE arguments fuse what the Qwen3 and
Llama attention forwards do with the kernel output (models/qwen3.py:257-309,
models/llama.py:169-205).
"""
from __future__ import annotations

import weakref

import torch

from .. import _lib

_OPERAND_DTYPES = (torch.bfloat16, torch.float16)


def head_dim_of(qkv_dim: int, num_q_heads: int, num_kv_heads: int) -> int:
    """head_dim = qkv_dim // (Hq + 2*Hkv), as every reference variant derives it."""
    return qkv_dim // (num_q_heads + 2 * num_kv_heads)


# Without the mixed rounding (the production and fp32 variants) the prefill
# projects x onto W * gamma (bfa_fold_rmsnorm_weight) and scales each row by
# 1 / rms, so no normalised operand is written.  The
# folded weight is made once per (weight, norm weight) pair and kept while both
# tensor objects are alive, with the same storage and version counter (an
# in-place update of either, or a new `.data`, makes the next call fold again).
# A write that bypasses torch's version counter (a raw-pointer kernel writing
# into the weight) needs clear_folded_weights().
_folded: dict = {}
# From 17 tokens: the column-pair decode kernel (17-64, shapes it takes) and the
# prefill projection's fused epilogue; fewer tokens fold the norm into their
# one decode launch already.
_FOLD_MIN_TOKENS = 17
_ERR_UNSUPPORTED = -2  # BFA_ERR_UNSUPPORTED: the folded entry does not take the shape


def _drop_folded(key, ref) -> None:
    ent = _folded.get(key)
    if ent is not None and (ent[0] is ref or ent[1] is ref):
        del _folded[key]


def folded_weight(w: torch.Tensor, norm_weight: torch.Tensor) -> torch.Tensor | None:
    """bf16(W * gamma) for (w, norm_weight), from the cache or folded now; None
    under graph capture when no folded copy exists yet (the caller then runs the
    unfolded path: a fold captured into a graph would be redone on every replay)."""
    key = (id(w), id(norm_weight))
    # storage, version counter and shape: a new `.data` or an in-place change
    # moves one of them
    state = (w.data_ptr(), w._version, w.shape, norm_weight.data_ptr(), norm_weight._version)
    ent = _folded.get(key)
    if ent is not None and ent[0]() is w and ent[1]() is norm_weight and ent[2] == state:
        return ent[3]
    if torch.cuda.is_current_stream_capturing():
        return None
    n, k = w.shape
    wf = torch.empty((n, k), dtype=w.dtype, device=w.device)
    _lib.call("bfa_fold_rmsnorm_weight", w.data_ptr(), _lib.dtype_code(w), n, k, w.stride(0),
              norm_weight.data_ptr(), _lib.dtype_code(norm_weight), wf.data_ptr(), wf.stride(0),
              _lib.stream_of(w.device))
    # once per pair: the fold is finished before any stream can read the copy
    torch.cuda.current_stream(w.device).synchronize()
    wr = weakref.ref(w, lambda r, key=key: _drop_folded(key, r))
    nr = weakref.ref(norm_weight, lambda r, key=key: _drop_folded(key, r))
    _folded[key] = (wr, nr, state, wf)
    return wf


def clear_folded_weights() -> int:
    """Drops every cached folded weight; returns how many there were."""
    n = len(_folded)
    _folded.clear()
    return n


def _matrix_weight(w: torch.Tensor) -> torch.Tensor:
    # The matrix cores take bf16 or fp16 operands.  An fp32 weight is rounded to
    # bf16, which is what the mixed/production Triton kernels do with every
    # weight tile (`weight_tile.to(tl.bfloat16)`).
    if w.dtype not in _OPERAND_DTYPES:
        w = w.to(torch.bfloat16)
    if w.stride(-1) != 1 or w.stride(0) % 8 != 0 or w.data_ptr() % 16 != 0:
        w = w.contiguous()
    return w


def fused_rmsnorm_qkv(
    input: torch.Tensor,
    norm_weight: torch.Tensor,
    qkv_weight: torch.Tensor,
    num_q_heads: int,
    num_kv_heads: int,
    eps: float,
    *,
    mixed_rounding: bool,
    qkv_dtype: torch.dtype,
    out_dtype: torch.dtype,
    qkv_bias: torch.Tensor | None = None,
    q_norm_weight: torch.Tensor | None = None,
    k_norm_weight: torch.Tensor | None = None,
    qk_norm_eps: float = 1e-6,
    qk_norm_out_dtype: torch.dtype | None = None,
    positions: torch.Tensor | None = None,
    cos_sin_cache: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    paged_kv=None,
) -> torch.Tensor:
    """Runs RMSNorm -> x @ W^T (+bias) [-> q/k RMSNorm] [-> RoPE] and returns the
    [tokens, qkv_dim] result (q | k | v columns) in `out_dtype`.  With
    ``paged_kv`` (a kv_cache_utils.PagedKVAppend) the k and v heads are also
    appended to that paged cache by the same call."""
    assert input.dim() == 2, f"Expected 2D input, got {input.dim()}D"
    tokens, hidden = input.shape
    qkv_dim = qkv_weight.shape[0]
    if input.stride(-1) != 1 or input.data_ptr() % 16 != 0:
        input = input.contiguous()
    orig_norm_weight = norm_weight
    if not norm_weight.is_contiguous():
        norm_weight = norm_weight.contiguous()
    w = _matrix_weight(qkv_weight)
    if qkv_bias is not None and not qkv_bias.is_contiguous():
        qkv_bias = qkv_bias.contiguous()
    dev = _lib.require_device(input, norm_weight, w, qkv_bias, q_norm_weight, k_norm_weight,
                              positions, cos_sin_cache)
    hd = head_dim_of(qkv_dim, num_q_heads, num_kv_heads)
    if q_norm_weight is not None and not q_norm_weight.is_contiguous():
        q_norm_weight = q_norm_weight.contiguous()
    if k_norm_weight is not None and not k_norm_weight.is_contiguous():
        k_norm_weight = k_norm_weight.contiguous()
    qn_dtype = (q_norm_weight if q_norm_weight is not None else k_norm_weight)
    if q_norm_weight is not None and k_norm_weight is not None and q_norm_weight.dtype != k_norm_weight.dtype:
        k_norm_weight = k_norm_weight.to(q_norm_weight.dtype)
    if cos_sin_cache is not None:
        if positions is None:
            raise ValueError("RoPE needs positions")
        if cos_sin_cache.dtype != torch.float32:
            raise TypeError("cos_sin_cache must be float32")
        if not cos_sin_cache.is_contiguous():
            cos_sin_cache = cos_sin_cache.contiguous()
        if cos_sin_cache.shape[-1] != hd:
            raise ValueError(f"cos_sin_cache width {cos_sin_cache.shape[-1]} != head_dim {hd}")
        if positions.dim() != 1:
            positions = positions.reshape(-1)
        if positions.numel() != tokens:
            raise ValueError(f"{positions.numel()} positions for {tokens} tokens")
        if positions.dtype not in (torch.int64, torch.int32):
            positions = positions.long()
        if not positions.is_contiguous():
            positions = positions.contiguous()
    if out is None:
        out = torch.empty((tokens, qkv_dim), dtype=out_dtype, device=dev)
    if paged_kv is not None:
        cache_args = paged_kv.c_args(tokens, num_kv_heads, hd)
    # the variants without the mixed rounding, at prefill: x projected onto the
    # folded weight (the unconverted weight and norm weight only, so that the
    # cache key is the caller's own tensors)
    # (decode counts: the column-pair kernel's shapes, bf16, at least 128 column
    # pairs; the C side has the last word and answers BFA_ERR_UNSUPPORTED otherwise)
    decode_ok = False
    if _FOLD_MIN_TOKENS <= tokens <= 64 and not mixed_rounding and input.dtype == torch.bfloat16 \
            and hd % 32 == 0 and hidden % 256 == 0:
        pair_mode = _lib.get_tuning("DECODE_PAIR")
        decode_ok = pair_mode != 0 and (qkv_dim // 32 >= 128 or pair_mode == 1)
    if (not mixed_rounding and tokens >= _FOLD_MIN_TOKENS
            and q_norm_weight is None and k_norm_weight is None
            and (decode_ok or (tokens > 64 and hd in (32, 64, 128)))
            and w is qkv_weight and norm_weight is orig_norm_weight and input.dtype == w.dtype
            and hidden % 8 == 0 and input.stride(0) % 8 == 0 and norm_weight.data_ptr() % 16 == 0
            and out.stride(-1) == 1 and out.stride(0) % 4 == 0 and out.data_ptr() % 16 == 0):
        wf = folded_weight(w, norm_weight)
        if wf is not None:
            size_fn = ("bfa_fused_rmsnorm_qkv_append_workspace_size" if paged_kv is not None
                       else "bfa_fused_rmsnorm_qkv_workspace_size")
            ws_bytes = _lib.workspace_size(size_fn, tokens, hidden, qkv_dim, hd)
            workspace = _lib.workspace(dev, ws_bytes)
            no_cache = (None, 0, 0, 0, 0, 0, 0, 0, None, 0, 0, None, None, 0, 0, None, 0, 0, 0)
            rc = _FOLDED()(
                input.data_ptr(), _lib.dtype_code(input), tokens, hidden, input.stride(0), float(eps),
                wf.data_ptr(), _lib.dtype_code(wf), qkv_dim, wf.stride(0),
                _lib.ptr(qkv_bias), _lib.dtype_code(qkv_bias) if qkv_bias is not None else 0,
                num_q_heads, num_kv_heads, _lib.dtype_code(qkv_dtype),
                _lib.ptr(positions), _lib.dtype_code(positions) if positions is not None else 0,
                _lib.ptr(cos_sin_cache), cos_sin_cache.shape[0] if cos_sin_cache is not None else 0,
                out.data_ptr(), _lib.dtype_code(out), out.stride(0),
                workspace.data_ptr(), workspace.numel(),
                *(cache_args if paged_kv is not None else no_cache),
                _lib.status_word(dev).data_ptr(), _lib.stream_of(dev),
            )
            if rc == 0:
                return out
            if rc != _ERR_UNSUPPORTED:
                _lib.raise_error(rc)
    if tokens == 0:
        return out
    if paged_kv is not None:
        ws_bytes = _lib.workspace_size("bfa_fused_rmsnorm_qkv_append_workspace_size", tokens, hidden,
                                       qkv_dim, hd)
        workspace = _lib.workspace(dev, ws_bytes)
        _lib.call(
            "bfa_fused_rmsnorm_qkv_append",
            input.data_ptr(), _lib.dtype_code(input), tokens, hidden, input.stride(0),
            norm_weight.data_ptr(), _lib.dtype_code(norm_weight), float(eps), int(mixed_rounding),
            w.data_ptr(), _lib.dtype_code(w), qkv_dim, w.stride(0),
            _lib.ptr(qkv_bias), _lib.dtype_code(qkv_bias) if qkv_bias is not None else 0,
            num_q_heads, num_kv_heads, _lib.dtype_code(qkv_dtype),
            _lib.ptr(q_norm_weight), _lib.ptr(k_norm_weight),
            _lib.dtype_code(qn_dtype) if qn_dtype is not None else 0, float(qk_norm_eps),
            _lib.dtype_code(qk_norm_out_dtype or input.dtype),
            _lib.ptr(positions), _lib.dtype_code(positions) if positions is not None else 0,
            _lib.ptr(cos_sin_cache), cos_sin_cache.shape[0] if cos_sin_cache is not None else 0,
            out.data_ptr(), _lib.dtype_code(out), out.stride(0),
            workspace.data_ptr(), workspace.numel(), *cache_args,
            _lib.status_word(dev).data_ptr(), _lib.stream_of(dev),
        )
        return out
    ws_bytes = _lib.workspace_size("bfa_fused_rmsnorm_qkv_workspace_size", tokens, hidden, qkv_dim, hd)
    workspace = _lib.workspace(dev, ws_bytes)
    rc = _FUSED()(
        input.data_ptr(), _lib.dtype_code(input), tokens, hidden, input.stride(0),
        norm_weight.data_ptr(), _lib.dtype_code(norm_weight), float(eps), int(mixed_rounding),
        w.data_ptr(), _lib.dtype_code(w), qkv_dim, w.stride(0),
        _lib.ptr(qkv_bias), _lib.dtype_code(qkv_bias) if qkv_bias is not None else 0,
        num_q_heads, num_kv_heads, _lib.dtype_code(qkv_dtype),
        _lib.ptr(q_norm_weight), _lib.ptr(k_norm_weight),
        _lib.dtype_code(qn_dtype) if qn_dtype is not None else 0, float(qk_norm_eps),
        _lib.dtype_code(qk_norm_out_dtype or input.dtype),
        _lib.ptr(positions), _lib.dtype_code(positions) if positions is not None else 0,
        _lib.ptr(cos_sin_cache), cos_sin_cache.shape[0] if cos_sin_cache is not None else 0,
        out.data_ptr(), _lib.dtype_code(out), out.stride(0),
        workspace.data_ptr(), workspace.numel(),
        _lib.status_word(dev).data_ptr(), _lib.stream_of(dev),
    )
    if rc < 0:
        _lib.raise_error(rc)
    return out


_fused_fn = None


def _FUSED():
    global _fused_fn
    if _fused_fn is None:
        _fused_fn = _lib.entry("bfa_fused_rmsnorm_qkv")
    return _fused_fn


_folded_fn = None


def _FOLDED():
    global _folded_fn
    if _folded_fn is None:
        _folded_fn = _lib.entry("bfa_fused_rmsnorm_qkv_folded")
    return _folded_fn


def split_heads(output: torch.Tensor, num_q_heads: int, num_kv_heads: int):
    """Splits the [T, qkv_dim] buffer into q/k/v views of shape [T, heads, head_dim]
    (the split/view sequence of the reference variants)."""
    tokens, qkv_dim = output.shape
    hd = head_dim_of(qkv_dim, num_q_heads, num_kv_heads)
    q, k, v = output.split([num_q_heads * hd, num_kv_heads * hd, num_kv_heads * hd], dim=-1)
    return (q.view(tokens, num_q_heads, hd), k.view(tokens, num_kv_heads, hd),
            v.view(tokens, num_kv_heads, hd))
