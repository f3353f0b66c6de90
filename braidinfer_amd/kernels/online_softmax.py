"""Online softmax state update on MI355X, under the name of
braidinfer/kernels/online_softmax.py (``online_softmax_update``, :214-297).

Updates the running maximum ``m_i``, sum ``l_i`` and accumulator ``acc_i``
(fp32, in place) of every (head, query) with a block of keys taken in order,
exactly the recurrence of the reference kernel (:80-125):
``m' = max(m, s)``, ``l = l e^(m-m') + e^(s-m')``, ``acc = acc e^(m-m') + e^(s-m') v``
with ``s = (q . k) * scale`` and keys past the query's position skipped when
causal.  The state tensors are updated where they are (any strides), which is
what the reference's callers expect of it.
"""
from __future__ import annotations

import torch

from .. import _lib


def online_softmax_update(
    query: torch.Tensor,            # [num_heads, batch_size, head_dim]
    key: torch.Tensor,              # [num_heads, num_tokens, head_dim]
    value: torch.Tensor,            # [num_heads, num_tokens, head_dim]
    m_i: torch.Tensor,              # [num_heads, batch_size] fp32, updated in place
    l_i: torch.Tensor,              # [num_heads, batch_size] fp32, updated in place
    acc_i: torch.Tensor,            # [num_heads, batch_size, head_dim] fp32, updated in place
    query_positions: torch.Tensor,  # [batch_size]
    key_positions: torch.Tensor,    # [num_tokens]
    scale: float,
    apply_causal_mask: bool = True,
) -> None:
    assert query.dim() == 3 and key.dim() == 3 and value.dim() == 3
    assert query.shape[0] == key.shape[0] == value.shape[0]  # num_heads
    assert query.shape[2] == key.shape[2] == value.shape[2]  # head_dim
    assert key.shape[1] == value.shape[1]  # num_tokens
    assert query_positions.shape[0] == query.shape[1]  # batch_size
    assert key_positions.shape[0] == key.shape[1]  # num_tokens
    for name, t in (("m_i", m_i), ("l_i", l_i), ("acc_i", acc_i)):
        if t.dtype != torch.float32:
            raise TypeError(f"{name} must be float32")
    num_heads, batch, head_dim = query.shape
    num_tokens = key.shape[1]
    if key.dtype != value.dtype:
        value = value.to(key.dtype)
    query = query if query.stride(-1) == 1 else query.contiguous()
    key = key if key.stride(-1) == 1 else key.contiguous()
    value = value if value.stride(-1) == 1 else value.contiguous()
    if acc_i.stride(-1) != 1:
        raise ValueError("acc_i must have unit stride along head_dim")
    qpos = query_positions.contiguous()
    kpos = key_positions.contiguous()
    if qpos.dtype not in (torch.int32, torch.int64):
        qpos = qpos.long()
    if kpos.dtype not in (torch.int32, torch.int64):
        kpos = kpos.long()
    dev = _lib.require_device(query, key, value, m_i, l_i, acc_i, qpos, kpos)
    _lib.call(
        "bfa_online_softmax_update",
        _lib.ptr(query), _lib.ptr(key), _lib.ptr(value), _lib.dtype_code(query),
        _lib.dtype_code(key), _lib.ptr(m_i), _lib.ptr(l_i), _lib.ptr(acc_i),
        _lib.ptr(qpos), _lib.dtype_code(qpos), _lib.ptr(kpos), _lib.dtype_code(kpos),
        num_heads, batch, num_tokens, head_dim,
        query.stride(0), query.stride(1), key.stride(0), key.stride(1),
        value.stride(0), value.stride(1), m_i.stride(0), m_i.stride(1),
        l_i.stride(0), l_i.stride(1), acc_i.stride(0), acc_i.stride(1),
        float(scale), int(bool(apply_causal_mask)), _lib.stream_of(dev),
    )
