"""VocabParallelEmbedding on MI355X, mirroring braidinfer/layers/embed_head.py:14-29.

The gather is a byte copy (bit-exact).  Out-of-range ids: F.embedding raises
IndexError; ids held on the host are checked here and raise the same way, and
ids on the device are checked by the kernel, which writes a zero row and sets
the device status word (raised by braidinfer_amd.check_device_status()).
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _lib


def _ids_on(ids: torch.Tensor, num_embeddings: int, dev: torch.device) -> torch.Tensor:
    if ids.device.type == "cpu":
        if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= num_embeddings):
            raise IndexError("index out of range in self")
        ids = ids.to(dev, non_blocking=True)
    if ids.dtype not in (torch.int64, torch.int32):
        raise TypeError(f"embedding ids must be int32/int64, got {ids.dtype}")
    return ids.contiguous()


def embedding(ids: torch.Tensor, weight: torch.Tensor, scale: float | None = None) -> torch.Tensor:
    """F.embedding(ids, weight) [* scale, rounded like a torch scalar multiply]."""
    dev = _lib.require_device(weight)
    ids = _ids_on(ids, weight.shape[0], dev)
    if weight.stride(-1) != 1:
        weight = weight.contiguous()
    num, dim = weight.shape
    out = torch.empty(tuple(ids.shape) + (dim,), dtype=weight.dtype, device=dev)
    status = _lib.status_word(dev)
    if scale is None:
        _lib.call("bfa_embedding", _lib.ptr(weight), num, dim, weight.stride(0),
                  weight.element_size(), _lib.ptr(ids), _lib.dtype_code(ids), ids.numel(),
                  _lib.ptr(out), dim, _lib.ptr(status), _lib.stream_of(dev))
    else:
        _lib.call("bfa_embedding_scaled", _lib.ptr(weight), num, dim, weight.stride(0),
                  _lib.dtype_code(weight), _lib.ptr(ids), _lib.dtype_code(ids), ids.numel(),
                  _lib.ptr(out), dim, float(scale), _lib.ptr(status), _lib.stream_of(dev))
    return out


class VocabParallelEmbedding(nn.Module):
    """Vocabulary embedding layer for single GPU."""

    def __init__(self, num_embeddings: int, embedding_dim: int):
        super().__init__()
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        self.weight = nn.Parameter(torch.empty(num_embeddings, embedding_dim))
        self.weight.weight_loader = self.weight_loader

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        assert param.data.size() == loaded_weight.size()
        param.data.copy_(loaded_weight)

    def forward(self, x: torch.Tensor):
        return embedding(x, self.weight)
