"""SiluAndMul on MI355X, mirroring braidinfer/layers/activation.py:6-13."""
from __future__ import annotations

import torch
from torch import nn

from .. import _lib


def silu_and_mul(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """y = silu(x[..., :I]) * x[..., I:], with the reference's two roundings."""
    two_i = x.shape[-1]
    if two_i % 2:
        raise ValueError("last dimension must be even (gate | up)")
    inter = two_i // 2
    x2 = x if (x.dim() == 2 and x.stride(-1) == 1) else x.reshape(-1, two_i)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    dev = _lib.require_device(x2)
    if out is None:
        out = torch.empty(x.shape[:-1] + (inter,), dtype=x.dtype, device=dev)
    o2 = out.view(-1, inter)
    _lib.call("bfa_silu_and_mul", _lib.ptr(x2), _lib.ptr(o2), _lib.dtype_code(x2), x2.shape[0],
              inter, x2.stride(0), o2.stride(0), _lib.stream_of(dev))
    return out


class SiluAndMul(nn.Module):

    def __init__(self):
        super().__init__()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return silu_and_mul(x)
