"""SiluAndMul on MI355X, mirroring braidinfer/layers/activation.py:6-13."""
from __future__ import annotations

import torch
from torch import nn

from .. import _lib


def silu_and_mul(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """y = silu(x[..., :I]) * x[..., I:], with the reference's two roundings."""
    shape = x.shape
    two_i = shape[-1]
    if two_i % 2:
        raise ValueError("last dimension must be even (gate | up)")
    inter = two_i // 2
    if x.dim() == 2 and x.stride(1) == 1:
        x2 = x
    else:
        x2 = x.reshape(-1, two_i)
        if x2.stride(-1) != 1:
            x2 = x2.contiguous()
    if not x2.is_cuda:
        _lib.require_device(x2)
    dev = x2.device
    if out is None:
        out = torch.empty(shape[:-1] + (inter,), dtype=x.dtype, device=dev)
        ostride = inter
    else:
        ostride = out.view(-1, inter).stride(0)
    rc = _SILU()(x2.data_ptr(), out.data_ptr(), _lib.dtype_code(x2), x2.shape[0], inter, x2.stride(0),
                 ostride, _lib.stream_of(dev))
    if rc < 0:
        _lib.raise_error(rc)
    return out


_silu_fn = None


def _SILU():
    global _silu_fn
    if _silu_fn is None:
        _silu_fn = _lib.entry("bfa_silu_and_mul")
    return _silu_fn


class SiluAndMul(nn.Module):

    def __init__(self):
        super().__init__()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return silu_and_mul(x)
