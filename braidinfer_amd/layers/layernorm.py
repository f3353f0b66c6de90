"""RMSNorm on MI355X, mirroring braidinfer/layers/layernorm.py:23-67.

Same module interface (weight Parameter initialised to ones, eps default
1e-6, forward(x, residual=None)) and the same aliasing: for an fp32 input the
reference normalises x in place and returns it (the `.to(float32)` calls are
no-ops), and add_rms_forward then returns that same tensor twice.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _lib


def _row_geometry(x: torch.Tensor):
    """(rows, rows_inner, stride_outer, stride_inner) of x seen as rows of its
    last dimension, or None when the layout needs a copy."""
    if x.stride(-1) != 1 and x.shape[-1] > 1:
        return None
    hidden = x.shape[-1]
    if x.dim() == 1:
        return 1, 1, hidden, 0
    if x.is_contiguous():
        return x.numel() // max(hidden, 1), 1, hidden, 0
    if x.dim() == 2:
        return x.shape[0], 1, x.stride(0), 0
    if x.dim() == 3:
        return x.shape[0] * x.shape[1], x.shape[1], x.stride(0), x.stride(1)
    return None


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, out: torch.Tensor | None = None):
    """RMSNorm.rms_forward (layernorm.py:35-44).  Writes a new tensor, or x
    itself when out is x (the fp32 in-place form)."""
    weight = weight.contiguous()
    dev = _lib.require_device(x, weight)
    hidden = x.shape[-1]
    src = x
    geo = _row_geometry(x)
    if geo is None:
        src = x.contiguous()
        geo = _row_geometry(src)
    rows, inner, so, si = geo
    if out is x and src is x:
        oso, osi = so, si
    else:
        if out is None:
            out = torch.empty(src.shape, dtype=src.dtype, device=dev)
        assert out.is_contiguous() and out.shape == src.shape
        oso, osi = inner * hidden, hidden
    _lib.call("bfa_rms_norm", _lib.ptr(src), _lib.ptr(out), _lib.ptr(weight),
              _lib.dtype_code(src), _lib.dtype_code(weight), rows, inner, hidden,
              so, si, oso, osi, float(eps), _lib.stream_of(dev))
    return out


_add_rms_fn = None


def _ADD_RMS():
    global _add_rms_fn
    if _add_rms_fn is None:
        _add_rms_fn = _lib.entry("bfa_add_rms_norm")
    return _add_rms_fn


class RMSNorm(nn.Module):

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.hidden_size = hidden_size
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def rms_forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype == torch.float32:
            if _row_geometry(x) is not None:
                return rms_norm(x, self.weight, self.eps, out=x)
            y = rms_norm(x, self.weight, self.eps)
            x.copy_(y)
            return x
        return rms_norm(x, self.weight, self.eps)

    def add_rms_forward(self, x: torch.Tensor, residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        # common case first: 16-bit x and residual of one contiguous shape on one device
        if ((x.dtype == torch.bfloat16 or x.dtype == torch.float16) and x.is_cuda and x.is_contiguous()
                and residual.is_contiguous()
                and residual.shape == x.shape and residual.dtype == x.dtype and residual.device == x.device):
            weight = self.weight
            if weight.is_cuda and weight.is_contiguous() and weight.device == x.device:
                hidden = x.shape[-1]
                y = torch.empty_like(x)
                res_out = torch.empty_like(x)
                code = _lib.DTYPE_CODE[x.dtype]
                rc = _ADD_RMS()(x.data_ptr(), residual.data_ptr(), y.data_ptr(), res_out.data_ptr(),
                                weight.data_ptr(), code, _lib.dtype_code(weight), x.numel() // hidden, hidden,
                                hidden, hidden, hidden, hidden, float(self.eps), _lib.stream_of(x.device))
                if rc < 0:
                    _lib.raise_error(rc)
                return y, res_out
        hidden = x.shape[-1]
        weight = self.weight
        if not weight.is_contiguous():
            weight = weight.contiguous()
        if x.is_cuda and residual.is_cuda and weight.is_cuda and x.device == residual.device == weight.device:
            dev = x.device
        else:
            dev = _lib.require_device(x, residual, weight)
        inplace = x.dtype == torch.float32
        # 2-D row views (views of x itself when its layout allows, so the fp32
        # in-place form writes through to the caller's tensor)
        x2 = x.view(-1, hidden) if x.is_contiguous() else (x if x.dim() == 2 and x.stride(-1) == 1 else None)
        work = x2 if x2 is not None else x.reshape(-1, hidden).contiguous()
        r2 = residual.reshape(-1, hidden)
        if r2.stride(-1) != 1:
            r2 = r2.contiguous()
        rows = work.shape[0]
        if inplace:
            # reference: x.add_(residual); residual = x (same tensor); x is then
            # normalised in place and returned twice
            _lib.call("bfa_add_rms_norm", _lib.ptr(work), _lib.ptr(r2), _lib.ptr(work), None,
                      _lib.ptr(weight), _lib.dtype_code(work), _lib.dtype_code(weight), rows,
                      hidden, work.stride(0), r2.stride(0), work.stride(0), 0, float(self.eps),
                      _lib.stream_of(dev))
            if x2 is None:
                x.copy_(work.view(x.shape))
            return x, x
        y = torch.empty(x.shape, dtype=x.dtype, device=dev)
        res_out = torch.empty(x.shape, dtype=x.dtype, device=dev)
        rc = _ADD_RMS()(work.data_ptr(), r2.data_ptr(), y.data_ptr(), res_out.data_ptr(), weight.data_ptr(),
                        _lib.dtype_code(work), _lib.dtype_code(weight), rows, hidden, work.stride(0),
                        r2.stride(0), hidden, hidden, float(self.eps), _lib.stream_of(dev))
        if rc < 0:
            _lib.raise_error(rc)
        return y, res_out

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        if residual is None:
            return self.rms_forward(x)
        return self.add_rms_forward(x, residual)
