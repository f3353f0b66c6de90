"""RMSNormF32 on MI355X.

Mirrors braidinfer/kernels/rmsnorm_f32.py:99-156: per row
rms = sqrt(sum(x^2)/H + eps), out = (x / rms) * weight, all in fp32, written
to a new fp32 tensor or to the caller's `output` buffer (which is returned).
"""
from __future__ import annotations

from typing import Optional

import torch

from .. import _lib


class RMSNormF32:
    """Standalone RMSNorm with full float32 precision."""

    @staticmethod
    def forward(
        input: torch.Tensor,
        norm_weight: torch.Tensor,
        eps: float = 1e-6,
        output: Optional[torch.Tensor] = None,
    ) -> torch.Tensor:
        assert input.dim() == 2, f"Expected 2D input, got {input.dim()}D"
        seq_len, hidden_dim = input.shape
        if output is None:
            output = torch.empty_like(input, dtype=torch.float32)
        else:
            assert output.dtype == torch.float32, "Output must be float32"
            assert output.shape == input.shape, "Output shape must match input"
        norm_weight = norm_weight.contiguous()
        dev = _lib.require_device(input, norm_weight, output)
        _lib.call(
            "bfa_rms_norm_f32", _lib.ptr(input), _lib.ptr(output), _lib.ptr(norm_weight),
            _lib.dtype_code(input), _lib.dtype_code(norm_weight), seq_len, hidden_dim,
            input.stride(0), input.stride(1), output.stride(0), output.stride(1), float(eps),
            _lib.stream_of(dev))
        return output
