"""Fused attention output projection (+ residual) on MI355X, under the names of
braidinfer/kernels/fused_attention_output.py.

``FusedAttentionOutput.gemv(x, W)`` = x W^T and ``FusedAttentionOutput.forward
(x, W, residual)`` = x W^T + residual, each accumulated in fp32 and stored
through an fp16 rounding (the reference kernels store ``acc.to(tl.float16)``
into an output of x's dtype, :72, :134), one GEMM launch with the epilogue
fused.  The class keeps the reference's shape checks (one token, :159-160,
:195); ``attention_output`` / ``attention_output_gemv`` take any number of
tokens.
"""
from __future__ import annotations

import torch

from .. import _lib
from ..layers.linear import _run


def attention_output_gemv(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """x W^T (fp32 accumulation) rounded to fp16, then to x's dtype; x [..., M],
    weight [N, M]."""
    return _run(x, weight.detach(), weight.shape[0], _lib.LINEAR_PLAIN, proj_dtype=_lib.F32,
                sum_dtype=_lib.F16)


def attention_output(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
    """x W^T + residual, in fp32, rounded to fp16, then to x's dtype."""
    return _run(x, weight.detach(), weight.shape[0], _lib.LINEAR_PLAIN, residual=residual,
                proj_dtype=_lib.F32, sum_dtype=_lib.F16)


class FusedAttentionOutput:
    """Fused attention output projection and residual addition (:137-225)."""

    @staticmethod
    def gemv(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        """x [1, M], weight [N, M] -> [1, N] (:139-171)."""
        batch_size, m = x.shape
        n = weight.shape[0]
        assert batch_size == 1, "This kernel is optimized for batch size 1"
        assert weight.shape == (n, m), f"Weight shape mismatch: expected ({n}, {m}), got {weight.shape}"
        return attention_output_gemv(x, weight)

    @staticmethod
    def forward(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        """x [1, 1, H], weight [H, H], residual [1, 1, H] -> [1, 1, H] (:173-225)."""
        batch_size, seq_len, hidden_size = x.shape
        assert batch_size == 1 and seq_len == 1, "Currently optimized for decode phase"
        y = attention_output(x.view(-1, hidden_size), weight, residual.view(-1, hidden_size))
        return y.view(batch_size, seq_len, hidden_size)
