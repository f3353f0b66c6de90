"""FusedRMSNormQKV on MI355X.

Mirrors braidinfer/kernels/fused_rmsnorm_qkv_production.py:142-229:
n = bf16((x / rms) * weight) computed in fp32, n @ W^T in bf16 with fp32
accumulation, bf16 output.  Returns q, k, v as views of one [T, qkv_dim]
bf16 buffer.
"""
from __future__ import annotations

from typing import Tuple

import torch

from ._qkv import fused_rmsnorm_qkv, split_heads


class FusedRMSNormQKV:
    """Fused RMSNorm + QKV projection (bf16 output)."""

    @staticmethod
    def forward(
        input: torch.Tensor,
        norm_weight: torch.Tensor,
        qkv_weight: torch.Tensor,
        num_q_heads: int,
        num_kv_heads: int,
        eps: float = 1e-6,
    ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        out = fused_rmsnorm_qkv(
            input, norm_weight, qkv_weight, num_q_heads, num_kv_heads, eps,
            mixed_rounding=False, qkv_dtype=torch.bfloat16, out_dtype=torch.bfloat16)
        return split_heads(out, num_q_heads, num_kv_heads)
