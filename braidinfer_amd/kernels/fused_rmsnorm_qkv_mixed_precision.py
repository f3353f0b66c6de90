"""FusedRMSNormQKVMixedPrecision on MI355X.

Mirrors braidinfer/kernels/fused_rmsnorm_qkv_mixed_precision.py:151-247 (the
variant Qwen3 uses, models/qwen3.py:236-246): variance in fp32,
n = bf16(x / rms) * weight in bf16, n @ W^T with fp32 accumulation, bias added
in fp32, result rounded to bf16 and stored in the input dtype.  Returns q, k,
v as views of one [T, qkv_dim] buffer, like the reference.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from ._qkv import fused_rmsnorm_qkv, split_heads


class FusedRMSNormQKVMixedPrecision:
    """Fused RMSNorm + QKV with mixed precision matching the standard path."""

    @staticmethod
    def forward(
        input: torch.Tensor,
        norm_weight: torch.Tensor,
        qkv_weight: torch.Tensor,
        qkv_bias: Optional[torch.Tensor],
        num_q_heads: int,
        num_kv_heads: int,
        eps: float = 1e-6,
    ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        out = fused_rmsnorm_qkv(
            input, norm_weight, qkv_weight, num_q_heads, num_kv_heads, eps,
            mixed_rounding=True, qkv_dtype=torch.bfloat16, out_dtype=input.dtype,
            qkv_bias=qkv_bias)
        return split_heads(out, num_q_heads, num_kv_heads)
