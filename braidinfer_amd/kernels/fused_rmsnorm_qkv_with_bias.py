"""FusedRMSNormQKVWithBias on MI355X.

Mirrors braidinfer/kernels/fused_rmsnorm_qkv_with_bias.py:119-228: the host
sanitises the bias exactly as the reference does (None -> no bias; NaN -> 0,
+-inf -> +-1e10; magnitudes above 1e10 are clamped with a printed warning,
`:155-167`), the projection is computed with fp32 output, the bias is added
in fp32 (fused into the kernel epilogue rather than a separate `output +=`),
and q, k, v come back as contiguous copies (`:224-226`).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from ._qkv import fused_rmsnorm_qkv, split_heads


def sanitize_bias(qkv_bias: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    """Host-side bias handling of the reference (fused_rmsnorm_qkv_with_bias.py:155-167)."""
    if qkv_bias is None:
        return None
    qkv_bias = qkv_bias.contiguous()
    qkv_bias = torch.nan_to_num(qkv_bias, nan=0.0, posinf=1e10, neginf=-1e10)
    bias_max = qkv_bias.abs().max().item()
    if bias_max > 1e10:
        qkv_bias = torch.clamp(qkv_bias, min=-1e10, max=1e10)
        print(f"Warning: Clamping extreme bias values (max was {bias_max:.2e})")
    return qkv_bias


class FusedRMSNormQKVWithBias:
    """Fused RMSNorm + QKV with bias support (fp32 output, contiguous q/k/v)."""

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
        bias = sanitize_bias(qkv_bias)
        out = fused_rmsnorm_qkv(
            input, norm_weight, qkv_weight, num_q_heads, num_kv_heads, eps,
            mixed_rounding=False, qkv_dtype=torch.float32, out_dtype=torch.float32,
            qkv_bias=bias)
        q, k, v = split_heads(out, num_q_heads, num_kv_heads)
        return q.contiguous(), k.contiguous(), v.contiguous()
