"""FusedRMSNormQKVMinimalF32 on MI355X.

Mirrors braidinfer/kernels/fused_rmsnorm_qkv_minimal_f32.py:128-214 (used by
Llama, TinyLlama and ERNIE, models/llama.py:169-176): n = (x / rms) * weight in
fp32, n @ W^T with fp32 accumulation, fp32 output returned as q, k, v views.

The reference's fp32 tl.dot runs on tensor cores in TF32 (10-bit mantissa
operands).  Here n is rounded once to the weight's bf16/fp16 type for the
MFMA units; the accumulation stays fp32.
"""
from __future__ import annotations

from typing import Tuple

import torch

from ._qkv import fused_rmsnorm_qkv, split_heads


class FusedRMSNormQKVMinimalF32:
    """Fused RMSNorm + QKV with fp32 accumulation and fp32 output."""

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
            mixed_rounding=False, qkv_dtype=torch.float32, out_dtype=torch.float32)
        return split_heads(out, num_q_heads, num_kv_heads)
