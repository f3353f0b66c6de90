"""The attention-input chains of the Qwen3 and Llama decoders as one kernel.

These reproduce, in one bfa_fused_rmsnorm_qkv launch (plus its normalisation
pre-pass), what the reference attention forwards do between the hidden state
and the attention call:

* Qwen3AttentionFused.forward (models/qwen3.py:236-309):
  FusedRMSNormQKVMixedPrecision -> q_norm(q.float()).to(dtype),
  k_norm(k.float()).to(dtype) -> rotary_emb(positions, q, k)
* LlamaAttentionFused.forward (models/llama.py:169-205):
  FusedRMSNormQKVMinimalF32 (fp32) -> rotary_emb on fp32 q/k -> .to(dtype)

Both return (q_flat, k_flat, v_flat) of shapes [T, Hq*D], [T, Hkv*D],
[T, Hkv*D] in the hidden-state dtype, as views of one [T, qkv_dim] buffer.
With ``paged_kv`` (kernels.kv_cache_utils.PagedKVAppend) the same call also
appends k and v to the layer's paged cache, which the reference's attention
layer does next (layers/attention.py:191-205 -> kernels/kv_cache_utils.py:9-78).
"""
from __future__ import annotations

import torch

from ..kernels._qkv import fused_rmsnorm_qkv, head_dim_of


def _split_flat(out: torch.Tensor, num_heads: int, num_kv_heads: int):
    hd = head_dim_of(out.shape[1], num_heads, num_kv_heads)
    return out.split([num_heads * hd, num_kv_heads * hd, num_kv_heads * hd], dim=-1)


def qwen3_attention_input(hidden_states: torch.Tensor, layernorm_weight: torch.Tensor,
                          qkv_weight: torch.Tensor, qkv_bias: torch.Tensor | None,
                          num_heads: int, num_kv_heads: int, rms_norm_eps: float,
                          positions: torch.Tensor, cos_sin_cache: torch.Tensor,
                          q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor,
                          qk_norm_eps: float | None = None, paged_kv=None):
    dtype = hidden_states.dtype
    out = fused_rmsnorm_qkv(
        hidden_states, layernorm_weight, qkv_weight, num_heads, num_kv_heads, rms_norm_eps,
        mixed_rounding=True, qkv_dtype=torch.bfloat16, out_dtype=dtype, qkv_bias=qkv_bias,
        q_norm_weight=q_norm_weight, k_norm_weight=k_norm_weight,
        qk_norm_eps=rms_norm_eps if qk_norm_eps is None else qk_norm_eps,
        qk_norm_out_dtype=dtype, positions=positions, cos_sin_cache=cos_sin_cache, paged_kv=paged_kv)
    return _split_flat(out, num_heads, num_kv_heads)


def llama_attention_input(hidden_states: torch.Tensor, layernorm_weight: torch.Tensor,
                          qkv_weight: torch.Tensor, num_heads: int, num_kv_heads: int,
                          rms_norm_eps: float, positions: torch.Tensor,
                          cos_sin_cache: torch.Tensor, paged_kv=None):
    dtype = hidden_states.dtype
    out = fused_rmsnorm_qkv(
        hidden_states, layernorm_weight, qkv_weight, num_heads, num_kv_heads, rms_norm_eps,
        mixed_rounding=False, qkv_dtype=torch.float32, out_dtype=dtype,
        positions=positions, cos_sin_cache=cos_sin_cache, paged_kv=paged_kv)
    return _split_flat(out, num_heads, num_kv_heads)
