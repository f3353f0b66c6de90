"""MI355X kernels under the module and class names of braidinfer/kernels."""
from ._qkv import clear_folded_weights
from .fused_attention_output import FusedAttentionOutput, attention_output, attention_output_gemv
from .fused_rmsnorm_qkv_minimal_f32 import FusedRMSNormQKVMinimalF32
from .fused_rmsnorm_qkv_mixed_precision import FusedRMSNormQKVMixedPrecision
from .fused_rmsnorm_qkv_production import FusedRMSNormQKV
from .fused_rmsnorm_qkv_with_bias import FusedRMSNormQKVWithBias
from .kv_cache_utils import (PagedKVAppend, append_paged_kv_batch, append_to_paged_kv_cache_custom,
                             build_paged_kv_indices)
from .online_softmax import online_softmax_update
from .rmsnorm_f32 import RMSNormF32

__all__ = [
    "FusedAttentionOutput",
    "FusedRMSNormQKV",
    "FusedRMSNormQKVMinimalF32",
    "FusedRMSNormQKVMixedPrecision",
    "FusedRMSNormQKVWithBias",
    "PagedKVAppend",
    "RMSNormF32",
    "append_paged_kv_batch",
    "attention_output",
    "attention_output_gemv",
    "append_to_paged_kv_cache_custom",
    "build_paged_kv_indices",
    "clear_folded_weights",
    "online_softmax_update",
]
