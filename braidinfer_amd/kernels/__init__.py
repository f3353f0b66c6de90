"""MI355X kernels under the module and class names of braidinfer/kernels."""
from .fused_rmsnorm_qkv_minimal_f32 import FusedRMSNormQKVMinimalF32
from .fused_rmsnorm_qkv_mixed_precision import FusedRMSNormQKVMixedPrecision
from .fused_rmsnorm_qkv_production import FusedRMSNormQKV
from .fused_rmsnorm_qkv_with_bias import FusedRMSNormQKVWithBias
from .rmsnorm_f32 import RMSNormF32

__all__ = [
    "FusedRMSNormQKV",
    "FusedRMSNormQKVMinimalF32",
    "FusedRMSNormQKVMixedPrecision",
    "FusedRMSNormQKVWithBias",
    "RMSNormF32",
]
