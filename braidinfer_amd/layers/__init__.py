"""MI355X layers under the module and class names of braidinfer/layers."""
from .activation import SiluAndMul, silu_and_mul
from .cascade_attention import CascadeAttention, CascadeLevel
from .cascade_rope import rerotate_paged_k
from .embed_head import VocabParallelEmbedding, embedding
from .fused_attention_input import llama_attention_input, qwen3_attention_input
from .layernorm import RMSNorm, rms_norm
from .linear import (ColumnParallelLinear, LinearBase, MergedColumnParallelLinear,
                     QKVParallelLinear, ReplicatedLinear, RowParallelLinear, gate_up_silu_and_mul,
                     linear, linear_add_residual)
from .rotary_embedding import RotaryEmbedding, apply_rotary_emb, get_rope

__all__ = [
    "CascadeAttention", "CascadeLevel", "ColumnParallelLinear", "LinearBase",
    "MergedColumnParallelLinear", "QKVParallelLinear", "RMSNorm", "ReplicatedLinear",
    "RotaryEmbedding", "RowParallelLinear", "SiluAndMul", "VocabParallelEmbedding",
    "apply_rotary_emb", "embedding", "gate_up_silu_and_mul", "get_rope", "linear",
    "linear_add_residual", "llama_attention_input", "qwen3_attention_input",
    "rerotate_paged_k", "rms_norm", "silu_and_mul",
]
