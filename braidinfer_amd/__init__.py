"""braidinfer_amd: MI355X (gfx950) HIP kernels for braidinfer's fused per-layer hot path.

Drop-in modules mirror the reference package layout:
  braidinfer_amd.kernels  <-> braidinfer.kernels  (FusedRMSNormQKV*, RMSNormF32)
  braidinfer_amd.layers   <-> braidinfer.layers   (RMSNorm, RotaryEmbedding, get_rope,
                                                    apply_rotary_emb, SiluAndMul,
                                                    VocabParallelEmbedding)
plus rerotate_paged_k (one launch for the cascade differential-RoPE loop) and
the fused Qwen3 / Llama attention-input chains.  Everything runs through the
C-ABI library braidinfer_amd/lib/libbraidinfer_amd.so; there is no fallback.
"""
from ._lib import LIB_PATH, BraidinferAMDError, check_device_status, load

__version__ = "0.1.0"
__all__ = ["BraidinferAMDError", "LIB_PATH", "check_device_status", "load"]
