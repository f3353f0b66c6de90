"""fp32-mode restatement of the hot-path ops (test infrastructure only).

Where oracle/torch_ref.py reproduces the reference's own rounding points (a
bf16 rounding after the normalisation, after the projection, after the head
norm, ...), the functions here compute each op chain in fp32 from the same
bf16 inputs and round once, to the output dtype of the reference op.  This is
the "fp32 reference after bf16 rounding" that the accuracy target is stated
against; the difference between the two modes is the reference's own rounding
error, and the GPU path is checked against both.

Same op order as the cited reference lines; only the intermediate roundings
are dropped.
"""
from __future__ import annotations

import torch


def _f(t):
    return None if t is None else t.to(torch.float32)


def _rms_scale(x32: torch.Tensor, eps: float) -> torch.Tensor:
    return torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + eps)


# --------------------------------------------------------------------- norms
def rms_forward(x, weight, eps):
    """RMSNorm.rms_forward (layers/layernorm.py:35-44) without the rounding
    before the gamma multiply."""
    x32 = _f(x)
    return (x32 * _rms_scale(x32, eps) * _f(weight)).to(x.dtype)


def add_rms_forward(x, residual, weight, eps):
    """RMSNorm.add_rms_forward (layers/layernorm.py:46-57): y from the fp32 sum,
    one rounding; residual_out = to(dtype)(x + residual) as in the reference."""
    s = _f(x) + _f(residual)
    return (s * _rms_scale(s, eps) * _f(weight)).to(x.dtype), s.to(x.dtype)


# -------------------------------------------------------------------- SwiGLU
def silu_and_mul(x):
    """SiluAndMul (layers/activation.py:11-13): silu(g) * u in fp32, one rounding."""
    g, u = _f(x).chunk(2, -1)
    return (g * torch.sigmoid(g) * u).to(x.dtype)


# ---------------------------------------------------------------------- RoPE
def _rotate(x32, cos, sin):
    x1, x2 = torch.chunk(x32, 2, dim=-1)
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1)


def _rope_rows(cache, positions, x32, head_dim):
    """x32 [T, heads * D] rotated per head by cache[positions] (neox half split,
    layers/rotary_embedding.py:6-24, 49-65), kept in fp32."""
    t = positions.size(0)
    cos, sin = cache[positions].to(torch.float32).chunk(2, dim=-1)
    return _rotate(x32.reshape(t, -1, head_dim), cos.unsqueeze(-2), sin.unsqueeze(-2)).reshape(t, -1)


# ------------------------------------------------------- fused RMSNorm + QKV
def qkv(x, norm_weight, qkv_weight, qkv_bias, eps, out_dtype):
    """Every fused RMSNorm+QKV variant (kernels/fused_rmsnorm_qkv_*.py) in fp32:
    n = (x / rms) * w, acc = n @ W^T (+ bias), one rounding to out_dtype."""
    x32 = _f(x)
    n = x32 * _rms_scale(x32, eps) * _f(norm_weight)
    acc = n @ _f(qkv_weight).t()
    if qkv_bias is not None:
        acc = acc + _f(qkv_bias)
    return acc.to(out_dtype)


def _head_norm(x32, hd, w, eps):
    """RMSNorm over each head_dim slice of [T, heads * hd], fp32."""
    t = x32.shape[0]
    h = x32.reshape(t, -1, hd)
    return (h * _rms_scale(h, eps) * _f(w)).reshape(t, -1)


def qwen3_attention_input(x, ln_w, qkv_w, qkv_b, hq, hkv, eps, positions, cache, q_norm_w, k_norm_w):
    """Qwen3AttentionFused.forward up to the attention call (models/qwen3.py:236-336)
    in fp32: QKV (+bias) -> q/k head RMSNorm -> RoPE, one rounding to x's dtype."""
    x32 = _f(x)
    n = x32 * _rms_scale(x32, eps) * _f(ln_w)
    acc = n @ _f(qkv_w).t()
    if qkv_b is not None:
        acc = acc + _f(qkv_b)
    hd = acc.shape[1] // (hq + 2 * hkv)
    q, k, v = acc.split([hq * hd, hkv * hd, hkv * hd], dim=-1)
    q = _rope_rows(cache, positions, _head_norm(q, hd, q_norm_w, eps), hd)
    k = _rope_rows(cache, positions, _head_norm(k, hd, k_norm_w, eps), hd)
    return q.to(x.dtype), k.to(x.dtype), v.to(x.dtype)


def llama_attention_input(x, ln_w, qkv_w, hq, hkv, eps, positions, cache):
    """LlamaAttentionFused.forward up to the attention call (models/llama.py:169-205)
    in fp32: QKV -> RoPE, one rounding to x's dtype."""
    x32 = _f(x)
    n = x32 * _rms_scale(x32, eps) * _f(ln_w)
    acc = n @ _f(qkv_w).t()
    hd = acc.shape[1] // (hq + 2 * hkv)
    q, k, v = acc.split([hq * hd, hkv * hd, hkv * hd], dim=-1)
    return (_rope_rows(cache, positions, q, hd).to(x.dtype), _rope_rows(cache, positions, k, hd).to(x.dtype),
            v.to(x.dtype))


# ------------------------------------------------------ linear layer fusions
def linear(x, weight, bias=None, residual=None):
    """F.linear(x, W, b) (+ residual) in fp32, one rounding to x's dtype."""
    acc = _f(x) @ _f(weight).t()
    if bias is not None:
        acc = acc + _f(bias)
    if residual is not None:
        acc = acc + _f(residual)
    return acc.to(x.dtype)


def gate_up_silu_and_mul(x, gate_up_weight):
    """SiluAndMul()(gate_up_proj(x)) in fp32, one rounding."""
    gu = _f(x) @ _f(gate_up_weight).t()
    g, u = gu.chunk(2, -1)
    return (g * torch.sigmoid(g) * u).to(x.dtype)
