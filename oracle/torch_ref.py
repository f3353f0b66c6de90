"""torch-CPU restatement of the reference hot-path ops (test infrastructure only).

Each function follows the cited reference lines op for op, with the same
rounding points, on CPU tensors.  Inputs are never mutated (the reference's
in-place fp32 forms are restated on a clone; the aliasing itself is tested
against the product separately).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


# --------------------------------------------------------------------- norms
def rms_forward(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm.rms_forward, braidinfer/layers/layernorm.py:35-44."""
    orig_dtype = x.dtype
    x = x.to(torch.float32).clone()
    var = x.pow(2).mean(dim=-1, keepdim=True)
    x.mul_(torch.rsqrt(var + eps))
    x = x.to(orig_dtype)
    return x.mul_(weight)


def add_rms_forward(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                    eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """RMSNorm.add_rms_forward, braidinfer/layers/layernorm.py:46-57.
    Returns (y, residual_out); for fp32 inputs the reference returns one tensor
    twice, holding y."""
    orig_dtype = x.dtype
    x = x.to(torch.float32).clone().add_(residual.to(torch.float32))
    residual_out = x.to(orig_dtype).clone()
    var = x.pow(2).mean(dim=-1, keepdim=True)
    x.mul_(torch.rsqrt(var + eps))
    x = x.to(orig_dtype)
    y = x.mul_(weight)
    if orig_dtype == torch.float32:
        return y, y
    return y, residual_out


def rmsnorm_f32(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNormF32 kernel, braidinfer/kernels/rmsnorm_f32.py:47-96:
    rms = sqrt(sum(x^2)/H + eps); out = (x / rms) * w, fp32."""
    x32 = x.to(torch.float32)
    acc = (x32 * x32).sum(dim=-1, keepdim=True)
    rms = torch.sqrt(acc / x.shape[-1] + eps)
    return (x32 / rms) * weight.to(torch.float32)


# ----------------------------------------------------------------- embedding
def embedding(ids: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """VocabParallelEmbedding.forward, braidinfer/layers/embed_head.py:28-29."""
    return F.embedding(ids, weight)


def embedding_scaled(ids: torch.Tensor, weight: torch.Tensor, hidden_size: int) -> torch.Tensor:
    """Qwen3Model.forward embedding + scaling, braidinfer/models/qwen3.py:463-465."""
    h = F.embedding(ids, weight)
    return h * (1.0 / (hidden_size ** 0.5))


# -------------------------------------------------------------------- SwiGLU
def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """SiluAndMul.forward, braidinfer/layers/activation.py:11-13."""
    g, u = x.chunk(2, -1)
    return F.silu(g) * u


# ---------------------------------------------------------------------- RoPE
def cos_sin_cache(head_size: int, max_position: int, base: float) -> torch.Tensor:
    """RotaryEmbedding.__init__ table, braidinfer/layers/rotary_embedding.py:29-47."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_size, 2, dtype=torch.float32) / head_size))
    t = torch.arange(max_position, dtype=torch.float32)
    freqs = torch.einsum("i,j -> ij", t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).to(torch.float32)


def apply_rotary_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """apply_rotary_emb, braidinfer/layers/rotary_embedding.py:6-24."""
    original_dtype = x.dtype
    cos = cos.unsqueeze(-2).to(torch.float32)
    sin = sin.unsqueeze(-2).to(torch.float32)
    x_f32 = x.to(torch.float32)
    x1, x2 = torch.chunk(x_f32, 2, dim=-1)
    y1 = x1 * cos - x2 * sin
    y2 = x2 * cos + x1 * sin
    return torch.cat((y1, y2), dim=-1).to(original_dtype)


def rotary_forward(cache: torch.Tensor, head_size: int, positions: torch.Tensor,
                   query: torch.Tensor, key: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """RotaryEmbedding.forward, braidinfer/layers/rotary_embedding.py:49-65."""
    num_tokens = positions.size(0)
    cos, sin = cache[positions].chunk(2, dim=-1)
    q = apply_rotary_emb(query.reshape(num_tokens, -1, head_size), cos, sin).view(query.shape)
    k = apply_rotary_emb(key.reshape(num_tokens, -1, head_size), cos, sin).view(key.shape)
    return q, k


# ---------------------------------------------------------- differential RoPE
def rerotate_paged_k(kv_cache_layer: torch.Tensor, page_indices: torch.Tensor,
                     chunk_indptr: torch.Tensor, chunk_delta: torch.Tensor,
                     last_page_len: torch.Tensor, cache: torch.Tensor,
                     k_norm_weight: torch.Tensor | None = None, k_norm_eps: float = 1e-6):
    """Per-page loop of CascadeAttention.forward, braidinfer/layers/cascade_attention.py:116-178:
    page_k = kv_cache[page, 0, :, :tokens, :].transpose(0, 1); if the chunk's
    positions moved, rotary_emb(pos_diff, zeros, page_k) (cos_sin_cache[pos_diff],
    torch negative-index wrap); then k_norm.  Returns the page-padded
    [entries, page_size, Hkv, D] stack of those page_k tensors."""
    n_pages, _, hkv, page_size, d = kv_cache_layer.shape
    entries = page_indices.numel()
    out = torch.zeros((entries, page_size, hkv, d), dtype=kv_cache_layer.dtype)
    for c in range(chunk_delta.numel()):
        start, end = int(chunk_indptr[c]), int(chunk_indptr[c + 1])
        delta = int(chunk_delta[c])
        for local, e in enumerate(range(start, end)):
            tokens = int(last_page_len[c]) if e == end - 1 else page_size
            if tokens <= 0:
                continue
            page = int(page_indices[e])
            page_k = kv_cache_layer[page, 0, :, :tokens, :].transpose(0, 1)
            if delta != 0:
                pos_diff = torch.full((tokens,), delta, dtype=torch.int64)
                flat = page_k.reshape(tokens, hkv * d)
                _, rot = rotary_forward(cache, d, pos_diff, torch.zeros_like(flat), flat)
                page_k = rot.reshape(tokens, hkv, d)
            if k_norm_weight is not None:
                page_k = rms_forward(page_k, k_norm_weight, k_norm_eps)
            out[e, :tokens] = page_k
    return out


# ---------------------------------------------------------- paged KV append
def append_to_paged_kv_cache(k: torch.Tensor, v: torch.Tensor, layer_cache: torch.Tensor,
                             kv_indices: torch.Tensor, positions: torch.Tensor, page_size: int,
                             kv_layout: str = "HND") -> tuple[torch.Tensor, list[int]]:
    """append_to_paged_kv_cache_custom, braidinfer/kernels/kv_cache_utils.py:9-78, applied
    to a clone of layer_cache: per token, page_offset = pos // page_size (Python
    floor), pos_in_page = pos % page_size; a token with page_offset >=
    len(kv_indices) is skipped; otherwise K and V are assigned into page
    kv_indices[page_offset] (torch indexing, so negative offsets and page ids
    wrap and out-of-range ones raise IndexError).  Returns (cache, skipped tokens)."""
    if kv_layout not in ("HND", "NHD"):
        raise ValueError(f"Unknown kv_layout: {kv_layout}")
    cache = layer_cache.clone()
    skipped = []
    for t in range(k.shape[0]):
        seq_pos = int(positions[t])
        page_offset = seq_pos // page_size
        pos_in_page = seq_pos % page_size
        if page_offset < len(kv_indices):
            page_idx = int(kv_indices[page_offset])
            if kv_layout == "HND":
                cache[page_idx, 0, :, pos_in_page, :] = k[t]
                cache[page_idx, 1, :, pos_in_page, :] = v[t]
            else:
                cache[page_idx, 0, pos_in_page, :, :] = k[t]
                cache[page_idx, 1, pos_in_page, :, :] = v[t]
        else:
            skipped.append(t)
    return cache, skipped


def append_paged_kv_batch(k, v, layer_cache, kv_indices, kv_indptr, batch_indices, positions,
                          page_size, kv_layout="HND"):
    """The batched append as the reference's page manager composes it
    (engine/page_manager.py:180-210): append_to_paged_kv_cache_custom once per
    sequence s, with the tokens of s (in order) and its slice
    kv_indices[kv_indptr[s]:kv_indptr[s+1]] of the CSR page table."""
    cache, skipped = layer_cache.clone(), []
    for s in range(kv_indptr.numel() - 1):
        toks = [t for t in range(k.shape[0]) if int(batch_indices[t]) == s]
        if not toks:
            continue
        sel = torch.tensor(toks)
        table = kv_indices[int(kv_indptr[s]):int(kv_indptr[s + 1])]
        cache, sk = append_to_paged_kv_cache(k[sel], v[sel], cache, table, positions[sel],
                                             page_size, kv_layout)
        skipped += [toks[i] for i in sk]
    return cache, sorted(skipped)


# ---------------------------------------------------------- cascade attention
def online_softmax_update(query, key, value, m_i, l_i, acc_i, query_positions, key_positions,
                          scale, apply_causal_mask=True):
    """The recurrence of online_softmax_kernel, braidinfer/kernels/online_softmax.py:80-125,
    in fp32, keys in order: s = (q . k) * scale; m' = max(m, s);
    l = l e^(m-m') + e^(s-m'); acc = acc e^(m-m') + e^(s-m') v; a key whose position
    exceeds the query's is skipped when causal.  query [H, B, D], key/value [H, N, D];
    returns new (m [H, B], l [H, B], acc [H, B, D])."""
    m, l, acc = m_i.clone().float(), l_i.clone().float(), acc_i.clone().float()
    q, k, v = query.float(), key.float(), value.float()
    for t in range(key.shape[1]):
        use = torch.ones(query.shape[1], dtype=torch.bool)
        if apply_causal_mask:
            use = key_positions[t] <= query_positions
        s = (q * k[:, t].unsqueeze(1)).sum(-1) * scale  # [H, B]
        m_new = torch.maximum(m, s)
        alpha = torch.exp(m - m_new)
        beta = torch.exp(s - m_new)
        u = use.unsqueeze(0)
        l = torch.where(u, l * alpha + beta, l)
        acc = torch.where(u.unsqueeze(-1), alpha.unsqueeze(-1) * acc + beta.unsqueeze(-1) * v[:, t].unsqueeze(1), acc)
        m = torch.where(u, m_new, m)
    return m, l, acc


def cascade_attention(query, query_positions, kv_cache, cascade_levels, num_heads, num_kv_heads,
                      scale, page_size, cos_sin_cache=None, k_norm_weight=None, k_norm_eps=1e-6,
                      causal_mask=True):
    """CascadeAttention.forward, braidinfer/layers/cascade_attention.py:50-231, page by page:
    K of each page is rotated by cos_sin_cache[global - cached position start] when the
    chunk moved (and a table is given), then RMS-normalised when k_norm_weight is given;
    GQA by repeat_interleave; the online softmax recurrence above per page with key
    positions counted over the attended chunks.  Levels and chunks are any objects with
    the reference's attributes (kv_page_indices / kv_page_indptr / kv_last_page_len /
    chunks; page_table / kv_length / global_position_start / cached_position_start).
    query [T, H, D]; returns [T, H * D] in the query dtype."""
    t_, h, d = query.shape
    q = query.transpose(0, 1)
    m = torch.full((h, t_), float("-inf"))
    l = torch.zeros(h, t_)
    acc = torch.zeros(h, t_, d)
    cumulative = 0
    for level in cascade_levels:
        for ci, chunk in enumerate(level.chunks):
            if not chunk.page_table or chunk.kv_length == 0:
                continue
            start, end = int(level.kv_page_indptr[ci]), int(level.kv_page_indptr[ci + 1])
            chunk_pages = level.kv_page_indices[start:end]
            for local, page in enumerate(chunk_pages):
                page = int(page)
                tokens = int(level.kv_last_page_len[ci]) if local == len(chunk_pages) - 1 else page_size
                if tokens <= 0:
                    continue
                page_k = kv_cache[page, 0, :, :tokens, :].transpose(0, 1)
                page_v = kv_cache[page, 1, :, :tokens, :].transpose(0, 1)
                if cos_sin_cache is not None and hasattr(chunk, "global_position_start"):
                    before = local * page_size
                    cached = getattr(chunk, "cached_position_start", 0)
                    glob = getattr(chunk, "global_position_start", cached)
                    cpos = torch.arange(cached + before, cached + before + tokens)
                    gpos = torch.arange(glob + before, glob + before + tokens)
                    if not torch.equal(cpos, gpos):
                        flat = page_k.reshape(tokens, num_kv_heads * d)
                        _, rot = rotary_forward(cos_sin_cache, d, gpos - cpos, torch.zeros_like(flat), flat)
                        page_k = rot.reshape(tokens, num_kv_heads, d)
                if k_norm_weight is not None:
                    page_k = rms_forward(page_k, k_norm_weight, k_norm_eps)
                if num_kv_heads != num_heads:
                    rep = num_heads // num_kv_heads
                    page_k = page_k.repeat_interleave(rep, dim=1)
                    page_v = page_v.repeat_interleave(rep, dim=1)
                kpos = torch.arange(cumulative + local * page_size, cumulative + local * page_size + tokens)
                m, l, acc = online_softmax_update(q, page_k.transpose(0, 1), page_v.transpose(0, 1), m, l,
                                                  acc, query_positions, kpos, scale, causal_mask)
            cumulative += chunk.kv_length
    out = (acc / torch.clamp(l, min=1e-12).unsqueeze(-1)).to(query.dtype)
    return out.transpose(0, 1).contiguous().view(-1, h * d)


# ------------------------------------------------------- fused RMSNorm + QKV
def _rms(x32: torch.Tensor, eps: float) -> torch.Tensor:
    # tl.sqrt(acc_var / hidden_dim + eps) with acc_var = sum(x*x) in fp32
    return torch.sqrt((x32 * x32).sum(dim=-1, keepdim=True) / x32.shape[-1] + eps)


def qkv_mixed_precision(x, norm_weight, qkv_weight, qkv_bias, eps):
    """fused_rmsnorm_qkv_mixed_precision_kernel, braidinfer/kernels/
    fused_rmsnorm_qkv_mixed_precision.py:57-148 (+ the output dtype of :190-195):
    n = bf16(x / rms) * w (bf16), acc = n @ bf16(W)^T (fp32), + bias (fp32),
    -> bf16 -> x.dtype.  Returns the [T, N] buffer."""
    x32 = x.to(torch.float32)
    n = (x32 / _rms(x32, eps)).to(torch.bfloat16)
    n = n * norm_weight.to(torch.bfloat16)
    acc = n.to(torch.float32) @ qkv_weight.to(torch.bfloat16).to(torch.float32).t()
    if qkv_bias is not None:
        acc = acc + qkv_bias.to(torch.float32)
    return acc.to(torch.bfloat16).to(x.dtype)


def qkv_production(x, norm_weight, qkv_weight, eps):
    """fused_rmsnorm_qkv_kernel, braidinfer/kernels/fused_rmsnorm_qkv_production.py:57-139:
    n = bf16((x / rms) * w) in fp32, acc = n @ bf16(W)^T, -> bf16."""
    x32 = x.to(torch.float32)
    n = ((x32 / _rms(x32, eps)) * norm_weight.to(torch.float32)).to(torch.bfloat16)
    acc = n.to(torch.float32) @ qkv_weight.to(torch.bfloat16).to(torch.float32).t()
    return acc.to(torch.bfloat16)


def qkv_minimal_f32(x, norm_weight, qkv_weight, eps):
    """fused_rmsnorm_qkv_minimal_f32_kernel, braidinfer/kernels/
    fused_rmsnorm_qkv_minimal_f32.py:54-125: n = (x / rms) * w in fp32,
    acc = n @ W^T in fp32, fp32 output (computed here without TF32)."""
    x32 = x.to(torch.float32)
    n = (x32 / _rms(x32, eps)) * norm_weight.to(torch.float32)
    return n @ qkv_weight.to(torch.float32).t()


def sanitize_bias(qkv_bias):
    """Host bias handling, braidinfer/kernels/fused_rmsnorm_qkv_with_bias.py:155-167."""
    if qkv_bias is None:
        return None
    b = torch.nan_to_num(qkv_bias, nan=0.0, posinf=1e10, neginf=-1e10)
    if b.abs().max().item() > 1e10:
        b = torch.clamp(b, min=-1e10, max=1e10)
    return b


def qkv_with_bias(x, norm_weight, qkv_weight, qkv_bias, eps):
    """FusedRMSNormQKVWithBias.forward, braidinfer/kernels/fused_rmsnorm_qkv_with_bias.py:123-228."""
    out = qkv_minimal_f32(x, norm_weight, qkv_weight, eps)
    b = sanitize_bias(qkv_bias)
    if b is None:
        b = torch.zeros(qkv_weight.shape[0], dtype=x.dtype)
    return out + b.to(torch.float32)


def split_qkv(out: torch.Tensor, num_q_heads: int, num_kv_heads: int):
    """The split/view of every variant (e.g. fused_rmsnorm_qkv_mixed_precision.py:236-247)."""
    t, n = out.shape
    hd = n // (num_q_heads + 2 * num_kv_heads)
    q, k, v = out.split([num_q_heads * hd, num_kv_heads * hd, num_kv_heads * hd], dim=-1)
    return q.reshape(t, num_q_heads, hd), k.reshape(t, num_kv_heads, hd), v.reshape(t, num_kv_heads, hd)


# ---------------------------------------------------- model attention inputs
def qwen3_attention_input(x, ln_w, qkv_w, qkv_b, hq, hkv, eps, positions, cache,
                          q_norm_w, k_norm_w):
    """Qwen3AttentionFused.forward up to the attention call, braidinfer/models/qwen3.py:236-336:
    mixed QKV -> q_norm(q.float()).to(dtype), k_norm(k.float()).to(dtype) -> RoPE."""
    dtype = x.dtype
    q, k, v = split_qkv(qkv_mixed_precision(x, ln_w, qkv_w, qkv_b, eps), hq, hkv)
    q = rms_forward(q.float(), q_norm_w, eps).to(dtype)
    k = rms_forward(k.float(), k_norm_w, eps).to(dtype)
    t = x.shape[0]
    qf, kf = rotary_forward(cache, q.shape[-1], positions, q.reshape(t, -1), k.reshape(t, -1))
    return qf.to(dtype), kf.to(dtype), v.reshape(t, -1).to(dtype)


def llama_attention_input(x, ln_w, qkv_w, hq, hkv, eps, positions, cache):
    """LlamaAttentionFused.forward up to the attention call, braidinfer/models/llama.py:169-205:
    minimal_f32 QKV -> RoPE on fp32 q/k -> .to(dtype)."""
    dtype = x.dtype
    q, k, v = split_qkv(qkv_minimal_f32(x, ln_w, qkv_w, eps), hq, hkv)
    t = x.shape[0]
    qf, kf = rotary_forward(cache, q.shape[-1], positions, q.reshape(t, -1), k.reshape(t, -1))
    return qf.to(dtype), kf.to(dtype), v.reshape(t, -1).to(dtype)


# ------------------------------------------------------ linear layer fusions
def linear(x, weight, bias=None):
    """F.linear(x, weight, bias) of ReplicatedLinear / ColumnParallelLinear /
    RowParallelLinear.forward (braidinfer/layers/linear.py:37-38, 159-160): fp32
    products and sums, the bias added in fp32, one rounding to x's dtype."""
    acc = x.to(torch.float32) @ weight.to(torch.float32).t()
    if bias is not None:
        acc = acc + bias.to(torch.float32)
    return acc.to(x.dtype)


def linear_add_residual(x, weight, residual, bias=None):
    """residual + F.linear(x, weight, bias) in torch's rounding: the projection
    rounded to x's dtype, the sum formed in fp32 and rounded again (the o_proj /
    down_proj output joining the residual stream, braidinfer/models/qwen3.py:
    336-366, 388-392)."""
    return (linear(x, weight, bias).to(torch.float32) + residual.to(torch.float32)).to(x.dtype)


def gate_up_silu_and_mul(x, gate_up_weight):
    """SiluAndMul()(gate_up_proj(x)), braidinfer/models/qwen3.py:388-392 with
    layers/linear.py:64-75 and layers/activation.py:11-13."""
    return silu_and_mul(linear(x, gate_up_weight))


def fused_attention_output(x, weight, residual=None):
    """fused_o_proj_add_residual_kernel / tiled_gemv_kernel, braidinfer/kernels/
    fused_attention_output.py:17-72, 76-134: acc = x W^T in fp32 (+ residual in
    fp32), stored as acc.to(float16) into an output of x's dtype."""
    acc = x.to(torch.float32) @ weight.to(torch.float32).t()
    if residual is not None:
        acc = acc + residual.to(torch.float32)
    return acc.to(torch.float16).to(x.dtype)
