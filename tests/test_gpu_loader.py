"""GPU parity of the fused kernels on weights read by utils/loader.py.

A tiny Llama- and Qwen3-shaped decoder layer is written to disk with the split
checkpoint names (``q_proj`` / ``k_proj`` / ``v_proj``, ``gate_proj`` /
``up_proj``), as safetensors and as a ``.bin`` file.  ``load_model`` packs the
pieces into device ``QKVParallelLinear`` / ``MergedColumnParallelLinear``
parameters (braidinfer/utils/loader.py:14-104 with models/qwen3.py:474-480 and
models/llama.py's mapping), and the fused attention-input chains
(models/llama.py:169-205, models/qwen3.py:236-309) and the gate_up SwiGLU
(layers/linear.py:63-75 + layers/activation.py:6-13) run on those parameters.
The oracle is fed ``torch.cat`` of the raw split tensors, so a shard placed at
the wrong row offset or a transposed piece fails the comparison.

Token counts cover the single-token decode path, the whole-K column-pair decode
kernel (40 tokens) and the MFMA prefill tiles (300 tokens).  Tolerance:
|d| <= 2e-2 + 1e-2 |r| elementwise (tests/helpers.py).
"""
from __future__ import annotations

import pytest
import torch
from safetensors.torch import save_file
from torch import nn

import braidinfer_amd
from braidinfer_amd.layers import (MergedColumnParallelLinear, QKVParallelLinear, RMSNorm,
                                   llama_attention_input, qwen3_attention_input)
from braidinfer_amd.utils import load_model
from oracle import torch_ref as R
from tests.helpers import assert_close, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"

MAPPING = {"q_proj": ("qkv_proj", "q"), "k_proj": ("qkv_proj", "k"), "v_proj": ("qkv_proj", "v"),
           "gate_proj": ("gate_up_proj", 0), "up_proj": ("gate_up_proj", 1)}

# name: hidden, q heads, kv heads, head_dim, intermediate, qkv bias, q/k norm, rope base
ARCH = {
    "llama": dict(h=512, hq=8, hkv=2, d=64, inter=1024, bias=False, qk_norm=False, base=5e5),
    "qwen3": dict(h=256, hq=4, hkv=2, d=128, inter=768, bias=True, qk_norm=True, base=1e6),
}


class _Attn(nn.Module):
    def __init__(self, a):
        super().__init__()
        self.qkv_proj = QKVParallelLinear(a["h"], a["d"], a["hq"], a["hkv"], bias=a["bias"])
        if a["qk_norm"]:
            self.q_norm, self.k_norm = RMSNorm(a["d"]), RMSNorm(a["d"])


class _Mlp(nn.Module):
    def __init__(self, a):
        super().__init__()
        self.gate_up_proj = MergedColumnParallelLinear(a["h"], [a["inter"], a["inter"]])


class _Layer(nn.Module):
    def __init__(self, a):
        super().__init__()
        self.input_layernorm = RMSNorm(a["h"])
        self.self_attn, self.mlp = _Attn(a), _Mlp(a)


class _Model(nn.Module):
    packed_modules_mapping = MAPPING

    def __init__(self, a):
        super().__init__()
        self.model = nn.Module()
        self.model.layers = nn.ModuleList([_Layer(a)])


def _checkpoint(a, seed):
    """Split-name tensors of one decoder layer, bf16 as checkpoints store them."""
    g = gen(seed)
    h, d, hq, hkv, inter = a["h"], a["d"], a["hq"], a["hkv"], a["inter"]
    p = "model.layers.0."
    t = {p + "input_layernorm.weight": randn(g, h, mean=1.0, std=0.1),
         p + "self_attn.q_proj.weight": randn(g, hq * d, h, std=0.02),
         p + "self_attn.k_proj.weight": randn(g, hkv * d, h, std=0.02),
         p + "self_attn.v_proj.weight": randn(g, hkv * d, h, std=0.02),
         p + "mlp.gate_proj.weight": randn(g, inter, h, std=0.03),
         p + "mlp.up_proj.weight": randn(g, inter, h, std=0.03)}
    if a["bias"]:
        for s, rows in (("q", hq * d), ("k", hkv * d), ("v", hkv * d)):
            t[p + f"self_attn.{s}_proj.bias"] = randn(g, rows, std=0.05)
    if a["qk_norm"]:
        t[p + "self_attn.q_norm.weight"] = randn(g, d, mean=1.0, std=0.1)
        t[p + "self_attn.k_norm.weight"] = randn(g, d, mean=1.0, std=0.1)
    return t


def _write(t, path, fmt):
    if fmt == "safetensors":
        names = sorted(t)
        half = len(names) // 2  # two files, as sharded checkpoints come
        save_file({k: t[k] for k in names[:half]}, str(path / "model-00001-of-00002.safetensors"))
        save_file({k: t[k] for k in names[half:]}, str(path / "model-00002-of-00002.safetensors"))
    else:
        torch.save(t, str(path / "pytorch_model.bin"))


def _loaded(arch, fmt, tmp_path, seed):
    a = ARCH[arch]
    t = _checkpoint(a, seed)
    _write(t, tmp_path, fmt)
    model = _Model(a).to(device=DEV, dtype=torch.bfloat16)
    report = load_model(model, str(tmp_path))
    assert sorted(report.loaded) == sorted(t) and not report.skipped
    return a, t, model.model.layers[0]


@pytest.mark.parametrize("fmt", ["safetensors", "bin"])
@pytest.mark.parametrize("tokens", [1, 40, 300])
@pytest.mark.parametrize("arch", ["llama", "qwen3"])
def test_fused_kernels_on_loaded_weights(arch, tokens, fmt, tmp_path):
    a, t, layer = _loaded(arch, fmt, tmp_path, seed=900 + tokens)
    p = "model.layers.0."
    hq, hkv, d = a["hq"], a["hkv"], a["d"]
    qkv = layer.self_attn.qkv_proj
    gu = layer.mlp.gate_up_proj
    assert qkv.weight.device.type == "cuda" and qkv.weight.dtype == torch.bfloat16
    # the oracle's operands: the raw split tensors, concatenated here
    w_qkv = torch.cat([t[p + f"self_attn.{s}_proj.weight"] for s in "qkv"])
    b_qkv = torch.cat([t[p + f"self_attn.{s}_proj.bias"] for s in "qkv"]) if a["bias"] else None
    w_gu = torch.cat([t[p + "mlp.gate_proj.weight"], t[p + "mlp.up_proj.weight"]])
    ln = t[p + "input_layernorm.weight"]

    g = gen(1000 + tokens)
    x = randn(g, tokens, a["h"])
    pos = torch.randint(0, 4096, (tokens,), generator=g)
    cache = R.cos_sin_cache(d, 4096, a["base"])
    xd, posd, cached = x.to(DEV), pos.to(DEV), cache.to(DEV)
    lnd = layer.input_layernorm.weight
    if arch == "qwen3":
        qn, kn = t[p + "self_attn.q_norm.weight"], t[p + "self_attn.k_norm.weight"]
        got = qwen3_attention_input(xd, lnd, qkv.weight, qkv.bias, hq, hkv, 1e-6, posd, cached,
                                    layer.self_attn.q_norm.weight, layer.self_attn.k_norm.weight)
        exp = R.qwen3_attention_input(x, ln, w_qkv, b_qkv, hq, hkv, 1e-6, pos, cache, qn, kn)
    else:
        got = llama_attention_input(xd, lnd, qkv.weight, hq, hkv, 1e-5, posd, cached)
        exp = R.llama_attention_input(x, ln, w_qkv, hq, hkv, 1e-5, pos, cache)
    for gt, ex, name in zip(got, exp, "qkv"):
        assert gt.shape == ex.shape
        assert_close(gt, ex, what=f"{arch} {fmt} t{tokens} {name}")

    y = gu.forward_silu_and_mul(xd)
    assert y.shape == (tokens, a["inter"])
    assert_close(y, R.gate_up_silu_and_mul(x, w_gu), what=f"{arch} {fmt} t{tokens} gate_up silu")
    braidinfer_amd.check_device_status()


def test_loaded_blocks_are_the_split_tensors(tmp_path):
    """The device parameters hold the split tensors at the [q; k; v] and
    [gate; up] row offsets, bit for bit."""
    a, t, layer = _loaded("qwen3", "safetensors", tmp_path, seed=7)
    p = "model.layers.0."
    qkv = layer.self_attn.qkv_proj.weight.detach().cpu()
    q_rows, kv_rows = a["hq"] * a["d"], a["hkv"] * a["d"]
    assert torch.equal(qkv[:q_rows], t[p + "self_attn.q_proj.weight"])
    assert torch.equal(qkv[q_rows:q_rows + kv_rows], t[p + "self_attn.k_proj.weight"])
    assert torch.equal(qkv[q_rows + kv_rows:], t[p + "self_attn.v_proj.weight"])
    bias = layer.self_attn.qkv_proj.bias.detach().cpu()
    assert torch.equal(bias[q_rows:q_rows + kv_rows], t[p + "self_attn.k_proj.bias"])
    gu = layer.mlp.gate_up_proj.weight.detach().cpu()
    assert torch.equal(gu[:a["inter"]], t[p + "mlp.gate_proj.weight"])
    assert torch.equal(gu[a["inter"]:], t[p + "mlp.up_proj.weight"])
