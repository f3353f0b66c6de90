"""Checkpoint loading into the packed layouts (braidinfer/utils/loader.py:14-104):
a tiny decoder written with Hugging Face tensor names must land in the
[q; k; v] and [gate; up] row blocks the fused kernels read.  CPU only."""
from __future__ import annotations

import pytest
import torch
from safetensors.torch import save_file
from torch import nn

from braidinfer_amd.layers import (MergedColumnParallelLinear, QKVParallelLinear, RMSNorm, RowParallelLinear,
                                   VocabParallelEmbedding)
from braidinfer_amd.utils import load_model
from braidinfer_amd.utils.loader import route

H, HQ, HKV, D, I, V = 64, 4, 2, 16, 96, 50


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.qkv_proj = QKVParallelLinear(H, D, HQ, HKV)
        self.o_proj = RowParallelLinear(HQ * D, H)


class _Mlp(nn.Module):
    def __init__(self):
        super().__init__()
        self.gate_up_proj = MergedColumnParallelLinear(H, [I, I])
        self.down_proj = RowParallelLinear(I, H)


class _Layer(nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn, self.mlp = _Attn(), _Mlp()
        self.input_layernorm = RMSNorm(H)


class _Inner(nn.Module):
    def __init__(self):
        super().__init__()
        self.embed_tokens = VocabParallelEmbedding(V, H)
        self.layers = nn.ModuleList([_Layer(), _Layer()])


class _Model(nn.Module):
    packed_modules_mapping = {"q_proj": ("qkv_proj", "q"), "k_proj": ("qkv_proj", "k"),
                              "v_proj": ("qkv_proj", "v"), "gate_proj": ("gate_up_proj", 0),
                              "up_proj": ("gate_up_proj", 1)}

    def __init__(self):
        super().__init__()
        self.model = _Inner()


def _checkpoint(g):
    t = {"model.embed_tokens.weight": torch.randn(V, H, generator=g),
         "lm_head.weight": torch.randn(V, H, generator=g)}  # not in the model: skipped
    for i in range(2):
        p = f"model.layers.{i}."
        t[p + "self_attn.q_proj.weight"] = torch.randn(HQ * D, H, generator=g)
        t[p + "self_attn.k_proj.weight"] = torch.randn(HKV * D, H, generator=g)
        t[p + "self_attn.v_proj.weight"] = torch.randn(HKV * D, H, generator=g)
        t[p + "self_attn.q_proj.bias"] = torch.randn(HQ * D, generator=g)  # the model has no bias
        t[p + "self_attn.o_proj.weight"] = torch.randn(H, HQ * D, generator=g)
        t[p + "mlp.gate_proj.weight"] = torch.randn(I, H, generator=g)
        t[p + "mlp.up_proj.weight"] = torch.randn(I, H, generator=g)
        t[p + "mlp.down_proj.weight"] = torch.randn(H, I, generator=g)
        t[p + "input_layernorm.weight"] = torch.randn(H, generator=g)
    return t


def _check(model, t):
    assert torch.equal(model.model.embed_tokens.weight.data, t["model.embed_tokens.weight"])
    for i, layer in enumerate(model.model.layers):
        p = f"model.layers.{i}."
        qkv = torch.cat([t[p + "self_attn.q_proj.weight"], t[p + "self_attn.k_proj.weight"],
                         t[p + "self_attn.v_proj.weight"]])
        assert torch.equal(layer.self_attn.qkv_proj.weight.data, qkv)
        assert torch.equal(layer.mlp.gate_up_proj.weight.data,
                           torch.cat([t[p + "mlp.gate_proj.weight"], t[p + "mlp.up_proj.weight"]]))
        assert torch.equal(layer.self_attn.o_proj.weight.data, t[p + "self_attn.o_proj.weight"])
        assert torch.equal(layer.mlp.down_proj.weight.data, t[p + "mlp.down_proj.weight"])
        assert torch.equal(layer.input_layernorm.weight.data, t[p + "input_layernorm.weight"])


def test_safetensors_checkpoint_lands_in_packed_blocks(tmp_path):
    t = _checkpoint(torch.Generator().manual_seed(1))
    names = list(t)
    half = len(names) // 2  # two shards, as large checkpoints come
    save_file({k: t[k] for k in names[:half]}, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file({k: t[k] for k in names[half:]}, str(tmp_path / "model-00002-of-00002.safetensors"))
    model = _Model()
    report = load_model(model, str(tmp_path))
    _check(model, t)
    # lm_head has no parameter here and the model was built without a q bias:
    # both are skipped and reported, everything else is loaded
    assert sorted(report.skipped) == ["lm_head.weight", "model.layers.0.self_attn.q_proj.bias",
                                      "model.layers.1.self_attn.q_proj.bias"]
    assert sorted(report.loaded) == sorted(set(t) - set(report.skipped))


def test_bin_checkpoint_with_split_names_is_packed(tmp_path):
    """A .bin checkpoint goes through the same routing as safetensors: split
    q/k/v and gate/up tensors land in the packed blocks."""
    t = _checkpoint(torch.Generator().manual_seed(2))
    torch.save(t, str(tmp_path / "pytorch_model.bin"))
    model = _Model()
    load_model(model, str(tmp_path))
    _check(model, t)


def test_single_file_path(tmp_path):
    t = _checkpoint(torch.Generator().manual_seed(3))
    save_file(t, str(tmp_path / "one.safetensors"))
    model = _Model()
    load_model(model, str(tmp_path / "one.safetensors"))
    _check(model, t)


def test_packed_state_dict_round_trip(tmp_path):
    """A checkpoint written from the model itself (packed names) reloads as is."""
    g = torch.Generator().manual_seed(4)
    model = _Model()
    sd = {k: torch.randn(v.shape, generator=g) for k, v in model.state_dict().items()}
    torch.save(sd, str(tmp_path / "pytorch_model.bin"))
    load_model(model, str(tmp_path))
    for k, v in model.state_dict().items():
        assert torch.equal(v, sd[k])


def test_missing_shard_raises(tmp_path):
    t = _checkpoint(torch.Generator().manual_seed(5))
    del t["model.layers.1.self_attn.v_proj.weight"]
    save_file(t, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match=r"layers\.1\.self_attn\.qkv_proj\.weight \(shards \['v'\] missing\)"):
        load_model(_Model(), str(tmp_path))
    # not strict: loads what is there and leaves the rest to the caller
    model = _Model()
    load_model(model, str(tmp_path), strict=False)
    assert torch.equal(model.model.layers[0].self_attn.qkv_proj.weight.data[:HQ * D],
                       t["model.layers.0.self_attn.q_proj.weight"])


def test_missing_whole_parameter_raises(tmp_path):
    t = _checkpoint(torch.Generator().manual_seed(6))
    del t["model.layers.0.input_layernorm.weight"]
    save_file(t, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match=r"model\.layers\.0\.input_layernorm\.weight"):
        load_model(_Model(), str(tmp_path))


def test_shape_mismatch_raises(tmp_path):
    t = _checkpoint(torch.Generator().manual_seed(7))
    t["model.layers.0.mlp.down_proj.weight"] = torch.zeros(H, I + 1)
    save_file(t, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="down_proj"):
        load_model(_Model(), str(tmp_path))
    t = _checkpoint(torch.Generator().manual_seed(7))
    t["model.layers.0.self_attn.k_proj.weight"] = torch.zeros(HKV * D + 1, H)  # packed shard too large
    save_file(t, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match=r"k_proj.*shard 'k'"):
        load_model(_Model(), str(tmp_path))


class _TiedModel(_Model):
    def __init__(self):
        super().__init__()
        self.lm_head = VocabParallelEmbedding(V, H)
        self.lm_head.weight.data = self.model.embed_tokens.weight.data  # tied, as Qwen3-0.6B is


def test_tied_parameter_counts_as_loaded(tmp_path):
    t = _checkpoint(torch.Generator().manual_seed(8))
    del t["lm_head.weight"]
    save_file(t, str(tmp_path / "model.safetensors"))
    model = _TiedModel()
    load_model(model, str(tmp_path))
    assert torch.equal(model.lm_head.weight.data, t["model.embed_tokens.weight"])


def test_no_checkpoint_raises(tmp_path):
    with pytest.raises(FileNotFoundError):
        load_model(_Model(), str(tmp_path))
    with pytest.raises(FileNotFoundError):
        load_model(_Model(), str(tmp_path / "absent"))


def test_route_matches_whole_name_components():
    packed = _Model.packed_modules_mapping
    params = {"a.qkv_proj.weight", "a.my_q_proj_x.weight"}
    assert route("a.k_proj.weight", packed, params) == ("a.qkv_proj.weight", "k")
    assert route("a.my_q_proj_x.weight", packed, params) == ("a.my_q_proj_x.weight", None)
    assert route("b.k_proj.weight", packed, params) is None
