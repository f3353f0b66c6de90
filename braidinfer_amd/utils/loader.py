"""Checkpoint loading into the packed layouts, mirroring braidinfer/utils/loader.py.

``load_model(model, path)`` reads every ``*.safetensors`` file of a local
directory (or of a cached Hugging Face model id) and hands each tensor to its
parameter's ``weight_loader``.  Names listed in the model's
``packed_modules_mapping`` are routed to the packed parameter with their shard
id -- ``q_proj`` / ``k_proj`` / ``v_proj`` into ``qkv_proj`` as "q" / "k" / "v",
``gate_proj`` / ``up_proj`` into ``gate_up_proj`` as 0 / 1 (Qwen3ForCausalLM and
LlamaForCausalLM, models/qwen3.py:474-480) -- so the weights land in the
``[q; k; v]`` and ``[gate; up]`` row blocks the fused kernels read
(layers/linear.py:64-114).  Other names go to the parameter of the same name
(GPT-2's unprefixed names get ``transformer.``), with ``default_weight_loader``
when the parameter has none (utils/loader.py:14-104).

One difference: ``*.bin`` checkpoints are read with
``torch.load(..., weights_only=True)``, which refuses pickled objects other
than tensors; the reference unpickles them unrestricted.
"""
from __future__ import annotations

import os
from glob import glob

import torch
from torch import nn


def default_weight_loader(param: nn.Parameter, loaded_weight: torch.Tensor):
    """utils/loader.py:10-11."""
    param.data.copy_(loaded_weight)


def _gpt2_name(model: nn.Module, name: str) -> str:
    if hasattr(model, "transformer") and not name.startswith("transformer."):
        if name.startswith(("wte.", "wpe.", "h.", "ln_f.")):
            return f"transformer.{name}"
    return name


def _load_state_dict_file(model: nn.Module, file: str) -> None:
    state_dict = torch.load(file, map_location="cpu", weights_only=True)
    params = model.state_dict()
    for name, tensor in state_dict.items():
        mapped = _gpt2_name(model, name)
        if mapped in params:
            params[mapped].copy_(tensor)
        else:
            print(f"Warning: Skipping weight {name}")


def _weight_files(model: nn.Module, model_name_or_path: str):
    """The safetensors files to read, or None after a .bin checkpoint was loaded."""
    if os.path.isdir(model_name_or_path):
        files = glob(os.path.join(model_name_or_path, "*.safetensors"))
        if files:
            return files
        bins = glob(os.path.join(model_name_or_path, "*.bin"))
        for file in bins:
            _load_state_dict_file(model, file)
        return None if bins else []
    from transformers.utils import cached_file
    try:
        file = cached_file(model_name_or_path, "model.safetensors", _raise_exceptions_for_missing_entries=False,
                           _raise_exceptions_for_connection_errors=False)
    except Exception:
        file = None
    if file:
        return [file]
    try:
        file = cached_file(model_name_or_path, "pytorch_model.bin", _raise_exceptions_for_missing_entries=False,
                           _raise_exceptions_for_connection_errors=False)
    except Exception:
        file = None
    if not file:
        raise ValueError(f"Could not find model weights for {model_name_or_path}")
    _load_state_dict_file(model, file)
    return None


def load_model(model: nn.Module, model_name_or_path: str) -> None:
    """Loads the checkpoint at `model_name_or_path` into `model` (utils/loader.py:14-104)."""
    from safetensors import safe_open

    packed_modules_mapping = getattr(model, "packed_modules_mapping", {})
    files = _weight_files(model, model_name_or_path)
    if files is None:
        return
    for file in files:
        with safe_open(file, "pt", "cpu") as f:
            for weight_name in f.keys():
                for k, (v, shard_id) in packed_modules_mapping.items():
                    if k not in weight_name:
                        continue
                    param_name = weight_name.replace(k, v)
                    try:
                        param = model.get_parameter(param_name)
                    except AttributeError:
                        if param_name.endswith(".bias"):  # a bias the model does not have
                            print(f"[INFO] Skipping bias parameter '{param_name}' as model has no bias")
                            break
                        raise
                    param.weight_loader(param, f.get_tensor(weight_name), shard_id)
                    break
                else:
                    mapped = _gpt2_name(model, weight_name)
                    try:
                        param = model.get_parameter(mapped)
                    except AttributeError:
                        print(f"Warning: Skipping weight {weight_name} -> {mapped}")
                        continue
                    getattr(param, "weight_loader", default_weight_loader)(param, f.get_tensor(weight_name))
