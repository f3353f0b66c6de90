"""Checkpoint reading into the packed weight layouts the fused kernels use.

The fused kernels read two packed matrices per decoder layer: W_qkv, whose rows
are ``[q (Hq*D); k (Hkv*D); v (Hkv*D)]`` (``QKVParallelLinear``,
layers/linear.py:78-114), and W_gate_up, ``[gate (I); up (I)]``
(``MergedColumnParallelLinear``, layers/linear.py:64-75).  Checkpoints store
the pieces separately (``q_proj`` / ``k_proj`` / ``v_proj``, ``gate_proj`` /
``up_proj``); the model class says where each piece goes through its
``packed_modules_mapping`` (models/qwen3.py:474-480).  ``load_model`` is the
drop-in for braidinfer's ``utils/loader.py:14`` with this structure:

1. ``checkpoint_tensors(path)`` lists ``(name, read)`` pairs of a local
   checkpoint: every ``*.safetensors`` file of a directory, else every
   ``*.bin`` file (read with ``torch.load(weights_only=True)``, which refuses
   pickled objects other than tensors), or one such file named directly.
   Nothing is fetched: the path must exist.
2. ``route(name, packed, params)`` resolves one checkpoint name to the model
   parameter it fills and the shard id (None for a whole parameter).  A
   packed piece is recognised by a dotted name component equal to a key of
   the mapping, so ``...self_attn.k_proj.weight`` becomes
   ``...self_attn.qkv_proj.weight`` with shard "k".  The same routing serves
   both file formats.
3. Every parameter records what it received.  Policy:

   * a checkpoint tensor with no destination in the model (an ``lm_head`` the
     model ties to its embedding, a bias the model was built without, rotary
     buffers some exporters save) is skipped and listed in the report;
   * a tensor whose shape does not fit its destination raises ``ValueError``;
   * with ``strict`` (the default), a parameter left without data -- a whole
     parameter never named, or a packed parameter missing one of its shards
     -- raises ``ValueError`` naming it, instead of leaving uninitialised
     memory in the model.  Parameters that share storage with a loaded one
     (tied embeddings) count as loaded.

The returned ``LoadReport`` lists what was loaded and what was skipped;
skipped names are also logged at INFO level.
"""
from __future__ import annotations

import logging
import os
from dataclasses import dataclass, field
from glob import glob
from typing import Callable, Iterator

import torch
from torch import nn

log = logging.getLogger(__name__)


def default_weight_loader(param: nn.Parameter, loaded_weight: torch.Tensor):
    """Copies a whole tensor into a parameter without a loader of its own
    (utils/loader.py:10-11)."""
    param.data.copy_(loaded_weight)


@dataclass
class LoadReport:
    loaded: list = field(default_factory=list)   # checkpoint names written into the model
    skipped: list = field(default_factory=list)  # checkpoint names with no destination


def checkpoint_tensors(path: str) -> Iterator[tuple[str, Callable[[], torch.Tensor]]]:
    """(name, read) for every tensor of the checkpoint at ``path``: a directory
    of ``*.safetensors`` files (or, when it has none, ``*.bin`` files), or one
    file of either kind.  ``read()`` returns the tensor on the CPU."""
    if os.path.isdir(path):
        files = sorted(glob(os.path.join(path, "*.safetensors"))) or sorted(glob(os.path.join(path, "*.bin")))
        if not files:
            raise FileNotFoundError(f"no *.safetensors or *.bin checkpoint files in {path}")
    elif os.path.isfile(path):
        files = [path]
    else:
        raise FileNotFoundError(f"checkpoint path {path} does not exist (only local checkpoints are read)")
    for file in files:
        if file.endswith(".safetensors"):
            from safetensors import safe_open
            with safe_open(file, "pt", "cpu") as f:
                for name in f.keys():
                    yield name, (lambda f=f, name=name: f.get_tensor(name))
        else:
            state = torch.load(file, map_location="cpu", weights_only=True)
            for name, tensor in state.items():
                yield name, (lambda t=tensor: t)


def route(name: str, packed: dict, params: dict) -> tuple[str, object] | None:
    """The (parameter name, shard id) that checkpoint tensor ``name`` fills, or
    None when the model has no such parameter.  ``packed`` maps a module name
    to (packed module name, shard id); ``params`` holds the model's parameter
    names."""
    parts = name.split(".")
    for i, part in enumerate(parts):
        if part in packed:
            target, shard = packed[part]
            mapped = ".".join(parts[:i] + [target] + parts[i + 1:])
            return (mapped, shard) if mapped in params else None
    return (name, None) if name in params else None


def _expected_shards(packed: dict) -> dict:
    """Packed module name -> the set of shard ids that fill it."""
    out: dict = {}
    for target, shard in packed.values():
        out.setdefault(target, set()).add(shard)
    return out


def load_model(model: nn.Module, model_name_or_path: str, strict: bool = True) -> LoadReport:
    """Reads the local checkpoint at ``model_name_or_path`` into ``model``,
    packing split q/k/v and gate/up tensors into their fused matrices through
    the parameters' ``weight_loader`` (utils/loader.py:14-104)."""
    packed = dict(getattr(model, "packed_modules_mapping", {}) or {})
    shards_of = _expected_shards(packed)
    params = dict(model.named_parameters(remove_duplicate=False))
    received: dict = {}  # parameter name -> set of shard ids (None for a whole tensor)
    report = LoadReport()
    for name, read in checkpoint_tensors(model_name_or_path):
        dest = route(name, packed, params)
        if dest is None:
            report.skipped.append(name)
            log.info("checkpoint tensor %s has no parameter in %s; skipped", name, type(model).__name__)
            continue
        pname, shard = dest
        param = params[pname]
        tensor = read()
        try:
            if shard is None:
                if tuple(tensor.shape) != tuple(param.shape):
                    raise ValueError(f"shape {tuple(tensor.shape)} does not fit parameter of shape "
                                     f"{tuple(param.shape)}")
                # a packed parameter saved whole (a checkpoint of this model's own
                # state) is copied as is; its loader takes one shard at a time
                whole = default_weight_loader if _module_of(pname) in shards_of else None
                (whole or getattr(param, "weight_loader", default_weight_loader))(param, tensor)
            else:
                param.weight_loader(param, tensor, shard)
        except (RuntimeError, ValueError, AssertionError) as e:
            raise ValueError(f"checkpoint tensor {name} -> {pname}"
                             f"{'' if shard is None else f' shard {shard!r}'}: {e}") from e
        received.setdefault(pname, set()).add(shard)
        report.loaded.append(name)
    if strict:
        _check_coverage(params, received, shards_of)
    return report


def _check_coverage(params: dict, received: dict, shards_of: dict) -> None:
    loaded_storage = {params[n].data_ptr() for n in received if _complete(n, received, shards_of)}
    missing = []
    for pname, param in params.items():
        if _complete(pname, received, shards_of):
            continue
        if param.numel() and param.data_ptr() in loaded_storage:
            continue  # tied to a parameter that was loaded
        got = received.get(pname)
        want = shards_of.get(_module_of(pname))
        if got and want:
            missing.append(f"{pname} (shards {sorted(map(str, want - got))} missing)")
        else:
            missing.append(pname)
    if missing:
        raise ValueError("checkpoint left parameters without data: " + ", ".join(missing))


def _complete(pname: str, received: dict, shards_of: dict) -> bool:
    got = received.get(pname)
    if not got:
        return False
    if None in got:
        return True
    return shards_of.get(_module_of(pname), set()) <= got


def _module_of(pname: str) -> str:
    """The module component of a parameter name ("...qkv_proj.weight" -> "qkv_proj")."""
    parts = pname.split(".")
    return parts[-2] if len(parts) >= 2 else pname
