"""Linear layers on MI355X, mirroring braidinfer/layers/linear.py.

Every ``forward`` is ``F.linear(x, weight, bias)`` computed by the projection
GEMM of the native library (``bfa_linear``): bf16/fp16 MFMA with fp32
accumulation, the bias added in fp32, the result rounded to x's dtype.  The
fused forms are the GEMM-epilogue fusions of the layers' callers:

* ``MergedColumnParallelLinear.forward_silu_and_mul(x)`` =
  ``SiluAndMul()(gate_up_proj(x))`` (models/qwen3.py:388-392,
  layers/activation.py:11-13) without the [tokens, 2 I] intermediate;
* ``RowParallelLinear.forward_add_residual(x, residual)`` =
  ``residual + F.linear(x, W)`` in torch's rounding (the o_proj / down_proj
  output joining the residual stream).

The weight loaders are the reference's (shard offsets of the packed
[q; k; v] and [gate; up] matrices, layers/linear.py:36-114).
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _lib

_F32 = _lib.F32


def _rows(x: torch.Tensor, k: int) -> torch.Tensor:
    """x as a [tokens, k] matrix with unit column stride and a 16-byte aligned
    row stride (a copy only when the view does not qualify)."""
    if x.shape[-1] != k:
        raise ValueError(f"input has {x.shape[-1]} features, the layer takes {k}")
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2


def _check_weight(w: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    if w.dtype != x.dtype:
        raise TypeError(f"weight dtype {w.dtype} does not match input dtype {x.dtype}")
    if w.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("the projection GEMM takes bf16 or fp16 operands")
    if w.stride(-1) != 1 or w.stride(0) % 8 or w.data_ptr() % 16:
        w = w.contiguous()
    return w


def _run(x: torch.Tensor, weight: torch.Tensor, n: int, mode: int, bias=None, residual=None,
         proj_dtype=None, sum_dtype: int = _F32, out_dtype=None) -> torch.Tensor:
    """Shared driver of bfa_linear: returns [..., n] in out_dtype (default x's)."""
    k = weight.shape[1]
    x2 = _rows(x, k)
    weight = _check_weight(weight, x2)
    dev = _lib.require_device(x2, weight, bias, residual)
    out_t = x.dtype if out_dtype is None else out_dtype
    tokens = x2.shape[0]
    out = torch.empty(tokens, n, dtype=out_t, device=dev)
    r2 = None
    if residual is not None:
        if residual.shape[-1] != n or residual.numel() != tokens * n:
            raise ValueError(f"residual of shape {tuple(residual.shape)} does not match [{tokens}, {n}]")
        r2 = residual.reshape(tokens, n)
        if r2.stride(-1) != 1:
            r2 = r2.contiguous()
    if bias is not None:
        if bias.numel() != n:
            raise ValueError(f"bias has {bias.numel()} elements, the layer has {n} outputs")
        bias = bias.detach().contiguous()
    ws_bytes = _lib.workspace_size("bfa_linear_workspace_size", tokens, k, n, mode)
    ws = _lib.workspace(dev, ws_bytes)
    _lib.call(
        "bfa_linear", _lib.ptr(x2), _lib.dtype_code(x2), tokens, k, x2.stride(0),
        _lib.ptr(weight), n, weight.stride(0), _lib.ptr(bias),
        _lib.dtype_code(bias) if bias is not None else 0, mode,
        _lib.dtype_code(x2) if proj_dtype is None else proj_dtype,
        _lib.ptr(r2), _lib.dtype_code(r2) if r2 is not None else 0, r2.stride(0) if r2 is not None else n,
        sum_dtype, _lib.ptr(out), _lib.dtype_code(out), out.stride(0), _lib.ptr(ws), ws.numel(),
        _lib.stream_of(dev))
    return out.view(*x.shape[:-1], n)


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """F.linear(x, weight, bias) for bf16 / fp16 x and weight."""
    return _run(x, weight.detach(), weight.shape[0], _lib.LINEAR_PLAIN, bias=bias)


def linear_add_residual(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor,
                        bias: torch.Tensor | None = None) -> torch.Tensor:
    """residual + F.linear(x, weight, bias): the projection rounded to x's dtype,
    then added to the residual in fp32 and rounded to x's dtype, as torch's
    bf16 / fp16 addition does."""
    return _run(x, weight.detach(), weight.shape[0], _lib.LINEAR_PLAIN, bias=bias, residual=residual,
                sum_dtype=_lib.dtype_code(x))


def gate_up_silu_and_mul(x: torch.Tensor, gate_up_weight: torch.Tensor) -> torch.Tensor:
    """SiluAndMul()(F.linear(x, gate_up_weight)) for the packed [gate; up]
    weight [2 I, H]: y = silu(g) * u with g, u the projection rounded to x's
    dtype and silu(g) rounded again, as F.silu on a bf16 / fp16 tensor does."""
    two_i = gate_up_weight.shape[0]
    if two_i % 2:
        raise ValueError("gate_up weight must have an even number of rows (gate | up)")
    return _run(x, gate_up_weight.detach(), two_i // 2, _lib.LINEAR_SILU_AND_MUL)


class LinearBase(nn.Module):
    """layers/linear.py:10-17."""

    def __init__(self, input_size: int, output_size: int):
        super().__init__()
        self.input_size = input_size
        self.output_size = output_size

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError


class ReplicatedLinear(LinearBase):
    """layers/linear.py:20-38."""

    def __init__(self, input_size: int, output_size: int, bias: bool = False):
        super().__init__(input_size, output_size)
        self.weight = nn.Parameter(torch.empty(self.output_size, self.input_size))
        self.weight.weight_loader = self.weight_loader
        if bias:
            self.bias = nn.Parameter(torch.empty(self.output_size))
            self.bias.weight_loader = self.weight_loader
        else:
            self.register_parameter("bias", None)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        param.data.copy_(loaded_weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return linear(x, self.weight, self.bias)


class ColumnParallelLinear(ReplicatedLinear):
    """layers/linear.py:41-61 (one GPU: a plain linear layer)."""


class MergedColumnParallelLinear(ColumnParallelLinear):
    """layers/linear.py:64-75: the [gate; up] (or any list of) row blocks in one
    weight."""

    def __init__(self, input_size: int, output_sizes: list, bias: bool = False):
        self.output_sizes = output_sizes
        super().__init__(input_size, sum(output_sizes), bias=bias)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor, loaded_shard_id: int):
        shard_offset = sum(self.output_sizes[:loaded_shard_id])
        shard_size = self.output_sizes[loaded_shard_id]
        param.data.narrow(0, shard_offset, shard_size).copy_(loaded_weight)

    def forward_silu_and_mul(self, x: torch.Tensor) -> torch.Tensor:
        """SiluAndMul()(self(x)) in one GEMM, for the two-block [gate; up] layer."""
        if len(self.output_sizes) != 2 or self.output_sizes[0] != self.output_sizes[1]:
            raise ValueError("forward_silu_and_mul needs two equal output blocks (gate, up)")
        if self.bias is not None:
            raise ValueError("forward_silu_and_mul has no bias term (gate_up_proj is bias-free)")
        return gate_up_silu_and_mul(x, self.weight)


class QKVParallelLinear(ColumnParallelLinear):
    """layers/linear.py:78-114: packed [q; k; v] rows."""

    def __init__(self, hidden_size: int, head_size: int, total_num_heads: int,
                 total_num_kv_heads: int | None = None, bias: bool = False):
        self.head_size = head_size
        self.total_num_heads = total_num_heads
        self.total_num_kv_heads = total_num_kv_heads or total_num_heads
        self.num_heads = self.total_num_heads
        self.num_kv_heads = self.total_num_kv_heads
        output_size = (self.total_num_heads + 2 * self.total_num_kv_heads) * self.head_size
        super().__init__(hidden_size, output_size, bias)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor, loaded_shard_id: str):
        assert loaded_shard_id in ["q", "k", "v"]
        q_size = self.num_heads * self.head_size
        kv_size = self.num_kv_heads * self.head_size
        if loaded_shard_id == "q":
            shard_offset, shard_size = 0, q_size
        elif loaded_shard_id == "k":
            shard_offset, shard_size = q_size, kv_size
        else:
            shard_offset, shard_size = q_size + kv_size, kv_size
        param.data.narrow(0, shard_offset, shard_size).copy_(loaded_weight)


class RowParallelLinear(ReplicatedLinear):
    """layers/linear.py:136-160 (one GPU: a plain linear layer)."""

    def forward_add_residual(self, x: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        """residual + self(x), with the addition in the GEMM epilogue."""
        return linear_add_residual(x, self.weight, residual, self.bias)
