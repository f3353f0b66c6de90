"""The C-ABI library loads and exports every entry point include/*.h declares;
host-side argument validation returns errors without touching a GPU."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

import braidinfer_amd
from braidinfer_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "braidinfer_amd.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(bfa_\w+)\s*\(", text, re.M)))


def test_library_loads_and_exports_header_symbols():
    lib = braidinfer_amd.load()
    names = declared_symbols()
    assert len(names) >= 14
    for name in names:
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"
    assert sorted(_lib.exported_symbols()) == names, "ctypes signatures must cover the header exactly"
    assert lib.bfa_abi_version() == _lib.ABI_VERSION


def test_invalid_arguments_are_rejected_on_the_host():
    lib = braidinfer_amd.load()
    rc = lib.bfa_rms_norm(None, None, None, 2, 2, 4, 1, 64, 64, 0, 64, 0, ctypes.c_float(1e-6), None)
    assert rc == -1 and b"null pointer" in lib.bfa_last_error()
    rc = lib.bfa_silu_and_mul(None, None, 9, 1, 8, 16, 8, None)
    assert rc == -1 and b"dtype" in lib.bfa_last_error()
    rc = lib.bfa_rerotate_paged_k(None, 2, 1, 1, 16, 24, None, 1, None, None, None, 4, 1, None,
                                  16, None, 0, ctypes.c_float(1e-6), None, None, None)
    assert rc == -1 and b"head_dim" in lib.bfa_last_error()
    with pytest.raises(ValueError):
        _lib.call("bfa_silu_and_mul", None, None, 9, 1, 8, 16, 8, None)


def test_workspace_size_plan():
    # decode: operand + split-K partials; prefill with a fused epilogue: operand only
    ws = _lib.call("bfa_fused_rmsnorm_qkv_workspace_size", 64, 4096, 6144, 128)
    assert ws >= 64 * 4096 * 2 + 64 * 6144 * 4
    ws = _lib.call("bfa_fused_rmsnorm_qkv_workspace_size", 8192, 4096, 6144, 128)
    assert ws == 8192 * 4096 * 2
    ws = _lib.call("bfa_fused_rmsnorm_qkv_workspace_size", 300, 512, 800, 80)
    assert ws == (300 * 512 * 2 + 255) // 256 * 256 + (300 * 800 * 4 + 255) // 256 * 256


def test_cascade_workspace_size_plan(tuning):
    """Cascade attention's workspace: split partials (m, l and 128 accumulators
    per row) for the decode form and the fused kernel; from 97 query rows per kv
    head also the flat form's K and V^T copies of the padded keys and their
    positions.  Qwen3 geometry over 4096 keys (256 pages of 16)."""
    def a256(v):
        return (v + 255) // 256 * 256

    hq, hkv, d, entries, ps = 16, 8, 128, 256, 16
    part = lambda splits, rows: splits * hkv * rows * (d + 2) * 4
    copies = 2 * a256(hkv * 4096 * d * 2) + a256(4096 * 4)
    # 256 queries = 512 rows: flat form, 4 row blocks of 128 x 8 heads, split 8 ways
    assert _lib.call("bfa_cascade_attention_workspace_size", 256, hq, hkv, d, entries, ps) == \
        a256(part(8, 512)) + copies
    # 48 queries = 96 rows: the fused kernel, 2 x 8 row blocks split 32 ways, no copies
    assert _lib.call("bfa_cascade_attention_workspace_size", 48, hq, hkv, d, entries, ps) == part(32, 96)
    # forcing the fused kernel drops the copies (256 queries: 8 x 8 blocks, 8 splits)
    tuning("CASCADE_FLAT", 0)
    assert _lib.call("bfa_cascade_attention_workspace_size", 256, hq, hkv, d, entries, ps) == part(8, 512)
    # no attended pages: nothing to copy or merge
    assert _lib.call("bfa_cascade_attention_workspace_size", 256, hq, hkv, d, 0, ps) == 0


def test_no_cpu_path():
    """The product path refuses CPU tensors instead of falling back."""
    from braidinfer_amd.layers import RMSNorm, SiluAndMul
    with pytest.raises(RuntimeError, match="ROCm"):
        RMSNorm(64)(torch.randn(2, 64))
    with pytest.raises(RuntimeError, match="ROCm"):
        SiluAndMul()(torch.randn(2, 64))
