"""Host-side logic of the Python mirror that runs without a GPU."""
from __future__ import annotations

import torch

from braidinfer_amd.kernels.fused_rmsnorm_qkv_with_bias import sanitize_bias
from braidinfer_amd.layers import get_rope
from braidinfer_amd.layers.rotary_embedding import RotaryEmbedding
from oracle import torch_ref as R


def test_bias_sanitization_matches_reference():
    b = torch.tensor([float("nan"), float("inf"), -float("inf"), 1e30, 0.25], dtype=torch.float32)
    assert torch.equal(sanitize_bias(b), R.sanitize_bias(b))
    assert sanitize_bias(None) is None


def test_rope_table_is_the_reference_table():
    rope = RotaryEmbedding(128, 128, 8192, 5e5)
    assert rope.cos_sin_cache.dtype == torch.float32
    assert torch.equal(rope.cos_sin_cache, R.cos_sin_cache(128, 8192, 5e5))
    assert "cos_sin_cache" not in rope.state_dict()  # non-persistent buffer


def test_get_rope_is_cached():
    a = get_rope(64, 64, 2048, 10000.0)
    assert get_rope(64, 64, 2048, 10000.0) is a
