"""Host-side logic of the Python mirror that runs without a GPU."""
from __future__ import annotations

import pytest
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


def _level(chunks, pages, indptr, last):
    from braidinfer_amd.layers import CascadeLevel
    i32 = torch.int32
    return CascadeLevel(chunks, torch.tensor(pages, dtype=i32), torch.tensor(indptr, dtype=i32),
                        torch.tensor(last, dtype=i32), 0)


def test_cascade_plan_walks_pages_like_the_reference():
    """The per-entry arrays of the cascade plan, worked out by hand from
    cascade_attention.py:112-224 for page_size 4: a system chunk of 7 tokens on two
    pages; a chunk with no pages and one with pages but no tokens (both skipped,
    neither advances the key position); a moved chunk of 12 tokens (rotated by
    -10); a chunk without global_position_start (never rotated); a chunk whose
    last page holds 0 tokens (that page dropped); a one-page chunk on page -1
    moved by 3."""
    from types import SimpleNamespace as NS
    from braidinfer_amd.layers import CascadeAttention

    a = NS(page_table=[5, 6], kv_length=7, cached_position_start=0, global_position_start=0)
    b = NS(page_table=[], kv_length=0, cached_position_start=0, global_position_start=50)
    c = NS(page_table=[9], kv_length=0, cached_position_start=0, global_position_start=50)
    d = NS(page_table=[1, 2, 3], kv_length=12, cached_position_start=100, global_position_start=90)
    e = NS(page_table=[4], kv_length=3, cached_position_start=40)
    f = NS(page_table=[7, 8], kv_length=4, cached_position_start=10, global_position_start=10)
    h = NS(page_table=[-1], kv_length=2, cached_position_start=0, global_position_start=3)
    levels = [_level([a], [5, 6], [0, 2], [3]),
              _level([b, c, d, e, f, h], [9, 1, 2, 3, 4, 7, 8, -1], [0, 0, 1, 4, 5, 7, 8],
                     [0, 0, 4, 3, 0, 2])]
    att = CascadeAttention(4, 128, 1.0, 2, page_size=4, rotary_emb=NS())
    meta = att._chunk_meta(levels)
    page, kstart, delta, info = att._plan(levels, meta, torch.device("cpu"))
    rot = 1 << 16
    assert page.tolist() == [5, 6, 1, 2, 3, 4, 7, -1]
    assert kstart.tolist() == [0, 4, 7, 11, 15, 19, 22, 26]
    assert delta.tolist() == [0, 0, -10, -10, -10, 0, 0, 3]
    assert info.tolist() == [4, 3, 4 | rot, 4 | rot, 4 | rot, 3, 4, 2 | rot]
    # no rotary table: nothing rotates
    plain = CascadeAttention(4, 128, 1.0, 2, page_size=4)
    _, _, _, info2 = plain._plan(levels, plain._chunk_meta(levels), torch.device("cpu"))
    assert info2.tolist() == [4, 3, 4, 4, 4, 3, 4, 2]
    # the plan is cached per level set
    assert att._plan(levels, meta, torch.device("cpu"))[0] is page


def test_cascade_plan_follows_in_place_page_table_edits():
    """A level whose page table is edited in place must not reuse the cached plan."""
    from types import SimpleNamespace as NS
    from braidinfer_amd.layers import CascadeAttention

    a = NS(page_table=[5, 6], kv_length=7, cached_position_start=0, global_position_start=0)
    levels = [_level([a], [5, 6], [0, 2], [3])]
    att = CascadeAttention(4, 128, 1.0, 2, page_size=4)
    dev = torch.device("cpu")
    page, _, _, _ = att._plan(levels, att._chunk_meta(levels), dev)
    assert page.tolist() == [5, 6]
    levels[0].kv_page_indices[1] = 9  # in place, as a page manager might
    page2, _, _, _ = att._plan(levels, att._chunk_meta(levels), dev)
    assert page2.tolist() == [5, 9]


def test_cascade_plan_follows_reassigned_tensors_and_page_size():
    """A level tensor replaced by another object (whose version counter starts
    at 0 again) and a page_size changed on the instance both give a new plan."""
    from types import SimpleNamespace as NS
    from braidinfer_amd.layers import CascadeAttention

    a = NS(page_table=[5, 6], kv_length=7, cached_position_start=0, global_position_start=0)
    levels = [_level([a], [5, 6], [0, 2], [3])]
    att = CascadeAttention(4, 128, 1.0, 2, page_size=4)
    dev = torch.device("cpu")
    assert att._plan(levels, att._chunk_meta(levels), dev)[0].tolist() == [5, 6]
    levels[0].kv_page_indices = torch.tensor([7, 8], dtype=torch.int32)
    assert att._plan(levels, att._chunk_meta(levels), dev)[0].tolist() == [7, 8]
    # page_size 8: the first page now holds 8 tokens, the second starts at key 8
    att.page_size = 8
    _, kstart, _, info = att._plan(levels, att._chunk_meta(levels), dev)
    assert kstart.tolist() == [0, 8] and info.tolist() == [8, 3]


def test_cascade_plan_is_shared_across_layers_without_device_reads():
    """Every layer builds its own levels from the same chunks (the reference's
    Attention.forward calls create_cascade_levels per layer): the second layer
    gets the first layer's device arrays, and levels built by _create_level
    carry host copies, so planning reads nothing back from the device."""
    from types import SimpleNamespace as NS
    from braidinfer_amd.layers import CascadeAttention
    from braidinfer_amd.layers.cascade_attention import _level_arrays

    a = NS(page_table=[3, 4], kv_length=20, cached_position_start=0, global_position_start=0)
    l1 = [_level([a], [3, 4], [0, 2], [4])]
    l2 = [_level([a], [3, 4], [0, 2], [4])]
    att1 = CascadeAttention(4, 128, 1.0, 2, page_size=16)
    att2 = CascadeAttention(4, 128, 1.0, 2, page_size=16)
    dev = torch.device("cpu")
    p1 = att1._plan(l1, att1._chunk_meta(l1), dev)
    p2 = att2._plan(l2, att2._chunk_meta(l2), dev)
    assert p1[0] is p2[0]
    # a level with fresh host copies is not read from its tensors
    lv = _level([a], [3, 4], [0, 2], [4])
    _level_arrays(lv)
    poisoned = lv.host_arrays
    lv.host_arrays = (poisoned[0] + 100,) + poisoned[1:]
    assert _level_arrays(lv)[0].tolist() == [103, 104]
    lv.kv_page_indices[0] = 5  # stale copy: read again
    assert _level_arrays(lv)[0].tolist() == [5, 4]


def test_cascade_query_shape_is_checked_before_launch():
    from braidinfer_amd.layers import CascadeAttention

    att = CascadeAttention(4, 128, 1.0, 2, page_size=16)
    cache = torch.zeros(2, 2, 2, 16, 128, dtype=torch.bfloat16)
    pos = torch.zeros(3, dtype=torch.int64)
    for bad in (torch.zeros(3, 2, 128), torch.zeros(3, 4, 64), torch.zeros(3, 4 * 128 - 8)):
        with pytest.raises(ValueError):
            att.forward(bad.bfloat16(), pos, cache, [], 0)


class _FoldSpy:
    """Stands in for the library and torch.cuda in the folded-weight cache: the
    fold call is counted, not run (no GPU here)."""

    def __init__(self, monkeypatch, capturing=False):
        from braidinfer_amd import _lib
        from braidinfer_amd.kernels import _qkv
        self.folds = 0
        self.capturing = capturing

        def call(name, *args):
            assert name == "bfa_fold_rmsnorm_weight"
            self.folds += 1
            return 0

        class _Stream:
            def synchronize(self):
                pass
        monkeypatch.setattr(_lib, "call", call)
        monkeypatch.setattr(_lib, "stream_of", lambda dev: 0)
        monkeypatch.setattr(_qkv.torch.cuda, "current_stream", lambda dev=None: _Stream())
        monkeypatch.setattr(_qkv.torch.cuda, "is_current_stream_capturing", lambda: self.capturing)
        _qkv.clear_folded_weights()


def test_folded_weight_cache_rules(monkeypatch):
    """The folded copy of (W, norm weight) is made once and reused while both
    tensors are the same objects with the same storage, version counter and
    shape; an in-place change, a new `.data`, a new tensor, or a dropped tensor
    changes that; under graph capture nothing is folded."""
    import gc

    from braidinfer_amd.kernels import _qkv
    spy = _FoldSpy(monkeypatch)
    w = torch.zeros(64, 32, dtype=torch.bfloat16)
    ln = torch.ones(32, dtype=torch.bfloat16)
    a = _qkv.folded_weight(w, ln)
    assert spy.folds == 1 and a.shape == w.shape and a.dtype == w.dtype
    assert _qkv.folded_weight(w, ln) is a and spy.folds == 1           # reused
    ln.mul_(2)                                                          # in place: version moves
    b = _qkv.folded_weight(w, ln)
    assert spy.folds == 2 and b is not a
    w[0].fill_(1)                                                       # in place through a view
    _qkv.folded_weight(w, ln)
    assert spy.folds == 3
    w.data = torch.zeros(64, 32, dtype=torch.bfloat16)                  # new storage
    _qkv.folded_weight(w, ln)
    assert spy.folds == 4 and len(_qkv._folded) == 1
    w2 = w.clone()                                                      # another tensor: its own entry
    _qkv.folded_weight(w2, ln)
    assert spy.folds == 5 and len(_qkv._folded) == 2
    del w2
    gc.collect()
    assert len(_qkv._folded) == 1                                       # dropped with its tensor
    spy.capturing = True
    assert _qkv.folded_weight(w.clone(), ln) is None and spy.folds == 5  # no fold under capture
    assert _qkv.folded_weight(w, ln) is not None and spy.folds == 5      # an existing copy is used
    assert _qkv.clear_folded_weights() == 1 and not _qkv._folded


def test_fold_algebra_in_float64():
    """The identity the folded path rests on, in float64 on the oracle's own
    operand: ((x / rms) * gamma) @ W^T == (x @ (W * gamma)^T) / rms, gamma along
    the hidden (K) axis of W.  Folding gamma along the other axis fails it."""
    g = torch.Generator().manual_seed(7)
    t, h = 5, 64
    x = torch.randn(t, h, generator=g, dtype=torch.float64)
    w = torch.randn(h, h, generator=g, dtype=torch.float64)  # square, so either axis fits
    gamma = torch.rand(h, generator=g, dtype=torch.float64) + 0.5
    inv = 1.0 / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-5)
    ref = ((x * inv) * gamma) @ w.t()
    folded = (x @ (w * gamma[None, :]).t()) * inv
    assert torch.allclose(folded, ref, rtol=1e-12, atol=1e-12)
    wrong_axis = (x @ (w * gamma[:, None]).t()) * inv
    assert not torch.allclose(wrong_axis, ref, rtol=1e-3, atol=1e-3)
