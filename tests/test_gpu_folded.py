"""GPU parity of the prefill with the RMSNorm weight folded into the QKV weight
(bfa_fold_rmsnorm_weight + bfa_fused_rmsnorm_qkv_folded): the variants without
the mixed rounding (kernels/fused_rmsnorm_qkv_{production,minimal_f32,with_bias}.py,
models/llama.py:169-205) project x onto bf16(W * gamma) and scale each row by
1 / rms, instead of projecting a normalised operand written by a pre-pass.

Checked here: the folded weight against its definition (bit for bit), the
folded path against the oracle and against the pre-pass path at the same
tolerance, at prefill and at the 17-64-token decode shapes of the column-pair
kernel (with and without the paged append), the cache of folded weights (an
in-place change of either weight, or a new tensor, folds again;
clear_folded_weights drops them), graph capture with and without a folded copy,
and the entry point's refusal of the other decode shapes.
The parity tests of the variants themselves (test_gpu_qkv.py,
test_gpu_fused_append.py, test_gpu_fp32_mode.py) run through this path at
prefill token counts."""
from __future__ import annotations

import pytest
import torch

import braidinfer_amd
from braidinfer_amd import _lib
from braidinfer_amd.kernels import FusedRMSNormQKV, FusedRMSNormQKVMinimalF32, _qkv
from braidinfer_amd.layers import llama_attention_input
from oracle import torch_ref as R
from tests.helpers import assert_close, bits, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make(seed, t, h, hq, hkv, d, gdtype=torch.bfloat16):
    g = gen(seed)
    n = (hq + 2 * hkv) * d
    return (randn(g, t, h), randn(g, h, mean=1.0, std=0.1).to(gdtype), randn(g, n, h, std=0.02), g)


@pytest.mark.parametrize("gdtype", [torch.bfloat16, torch.float32])
def test_fold_weight_definition(gdtype):
    """folded[n, k] = bf16(W[n, k] * gamma[k]) with the product in fp32."""
    _, ln, w, _ = make(501, 1, 1024, 8, 2, 64, gdtype)
    wd, lnd = w.to(DEV), ln.to(DEV)
    wf = _qkv.folded_weight(wd, lnd)
    exp = (w.float() * ln.float()[None, :]).to(torch.bfloat16)
    assert torch.equal(bits(wf.cpu()), bits(exp))
    _qkv.clear_folded_weights()


@pytest.mark.parametrize("t,h,hq,hkv,d", [(65, 1024, 8, 2, 128), (300, 2048, 32, 4, 64), (1024, 4096, 32, 8, 128)])
def test_folded_against_oracle_and_prepass(monkeypatch, t, h, hq, hkv, d):
    """The Llama chain (minimal_f32 + RoPE) and the production variant through the
    folded path, against the oracle and against the pre-pass path."""
    x, ln, w, g = make(502, t, h, hq, hkv, d)
    cache = R.cos_sin_cache(d, 8192, 5e5)
    pos = torch.randint(0, 8192, (t,), generator=g)
    args = (x.to(DEV), ln.to(DEV), w.to(DEV))
    ref = R.llama_attention_input(x, ln, w, hq, hkv, 1e-5, pos, cache)
    folded = llama_attention_input(*args, hq, hkv, 1e-5, pos.to(DEV), cache.to(DEV))
    for g_, e_, name in zip(folded, ref, "qkv"):
        assert_close(g_, e_, what=f"folded llama {name} t={t}")
    monkeypatch.setattr(_qkv, "_FOLD_MIN_TOKENS", 1 << 40)  # the pre-pass path
    prepass = llama_attention_input(*args, hq, hkv, 1e-5, pos.to(DEV), cache.to(DEV))
    for a, b, name in zip(folded, prepass, "qkv"):
        assert_close(a, b, what=f"folded against pre-pass {name} t={t}")
    monkeypatch.undo()
    ref = R.split_qkv(R.qkv_production(x, ln, w, 1e-6), hq, hkv)
    got = FusedRMSNormQKV.forward(*args, hq, hkv, eps=1e-6)
    for g_, e_ in zip(got, ref):
        assert_close(g_, e_, what=f"folded production t={t}")
    braidinfer_amd.check_device_status()
    _qkv.clear_folded_weights()


def test_folded_cache_follows_the_weights():
    """An in-place change of the norm weight or of W, and a new tensor, fold
    again; clear_folded_weights drops every copy."""
    t, h, hq, hkv, d = 128, 1024, 8, 2, 128
    x, ln, w, _ = make(503, t, h, hq, hkv, d)
    xd, lnd, wd = x.to(DEV), ln.to(DEV), w.to(DEV)
    _qkv.clear_folded_weights()

    def check(ln_cpu, w_cpu, what):
        got = FusedRMSNormQKVMinimalF32.forward(xd, lnd, wd, hq, hkv, eps=1e-5)
        ref = R.split_qkv(R.qkv_minimal_f32(x, ln_cpu, w_cpu, 1e-5), hq, hkv)
        for g_, e_ in zip(got, ref):
            assert_close(g_, e_, what=what)
    check(ln, w, "first call")
    assert len(_qkv._folded) == 1
    check(ln, w, "second call (cached)")
    assert len(_qkv._folded) == 1
    lnd.mul_(1.5)  # in place: the version counter moves
    check(ln.float().mul(1.5).to(ln.dtype), w, "norm weight changed in place")
    wd[: 3 * d].neg_()
    w2 = w.clone()
    w2[: 3 * d] = -w2[: 3 * d]
    check(ln.float().mul(1.5).to(ln.dtype), w2, "weight changed in place")
    assert len(_qkv._folded) == 1
    # a new weight tensor: a second entry, dropped with the tensor
    w3 = wd.clone()
    FusedRMSNormQKVMinimalF32.forward(xd, lnd, w3, hq, hkv, eps=1e-5)
    assert len(_qkv._folded) == 2
    del w3
    import gc
    gc.collect()
    assert len(_qkv._folded) == 1
    assert _qkv.clear_folded_weights() == 1 and not _qkv._folded
    braidinfer_amd.check_device_status()


@pytest.mark.parametrize("warm", [True, False])
def test_folded_graph_capture(warm):
    """Captured after a call has folded the weight, the graph runs the folded
    path; captured with no folded copy, the pre-pass path (no fold is captured).
    Every replay equals the eager call bit for bit."""
    t, h, hq, hkv, d = 256, 2048, 16, 4, 128
    x, ln, w, g = make(504, t, h, hq, hkv, d)
    xd, lnd, wd = x.to(DEV), ln.to(DEV), w.to(DEV)
    _qkv.clear_folded_weights()
    if warm:
        FusedRMSNormQKVMinimalF32.forward(xd, lnd, wd, hq, hkv, eps=1e-5)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = FusedRMSNormQKVMinimalF32.forward(xd, lnd, wd, hq, hkv, eps=1e-5)
    assert len(_qkv._folded) == (1 if warm else 0)
    for r in range(4):
        xd.copy_(randn(g, t, h).to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        replayed = [o.clone() for o in got]
        if not warm:
            # the eager call below would fold; compare with the pre-pass path instead
            _qkv.clear_folded_weights()
            old = _qkv._FOLD_MIN_TOKENS
            _qkv._FOLD_MIN_TOKENS = 1 << 40
            try:
                eager = FusedRMSNormQKVMinimalF32.forward(xd, lnd, wd, hq, hkv, eps=1e-5)
            finally:
                _qkv._FOLD_MIN_TOKENS = old
        else:
            eager = FusedRMSNormQKVMinimalF32.forward(xd, lnd, wd, hq, hkv, eps=1e-5)
        torch.cuda.synchronize()
        for a, b in zip(replayed, eager):
            assert torch.equal(bits(a.cpu()), bits(b.cpu())), f"replay {r} differs"
    braidinfer_amd.check_device_status()
    _qkv.clear_folded_weights()


def test_folded_entry_refuses_other_decode_shapes():
    """Below 65 tokens the folded entry point takes the column-pair kernel's shapes
    only: 64 tokens on 48 column pairs is BFA_ERR_UNSUPPORTED (and the Python
    layer runs the unfolded path for them)."""
    t, h, hq, hkv, d = 64, 1024, 8, 2, 128
    x, ln, w, _ = make(505, t, h, hq, hkv, d)
    xd, wd = x.to(DEV), w.to(DEV)
    n = (hq + 2 * hkv) * d
    out = torch.empty(t, n, dtype=torch.float32, device=DEV)
    ws = torch.empty(_lib.workspace_size("bfa_fused_rmsnorm_qkv_workspace_size", t, h, n, d), dtype=torch.uint8,
                     device=DEV)
    no_cache = (None, 0, 0, 0, 0, 0, 0, 0, None, 0, 0, None, None, 0, 0, None, 0, 0, 0)
    with pytest.raises(_lib.BraidinferAMDError, match="column-pair"):
        _lib.call("bfa_fused_rmsnorm_qkv_folded", xd.data_ptr(), _lib.BF16, t, h, h, 1e-5, wd.data_ptr(),
                  _lib.BF16, n, h, None, 0, hq, hkv, _lib.F32, None, 0, None, 0, out.data_ptr(), _lib.F32, n,
                  ws.data_ptr(), ws.numel(), *no_cache, _lib.status_word(torch.device(DEV)).data_ptr(),
                  _lib.stream_of(torch.device(DEV)))


@pytest.mark.parametrize("t", [17, 40, 64])
def test_folded_decode_pair(monkeypatch, t):
    """Llama-3-8B decode batches of 17-64 tokens: the column-pair kernel on x and
    the folded weight, against the oracle and against the in-kernel gamma form;
    with the paged append, the cache holds the output's k/v bit for bit."""
    h, hq, hkv, d = 4096, 32, 8, 128
    x, ln, w, g = make(506, t, h, hq, hkv, d)
    cache = R.cos_sin_cache(d, 8192, 5e5)
    pos = torch.randint(0, 8192, (t,), generator=g)
    args = (x.to(DEV), ln.to(DEV), w.to(DEV))
    _qkv.clear_folded_weights()
    ref = R.llama_attention_input(x, ln, w, hq, hkv, 1e-5, pos, cache)
    folded = llama_attention_input(*args, hq, hkv, 1e-5, pos.to(DEV), cache.to(DEV))
    assert len(_qkv._folded) == 1, "the decode batch did not take the folded path"
    for g_, e_, name in zip(folded, ref, "qkv"):
        assert_close(g_, e_, what=f"folded decode {name} t={t}")
    monkeypatch.setattr(_qkv, "_FOLD_MIN_TOKENS", 1 << 40)  # gamma on the weight fragments in the kernel
    unfolded = llama_attention_input(*args, hq, hkv, 1e-5, pos.to(DEV), cache.to(DEV))
    monkeypatch.undo()
    for a, b, name in zip(folded, unfolded, "qkv"):
        assert_close(a, b, what=f"folded against in-kernel gamma {name} t={t}")
    # with the paged append (HND cache, 16-slot pages, shuffled page list)
    from braidinfer_amd.kernels import PagedKVAppend
    ps, start = 16, 5
    need = (start + t + ps - 1) // ps
    kv_indices = torch.randperm(need + 3, generator=g)[:need].to(torch.int32)
    layer = torch.zeros(need + 3, 2, hkv, ps, d, dtype=torch.bfloat16, device=DEV)
    cpos = torch.arange(start, start + t, dtype=torch.int64)
    pkv = PagedKVAppend(layer, kv_indices.to(DEV), cpos.to(DEV), ps, "HND")
    q2, k2, v2 = llama_attention_input(*args, hq, hkv, 1e-5, pos.to(DEV), cache.to(DEV), paged_kv=pkv)
    torch.cuda.synchronize()
    for a, b in zip((q2, k2, v2), folded):
        assert torch.equal(bits(a.cpu()), bits(b.cpu())), "the append call's output differs from the plain call's"
    exp, skipped = R.append_to_paged_kv_cache(k2.cpu().reshape(t, hkv, d), v2.cpu().reshape(t, hkv, d),
                                              torch.zeros(need + 3, 2, hkv, ps, d, dtype=torch.bfloat16),
                                              kv_indices, cpos, ps, "HND")
    assert skipped == [] and torch.equal(bits(layer.cpu()), bits(exp))
    braidinfer_amd.check_device_status()
    _qkv.clear_folded_weights()
