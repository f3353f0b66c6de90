"""Golden fixtures (tests/golden/golden.npz, written by tests/golden/make_golden.py
from the float64 numpy restatement).

CPU: the committed file is exactly what the script produces, and the torch
oracle reproduces every expected output (bf16 results within one bf16 ulp,
fp32 results to float32 precision, the gather bit for bit).
GPU: the HIP path reproduces them through the C ABI, to the path's tolerance
|d| <= 2e-2 + 1e-2 |r| (tests/helpers.py), the gather bit for bit.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import torch_ref as R
from tests.golden.make_golden import build
from tests.helpers import assert_close

GOLDEN = Path(__file__).resolve().parent / "golden" / "golden.npz"
BF16_ULP = 2.0 ** -7


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN) as z:
        return {k: z[k] for k in z.files}


def bf(a) -> torch.Tensor:
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16)


def f32(a) -> torch.Tensor:
    return torch.from_numpy(np.asarray(a, np.float32))


def within_ulp(got: torch.Tensor, exp: np.ndarray, what: str, max_frac: float = 0.02):
    g = got.detach().double().cpu().numpy().reshape(exp.shape)
    e = exp.astype(np.float64)
    diff = np.abs(g - e)
    assert np.all(diff <= BF16_ULP * np.abs(e) + 1e-30), f"{what}: beyond one bf16 ulp ({diff.max():.3e})"
    assert float(np.mean(diff > 0)) <= max_frac, f"{what}: {np.mean(diff > 0):.3f} of elements differ"


# ------------------------------------------------------------------------ CPU
def test_fixture_file_is_what_the_script_writes(gold):
    fresh = build()
    assert sorted(fresh) == sorted(gold)
    for k, v in fresh.items():
        assert v.dtype == gold[k].dtype and np.array_equal(v, gold[k]), k


def test_torch_oracle_reproduces_golden(gold):
    g = gold
    eps = float(g["rms.eps"])
    within_ulp(R.rms_forward(bf(g["rms.x"]), bf(g["rms.w"]), eps), g["rms.y"], "rms")
    y, r = R.add_rms_forward(bf(g["rms.x"]), bf(g["rms.res"]), bf(g["rms.w"]), eps)
    within_ulp(y, g["add_rms.y"], "add_rms y")
    within_ulp(r, g["add_rms.res_out"], "add_rms residual")
    np.testing.assert_allclose(R.rmsnorm_f32(bf(g["rmsf32.x"]), bf(g["rmsf32.w"]), 1e-6).numpy(),
                               g["rmsf32.y"], rtol=2e-6, atol=1e-6)
    emb = R.embedding(torch.from_numpy(g["emb.ids"]), bf(g["emb.table"]))
    assert np.array_equal(emb.float().numpy(), g["emb.y"])
    within_ulp(R.silu_and_mul(bf(g["silu.x"])), g["silu.y"], "silu")
    q, k = R.rotary_forward(f32(g["rope.table"]), 64, torch.from_numpy(g["rope.pos"]),
                            bf(g["rope.q"]), bf(g["rope.k"]))
    within_ulp(q, g["rope.q_out"], "rope q")
    within_ulp(k, g["rope.k_out"], "rope k")
    x, ln, w, b = bf(g["qkv.x"]), bf(g["qkv.ln"]), bf(g["qkv.w"]), bf(g["qkv.b"])
    within_ulp(R.qkv_mixed_precision(x, ln, w, b, 1e-6), g["qkv.mixed"], "qkv mixed", 0.05)
    within_ulp(R.qkv_production(x, ln, w, 1e-6), g["qkv.production"], "qkv production", 0.05)
    np.testing.assert_allclose(R.qkv_minimal_f32(x, ln, w, 1e-6).numpy(), g["qkv.f32"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(R.qkv_with_bias(x, ln, w, b, 1e-6).numpy(), g["qkv.with_bias"],
                               rtol=1e-5, atol=1e-6)
    hq, hkv, d = (int(v) for v in g["qkv.geom"])
    pos, tab = torch.from_numpy(g["chain.pos"]), f32(g["chain.table"])
    q, k, v = R.qwen3_attention_input(x, ln, w, None, hq, hkv, 1e-6, pos, tab,
                                      bf(g["chain.qn"]), bf(g["chain.kn"]))
    for got, name in ((q, "q"), (k, "k"), (v, "v")):
        within_ulp(got, g[f"qwen3.{name}"], f"qwen3 {name}", 0.05)
    q, k, v = R.llama_attention_input(x, ln, w, hq, hkv, 1e-5, pos, tab)
    for got, name in ((q, "q"), (k, "k"), (v, "v")):
        within_ulp(got, g[f"llama.{name}"], f"llama {name}", 0.05)
    out = R.rerotate_paged_k(bf(g["rerot.kv"]), torch.from_numpy(g["rerot.pidx"]),
                             torch.from_numpy(g["rerot.indptr"]), torch.from_numpy(g["rerot.delta"]),
                             torch.from_numpy(g["rerot.last"]), f32(g["rerot.table"]))
    within_ulp(out, g["rerot.out"], "rerotate")
    cache, skipped = R.append_to_paged_kv_cache(bf(g["kvapp.k"]), bf(g["kvapp.v"]), bf(g["kvapp.cache"]),
                                                torch.from_numpy(g["kvapp.ptab"]),
                                                torch.from_numpy(g["kvapp.pos"]), 4)
    assert skipped == [9]
    assert np.array_equal(cache.float().numpy(), g["kvapp.out"]), "KV append must be bit-exact"


# ------------------------------------------------------------------------ GPU
@pytest.mark.gpu
def test_hip_path_reproduces_golden(gold):
    from braidinfer_amd.kernels import (FusedRMSNormQKV, FusedRMSNormQKVMinimalF32,
                                        FusedRMSNormQKVMixedPrecision, FusedRMSNormQKVWithBias,
                                        RMSNormF32)
    from braidinfer_amd.layers import (RMSNorm, RotaryEmbedding, embedding, llama_attention_input,
                                       qwen3_attention_input, rerotate_paged_k, rms_norm,
                                       silu_and_mul)
    g, dev = gold, "cuda"

    def on(t):
        return t.to(dev)

    def close(got, key, what=None):
        assert_close(got.cpu(), torch.from_numpy(np.asarray(g[key], np.float64)).reshape(got.shape),
                     what=what or key)

    eps = float(g["rms.eps"])
    close(rms_norm(on(bf(g["rms.x"])), on(bf(g["rms.w"])), eps), "rms.y")
    norm = RMSNorm(256, eps).to(dev)
    with torch.no_grad():
        norm.weight.data = on(bf(g["rms.w"]))
    y, r = norm(on(bf(g["rms.x"])), on(bf(g["rms.res"])))
    close(y, "add_rms.y")
    close(r, "add_rms.res_out")
    close(RMSNormF32.forward(on(bf(g["rmsf32.x"])), on(bf(g["rmsf32.w"])), 1e-6), "rmsf32.y")
    emb = embedding(on(torch.from_numpy(g["emb.ids"])), on(bf(g["emb.table"])))
    assert np.array_equal(emb.float().cpu().numpy(), g["emb.y"]), "gather must be bit-exact"
    close(silu_and_mul(on(bf(g["silu.x"]))), "silu.y")
    rope = RotaryEmbedding(64, 64, 64, 1e4).to(dev)
    rope.cos_sin_cache = on(f32(g["rope.table"]))
    q, k = rope(on(torch.from_numpy(g["rope.pos"])), on(bf(g["rope.q"])), on(bf(g["rope.k"])))
    close(q, "rope.q_out")
    close(k, "rope.k_out")
    x, ln, w, b = (on(bf(g[f"qkv.{n}"])) for n in ("x", "ln", "w", "b"))
    hq, hkv, d = (int(v) for v in g["qkv.geom"])
    for cls, key, args in ((FusedRMSNormQKVMixedPrecision, "qkv.mixed", (x, ln, w, b)),
                           (FusedRMSNormQKV, "qkv.production", (x, ln, w)),
                           (FusedRMSNormQKVMinimalF32, "qkv.f32", (x, ln, w)),
                           (FusedRMSNormQKVWithBias, "qkv.with_bias", (x, ln, w, b))):
        q, k, v = cls.forward(*args, hq, hkv, eps=1e-6)
        close(torch.cat([t.reshape(x.shape[0], -1) for t in (q, k, v)], dim=1), key)
    pos, tab = on(torch.from_numpy(g["chain.pos"])), on(f32(g["chain.table"]))
    q, k, v = qwen3_attention_input(x, ln, w, None, hq, hkv, 1e-6, pos, tab,
                                    on(bf(g["chain.qn"])), on(bf(g["chain.kn"])))
    for got, name in ((q, "q"), (k, "k"), (v, "v")):
        close(got, f"qwen3.{name}")
    q, k, v = llama_attention_input(x, ln, w, hq, hkv, 1e-5, pos, tab)
    for got, name in ((q, "q"), (k, "k"), (v, "v")):
        close(got, f"llama.{name}")
    out = rerotate_paged_k(on(bf(g["rerot.kv"])), on(torch.from_numpy(g["rerot.pidx"])),
                           on(torch.from_numpy(g["rerot.indptr"])), on(torch.from_numpy(g["rerot.delta"])),
                           on(torch.from_numpy(g["rerot.last"])), on(f32(g["rerot.table"])))
    close(out, "rerot.out")
    from braidinfer_amd.kernels import append_to_paged_kv_cache_custom
    import braidinfer_amd
    braidinfer_amd.check_device_status()
    cache = on(bf(g["kvapp.cache"]))
    with pytest.warns(RuntimeWarning, match="skipped"):
        append_to_paged_kv_cache_custom(on(bf(g["kvapp.k"])), on(bf(g["kvapp.v"])), cache,
                                        on(torch.from_numpy(g["kvapp.ptab"])),
                                        on(torch.from_numpy(g["kvapp.pos"])), 4)
        braidinfer_amd.check_device_status()
    assert np.array_equal(cache.float().cpu().numpy(), g["kvapp.out"]), "KV append must be bit-exact"
