"""Writes tests/golden/golden.npz: small seeded inputs and the expected outputs of
every function on the path, computed by the float64 numpy restatement
(oracle/numpy_ref.py) with the reference's rounding points emulated.

The fixtures pin the torch restatement on the CPU (tests/test_golden.py) and
the HIP kernels on the GPU independently of the torch version a machine has.
bf16-valued arrays are stored as float32 (every bf16 value is exactly
representable); fp32-result arrays are stored as float64.

    python -m tests.golden.make_golden          # rewrites golden.npz
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

from oracle import numpy_ref as N

OUT = Path(__file__).resolve().parent / "golden.npz"
SEED = 20240611


def _bf16(rng, shape, std=1.0, mean=0.0):
    return N.round_bf16(rng.standard_normal(shape) * std + mean)


def build() -> dict:
    rng = np.random.default_rng(SEED)
    f = {}

    # RMSNorm / add+RMSNorm (layers/layernorm.py:35-57)
    x = _bf16(rng, (8, 256))
    res = _bf16(rng, (8, 256))
    w = _bf16(rng, (256,), 0.1, 1.0)
    f["rms.x"], f["rms.res"], f["rms.w"] = x, res, w
    f["rms.eps"] = np.array(1e-5)
    f["rms.y"] = N.rms_forward(x, w, 1e-5)
    y, r = N.add_rms_forward(x, res, w, 1e-5)
    f["add_rms.y"], f["add_rms.res_out"] = y, r

    # RMSNormF32 with an extreme gamma column (tests/test_rmsnorm_f32.py:71-96)
    x = _bf16(rng, (4, 128))
    w = _bf16(rng, (128,), 0.1, 1.0)
    w[0] = 96.5
    f["rmsf32.x"], f["rmsf32.w"] = x, w
    f["rmsf32.y"] = N.rmsnorm_f32(x, w, 1e-6)

    # embedding gather (layers/embed_head.py:28-29): bit-exact
    table = _bf16(rng, (512, 64), 0.02)
    ids = np.concatenate([[0, 511], rng.integers(0, 512, 35)]).astype(np.int64)
    f["emb.table"], f["emb.ids"] = table, ids
    f["emb.y"] = N.embedding(ids, table)

    # SiLU * mul (layers/activation.py:11-13)
    x = _bf16(rng, (16, 192))
    f["silu.x"] = x
    f["silu.y"] = N.silu_and_mul(x)

    # RoPE (layers/rotary_embedding.py:6-65), neox half split, table in float32
    d, maxp = 64, 64
    tab = N.to_f32(N.cos_sin_table(d, maxp, 1e4)).astype(np.float64)
    pos = np.concatenate([[0, maxp - 1], rng.integers(0, maxp, 10)]).astype(np.int64)
    q = _bf16(rng, (12, 4 * d))
    k = _bf16(rng, (12, 2 * d))
    f["rope.table"], f["rope.pos"], f["rope.q"], f["rope.k"] = tab, pos, q, k
    f["rope.q_out"] = N.rotary_forward(tab, pos, q, d)
    f["rope.k_out"] = N.rotary_forward(tab, pos, k, d)

    # fused RMSNorm+QKV, all variants (kernels/fused_rmsnorm_qkv_*.py)
    t, h, hq, hkv, d = 6, 128, 4, 2, 32
    n = (hq + 2 * hkv) * d
    x = _bf16(rng, (t, h))
    ln = _bf16(rng, (h,), 0.1, 1.0)
    wq = _bf16(rng, (n, h), 0.05)
    b = _bf16(rng, (n,), 0.05)
    f["qkv.x"], f["qkv.ln"], f["qkv.w"], f["qkv.b"] = x, ln, wq, b
    f["qkv.geom"] = np.array([hq, hkv, d])
    f["qkv.mixed"] = N.qkv(x, ln, wq, b, 1e-6, "mixed")
    f["qkv.production"] = N.qkv(x, ln, wq, None, 1e-6, "production")
    f["qkv.f32"] = N.qkv(x, ln, wq, None, 1e-6, "f32")
    f["qkv.with_bias"] = N.qkv(x, ln, wq, b, 1e-6, "with_bias")

    # Qwen3 chain: mixed QKV -> per-head q/k RMSNorm (extreme k gamma) -> RoPE
    # (models/qwen3.py:236-309), and the Llama chain: fp32 QKV -> RoPE in fp32 ->
    # bf16 (models/llama.py:169-205)
    qn = _bf16(rng, (d,), 0.1, 1.0)
    kn = N.round_bf16(np.exp(rng.uniform(np.log(0.05), np.log(100.0), d)))
    ctab = N.to_f32(N.cos_sin_table(d, 128, 1e6)).astype(np.float64)
    cpos = rng.integers(0, 128, t).astype(np.int64)
    f["chain.qn"], f["chain.kn"], f["chain.table"], f["chain.pos"] = qn, kn, ctab, cpos
    base = N.qkv(x, ln, wq, None, 1e-6, "mixed")
    nq = N.head_norm(base[:, : hq * d].reshape(t, hq, d), qn, 1e-6, "bf16")
    nk = N.head_norm(base[:, hq * d:(hq + hkv) * d].reshape(t, hkv, d), kn, 1e-6, "bf16")
    f["qwen3.q"] = N.rotary_forward(ctab, cpos, nq.reshape(t, -1), d).reshape(t, hq, d)
    f["qwen3.k"] = N.rotary_forward(ctab, cpos, nk.reshape(t, -1), d).reshape(t, hkv, d)
    f["qwen3.v"] = base[:, (hq + hkv) * d:].reshape(t, hkv, d)
    base = N.qkv(x, ln, wq, None, 1e-5, "f32")
    f["llama.q"] = N.round_bf16(N.rotary_forward(ctab, cpos, base[:, : hq * d], d, "f32")).reshape(t, hq, d)
    f["llama.k"] = N.round_bf16(
        N.rotary_forward(ctab, cpos, base[:, hq * d:(hq + hkv) * d], d, "f32")).reshape(t, hkv, d)
    f["llama.v"] = N.round_bf16(base[:, (hq + hkv) * d:]).reshape(t, hkv, d)

    # differential-RoPE re-rotation of paged K (layers/cascade_attention.py:143-174):
    # HND cache [pages, 2, Hkv, page, D], two chunks, a negative delta wraps
    pages, hkv, ps, d = 6, 2, 4, 32
    kv = _bf16(rng, (pages, 2, hkv, ps, d))
    pidx = np.array([4, 1, 5, 0, 2], dtype=np.int32)
    indptr = np.array([0, 2, 5], dtype=np.int32)
    delta = np.array([37, -5], dtype=np.int64)
    last = np.array([4, 3], dtype=np.int32)
    rtab = N.to_f32(N.cos_sin_table(d, 64, 1e4)).astype(np.float64)
    out = np.zeros((len(pidx), ps, hkv, d))
    for c in range(2):
        p = int(delta[c]) % rtab.shape[0]
        for e in range(int(indptr[c]), int(indptr[c + 1])):
            nrow = int(last[c]) if e == int(indptr[c + 1]) - 1 else ps
            page = kv[int(pidx[e]), 0, :, :nrow].transpose(1, 0, 2)  # [n, hkv, d]
            out[e, :nrow] = N.rope(page, rtab[p, : d // 2], rtab[p, d // 2:])
    f["rerot.kv"], f["rerot.pidx"], f["rerot.indptr"] = kv, pidx, indptr
    f["rerot.delta"], f["rerot.last"], f["rerot.table"], f["rerot.out"] = delta, last, rtab, out

    # paged KV append (kernels/kv_cache_utils.py:9-78): HND cache, shuffled page
    # table, one negative position (lands on the last page of the table through
    # Python floor division and negative indexing) and one past the table (skipped)
    pages, hkv, ps, d = 7, 2, 4, 16
    cache0 = _bf16(rng, (pages, 2, hkv, ps, d))
    ptab = np.array([5, 2, 6, 0], dtype=np.int32)
    kpos = np.array([0, 1, 2, 3, 4, 9, 14, 15, -3, 16], dtype=np.int64)
    ka = _bf16(rng, (len(kpos), hkv, d))
    va = _bf16(rng, (len(kpos), hkv, d))
    app, skipped = N.append_paged_kv(ka, va, cache0, ptab, kpos, ps)
    assert skipped == [9]
    f["kvapp.cache"], f["kvapp.ptab"], f["kvapp.pos"] = cache0, ptab, kpos
    f["kvapp.k"], f["kvapp.v"], f["kvapp.out"] = ka, va, app

    # bf16-valued arrays and the float32 RoPE tables fit float32 exactly;
    # fp32 results computed in float64 keep float64
    keep64 = {"rmsf32.y", "qkv.f32", "qkv.with_bias"}
    return {k: (v.astype(np.float32) if v.dtype == np.float64 and k not in keep64 else v)
            for k, v in f.items()}


def main() -> None:
    np.savez_compressed(OUT, **build())
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
