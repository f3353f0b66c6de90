"""The allocation-free QKV entry point (bfa_fused_rmsnorm_qkv_noalloc) against
bfa_fused_rmsnorm_qkv with a caller workspace, through the C ABI.  Both run the
same kernels with the same plan, so the outputs must agree bit for bit; two
calls in a row, the second smaller, check that the scratch the library keeps
between calls does not leak into the next result."""
from __future__ import annotations

import pytest
import torch

from braidinfer_amd import _lib
from oracle import torch_ref as R
from tests.helpers import gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(seed, t, h, hq, hkv, d, theta, qk_norm):
    g = gen(seed)
    n = (hq + 2 * hkv) * d
    x = randn(g, t, h).to(DEV)
    ln = randn(g, h, mean=1.0, std=0.1).to(DEV)
    w = randn(g, n, h, std=0.02).to(DEV)
    pos = torch.randint(0, 2048, (t,), generator=g).to(DEV)
    cs = R.cos_sin_cache(d, 4096, theta).to(DEV)
    qn = kn = None
    if qk_norm:
        qn = randn(g, d, mean=1.0, std=0.1).to(DEV)
        kn = torch.exp(torch.empty(d).uniform_(-3.0, 4.6, generator=g)).bfloat16().to(DEV)
    return x, ln, w, pos, cs, qn, kn


def _args(x, ln, w, pos, cs, qn, kn, hq, hkv, out, f32):
    t, h = x.shape
    n = w.shape[0]
    dev = x.device
    return [
        _lib.ptr(x), _lib.dtype_code(x), t, h, x.stride(0), _lib.ptr(ln), _lib.dtype_code(ln), 1e-5,
        0 if f32 else 1, _lib.ptr(w), _lib.dtype_code(w), n, w.stride(0), None, 0, hq, hkv,
        _lib.F32 if f32 else _lib.BF16, _lib.ptr(qn), _lib.ptr(kn), _lib.BF16 if qn is not None else 0,
        1e-6, _lib.BF16, _lib.ptr(pos), _lib.I64, _lib.ptr(cs), cs.shape[0],
        _lib.ptr(out), _lib.dtype_code(out), out.stride(0)], _lib.ptr(_lib.status_word(dev)), _lib.stream_of(dev)


def _with_workspace(x, ln, w, pos, cs, qn, kn, hq, hkv, f32):
    t, h = x.shape
    n = w.shape[0]
    out = torch.empty(t, n, dtype=torch.float32 if f32 else torch.bfloat16, device=DEV)
    ws_bytes = _lib.call("bfa_fused_rmsnorm_qkv_workspace_size", t, h, n, n // (hq + 2 * hkv))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=DEV)
    a, status, stream = _args(x, ln, w, pos, cs, qn, kn, hq, hkv, out, f32)
    _lib.call("bfa_fused_rmsnorm_qkv", *a, _lib.ptr(ws), ws.numel(), status, stream)
    return out


def _no_alloc(x, ln, w, pos, cs, qn, kn, hq, hkv, f32):
    out = torch.full((x.shape[0], w.shape[0]), float("nan"), dtype=torch.float32 if f32 else torch.bfloat16,
                     device=DEV)
    a, status, stream = _args(x, ln, w, pos, cs, qn, kn, hq, hkv, out, f32)
    _lib.call("bfa_fused_rmsnorm_qkv_noalloc", *a, status, stream)
    return out


CASES = [
    # (first call, second smaller call): t, h, hq, hkv, d, theta, qk_norm, fp32 output
    ((64, 4096, 32, 8, 128, 5e5, False, True), (8, 4096, 32, 8, 128, 5e5, False, True)),      # Llama-3-8B decode
    ((300, 1024, 16, 8, 128, 1e6, True, False), (5, 1024, 16, 8, 128, 1e6, True, False)),     # Qwen3 prefill, decode
    ((2048, 4096, 32, 8, 128, 5e5, False, False), (33, 4096, 32, 8, 128, 5e5, False, False)),  # largest that fits
]


@pytest.mark.parametrize("first,second", CASES)
def test_no_alloc_matches_workspace_entry_point(first, second):
    for seed, (t, h, hq, hkv, d, theta, qk, f32) in enumerate((first, second)):
        print(f"no_alloc case t={t} h={h} hq={hq} hkv={hkv} d={d} qk_norm={qk} f32={f32}", flush=True)
        inp = _inputs(700 + seed, t, h, hq, hkv, d, theta, qk)
        ref = _with_workspace(*inp, hq, hkv, f32)
        got = _no_alloc(*inp, hq, hkv, f32)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16 if not f32 else torch.int32),
                           ref.view(torch.int16 if not f32 else torch.int32)), f"t={t}: outputs differ"
    _lib.check_device_status()


def test_no_alloc_rejects_shapes_beyond_its_scratch():
    """2049 tokens at hidden 4096 need 16 MiB + 8 KiB of operand scratch: a
    clear error before any launch."""
    inp = _inputs(710, 4, 4096, 32, 8, 128, 5e5, False)
    x, ln, w, pos, cs, qn, kn = inp
    out = torch.empty(4, w.shape[0], dtype=torch.bfloat16, device=DEV)
    a, status, stream = _args(x, ln, w, pos, cs, qn, kn, 32, 8, out, False)
    a[2] = 2049  # tokens: the host check refuses before reading any row
    with pytest.raises(ValueError, match="scratch"):
        _lib.call("bfa_fused_rmsnorm_qkv_noalloc", *a, status, stream)
