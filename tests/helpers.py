"""Shared test helpers: seeded inputs and the tolerance checks."""
from __future__ import annotations

import torch

# Tolerance for floating-point kernels (elementwise allclose form):
#   |actual - expected| <= ATOL + RTOL * |expected|
# with max-abs 2e-2 / max-rel 1e-2 against the fp32 reference after bf16 rounding.
ATOL = 2e-2
RTOL = 1e-2


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(g, *shape, mean=0.0, std=1.0, dtype=torch.bfloat16):
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * std + mean).to(dtype)


def assert_close(actual: torch.Tensor, expected: torch.Tensor, atol=ATOL, rtol=RTOL, what=""):
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    fin = torch.isfinite(e)
    assert torch.equal(torch.isfinite(a), fin), f"{what}: non-finite pattern differs"
    diff = (a - e).abs()[fin]
    bound = (atol + rtol * e.abs())[fin]
    bad = diff > bound
    if bad.any():
        i = int(torch.argmax((diff - bound)))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{diff.numel()} elements outside |d| <= {atol} + {rtol}|r|; "
            f"max abs {diff.max().item():.3e}, worst d={diff[i].item():.3e} at r={e[fin][i].item():.3e}")


def max_errors(actual: torch.Tensor, expected: torch.Tensor):
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    d = (a - e).abs()
    return d.max().item(), (d.max() / e.abs().max().clamp_min(1e-30)).item()


def bits(t: torch.Tensor) -> torch.Tensor:
    """Raw bit pattern, for bit-exact comparisons."""
    t = t.detach().cpu().contiguous()
    if t.element_size() == 2:
        return t.view(torch.int16)
    if t.element_size() == 4:
        return t.view(torch.int32)
    return t.view(torch.int64)
