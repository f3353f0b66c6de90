"""Shared test helpers: seeded inputs and the tolerance checks."""
from __future__ import annotations

import torch

# Tolerance for floating-point kernels (elementwise allclose form):
#   |actual - expected| <= ATOL + RTOL * |expected|
# with max-abs 2e-2 / max-rel 1e-2 against the fp32 reference after bf16 rounding.
ATOL = 2e-2
RTOL = 1e-2


# Every use of a documented rounding allowance, for the session summary that
# tests/conftest.py prints: (what, elements beyond the strict bound, elements).
ALLOWANCE_LOG: list = []


def record_allowance(what: str, used: int, numel: int) -> None:
    ALLOWANCE_LOG.append((what, int(used), int(numel)))


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(g, *shape, mean=0.0, std=1.0, dtype=torch.bfloat16):
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * std + mean).to(dtype)


def assert_close(actual: torch.Tensor, expected: torch.Tensor, atol=ATOL, rtol=RTOL, what="",
                 slack: torch.Tensor | None = None, max_slack_frac: float = 1e-4):
    """Elementwise |actual - expected| <= atol + rtol |expected|.

    `slack` is an elementwise allowance for a documented rounding effect (see
    rope_flip_slack); at most `max_slack_frac` of the elements may need it, so
    a systematic error still fails."""
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    fin = torch.isfinite(e)
    assert torch.equal(torch.isfinite(a), fin), f"{what}: non-finite pattern differs"
    diff = (a - e).abs()[fin]
    bound = atol + rtol * e.abs()
    if slack is not None:
        strict = bound[fin]
        bound = bound + slack.detach().float().cpu().reshape(e.shape)
        used = int((diff > strict).sum())
        record_allowance(what, used, diff.numel())
        assert used <= max_slack_frac * diff.numel(), (
            f"{what}: {used}/{diff.numel()} elements need the rounding allowance (> {max_slack_frac:g})")
    bound = bound[fin]
    bad = diff > bound
    if bad.any():
        i = int(torch.argmax((diff - bound)))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{diff.numel()} elements outside |d| <= {atol} + {rtol}|r|; "
            f"max abs {diff.max().item():.3e}, worst d={diff[i].item():.3e} at r={e[fin][i].item():.3e}")


def rope_flip_slack(pre: torch.Tensor) -> torch.Tensor:
    """Two bf16 ulps of each input of the neox rotation, per output element.

    RoPE forms x1 cos - x2 sin and x2 cos + x1 sin from bf16-rounded inputs.  A
    projection summed in another order can round one element an ulp away from
    the oracle's; through the second rounding (of the normalised value) that is
    up to two ulps of the RoPE input, and where the two terms cancel (inputs of
    ~100 after a Qwen3 k_norm weight of 100, output ~10) it passes to the output
    unreduced.  The allowance is 2 * 2^-7 (|x1| + |x2|) for both outputs of the
    pair; `pre` holds the oracle's RoPE inputs [..., D]."""
    p = pre.detach().float().cpu().abs()
    h = p.shape[-1] // 2
    pair = p[..., :h] + p[..., h:]
    return torch.cat([pair, pair], dim=-1) * 2.0 ** -6


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
