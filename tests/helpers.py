"""Shared test helpers."""

import torch


def rel_fro(actual: torch.Tensor, expected: torch.Tensor) -> float:
    """||actual - expected||_F / ||expected||_F in float64 (0 if both are zero)."""
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    den = e.norm().item()
    num = (a - e).norm().item()
    return num if den == 0 else num / den


def assert_close_pct(actual, expected, *, rtol, atol, max_mismatch_pct, msg=""):
    """Elementwise closeness in fp32 with a budget of mismatched elements."""
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    bad = ~torch.isclose(a, e, rtol=rtol, atol=atol)
    pct = 100.0 * bad.sum().item() / max(bad.numel(), 1)
    assert pct <= max_mismatch_pct, (
        f"{msg}\n{pct:.4f}% of elements mismatched (allowed {max_mismatch_pct}%) "
        f"at rtol={rtol}, atol={atol}"
    )
