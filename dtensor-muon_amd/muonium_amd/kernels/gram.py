"""Gram kernel entry points on the MI355X SYRK (libmuon_amd ``muon_gram``).

Mirrors muonium/kernels/gram.py:109-165, including its contract checks and their
AssertionError messages (pinned by the reference's tests/kernels/test_gram.py:117-164).
"""

from __future__ import annotations

import torch

from .. import _ops


def gram_(d_in: torch.Tensor, d_out: torch.Tensor) -> None:
    """d_out[...] = d_in @ d_in^T; d_in (..., M, K), d_out (..., M, M) contiguous.

    Only upper-triangle tiles are computed; the lower triangle is a mirrored copy, so
    the output is exactly symmetric."""
    assert d_in.is_cuda and d_out.is_cuda
    assert d_in.device == d_out.device
    assert d_in.dtype == d_out.dtype
    assert d_in.ndim >= 2 and d_out.ndim >= 2
    assert d_in.shape[:-2] == d_out.shape[:-2]

    M, K = d_in.shape[-2], d_in.shape[-1]
    assert d_out.shape[-2:] == (M, M)

    x = d_in.contiguous()
    assert d_out.is_contiguous(), (
        "d_out must be contiguous (or you must write into a contiguous temp and copy_ back)"
    )
    assert x.dtype in (torch.bfloat16, torch.float32), f"unsupported dtype {x.dtype}"
    if x.numel() == 0 and d_out.numel() == 0:
        return
    _ops.gram_(x, d_out)  # K == 0 writes zeros


def gram(d_in: torch.Tensor) -> torch.Tensor:
    """Allocating form: returns d_in @ d_in^T over the last two dims."""
    assert d_in.ndim >= 2
    M = d_in.size(-2)
    d_out = torch.empty((*d_in.shape[:-2], M, M), device=d_in.device, dtype=d_in.dtype)
    gram_(d_in, d_out)
    return d_out
