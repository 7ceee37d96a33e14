"""Quintic Newton-Schulz iteration on the MI355X kernels.

Mirrors muonium/orthogonalize/newton_schulz.py: ``ns_loop`` (:16-57) and
``ns_loop_triton`` (:60-107) compute the same iteration; here both names run the HIP
path (bf16 or fp32 iteration by input dtype), so ``use_triton`` only selects a name.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _ops

# newton_schulz.py:21-23 (a, b, c)
NS_COEFFS: tuple[float, float, float] = (3.4445, -4.7750, 2.0315)


def _iteration_dtype(X: Tensor) -> torch.dtype:
    return torch.float32 if X.dtype == torch.float32 else torch.bfloat16


def run_loop(X: Tensor, coeffs, *, prescale: float, eps: float) -> Tensor:
    """Shared body of the NS / PE loops: (..., N, M) in, same shape and dtype out.

    The iteration runs in fp32 for fp32 inputs and in bf16 (fp32 accumulation)
    otherwise; matrices with N > M are transposed inside the kernels."""
    assert X.ndim >= 2
    if X.size(0) == 0 or X.numel() == 0:
        return X
    assert X.is_cuda, "muonium_amd: the orthogonalization runs on a HIP device"
    Xc = X.contiguous()
    it = _iteration_dtype(X)
    out_dtype = X.dtype if X.dtype in (torch.float32, torch.bfloat16, torch.float16) else it
    U = _ops.orthogonalize([Xc], coeffs, prescale=prescale, eps=eps, iter_dtype=it,
                           out_dtype=out_dtype)
    return U[0]


def ns_loop(
    X: Tensor,
    steps: int = 5,
    *,
    a: float = NS_COEFFS[0],
    b: float = NS_COEFFS[1],
    c: float = NS_COEFFS[2],
    eps: float = 1e-7,
) -> Tensor:
    """Newton-Schulz iteration (newton_schulz.py:16-57): X / (||X||_F + eps), then
    ``steps`` times A = X X^T, B = b A + c A^2, X = a X + B X."""
    return run_loop(X, [(a, b, c)] * steps, prescale=1.0, eps=eps)


def ns_loop_triton(
    X: Tensor,
    steps: int = 5,
    *,
    a: float = NS_COEFFS[0],
    b: float = NS_COEFFS[1],
    c: float = NS_COEFFS[2],
    eps: float = 1e-7,
) -> Tensor:
    """Name kept for drop-in compatibility with newton_schulz.py:60-107; same kernels."""
    return ns_loop(X, steps, a=a, b=b, c=c, eps=eps)
