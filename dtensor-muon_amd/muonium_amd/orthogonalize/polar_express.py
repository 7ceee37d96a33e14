"""Polar Express orthogonalization on the MI355X kernels.

Mirrors muonium/orthogonalize/polar_express.py (arXiv:2505.16932): ``pe_loop``
(:28-68) and ``pe_loop_triton`` (:71-115); both names run the HIP path.
"""

from __future__ import annotations

from torch import Tensor

from .newton_schulz import run_loop

# Per-step (a, b, c) of the published Polar Express schedule (polar_express.py:19-25).
POLAR_EXPRESS_COEFFS = [
    (8.156554524902461, -22.48329292557795, 15.878769915207462),
    (4.042929935166739, -2.808917465908714, 0.5000178451051316),
    (3.8916678022926607, -2.772484153217685, 0.5060648178503393),
    (3.285753657755655, -2.3681294933425376, 0.46449024233003106),
    (2.3465413258596377, -1.7097828382687081, 0.42323551169305323),
]


def pe_loop(X: Tensor, steps: int = 5, *, eps: float = 1e-6) -> Tensor:
    """X / (1.02 ||X||_F + eps), then per schedule entry (a, b, c):
    A = X X^T, B = b A + c A^2, X = a X + B X (at most 5 steps)."""
    return run_loop(X, POLAR_EXPRESS_COEFFS[:steps], prescale=1.02, eps=eps)


def pe_loop_triton(X: Tensor, steps: int = 5, *, eps: float = 1e-6) -> Tensor:
    """Name kept for drop-in compatibility with polar_express.py:71-115; same kernels."""
    return pe_loop(X, steps, eps=eps)
