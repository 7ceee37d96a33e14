"""CPU restatement of the Muon step arithmetic (test infrastructure only; see __init__).

All functions are functional: they return new tensors and never mutate their inputs,
so tests can feed the same inputs to the HIP path and to the oracle.
"""

from __future__ import annotations

import math
from typing import Callable, Sequence

import torch
from torch import Tensor

# Polar Express per-step (a, b, c): muonium/orthogonalize/polar_express.py:19-25
# (published in arXiv:2505.16932).
POLAR_EXPRESS_COEFFS: list[tuple[float, float, float]] = [
    (8.156554524902461, -22.48329292557795, 15.878769915207462),
    (4.042929935166739, -2.808917465908714, 0.5000178451051316),
    (3.8916678022926607, -2.772484153217685, 0.5060648178503393),
    (3.285753657755655, -2.3681294933425376, 0.46449024233003106),
    (2.3465413258596377, -1.7097828382687081, 0.42323551169305323),
]
# Quintic Newton-Schulz (a, b, c): muonium/orthogonalize/newton_schulz.py:21-23.
NS_COEFFS: tuple[float, float, float] = (3.4445, -4.7750, 2.0315)


def polar_iteration(
    X: Tensor, coeffs: Sequence[tuple[float, float, float]], *, prescale: float, eps: float
) -> Tensor:
    """Odd-polynomial iteration shared by both strategies, computed in X's dtype.

    Follows the eager bodies of pe_loop (polar_express.py:28-68) and ns_loop
    (newton_schulz.py:16-57): empty batch passes through; matrices with more rows
    than columns are transposed; X /= ||X||_F * prescale + eps; then per (a, b, c):
    A = X X^T, B = b A + c A A, X = a X + B X.
    """
    if X.size(0) == 0:
        return X
    tall = X.size(-2) > X.size(-1)
    if tall:
        X = X.transpose(-2, -1)
    X = X / (X.norm(dim=(-2, -1), keepdim=True) * prescale + eps)
    for a, b, c in coeffs:
        A = X @ X.transpose(-2, -1)
        B = b * A + c * (A @ A)
        X = a * X + B @ X
    return X.transpose(-2, -1) if tall else X


def _bf(t: Tensor) -> Tensor:
    return t.to(torch.bfloat16).to(torch.float32)


def polar_iteration_bf16(
    X: Tensor, coeffs: Sequence[tuple[float, float, float]], *, prescale: float, eps: float,
    rounding: str = "fused",
) -> Tensor:
    """The same iteration with bf16 storage and fp32 accumulation, at the storage
    points of a given implementation (returned in bf16):

    * ``"fused"`` — X, A and B stored in bf16, each product accumulated in fp32 and
      combined with its polynomial term before one rounding: A = bf16(X X^T),
      B = bf16(b A + c A A), X = bf16(a X + B X). The Frobenius prescale
      s = 1 / (||X||_F * prescale + eps) (fp32) is folded into the first step
      (A = bf16(s^2 X X^T), X = bf16(s B X + a s X)). This is the HIP path's scheme.
    * ``"triton"`` — the rounding points of the reference's compiled pe_loop_triton /
      ns_loop_triton (polar_express.py:71-115): X = bf16(X / (...)) first, then
      A = bf16(X X^T), A2 = bf16(A A), B = bf16(c A2 + b A), BX = bf16(B X),
      X = bf16(a X + BX) (compiled pointwise chains round once).
    """
    if X.size(0) == 0:
        return X.bfloat16()
    tall = X.size(-2) > X.size(-1)
    X = X.to(torch.float32)
    if tall:
        X = X.transpose(-2, -1)
    X = _bf(X)
    norm = X.double().pow(2).sum(dim=(-2, -1), keepdim=True).sqrt().float()
    s = 1.0 / (norm * prescale + eps)
    if rounding == "triton":
        X = _bf(X * s)
        for a, b, c in coeffs:
            A = _bf(X @ X.transpose(-2, -1))
            A2 = _bf(A @ A.transpose(-2, -1))
            B = _bf(c * A2 + b * A)
            X = _bf(a * X + _bf(B @ X))
    elif rounding == "fused":
        if len(coeffs) == 0:
            X = _bf(X * s)
        for i, (a, b, c) in enumerate(coeffs):
            if i == 0:
                A = _bf((s * s) * (X @ X.transpose(-2, -1)))
                B = _bf(c * (A @ A) + b * A)
                X = _bf(s * (B @ X) + (a * s) * X)
            else:
                A = _bf(X @ X.transpose(-2, -1))
                B = _bf(c * (A @ A) + b * A)
                X = _bf((B @ X) + a * X)
    else:
        raise ValueError(rounding)
    X = X.transpose(-2, -1) if tall else X
    return X.bfloat16()


def pe_loop(X: Tensor, steps: int = 5, *, eps: float = 1e-6) -> Tensor:
    """polar_express.py:28-68 (prescale 1.02, default eps 1e-6)."""
    return polar_iteration(X, POLAR_EXPRESS_COEFFS[:steps], prescale=1.02, eps=eps)


def ns_loop(
    X: Tensor,
    steps: int = 5,
    *,
    a: float = NS_COEFFS[0],
    b: float = NS_COEFFS[1],
    c: float = NS_COEFFS[2],
    eps: float = 1e-7,
) -> Tensor:
    """newton_schulz.py:16-57 (prescale 1.0, default eps 1e-7)."""
    return polar_iteration(X, [(a, b, c)] * steps, prescale=1.0, eps=eps)


def strategy_coeffs(strategy: str, steps: int) -> tuple[list[tuple[float, float, float]], float]:
    """(coefficients, prescale) for a strategy name (orthogonalize.py:48-65)."""
    if strategy == "polar_express":
        assert steps <= 5, "polar express orthogonalization only supports up to 5 optimization steps."
        return POLAR_EXPRESS_COEFFS[:steps], 1.02
    if strategy == "newton_schulz":
        return [NS_COEFFS] * steps, 1.0
    raise ValueError(f"Unknown orthogonalization strategy: {strategy}")


def zeropower(G: Tensor, steps: int = 5, eps: float = 1e-7, strategy: str = "newton_schulz") -> Tensor:
    """orthogonalize.py:68-102 plain branch: cast to bf16, run the loop (eps 1e-7)."""
    coeffs, prescale = strategy_coeffs(strategy, steps)
    return polar_iteration(G.bfloat16(), coeffs, prescale=prescale, eps=eps)


def foreach_zeropower(
    Gs: list[Tensor], steps: int = 5, eps: float = 1e-7, strategy: str = "newton_schulz"
) -> list[Tensor]:
    """orthogonalize.py:105-162 plain branch: stack, cast, loop, unbind."""
    coeffs, prescale = strategy_coeffs(strategy, steps)
    X = torch.stack(list(Gs)).bfloat16()
    return list(polar_iteration(X, coeffs, prescale=prescale, eps=eps).unbind(0))


def prescale_fp32(G: Tensor, *, prescale: float, eps: float) -> Tensor:
    """The steps == 0 output with the norm and divisor held in fp32 (how the HIP path
    computes it): bf16(X * (1 / (||X||_F * prescale + eps))), X = bf16(G) in its
    wide orientation, returned in the stored orientation."""
    X = G.bfloat16().float()
    norm = X.double().pow(2).sum(dim=(-2, -1), keepdim=True).sqrt().float()
    s = 1.0 / (norm * prescale + eps)
    return (X * s).bfloat16()


def gram(x: Tensor) -> Tensor:
    """kernels/gram.py:155-165 semantics: x @ x^T over the last two dims in fp32,
    returned in x's dtype."""
    return (x.float() @ x.float().transpose(-2, -1)).to(x.dtype)


# ---- optimizer-side helpers ------------------------------------------------------------


def transform_grad(grad: Tensor, flatten: bool) -> Tensor:
    """optim.py:395-401: 3D+ gradients become one (dim0, -1) matrix with flatten, else
    4D+ fold their leading dims into one batch dim."""
    if grad.ndim > 2:
        if flatten:
            return grad.reshape(grad.size(0), -1)
        if grad.ndim > 3:
            return grad.flatten(end_dim=-3)
    return grad


def lr_ratio(shape: Sequence[int]) -> float:
    """optim.py:411-413: sqrt(max(1, rows / cols)) of the transformed gradient,
    as the 0-dim fp32 tensor the optimizer stores."""
    return float(torch.tensor(math.sqrt(max(1.0, shape[-2] / shape[-1]))))


def split_lr_scales(shape: Sequence[int], split_sizes: Sequence[int]) -> tuple[float, ...]:
    """base.py:56-70."""
    rows, cols = shape[-2], shape[-1]
    full = math.sqrt(max(1.0, rows / cols))
    return tuple(math.sqrt(max(1.0, h / cols)) / full for h in split_sizes)


def split_orthogonalize(
    g: Tensor,
    split_sizes: Sequence[int],
    *,
    ns_steps: int,
    strategy: str,
    orth: Callable[[list[Tensor]], list[Tensor]] | None = None,
) -> Tensor:
    """base.py:73-99: orthogonalize equal-height row blocks together, scale each block
    by split_lr_scales, concatenate."""
    scales = split_lr_scales(g.shape, split_sizes)
    blocks = list(g.split(list(split_sizes), dim=-2))
    by_height: dict[int, list[int]] = {}
    for i, blk in enumerate(blocks):
        by_height.setdefault(blk.size(-2), []).append(i)
    out: list[Tensor | None] = [None] * len(blocks)
    for idx in by_height.values():
        group = [blocks[i] for i in idx]
        us = orth(group) if orth else foreach_zeropower(group, steps=ns_steps, strategy=strategy)
        for i, u in zip(idx, us):
            out[i] = u * scales[i]
    return torch.cat([u for u in out if u is not None], dim=-2)


def orthogonalize_single(g, *, ns_steps, strategy, split_sizes=None, orth_single=None, orth_batch=None):
    """base.py:102-131 (plain tensors)."""
    if split_sizes is None:
        return orth_single(g) if orth_single else zeropower(g, steps=ns_steps, strategy=strategy)
    return split_orthogonalize(g, split_sizes, ns_steps=ns_steps, strategy=strategy, orth=orth_batch)


def muon_update(
    param: Tensor,
    grad: Tensor,
    momentum_buffer: Tensor,
    lr_ratio_: float,
    *,
    lr: float,
    weight_decay: float,
    cautious_wd: bool,
    momentum: float,
    nesterov: bool,
    maximize: bool,
    ns_steps: int = 5,
    strategy: str = "polar_express",
    split_sizes=None,
    orth_single=None,
    orth_batch=None,
):
    """MuonBaseline.update (muon.py:21-77), functional.

    ``param`` is given in its own shape, ``grad`` / ``momentum_buffer`` in the
    transformed-gradient shape. Returns (new_param, new_buffer, g_prime, u) where
    g_prime is the fp32 orthogonalization input and u the orthogonalized update.
    """
    if maximize:
        grad = -grad
    p32 = param.to(torch.float32)
    g32 = grad.to(torch.float32)
    buf32 = momentum_buffer.to(torch.float32) * momentum + g32
    new_buf = buf32.to(momentum_buffer.dtype)
    gq = g32 + buf32 * momentum if nesterov else buf32
    u = orthogonalize_single(
        gq, ns_steps=ns_steps, strategy=strategy, split_sizes=split_sizes,
        orth_single=orth_single, orth_batch=orth_batch,
    )
    u = u.reshape(p32.shape)
    if weight_decay != 0:
        if cautious_wd:
            u = u + weight_decay * p32 * (u * p32 > 0)
        else:
            u = u + weight_decay * p32
    adjusted_lr = torch.tensor(lr_ratio_, dtype=torch.float32) * torch.tensor(lr, dtype=torch.float32)
    new_p = (p32 - adjusted_lr * u).to(param.dtype)
    return new_p, new_buf, gq, u


def normuon_normalize(u: Tensor, v: Tensor, beta2: float, split_sizes=None) -> tuple[Tensor, Tensor]:
    """normuon.py:16-55."""
    if split_sizes is not None:
        parts = [
            normuon_normalize(ub, vb, beta2)
            for ub, vb in zip(u.split(list(split_sizes), dim=-2), v.split(list(split_sizes), dim=-2))
        ]
        return torch.cat([p[0] for p in parts], dim=-2), torch.cat([p[1] for p in parts], dim=-2)
    u = u.to(v.dtype)
    norm_u = u.norm(p=2, dim=(-2, -1), keepdim=True)
    v_new = torch.lerp(v, (u * u).mean(dim=-1, keepdim=True), 1 - beta2)
    u = u / (v_new.sqrt() + 1e-8)
    norm_new = u.norm(p=2, dim=(-2, -1), keepdim=True).clamp(min=1e-8)
    return u * (norm_u / norm_new), v_new


def normuon_update(
    param, grad, momentum_buffer, variance, lr_ratio_, *, lr, weight_decay, cautious_wd,
    momentum, nesterov, maximize, ns_steps=5, strategy="polar_express", split_sizes=None,
    beta2=0.95, orth_single=None, orth_batch=None,
):
    """NorMuon.update (normuon.py:74-134), functional. Returns
    (new_param, new_buffer, new_variance, u_normalized)."""
    if maximize:
        grad = -grad
    p32 = param.to(torch.float32)
    g32 = grad.to(torch.float32)
    buf32 = momentum_buffer.to(torch.float32) * momentum + g32
    gq = g32 + buf32 * momentum if nesterov else buf32
    u = orthogonalize_single(
        gq, ns_steps=ns_steps, strategy=strategy, split_sizes=split_sizes,
        orth_single=orth_single, orth_batch=orth_batch,
    )
    u, v_new = normuon_normalize(u, variance.to(torch.float32), beta2, split_sizes)
    u = u.reshape(p32.shape)
    if weight_decay != 0:
        u = u + weight_decay * p32 * (u * p32 > 0) if cautious_wd else u + weight_decay * p32
    adjusted_lr = torch.tensor(lr_ratio_, dtype=torch.float32) * torch.tensor(lr, dtype=torch.float32)
    new_p = (p32 - adjusted_lr * u).to(param.dtype)
    return new_p, buf32.to(momentum_buffer.dtype), v_new.to(variance.dtype), u


class MuonRef:
    """The reference's per-parameter driver (optim.py:378-419 state init +
    optim.py:511-531 loop + muon.py:21-77 update), for plain CPU tensors.

    Used as the CPU baseline and as a multi-step trajectory oracle. State matches the
    checkpoint layout (step, momentum_buffer, lr_ratio)."""

    def __init__(self, params, *, lr=1e-3, wd=0.1, use_cautious_wd=True, momentum=0.95,
                 nesterov=True, ns_steps=5, strategy="polar_express", maximize=False,
                 flatten=False):
        self.params = list(params)
        self.hp = dict(lr=lr, weight_decay=wd, cautious_wd=use_cautious_wd, momentum=momentum,
                       nesterov=nesterov, maximize=maximize, ns_steps=ns_steps, strategy=strategy)
        self.flatten = flatten
        self.state: dict[int, dict] = {}

    @torch.no_grad()
    def step(self, grads: list[Tensor]):
        for i, (p, g) in enumerate(zip(self.params, grads)):
            if g is None:
                continue
            gt = transform_grad(g, self.flatten)
            st = self.state.get(i)
            if st is None:
                st = self.state[i] = {
                    "step": torch.tensor(0.0),
                    "momentum_buffer": torch.zeros_like(gt, dtype=torch.float32),
                    "lr_ratio": torch.tensor(math.sqrt(max(1.0, gt.shape[-2] / gt.shape[-1]))),
                }
            st["step"] += 1
            new_p, new_buf, _, _ = muon_update(
                p, gt, st["momentum_buffer"], float(st["lr_ratio"]), **self.hp
            )
            p.copy_(new_p)
            st["momentum_buffer"] = new_buf
