"""Strategy dispatch and the plain-tensor zero-power entry points.

Mirrors muonium/orthogonalize/orthogonalize.py:48-162 for plain tensors. The bf16 cast
and the stacking of a same-shape list happen inside the pre-pass kernel (it reads
every input in place and writes the batched bf16 workspace), so no stacked copy is
materialized. DTensor inputs belong to the multi-GPU paths, which this single-GPU
build does not provide.
"""

from __future__ import annotations

from typing import Literal

import torch
from torch import Tensor

from .. import _ops
from .newton_schulz import NS_COEFFS, ns_loop, ns_loop_triton
from .polar_express import POLAR_EXPRESS_COEFFS, pe_loop, pe_loop_triton

OrthogonalizationStrategy = Literal["newton_schulz", "polar_express"]


def _reject_dtensor(x) -> None:
    try:
        from torch.distributed.tensor import DTensor
    except Exception:  # pragma: no cover - torch without distributed
        return
    if isinstance(x, DTensor):
        raise NotImplementedError(
            "muonium_amd is a single-GPU build: DTensor parameters are not supported"
        )


def _get_orthogonalization_fn(strategy: OrthogonalizationStrategy, use_triton: bool = True):
    """orthogonalize.py:48-55. Both ``use_triton`` values select the HIP loop."""
    if strategy == "newton_schulz":
        return ns_loop_triton if use_triton else ns_loop
    elif strategy == "polar_express":
        return pe_loop_triton if use_triton else pe_loop
    else:
        raise ValueError(f"Unknown orthogonalization strategy: {strategy}")


def _validate_orthogonalization_args(strategy: OrthogonalizationStrategy, steps: int) -> None:
    """orthogonalize.py:58-65."""
    if strategy == "polar_express":
        assert steps <= 5, (
            "polar express orthogonalization only supports up to 5 optimization steps."
        )


def _schedule(strategy: OrthogonalizationStrategy, steps: int):
    if strategy == "polar_express":
        return list(POLAR_EXPRESS_COEFFS[:steps]), 1.02
    return [NS_COEFFS] * steps, 1.0


def _zeropower_stack(Gs: list[Tensor], steps: int, eps: float, strategy) -> Tensor:
    coeffs, prescale = _schedule(strategy, steps)
    for g in Gs:
        assert g.is_cuda, "muonium_amd: the orthogonalization runs on a HIP device"
    Gs = [g.contiguous() for g in Gs]
    return _ops.orthogonalize(Gs, coeffs, prescale=prescale, eps=eps,
                              iter_dtype=torch.bfloat16, out_dtype=torch.bfloat16)


def zeropower(
    G: Tensor,
    steps: int = 5,
    eps: float = 1e-7,
    use_triton: bool = True,
    strategy: OrthogonalizationStrategy = "newton_schulz",
) -> Tensor:
    """Zero-power (matrix sign) of one gradient tensor, returned in bf16
    (orthogonalize.py:68-102)."""
    _validate_orthogonalization_args(strategy, steps)
    _get_orthogonalization_fn(strategy, use_triton)
    _reject_dtensor(G)
    if G.ndim >= 2 and (G.size(0) == 0 or G.numel() == 0):
        return G.bfloat16()
    return _zeropower_stack([G], steps, eps, strategy)[0]


def foreach_zeropower(
    Gs: list[Tensor],
    steps: int = 5,
    eps: float = 1e-7,
    use_triton: bool = True,
    strategy: OrthogonalizationStrategy = "newton_schulz",
) -> list[Tensor]:
    """Zero-power of a same-shape list, batched in one launch sequence, returned as
    bf16 views of one stacked result (orthogonalize.py:105-162)."""
    _validate_orthogonalization_args(strategy, steps)
    _get_orthogonalization_fn(strategy, use_triton)
    Gs = list(Gs)
    _reject_dtensor(Gs[0])  # empty list -> IndexError, as torch.stack's caller sees
    shape = Gs[0].shape
    for g in Gs[1:]:
        if g.shape != shape:
            raise RuntimeError(
                f"stack expects each tensor to be equal size, but got {list(shape)} and "
                f"{list(g.shape)}"
            )
    if Gs[0].ndim >= 2 and (Gs[0].size(0) == 0 or Gs[0].numel() == 0):
        return list(torch.stack(Gs).bfloat16().unbind(0))
    return list(_zeropower_stack(Gs, steps, eps, strategy).unbind(0))


def is_fsdp_3d_sharded(xs) -> bool:
    """orthogonalize.py:165-174. Only DTensors can be FSDP-sharded, and this
    single-GPU build takes plain tensors only, so this is always False."""
    return False


def foreach_zeropower_3d_fsdp(Gs, steps: int = 5, eps: float = 1e-7, use_triton: bool = True,
                              strategy: OrthogonalizationStrategy = "newton_schulz"):
    """orthogonalize.py:177-204 is the FSDP local-shard path; single-GPU build."""
    raise NotImplementedError(
        "muonium_amd is a single-GPU build: the FSDP local-shard path is not provided"
    )
