"""Plugin ABI of Muon-family algorithms: base class, registry, shared helpers.

Mirrors muonium/optim/algorithms/base.py:20-310 (same names, signatures, reserved keys
and error messages). ``zeropower`` / ``foreach_zeropower`` are module attributes looked
up at call time, so callers (and tests) can substitute the orthogonalizer; the built-in
algorithms take their fused kernel path only while these are the library's own.
"""

from __future__ import annotations

import math
from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import Any, ClassVar, Literal, cast

import torch
from torch import Tensor

from muonium_amd.orthogonalize import (
    OrthogonalizationStrategy,
    foreach_zeropower,
    foreach_zeropower_3d_fsdp,
    is_fsdp_3d_sharded,
    zeropower,
)

BUILTIN_ZEROPOWER = zeropower
BUILTIN_FOREACH_ZEROPOWER = foreach_zeropower

# Group keys owned by the optimizer; algorithm options may not shadow them (base.py:20-37).
RESERVED_GROUP_KEYS = frozenset(
    {
        "params",
        "algorithm",
        "use_muon",
        "lr",
        "wd",
        "use_cautious_wd",
        "momentum",
        "nesterov",
        "ns_steps",
        "orthogonalization_strategy",
        "maximize",
        "flatten",
        "foreach",
        "split_sizes",
    }
)

# Names routed to the Adam path by the optimizer, never to this registry (base.py:39-40).
ADAM_ALGORITHMS = ("adam", "adamw")


@dataclass(frozen=True)
class BufferSpec:
    """One per-parameter state buffer: ``like="grad"`` is an fp32 buffer shaped like
    the (possibly flattened) gradient, ``like="grad_rows"`` one value per row
    (``grad[..., :1]``). ``signed`` is read by quantized-state optimizers."""

    like: Literal["grad", "grad_rows"]
    signed: bool = True


def split_lr_scales(
    shape: torch.Size | tuple[int, ...], split_sizes: tuple[int, ...]
) -> tuple[float, ...]:
    """Per-row-block correction ratio(block) / ratio(full) with
    ratio = sqrt(max(1, rows / cols)) (base.py:56-70)."""
    rows, cols = shape[-2], shape[-1]
    full_ratio = math.sqrt(max(1.0, rows / cols))
    return tuple(math.sqrt(max(1.0, h / cols)) / full_ratio for h in split_sizes)


def _split_orthogonalize_full(
    g: Tensor,
    split_sizes: tuple[int, ...],
    scales: tuple[float, ...],
    *,
    ns_steps: int,
    strategy: OrthogonalizationStrategy,
) -> Tensor:
    """Orthogonalize row blocks independently, equal heights batched together, each
    scaled by its split_lr_scales entry (base.py:73-99)."""
    blocks = [b.contiguous() for b in g.split(list(split_sizes), dim=-2)]
    by_height: dict[int, list[int]] = {}
    for i, block in enumerate(blocks):
        by_height.setdefault(block.size(-2), []).append(i)
    out: list[Tensor | None] = [None] * len(blocks)
    for indices in by_height.values():
        ortho = foreach_zeropower([blocks[i] for i in indices], steps=ns_steps, strategy=strategy)
        for i, u in zip(indices, ortho, strict=True):
            out[i] = u * scales[i]
    return torch.cat([u for u in out if u is not None], dim=-2)


def orthogonalize_single(
    g: Tensor,
    *,
    ns_steps: int,
    strategy: OrthogonalizationStrategy,
    split_sizes: tuple[int, ...] | None = None,
):
    """Orthogonalize one tensor (base.py:102-131, plain tensors)."""
    if split_sizes is None:
        return zeropower(g, steps=ns_steps, strategy=strategy)
    scales = split_lr_scales(g.shape, split_sizes)
    return _split_orthogonalize_full(g, split_sizes, scales, ns_steps=ns_steps, strategy=strategy)


def orthogonalize_batch(
    gs: list[Tensor],
    *,
    ns_steps: int,
    strategy: OrthogonalizationStrategy,
    split_sizes: tuple[int, ...] | None = None,
) -> list[Tensor]:
    """Orthogonalize a same-shape batch (base.py:134-168, plain tensors)."""
    if split_sizes is not None:
        scales = split_lr_scales(gs[0].shape, split_sizes)
        return [
            _split_orthogonalize_full(g, split_sizes, scales, ns_steps=ns_steps, strategy=strategy)
            for g in gs
        ]
    if is_fsdp_3d_sharded(gs):
        return cast(list[Tensor], foreach_zeropower_3d_fsdp(gs, steps=ns_steps, strategy=strategy))
    return cast(list[Tensor], foreach_zeropower(gs, steps=ns_steps, strategy=strategy))


class MuonAlgorithm(ABC):
    """A Muon-family update rule, selected per param group via ``"algorithm"``
    (base.py:171-268). Subclasses own the math; the optimizer owns group building,
    state allocation (``state_spec``), batching and offload."""

    name: ClassVar[str]
    options: ClassVar[dict[str, Any]] = {}
    state_spec: ClassVar[dict[str, BufferSpec]] = {
        "momentum_buffer": BufferSpec(like="grad", signed=True),
    }

    def validate_param(self, p: Tensor) -> None:
        if p.ndim < 2:
            raise ValueError(
                "Muon only supports 2D+ parameters; found a 1D tensor in a Muon group"
            )
        if torch.is_complex(p):
            raise NotImplementedError(
                "Complex parameters are not supported in Muon. Add these parameters "
                "to the Adam group or use a different optimizer."
            )

    @abstractmethod
    def update(
        self,
        param: Tensor,
        grad: Tensor,
        state: dict[str, Tensor],
        lr_ratio: Tensor,
        *,
        lr: Tensor,
        weight_decay: float,
        cautious_wd: bool,
        momentum: float,
        nesterov: bool,
        maximize: bool,
        ns_steps: int,
        orthogonalization_strategy: OrthogonalizationStrategy,
        split_sizes: tuple[int, ...] | None,
        **opts,
    ) -> None:
        """Per-tensor update; mutates ``param`` and ``state`` in place."""

    def foreach_update(
        self,
        params: list[Tensor],
        grads: list[Tensor],
        state: dict[str, list[Tensor]],
        lr_ratios: list[Tensor],
        *,
        lr: Tensor,
        weight_decay: float,
        cautious_wd: bool,
        momentum: float,
        nesterov: bool,
        maximize: bool,
        ns_steps: int,
        orthogonalization_strategy: OrthogonalizationStrategy,
        split_sizes: tuple[int, ...] | None,
        **opts,
    ) -> None:
        """Batched update over same-(device, dtype, shape) tensors; the default loops
        ``update``."""
        for i, (param, grad, lr_ratio) in enumerate(zip(params, grads, lr_ratios, strict=True)):
            self.update(
                param,
                grad,
                {key: buffers[i] for key, buffers in state.items()},
                lr_ratio,
                lr=lr,
                weight_decay=weight_decay,
                cautious_wd=cautious_wd,
                momentum=momentum,
                nesterov=nesterov,
                maximize=maximize,
                ns_steps=ns_steps,
                orthogonalization_strategy=orthogonalization_strategy,
                split_sizes=split_sizes,
                **opts,
            )


_REGISTRY: dict[str, MuonAlgorithm] = {}


def register_muon_algorithm(cls: type[MuonAlgorithm]) -> type[MuonAlgorithm]:
    """Register a MuonAlgorithm subclass under ``cls.name`` (base.py:274-294)."""
    name = getattr(cls, "name", None)
    if not isinstance(name, str) or not name:
        raise ValueError(f"{cls.__qualname__} must define a non-empty string `name`")
    name = name.lower()
    if name in ADAM_ALGORITHMS:
        raise ValueError(f"'{name}' is reserved for the Adam path")
    if name in _REGISTRY and type(_REGISTRY[name]).__qualname__ != cls.__qualname__:
        raise ValueError(f"Muon algorithm '{name}' is already registered")
    shadowed = RESERVED_GROUP_KEYS.intersection(cls.options)
    if shadowed:
        raise ValueError(
            f"{cls.__qualname__}.options shadow reserved group keys: {sorted(shadowed)}"
        )
    _REGISTRY[name] = cls()
    return cls


def get_algorithm(name: str) -> MuonAlgorithm:
    """Case-insensitive lookup (base.py:297-305)."""
    try:
        return _REGISTRY[name.lower()]
    except KeyError:
        raise ValueError(
            f"Unknown algorithm '{name}'. Registered Muon algorithms: "
            f"{sorted(_REGISTRY)}; 'adam' and 'adamw' select the Adam path."
        ) from None


def registered_algorithms() -> tuple[str, ...]:
    return tuple(sorted(_REGISTRY))
