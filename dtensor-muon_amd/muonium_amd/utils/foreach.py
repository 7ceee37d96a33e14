"""Foreach grouping helpers (muonium/utils/foreach.py:8-40)."""

from __future__ import annotations

from typing import Sequence

import torch
from torch import Tensor


def group_tensors_by_shape(
    tensorlist: list[Tensor],
) -> dict[tuple[int, ...], tuple[list[Tensor], list[int]]]:
    """Map each shape to (tensors with that shape, their indices), in first-seen
    order. dtype and device are not part of the key."""
    groups: dict[tuple[int, ...], tuple[list[Tensor], list[int]]] = {}
    for idx, t in enumerate(tensorlist):
        key = tuple(t.shape)
        entry = groups.get(key)
        if entry is None:
            groups[key] = ([t], [idx])
        else:
            entry[0].append(t)
            entry[1].append(idx)
    return groups


def move_tensors_to_device(
    tensors: Sequence[Tensor | None],
    device_in: torch.device,
    device_out: torch.device,
) -> list[Tensor | None]:
    """Same device type: the input list itself. Otherwise copies (None kept)."""
    if device_in.type == device_out.type:
        return tensors  # type: ignore[return-value]
    return [t.to(device_out, non_blocking=True) if t is not None else None for t in tensors]
