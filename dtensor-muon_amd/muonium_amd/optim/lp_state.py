"""Blockwise-quantized momentum state for MuonLP.

One object per tensor: uint8 ``codes`` (one per value for 8-bit / fp8, two per byte
for 4-bit with element 2i in the high nibble), one fp32 absmax ``scale`` per block of
``block_size`` consecutive values of the flattened tensor, and for the map formats the
fp32 ``qmap`` the codes index. The class names and ``zeros(...)`` constructors follow
the torchao 0.17.0 classes MuonLP allocates (optim_lp.py:118-133); the arithmetic
(``muon_lp_quantize`` / ``muon_lp_dequantize`` / ``muon_lp_prepass``) is this library's.
"""

from __future__ import annotations

import torch
from torch import Tensor

from muonium_amd import _lib, _ops


def create_dynamic_map(signed: bool = True, max_exponent_bits: int = 7, total_bits: int = 8):
    """Sorted dynamic quantization map with 2**total_bits fp32 entries: for exponent
    level i < max_exponent_bits, 10^(i - max_exponent_bits + 1) times the midpoints of
    an evenly spaced grid on [0.1, 1] (the grid doubles per level), mirrored when
    signed, plus 0 and 1 (the bitsandbytes/torchao dynamic map)."""
    data: list[float] = []
    non_sign = total_bits - 1
    extra = 2 ** (non_sign - max_exponent_bits) - 1
    level = 0
    for level in range(max_exponent_bits):
        k = (2 ** (level + non_sign - max_exponent_bits) if signed
             else 2 ** (level + non_sign - max_exponent_bits + 1))
        grid = torch.linspace(0.1, 1, k + 1)
        mid = (grid[:-1] + grid[1:]) / 2.0
        mag = 10 ** (level - max_exponent_bits + 1)
        data += (mag * mid).tolist()
        if signed:
            data += (-mag * mid).tolist()
    if extra > 0:
        grid = torch.linspace(0.1, 1, extra + 1)
        mid = (grid[:-1] + grid[1:]) / 2.0
        mag = 10 ** (level - max_exponent_bits + 1)
        data += (mag * mid).tolist()
        if signed:
            data += (-mag * mid).tolist()
    data += [0.0, 1.0]
    assert len(data) == 2**total_bits
    return sorted(data)


_QMAPS: dict[tuple[str, bool], list[float]] = {}


def qmap_values(fmt: str, signed: bool) -> list[float]:
    key = (fmt, signed)
    if key not in _QMAPS:
        if fmt == "8bit":
            _QMAPS[key] = create_dynamic_map(signed)
        elif signed:
            _QMAPS[key] = create_dynamic_map(True, 3, 4)
        else:
            _QMAPS[key] = torch.linspace(0, 1, 17)[1:].tolist()
    return _QMAPS[key]


class QuantizedState:
    """Quantized tensor-shaped optimizer state (see module docstring)."""

    qformat: int = -1
    fmt: str = ""

    def __init__(self, codes: Tensor, scale: Tensor, qmap: Tensor | None, signed: bool,
                 shape, block_size: int):
        self.codes = codes
        self.scale = scale
        self.qmap = qmap
        self.signed = signed
        self.shape = torch.Size(shape)
        self.block_size = block_size

    # tensor-like surface
    @property
    def device(self) -> torch.device:
        return self.codes.device

    @property
    def dtype(self) -> torch.dtype:
        return torch.float32

    @property
    def ndim(self) -> int:
        return len(self.shape)

    def numel(self) -> int:
        return self.shape.numel()

    def size(self, dim=None):
        return self.shape if dim is None else self.shape[dim]

    def __repr__(self) -> str:
        return (f"{type(self).__name__}(shape={tuple(self.shape)}, block_size={self.block_size}, "
                f"signed={self.signed}, device={self.device})")

    @classmethod
    def _codes_numel(cls, n: int) -> int:
        return n

    @classmethod
    def zeros(cls, shape, signed: bool = True, block_size: int = 256, device=None):
        shape = torch.Size(shape)
        n = shape.numel()
        codes = torch.zeros(cls._codes_numel(n), dtype=torch.uint8, device=device)
        scale = torch.zeros(n // block_size, dtype=torch.float32, device=device)
        qmap = None
        if cls.fmt != "fp8":
            qmap = torch.tensor(qmap_values(cls.fmt, signed), dtype=torch.float32, device=device)
        return cls(codes, scale, qmap, signed, shape, block_size)

    def dequantize(self, output_dtype: torch.dtype | None = None) -> Tensor:
        """Dense fp32 values, shaped like the state."""
        n = self.numel()
        if self.codes.is_cuda:
            out = torch.empty(n, dtype=torch.float32, device=self.device)
            _ops.lp_dequantize(self.codes, self.scale, self.qmap, self.qformat, self.block_size,
                               n, out)
        else:
            out = self._dequantize_host()
        out = out.view(self.shape)
        return out if output_dtype is None else out.to(output_dtype)

    def _dequantize_host(self) -> Tensor:
        # Inspection of host-resident state (e.g. a checkpoint loaded on the CPU);
        # the optimizer step never comes here.
        if self.fmt == "fp8":
            vals = self.codes.view(torch.float8_e4m3fn).float()
        else:
            codes = self.codes
            if self.fmt == "4bit":
                codes = torch.stack([codes >> 4, codes & 15], dim=-1).reshape(-1)
            vals = self.qmap[codes.long()]
        return (vals.view(-1, self.block_size) * self.scale.view(-1, 1)).reshape(-1)

    def copy_(self, src: Tensor) -> "QuantizedState":
        """Quantize ``src`` (same numel) into this state."""
        if isinstance(src, QuantizedState):
            self.codes.copy_(src.codes)
            self.scale.copy_(src.scale)
            return self
        _ops.lp_quantize(src.reshape(-1), self.codes, self.scale, self.qmap, self.qformat,
                         self.block_size)
        return self

    def to(self, *args, **kwargs):
        """Device moves return a moved state; dtype conversions return dense values."""
        dtype = kwargs.get("dtype")
        device = kwargs.get("device")
        for a in args:
            if isinstance(a, torch.dtype):
                dtype = a
            elif isinstance(a, (str, torch.device)):
                device = torch.device(a)
        if dtype is not None:
            dense = self.dequantize()
            return dense.to(device=device or dense.device, dtype=dtype)
        if device is None or torch.device(device) == self.device:
            return self
        move = lambda t: None if t is None else t.to(device, non_blocking=kwargs.get("non_blocking", False))
        return type(self)(move(self.codes), move(self.scale), move(self.qmap), self.signed,
                          self.shape, self.block_size)


class OptimState8bit(QuantizedState):
    """8-bit dynamic-map codes (256-entry map), one fp32 absmax scale per block."""

    qformat = _lib.Q_8BIT
    fmt = "8bit"


class OptimState4bit(QuantizedState):
    """4-bit codes (16-entry map), packed two per byte, one fp32 scale per block."""

    qformat = _lib.Q_4BIT
    fmt = "4bit"

    @classmethod
    def _codes_numel(cls, n: int) -> int:
        return n // 2


class OptimStateFp8(QuantizedState):
    """float8_e4m3fn codes of x / scale, scale = absmax / 448 per block."""

    qformat = _lib.Q_FP8
    fmt = "fp8"

    @classmethod
    def zeros(cls, shape, block_size: int = 256, device=None):  # type: ignore[override]
        return super().zeros(shape, True, block_size, device)


# A MuonLP checkpoint holds these objects as optimizer state. Their pickled form is the
# class plus a dict of plain tensors and scalars, which torch.load's default
# weights_only unpickler accepts once the classes are allow-listed.
torch.serialization.add_safe_globals([OptimState8bit, OptimState4bit, OptimStateFp8])
