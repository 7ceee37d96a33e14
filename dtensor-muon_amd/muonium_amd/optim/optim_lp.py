"""Low-precision Muon: quantized momentum state (drop-in for muonium/optim/optim_lp.py).

Same constructor (``block_size=2048``, ``bf16_stochastic_round`` stored only,
``foreach=False`` default), same eligibility rule for quantizing a buffer (local
numel >= 4096 and divisible by ``block_size``, else a plain zeros buffer in the
param's dtype) and the same subclass names. The step itself runs the fused
dequant -> momentum -> requant pre-pass of libmuon_amd, where the reference's
quantized subclasses raise NotImplementedError (tests/optim/test_optim_lp.py:211-222).
"""

from __future__ import annotations

import torch
from torch import Tensor

from muonium_amd.orthogonalize import OrthogonalizationStrategy

from .algorithms import BufferSpec
from .lp_state import OptimState4bit, OptimState8bit, OptimStateFp8
from .optim import Muon


class MuonLP(Muon):
    """Low-precision Muon with quantized optimizer states."""

    def __init__(
        self,
        params,
        lr: float = 1e-3,
        wd: float = 0.1,
        use_cautious_wd: bool = True,
        maximize: bool = False,
        momentum: float = 0.95,
        nesterov: bool = True,
        ns_steps: int = 5,
        orthogonalization_strategy: OrthogonalizationStrategy = "polar_express",
        amsgrad: bool = False,
        adam_betas: tuple[float, float] = (0.9, 0.95),
        adam_eps: float = 1e-8,
        is_adamw: bool = True,
        foreach_adam: bool | None = None,
        fused_adam: bool | None = None,
        foreach: bool | None = False,
        batch_size: int | None = None,
        block_size: int | None = 2048,
        bf16_stochastic_round: bool = False,
    ):
        super().__init__(
            params=params,
            lr=lr,
            wd=wd,
            use_cautious_wd=use_cautious_wd,
            maximize=maximize,
            momentum=momentum,
            nesterov=nesterov,
            ns_steps=ns_steps,
            orthogonalization_strategy=orthogonalization_strategy,
            amsgrad=amsgrad,
            adam_betas=adam_betas,
            adam_eps=adam_eps,
            is_adamw=is_adamw,
            fused_adam=fused_adam,
            foreach_adam=foreach_adam,
            foreach=foreach,
            batch_size=batch_size,
        )
        self.block_size = block_size
        self.bf16_stochastic_round = bf16_stochastic_round

    @staticmethod
    def _subclass_zeros(p: Tensor, signed: bool, block_size: int):
        """Override in subclasses to use quantized storage."""
        return torch.zeros_like(p)

    def _new_buffer(self, p: Tensor, signed: bool):
        """Quantized zeros when eligible (optim_lp.py:81-102, bitsandbytes' 4096
        threshold), else plain zeros in the param's dtype.

        ``block_size=None`` (an addition to the reference's API, whose blocks all have one
        size per optimizer) gives every quantized buffer a single block, i.e. one scale
        per tensor; the eligibility threshold is unchanged."""
        block = p.numel() if self.block_size is None else self.block_size
        if p.numel() >= 4096 and p.numel() % block == 0:
            out = self._subclass_zeros(p, signed, block)
        else:
            out = torch.zeros_like(p)
        return out.to(p.device)

    def _new_state_buffer(self, p: Tensor, grad: Tensor, spec: BufferSpec):
        """Grad-shaped buffers go through ``_new_buffer``; per-row buffers stay fp32
        (optim_lp.py:104-115)."""
        if spec.like == "grad":
            buf = self._new_buffer(p, signed=spec.signed)
            if isinstance(buf, Tensor) and buf.shape != grad.shape:
                buf = buf.view(grad.shape)
            return buf
        return super()._new_state_buffer(p, grad, spec)


class Muon8bit(MuonLP):
    @staticmethod
    def _subclass_zeros(p: Tensor, signed: bool, block_size: int):
        return OptimState8bit.zeros(p.shape, signed, block_size, p.device)


class Muon4bit(MuonLP):
    @staticmethod
    def _subclass_zeros(p: Tensor, signed: bool, block_size: int):
        return OptimState4bit.zeros(p.shape, signed, block_size, p.device)


class MuonFp8(MuonLP):
    @staticmethod
    def _subclass_zeros(p: Tensor, signed: bool, block_size: int):
        return OptimStateFp8.zeros(p.shape, block_size, p.device)
