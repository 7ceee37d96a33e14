"""Baseline Muon update rule on the MI355X kernels (muonium/optim/algorithms/muon.py).

Two launch plans, same arithmetic:

* fused (the normal case: the module-level orthogonalizer is this library's own and
  there are no ``split_sizes``): one momentum pre-pass writes the bf16 iteration input
  straight into the batched workspace, the iteration runs there, and the post-pass
  applies weight decay and the shape-scaled step reading the result in place;
* seam (a substituted ``zeropower`` / ``foreach_zeropower``, or ``split_sizes``): the
  momentum kernel produces g' as tensors, the module-level orthogonalizer is called
  on them exactly as the reference does, and the post-pass applies its output.

Quantized momentum buffers (MuonLP) take the dequant -> momentum -> requant pre-pass.
"""

from __future__ import annotations

from typing import Sequence

import torch
from torch import Tensor

from muonium_amd import _ops
from muonium_amd.orthogonalize import OrthogonalizationStrategy

from . import base as _base
from .base import (
    MuonAlgorithm,
    orthogonalize_batch,
    orthogonalize_single,
    register_muon_algorithm,
    split_lr_scales,
)


def fused_orth_available(split_sizes, batched: bool) -> bool:
    if split_sizes is not None:
        return False
    if batched:
        return _base.foreach_zeropower is _base.BUILTIN_FOREACH_ZEROPOWER
    return _base.zeropower is _base.BUILTIN_ZEROPOWER


def schedule(strategy: OrthogonalizationStrategy, ns_steps: int):
    """(coeffs, prescale) with the reference's validation (orthogonalize.py:48-65)."""
    if strategy == "polar_express":
        assert ns_steps <= 5, (
            "polar express orthogonalization only supports up to 5 optimization steps."
        )
    return _ops.coeffs_for(strategy, ns_steps)


class _Contig:
    """Contiguous working copies of non-contiguous tensors, copied back on exit."""

    def __init__(self, tensors: Sequence[Tensor]):
        self.orig = list(tensors)
        self.work = [t if t.is_contiguous() else t.contiguous() for t in self.orig]

    def writeback(self) -> None:
        for o, w in zip(self.orig, self.work):
            if o is not w:
                o.copy_(w)


def is_quantized(buf) -> bool:
    from muonium_amd.optim.lp_state import QuantizedState

    return isinstance(buf, QuantizedState)


def muon_step(
    params: Sequence[Tensor],
    grads: Sequence[Tensor],
    bufs: Sequence,
    lr_ratios: Sequence[Tensor],
    *,
    lr,
    weight_decay: float,
    cautious_wd: bool,
    momentum: float,
    nesterov: bool,
    maximize: bool,
    ns_steps: int,
    orthogonalization_strategy: OrthogonalizationStrategy,
    split_sizes,
    batched: bool,
) -> None:
    """The Muon step for a same-shape list (batched=True: the foreach semantics of
    muon.py:79-140, which update the gradient list in place under Nesterov;
    batched=False: the per-tensor semantics of muon.py:21-77)."""
    if not params[0].is_cuda:
        return _offloaded(muon_step, params, grads, bufs, lr_ratios, lr=lr,
                          weight_decay=weight_decay, cautious_wd=cautious_wd, momentum=momentum,
                          nesterov=nesterov, maximize=maximize, ns_steps=ns_steps,
                          orthogonalization_strategy=orthogonalization_strategy,
                          split_sizes=split_sizes, batched=batched)
    coeffs, prescale = schedule(orthogonalization_strategy, ns_steps)
    quantized = is_quantized(bufs[0])
    P = _Contig(params)
    G = _Contig(grads)
    B = None if quantized else _Contig(bufs)
    pview = [p.view(g.shape) for p, g in zip(P.work, G.work)]
    if split_sizes is not None and not quantized and G.work[0].dim() == 2 and \
            fused_orth_available(None, batched):
        _fused_split_step(
            pview, G.work, B.work, lr_ratios, lr, split_sizes, momentum=momentum,
            nesterov=nesterov,
            maximize=maximize, write_back_grad=batched and nesterov and not maximize,
            weight_decay=weight_decay, cautious_wd=cautious_wd, coeffs=coeffs,
            prescale=prescale,
        )
    elif fused_orth_available(split_sizes, batched):
        if quantized:
            _ops.fused_lp_step(
                pview, G.work, bufs, lr_ratios, lr, momentum=momentum, nesterov=nesterov,
                maximize=maximize, weight_decay=weight_decay, cautious_wd=cautious_wd,
                coeffs=coeffs, prescale=prescale,
            )
        else:
            _ops.fused_step(
                pview, G.work, B.work, lr_ratios, lr, momentum=momentum, nesterov=nesterov,
                maximize=maximize, write_back_grad=batched and nesterov and not maximize,
                weight_decay=weight_decay, cautious_wd=cautious_wd, coeffs=coeffs,
                prescale=prescale,
            )
    else:
        gq = momentum_seam(G.work, bufs if quantized else B.work, momentum=momentum,
                           nesterov=nesterov, maximize=maximize, batched=batched)
        if batched:
            us = orthogonalize_batch(gq, ns_steps=ns_steps, strategy=orthogonalization_strategy,
                                     split_sizes=split_sizes)
        else:
            us = [orthogonalize_single(g, ns_steps=ns_steps, strategy=orthogonalization_strategy,
                                       split_sizes=split_sizes) for g in gq]
        _ops.postpass(pview, [u.reshape(g.shape) for u, g in zip(us, G.work)], lr_ratios, lr,
                      weight_decay=weight_decay, cautious_wd=cautious_wd, shape=G.work[0].shape)
    P.writeback()
    if batched and nesterov and not maximize:
        G.writeback()
    if B is not None:
        B.writeback()


def _fused_split_step(params, grads, bufs, lr_ratios, lr, split_sizes, **kw) -> None:
    """The fused step for 2D tensors split into row blocks (base.py:56-99): every block is a
    contiguous row slice, i.e. a matrix of its own, so equal-height blocks of all tensors run
    through one prepass / iteration / post-pass sequence, each block's update rescaled by
    its split_lr_scales entry (rounded to the update's bf16, as `u * scales[i]` is)."""
    rows, cols = grads[0].shape
    scales = split_lr_scales((rows, cols), tuple(split_sizes))
    offsets, acc = [], 0
    for h in split_sizes:
        offsets.append(acc)
        acc += h
    by_height: dict[int, list[int]] = {}
    for j, h in enumerate(split_sizes):
        by_height.setdefault(h, []).append(j)
    for h, blocks in by_height.items():
        ps, gs, bs, block_ratios, block_scales = [], [], [], [], []
        for p, g, b, ratio in zip(params, grads, bufs, lr_ratios):
            for j in blocks:
                o = offsets[j]
                ps.append(p[o:o + h])
                gs.append(g[o:o + h])
                bs.append(b[o:o + h])
                block_ratios.append(ratio)
                block_scales.append(scales[j])
        _ops.fused_step(ps, gs, bs, block_ratios, lr, u_scales=block_scales, **kw)


def _offloaded(fn, params, grads, *state_lists, **kw):
    """Run ``fn`` on HIP-device copies of host-resident tensors and copy every
    result back (the same round trip the foreach driver makes, optim.py:546-595)."""
    if not torch.cuda.is_available():
        raise RuntimeError(
            "muonium_amd: the Muon step runs on a HIP device and none is available "
            f"(params on {params[0].device})"
        )
    dev = torch.device("cuda")
    moved = [[t.to(dev) for t in lst] for lst in (params, grads, *state_lists)]
    fn(*moved, **kw)
    for originals, copies in zip((params, grads, *state_lists), moved):
        for o, c in zip(originals, copies):
            if isinstance(o, Tensor) and o.dtype.is_floating_point:
                o.copy_(c.to(o.device))
            elif hasattr(o, "copy_") and not isinstance(o, Tensor):
                o.copy_(c.to(o.device))


def momentum_seam(grads, bufs, *, momentum, nesterov, maximize, batched) -> list[Tensor]:
    """Momentum step producing g' as tensors for a caller-supplied orthogonalizer.

    batched (foreach, muon.py:108-119): under Nesterov without maximize the gradient
    tensors themselves become g'; with maximize the negated copies do; without
    Nesterov g' is the momentum buffer. Per tensor (muon.py:39-56): g' is a new fp32
    tensor and the gradient is left untouched."""
    if is_quantized(bufs[0]):
        ms = [b.dequantize() for b in bufs]
        gq = [g.to(torch.float32, copy=True) for g in grads]
        _ops.momentum_only(gq, ms, momentum=momentum, nesterov=nesterov, maximize=maximize,
                           write_back_grad=True)
        for b, m in zip(bufs, ms):
            b.copy_(m)
        return gq if nesterov else ms
    if batched:
        if nesterov:
            gq = [g.clone() for g in grads] if maximize else list(grads)
            _ops.momentum_only(gq, bufs, momentum=momentum, nesterov=True, maximize=maximize,
                               write_back_grad=True)
            return gq
        _ops.momentum_only(list(grads), bufs, momentum=momentum, nesterov=False,
                           maximize=maximize, write_back_grad=False)
        return list(bufs)
    gq = [g.to(torch.float32, copy=True) for g in grads]
    _ops.momentum_only(gq, bufs, momentum=momentum, nesterov=nesterov, maximize=maximize,
                       write_back_grad=True)
    return gq


def batches_per_tensor(algorithm, cls, split_sizes) -> bool:
    """True when the per-parameter driver may group same-shape tensors of ``algorithm``
    into one `update_same_shape` call: the built-in `update` is in place (not replaced
    on the instance) and its step runs entirely in the fused kernels (this library's
    orthogonalizer, no row blocks)."""
    return (type(algorithm) is cls and "update" not in vars(algorithm)
            and fused_orth_available(split_sizes, batched=False))


@register_muon_algorithm
class MuonBaseline(MuonAlgorithm):
    """The original Muon update: momentum, orthogonalize, shape-scaled apply."""

    name = "muon"

    def batches_per_tensor(self, split_sizes) -> bool:
        return batches_per_tensor(self, MuonBaseline, split_sizes)

    def update_same_shape(self, params, grads, state, lr_ratios, *, lr, weight_decay,
                          cautious_wd, momentum, nesterov, maximize, ns_steps,
                          orthogonalization_strategy, split_sizes, **opts) -> None:
        """`update` for several same-shape tensors at once, per-tensor semantics
        (muon.py:21-77 for each): the gradients are left as they are."""
        muon_step(
            params, grads, state["momentum_buffer"], lr_ratios, lr=lr,
            weight_decay=weight_decay, cautious_wd=cautious_wd, momentum=momentum,
            nesterov=nesterov, maximize=maximize, ns_steps=ns_steps,
            orthogonalization_strategy=orthogonalization_strategy, split_sizes=split_sizes,
            batched=False,
        )

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
        muon_step(
            [param], [grad], [state["momentum_buffer"]], [lr_ratio], lr=lr,
            weight_decay=weight_decay, cautious_wd=cautious_wd, momentum=momentum,
            nesterov=nesterov, maximize=maximize, ns_steps=ns_steps,
            orthogonalization_strategy=orthogonalization_strategy, split_sizes=split_sizes,
            batched=False,
        )

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
        """Batched Muon update over same-shape, same-device tensors."""
        muon_step(
            params, grads, state["momentum_buffer"], lr_ratios, lr=lr,
            weight_decay=weight_decay, cautious_wd=cautious_wd, momentum=momentum,
            nesterov=nesterov, maximize=maximize, ns_steps=ns_steps,
            orthogonalization_strategy=orthogonalization_strategy, split_sizes=split_sizes,
            batched=True,
        )
