"""NorMuon: Muon with neuron-wise update normalization (arXiv:2510.05491).

Mirrors muonium/optim/algorithms/normuon.py:16-203. Momentum, orthogonalization, the
per-row normalization of the orthogonalized update and the weight-decay/apply pass all
run on the MI355X kernels (``muon_normuon_postpass``).
"""

from __future__ import annotations

import torch
from torch import Tensor

from muonium_amd import _ops
from muonium_amd.orthogonalize import OrthogonalizationStrategy

from .base import (
    BufferSpec,
    MuonAlgorithm,
    orthogonalize_batch,
    orthogonalize_single,
    register_muon_algorithm,
    split_lr_scales,
)
from .muon import (
    _Contig,
    _offloaded,
    batches_per_tensor,
    fused_orth_available,
    is_quantized,
    momentum_seam,
    schedule,
)


def _normuon_step(params, grads, bufs, variances, lr_ratios, *, lr, weight_decay, cautious_wd,
                  momentum, nesterov, maximize, ns_steps, orthogonalization_strategy,
                  split_sizes, muon_beta2, batched):
    if not params[0].is_cuda:
        # host-resident tensors (the per-parameter driver's default for them): run on
        # device copies and copy every result back
        return _offloaded(_normuon_step, params, grads, bufs, variances, lr_ratios, lr=lr,
                          weight_decay=weight_decay, cautious_wd=cautious_wd,
                          momentum=momentum, nesterov=nesterov, maximize=maximize,
                          ns_steps=ns_steps,
                          orthogonalization_strategy=orthogonalization_strategy,
                          split_sizes=split_sizes, muon_beta2=muon_beta2, batched=batched)
    coeffs, prescale = schedule(orthogonalization_strategy, ns_steps)
    quantized = is_quantized(bufs[0])
    P, G, V = _Contig(params), _Contig(grads), _Contig(variances)
    B = None if quantized else _Contig(bufs)
    pview = [p.view(g.shape) for p, g in zip(P.work, G.work)]
    if split_sizes is not None and not quantized and G.work[0].dim() == 2 and \
            fused_orth_available(None, batched):
        _fused_normuon_split_step(
            pview, G.work, B.work, V.work, lr_ratios, lr, split_sizes, momentum=momentum,
            nesterov=nesterov, maximize=maximize,
            write_back_grad=batched and nesterov and not maximize, weight_decay=weight_decay,
            cautious_wd=cautious_wd, coeffs=coeffs, prescale=prescale, beta2=muon_beta2,
        )
    elif not quantized and fused_orth_available(split_sizes, batched):
        _ops.fused_normuon_step(
            pview, G.work, B.work, V.work, lr_ratios, lr, momentum=momentum, nesterov=nesterov,
            maximize=maximize, write_back_grad=batched and nesterov and not maximize,
            weight_decay=weight_decay, cautious_wd=cautious_wd, coeffs=coeffs,
            prescale=prescale, beta2=muon_beta2,
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
        _ops.normuon_postpass(pview, [u.reshape(g.shape) for u, g in zip(us, G.work)], V.work,
                              lr_ratios, lr, weight_decay=weight_decay, cautious_wd=cautious_wd,
                              beta2=muon_beta2, split_sizes=split_sizes, shape=G.work[0].shape)
    P.writeback()
    if batched and nesterov and not maximize:
        G.writeback()
    if B is not None:
        B.writeback()
    V.writeback()


def _fused_normuon_split_step(params, grads, bufs, variances, lr_ratios, lr, split_sizes,
                              **kw) -> None:
    """The fused NorMuon step for 2D tensors split into row blocks (base.py:56-99 and
    normuon.py:16-42): every block is a contiguous row slice, a matrix of its own with its
    own slice of the per-row variance state, so equal-height blocks of all tensors run
    through one pre-pass / iteration / NorMuon post-pass sequence. Each block's update is
    rescaled by its split_lr_scales entry (rounded to bf16) before the normalization, as
    `u * scales[i]` precedes _normuon_normalize in the reference."""
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
        ps, gs, bs, vs, ratios, block_scales = [], [], [], [], [], []
        for p, g, b, v, ratio in zip(params, grads, bufs, variances, lr_ratios):
            for j in blocks:
                o = offsets[j]
                ps.append(p[o:o + h])
                gs.append(g[o:o + h])
                bs.append(b[o:o + h])
                vs.append(v[o:o + h])
                ratios.append(ratio)
                block_scales.append(scales[j])
        _ops.fused_normuon_step(ps, gs, bs, vs, ratios, lr, u_scales=block_scales, **kw)


@register_muon_algorithm
class NorMuon(MuonAlgorithm):
    """Muon plus a neuron-wise second-moment normalization of the update."""

    name = "normuon"
    options = {"muon_beta2": 0.95}
    state_spec = {
        "momentum_buffer": BufferSpec(like="grad", signed=True),
        "variance_neuron": BufferSpec(like="grad_rows", signed=False),
    }

    def batches_per_tensor(self, split_sizes) -> bool:
        return batches_per_tensor(self, NorMuon, split_sizes)

    def update_same_shape(self, params, grads, state, lr_ratios, *, lr, weight_decay,
                          cautious_wd, momentum, nesterov, maximize, ns_steps,
                          orthogonalization_strategy, split_sizes, muon_beta2=0.95,
                          **opts) -> None:
        """`update` for several same-shape tensors at once, per-tensor semantics."""
        _normuon_step(
            params, grads, state["momentum_buffer"], state["variance_neuron"], lr_ratios,
            lr=lr, weight_decay=weight_decay, cautious_wd=cautious_wd, momentum=momentum,
            nesterov=nesterov, maximize=maximize, ns_steps=ns_steps,
            orthogonalization_strategy=orthogonalization_strategy, split_sizes=split_sizes,
            muon_beta2=muon_beta2, batched=False,
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
        muon_beta2: float = 0.95,
        **opts,
    ) -> None:
        _normuon_step(
            [param], [grad], [state["momentum_buffer"]], [state["variance_neuron"]], [lr_ratio],
            lr=lr, weight_decay=weight_decay, cautious_wd=cautious_wd, momentum=momentum,
            nesterov=nesterov, maximize=maximize, ns_steps=ns_steps,
            orthogonalization_strategy=orthogonalization_strategy, split_sizes=split_sizes,
            muon_beta2=muon_beta2, batched=False,
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
        muon_beta2: float = 0.95,
        **opts,
    ) -> None:
        _normuon_step(
            params, grads, state["momentum_buffer"], state["variance_neuron"], lr_ratios,
            lr=lr, weight_decay=weight_decay, cautious_wd=cautious_wd, momentum=momentum,
            nesterov=nesterov, maximize=maximize, ns_steps=ns_steps,
            orthogonalization_strategy=orthogonalization_strategy, split_sizes=split_sizes,
            muon_beta2=muon_beta2, batched=True,
        )
