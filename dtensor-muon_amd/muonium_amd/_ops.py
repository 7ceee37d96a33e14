"""Device operations of the Muon step, each a short launch sequence on libmuon_amd.

Shapes: a Muon tensor is handed over as ``nb`` stored matrices of ``rows x cols``
(its transformed-gradient shape, optim.py:395-401), contiguous. Same-shape tensors
of a foreach bucket share one batched workspace, so one launch sequence covers the
whole bucket.
"""

from __future__ import annotations

import ctypes
import threading

import numpy as np
from typing import Optional, Sequence

import torch
from torch import Tensor

from . import _lib

# ---------------------------------------------------------------------------------
# workspace cache: one growable buffer per (device, stream, iteration dtype, padded m, n)
#
# A buffer is only ever used on the stream that allocated it. Buckets running on
# different streams (the foreach driver's side streams) therefore never share one,
# and a capacity regrow frees the old buffer on the only stream that used it, which
# the caching allocator orders behind that stream's earlier launches.

_ws_lock = threading.Lock()
_ws_cache: dict[tuple, tuple[int, Tensor]] = {}


def _padded_extents(dtype: torch.dtype, rows: int, cols: int) -> tuple[int, int]:
    """(m_pad, n_pad) of the library's workspace layout for one rows x cols matrix."""
    off, pitch, mst, trans = (ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64(),
                              ctypes.c_int())
    rc = _lib.load().muon_orth_result(_lib.dtype_code(dtype), 1, rows, cols, 0,
                                      ctypes.byref(off), ctypes.byref(pitch), ctypes.byref(mst),
                                      ctypes.byref(trans))
    if rc != 0:
        raise RuntimeError(f"muonium_amd: bad workspace request {rows}x{cols}: {_lib.last_error()}")
    return mst.value // pitch.value, pitch.value


def workspace(device: torch.device, dtype: torch.dtype, batch: int, rows: int, cols: int):
    """(buffer, capacity) with room for ``batch`` matrices of rows x cols.

    The layout only depends on the padded (min, max) extents and the capacity, so
    tall and wide matrices of the same extents share a buffer, on the current stream
    of ``device`` only. Contents need no initialization (every launch rewrites what
    it reads later)."""
    m, n = _padded_extents(dtype, rows, cols)
    key = (device, _lib.stream(device), dtype, m, n)
    with _ws_lock:
        hit = _ws_cache.get(key)
        if hit is not None and hit[0] >= batch:
            return hit[1], hit[0]
        nbytes = _lib.load().muon_orth_workspace_bytes(_lib.dtype_code(dtype), batch, rows, cols)
        if nbytes < 0:
            raise RuntimeError(f"muonium_amd: bad workspace request {batch}x{rows}x{cols}")
        if hit is not None:
            del _ws_cache[key]
            del hit
        buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
        _ws_cache[key] = (batch, buf)
        return buf, batch


def release_workspaces() -> None:
    """Drop every cached workspace (they are re-created on demand)."""
    with _ws_lock:
        _ws_cache.clear()


# ---------------------------------------------------------------------------------
# shape helpers


def matrix_view(t) -> tuple[int, int, int]:
    """(nb, rows, cols) of a 2D+ tensor (or shape) viewed as a batch of its last two
    dims."""
    shape = tuple(t.shape) if isinstance(t, Tensor) else tuple(t)
    rows, cols = shape[-2], shape[-1]
    nb = 1
    for d in shape[:-2]:
        nb *= d
    return nb, rows, cols


def _check_cuda_contig(ts: Sequence[Tensor], what: str) -> None:
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError(f"muonium_amd: {what} must live on a HIP device (got {t.device})")
        if not t.is_contiguous():
            raise RuntimeError(f"muonium_amd: {what} must be contiguous")


def coeffs_for(strategy: str, steps: int) -> tuple[list[tuple[float, float, float]], float]:
    from .orthogonalize.newton_schulz import NS_COEFFS
    from .orthogonalize.polar_express import POLAR_EXPRESS_COEFFS

    if strategy == "polar_express":
        return list(POLAR_EXPRESS_COEFFS[:steps]), 1.02
    if strategy == "newton_schulz":
        return [NS_COEFFS] * steps, 1.0
    raise ValueError(f"Unknown orthogonalization strategy: {strategy}")


def _flat_coeffs(coeffs: Sequence[float]):
    return _lib.f64_array(list(coeffs))


def _flatten_coeffs(coeffs) -> list[float]:
    """(a, b, c) triples -> [a0, b0, c0, a1, ...] (plain floats, as the ops take them)."""
    return [float(c) for abc in coeffs for c in abc]


def adjusted_lrs(lr_ratios: Sequence[Tensor], lr: Tensor | float) -> list[float]:
    """lr_ratio * lr as the fp32 product of two 0-dim fp32 tensors (muon.py:71,115)."""
    lr32 = np.float32(float(lr))
    return [float(np.float32(float(r)) * lr32) for r in lr_ratios]


def _as_tensor(lr) -> Tensor:
    return lr if isinstance(lr, Tensor) else torch.tensor(float(lr))


def _compiling() -> bool:
    return torch.compiler.is_compiling()


# ---------------------------------------------------------------------------------
# Device operations. Each runs its implementation (`_*_impl`) directly in eager mode.
# While an outer torch.compile traces the step (optim.py:616-623: the reference then
# runs its raw update inside the caller's graph), the same implementation is reached
# through a torch.library custom op of namespace "muonium_amd", whose fake (meta)
# implementation lets the tracer put the library call into the graph instead of
# breaking it: the ops declare which tensor lists they write (mutates_args).


def _gram_impl(x: Tensor, y: Tensor) -> None:
    lib = _lib.load()
    _lib.ensure_device(x.device)
    B, M, K = matrix_view(x)
    _lib.check(
        lib.muon_gram(x.data_ptr(), y.data_ptr(), _lib.dtype_code(x.dtype), B, M, K,
                      _lib.stream(x.device)),
        "muon_gram",
    )


def gram_(x: Tensor, y: Tensor) -> None:
    """y = x x^T over the last two dims; x (B, M, K) and y (B, M, M) contiguous."""
    if _compiling():
        torch.ops.muonium_amd.gram_(x, y)
    else:
        _gram_impl(x, y)


def _orthogonalize_impl(tensors: list[Tensor], coeffs: list[float], prescale: float, eps: float,
                        iter_dtype: torch.dtype, out_dtype: torch.dtype) -> Tensor:
    lib = _lib.load()
    t0 = tensors[0]
    device = t0.device
    _lib.ensure_device(device)
    _check_cuda_contig(tensors, "orthogonalization inputs")
    nb, rows, cols = matrix_view(t0)
    count = len(tensors)
    out = torch.empty((count, *t0.shape), dtype=out_dtype, device=device)
    if out.numel() == 0:
        return out
    ws, cap = workspace(device, iter_dtype, count * nb, rows, cols)
    wdt = _lib.dtype_code(iter_dtype)
    s = _lib.stream(device)
    steps = len(coeffs) // 3
    grads = _lib.ptr_array(tensors)
    _lib.check(
        lib.muon_prepass(count, grads, None, _lib.dtype_code(t0.dtype), 0, nb, rows, cols, 0.0,
                         0, 0, 0, ws.data_ptr(), wdt, cap, s),
        "muon_prepass",
    )
    _lib.check(
        lib.muon_orth_run(ws.data_ptr(), wdt, cap, count * nb, rows, cols, _flat_coeffs(coeffs),
                          steps, prescale, eps, s),
        "muon_orth_run",
    )
    _lib.check(
        lib.muon_orth_extract(ws.data_ptr(), wdt, cap, count * nb, rows, cols, steps,
                              out.data_ptr(), _lib.dtype_code(out_dtype), s),
        "muon_orth_extract",
    )
    return out


def orthogonalize(
    tensors: Sequence[Tensor],
    coeffs: Sequence[tuple[float, float, float]],
    *,
    prescale: float,
    eps: float,
    iter_dtype: torch.dtype,
    out_dtype: torch.dtype,
) -> Tensor:
    """Run the polynomial iteration on every matrix of ``tensors`` (same shape, any
    float dtype, cast to ``iter_dtype`` on the fly) and return the stacked result
    of shape (len(tensors), *shape) in ``out_dtype``."""
    args = (list(tensors), _flatten_coeffs(coeffs), float(prescale), float(eps), iter_dtype,
            out_dtype)
    if _compiling():
        return torch.ops.muonium_amd.orthogonalize(*args)
    return _orthogonalize_impl(*args)


# ---------------------------------------------------------------------------------
# the Muon step pieces


def _momentum_impl(grads: list[Tensor], bufs: list[Tensor], momentum: float, nesterov: bool,
                   maximize: bool, write_back_grad: bool) -> None:
    lib = _lib.load()
    g0 = grads[0]
    _lib.ensure_device(g0.device)
    _check_cuda_contig(list(grads) + list(bufs), "momentum inputs")
    nb, rows, cols = matrix_view(g0)
    _lib.check(
        lib.muon_prepass(len(grads), _lib.ptr_array(grads), _lib.ptr_array(bufs),
                         _lib.dtype_code(g0.dtype), _lib.dtype_code(bufs[0].dtype), nb, rows, cols,
                         momentum, int(nesterov), int(maximize), int(write_back_grad), None, 1,
                         0, _lib.stream(g0.device)),
        "muon_prepass(momentum)",
    )


def momentum_only(
    grads: Sequence[Tensor], bufs: Sequence[Tensor], *, momentum: float, nesterov: bool,
    maximize: bool, write_back_grad: bool,
) -> None:
    """buf' = buf*mu + g (and, with write_back_grad, grad <- g + mu*buf') in place."""
    args = (list(grads), list(bufs), float(momentum), bool(nesterov), bool(maximize),
            bool(write_back_grad))
    if _compiling():
        torch.ops.muonium_amd.momentum_only(*args)
    else:
        _momentum_impl(*args)


def _postpass_impl(params: list[Tensor], us: list[Tensor], lr_ratios: list[Tensor], lr: Tensor,
                   weight_decay: float, cautious_wd: bool, shape: list[int]) -> None:
    lib = _lib.load()
    p0 = params[0]
    _lib.ensure_device(p0.device)
    _check_cuda_contig(params, "params")
    lrs = adjusted_lrs(lr_ratios, lr)
    nb, rows, cols = matrix_view(shape)
    s = _lib.stream(p0.device)
    if len(us) == 1 and len(params) > 1:
        chunks = [(list(range(len(params))), us[0])]  # one stacked tensor for every param
    else:
        chunks = [([i], u) for i, u in enumerate(us)]
    for idx, u in chunks:
        u = u.contiguous()
        ps = [params[i] for i in idx]
        _lib.check(
            lib.muon_postpass(len(ps), _lib.ptr_array(ps), _lib.dtype_code(p0.dtype),
                              u.data_ptr(), _lib.dtype_code(u.dtype), None, 1, 0, 0, nb, rows,
                              cols, _lib.f32_array([lrs[i] for i in idx]), None,
                              float(weight_decay), int(cautious_wd), s),
            "muon_postpass",
        )


def postpass(
    params: Sequence[Tensor], us: Sequence[Tensor] | Tensor, lr_ratios: Sequence[Tensor], lr, *,
    weight_decay: float, cautious_wd: bool, shape=None,
) -> None:
    """p <- p - lr_ratio * lr * (u + wd * p * [u*p > 0]) elementwise.

    ``us`` is either one contiguous stacked tensor or a list of tensors with the
    elements of each param in the same order; ``shape`` (default: the params') gives
    the (..., rows, cols) matrix view."""
    us = [us] if isinstance(us, Tensor) else list(us)
    shape = list(params[0].shape if shape is None else shape)
    args = (list(params), us, list(lr_ratios), _as_tensor(lr), float(weight_decay),
            bool(cautious_wd), shape)
    if _compiling():
        torch.ops.muonium_amd.postpass(*args)
    else:
        _postpass_impl(*args)


def _fused_step_impl(params: list[Tensor], grads: list[Tensor], bufs: list[Tensor],
                     lr_ratios: list[Tensor], lr: Tensor, momentum: float, nesterov: bool,
                     maximize: bool, write_back_grad: bool, weight_decay: float,
                     cautious_wd: bool, coeffs: list[float], prescale: float, eps: float,
                     u_scales: Optional[list[float]]) -> None:
    lib = _lib.load()
    g0 = grads[0]
    device = g0.device
    _lib.ensure_device(device)
    _check_cuda_contig(list(params) + list(grads) + list(bufs), "Muon step tensors")
    lrs = adjusted_lrs(lr_ratios, lr)
    nb, rows, cols = matrix_view(g0)
    count = len(grads)
    ws, cap = workspace(device, torch.bfloat16, count * nb, rows, cols)
    s = _lib.stream(device)
    steps = len(coeffs) // 3
    _lib.check(
        lib.muon_prepass(count, _lib.ptr_array(grads), _lib.ptr_array(bufs),
                         _lib.dtype_code(g0.dtype), _lib.dtype_code(bufs[0].dtype), nb, rows, cols,
                         momentum, int(nesterov), int(maximize), int(write_back_grad),
                         ws.data_ptr(), _lib.DT_BF16, cap, s),
        "muon_prepass",
    )
    if u_scales is None:
        # the iteration and the apply in one call: the library fuses the apply into the last
        # X' = a X + B X where the shapes allow it, else runs the post-pass after it
        _lib.check(
            lib.muon_orth_run_apply(ws.data_ptr(), _lib.DT_BF16, cap, count * nb, rows, cols,
                                    _flat_coeffs(coeffs), steps, prescale, eps, count,
                                    _lib.ptr_array(params), _lib.dtype_code(params[0].dtype), nb,
                                    _lib.f32_array(lrs), float(weight_decay), int(cautious_wd),
                                    s),
            "muon_orth_run_apply",
        )
        return
    _lib.check(
        lib.muon_orth_run(ws.data_ptr(), _lib.DT_BF16, cap, count * nb, rows, cols,
                          _flat_coeffs(coeffs), steps, prescale, eps, s),
        "muon_orth_run",
    )
    _lib.check(
        lib.muon_postpass(count, _lib.ptr_array(params), _lib.dtype_code(params[0].dtype), None,
                          0, ws.data_ptr(), _lib.DT_BF16, cap, steps, nb, rows, cols,
                          _lib.f32_array(lrs), _lib.f32_array(u_scales),
                          float(weight_decay), int(cautious_wd), s),
        "muon_postpass",
    )


def fused_step(
    params: Sequence[Tensor],
    grads: Sequence[Tensor],
    bufs: Sequence[Tensor],
    lr_ratios: Sequence[Tensor],
    lr,
    *,
    momentum: float,
    nesterov: bool,
    maximize: bool,
    write_back_grad: bool,
    weight_decay: float,
    cautious_wd: bool,
    coeffs: Sequence[tuple[float, float, float]],
    prescale: float,
    eps: float = 1e-7,
    u_scales: Sequence[float] | None = None,
) -> None:
    """One Muon step over a same-shape bucket: momentum pre-pass into the batched bf16
    workspace, the iteration, and the weight-decay/apply post-pass reading the
    result straight from the workspace. ``u_scales`` (one per tensor) rescales each
    update first, rounded to bf16: the split_sizes row-block correction."""
    args = (list(params), list(grads), list(bufs), list(lr_ratios), _as_tensor(lr),
            float(momentum), bool(nesterov), bool(maximize), bool(write_back_grad),
            float(weight_decay), bool(cautious_wd), _flatten_coeffs(coeffs), float(prescale),
            float(eps), None if u_scales is None else [float(v) for v in u_scales])
    if _compiling():
        torch.ops.muonium_amd.fused_step(*args)
    else:
        _fused_step_impl(*args)


def _splits(split_sizes):
    if split_sizes is None:
        return None, 0
    return _lib.i64_array(list(split_sizes)), len(split_sizes)


def _fused_normuon_impl(params: list[Tensor], grads: list[Tensor], bufs: list[Tensor],
                        variances: list[Tensor], lr_ratios: list[Tensor], lr: Tensor,
                        momentum: float, nesterov: bool, maximize: bool, write_back_grad: bool,
                        weight_decay: float, cautious_wd: bool, coeffs: list[float],
                        prescale: float, beta2: float, eps: float,
                        u_scales: Optional[list[float]]) -> None:
    lib = _lib.load()
    g0 = grads[0]
    device = g0.device
    _lib.ensure_device(device)
    _check_cuda_contig(list(params) + list(grads) + list(bufs) + list(variances),
                       "NorMuon step tensors")
    lrs = adjusted_lrs(lr_ratios, lr)
    nb, rows, cols = matrix_view(g0)
    count = len(grads)
    ws, cap = workspace(device, torch.bfloat16, count * nb, rows, cols)
    s = _lib.stream(device)
    steps = len(coeffs) // 3
    _lib.check(
        lib.muon_prepass(count, _lib.ptr_array(grads), _lib.ptr_array(bufs),
                         _lib.dtype_code(g0.dtype), _lib.dtype_code(bufs[0].dtype), nb, rows, cols,
                         momentum, int(nesterov), int(maximize), int(write_back_grad),
                         ws.data_ptr(), _lib.DT_BF16, cap, s),
        "muon_prepass",
    )
    _lib.check(
        lib.muon_orth_run(ws.data_ptr(), _lib.DT_BF16, cap, count * nb, rows, cols,
                          _flat_coeffs(coeffs), steps, prescale, eps, s),
        "muon_orth_run",
    )
    _lib.check(
        lib.muon_normuon_postpass(
            count, _lib.ptr_array(params), _lib.dtype_code(params[0].dtype),
            _lib.ptr_array(variances), _lib.dtype_code(variances[0].dtype), None, 0,
            ws.data_ptr(), _lib.DT_BF16, cap, steps, nb, rows, cols, None, 0,
            _lib.f32_array(lrs), None if u_scales is None else _lib.f32_array(u_scales),
            float(weight_decay), int(cautious_wd), float(beta2), s,
        ),
        "muon_normuon_postpass",
    )


def fused_normuon_step(
    params: Sequence[Tensor],
    grads: Sequence[Tensor],
    bufs: Sequence[Tensor],
    variances: Sequence[Tensor],
    lr_ratios: Sequence[Tensor],
    lr,
    *,
    momentum: float,
    nesterov: bool,
    maximize: bool,
    write_back_grad: bool,
    weight_decay: float,
    cautious_wd: bool,
    coeffs: Sequence[tuple[float, float, float]],
    prescale: float,
    beta2: float,
    eps: float = 1e-7,
    u_scales: Sequence[float] | None = None,
) -> None:
    """fused_step for the "normuon" algorithm: the post-pass normalizes U per stored row
    (second-moment EMA into ``variances``, Frobenius rescale) before the apply.
    ``u_scales`` (one per tensor) rescales each U first, rounded to bf16: the split_sizes
    row-block correction, applied before the normalization as the reference does."""
    args = (list(params), list(grads), list(bufs), list(variances), list(lr_ratios),
            _as_tensor(lr), float(momentum), bool(nesterov), bool(maximize),
            bool(write_back_grad), float(weight_decay), bool(cautious_wd),
            _flatten_coeffs(coeffs), float(prescale), float(beta2), float(eps),
            None if u_scales is None else [float(v) for v in u_scales])
    if _compiling():
        torch.ops.muonium_amd.fused_normuon_step(*args)
    else:
        _fused_normuon_impl(*args)


def _normuon_postpass_impl(params: list[Tensor], us: list[Tensor], variances: list[Tensor],
                           lr_ratios: list[Tensor], lr: Tensor, weight_decay: float,
                           cautious_wd: bool, beta2: float, split_sizes: Optional[list[int]],
                           shape: list[int]) -> None:
    lib = _lib.load()
    p0 = params[0]
    _lib.ensure_device(p0.device)
    _check_cuda_contig(list(params) + list(variances), "NorMuon tensors")
    lrs = adjusted_lrs(lr_ratios, lr)
    nb, rows, cols = matrix_view(shape)
    ws, cap = workspace(p0.device, torch.bfloat16, nb, rows, cols)
    sp, nsp = _splits(split_sizes)
    s = _lib.stream(p0.device)
    for p, u, v, lr_t in zip(params, us, variances, lrs):
        u = u.contiguous()
        _lib.check(
            lib.muon_normuon_postpass(
                1, _lib.ptr_array([p]), _lib.dtype_code(p.dtype), _lib.ptr_array([v]),
                _lib.dtype_code(v.dtype), u.data_ptr(), _lib.dtype_code(u.dtype), ws.data_ptr(),
                _lib.DT_BF16, cap, 0, nb, rows, cols, sp, nsp, _lib.f32_array([lr_t]), None,
                float(weight_decay), int(cautious_wd), float(beta2), s,
            ),
            "muon_normuon_postpass",
        )


def normuon_postpass(
    params: Sequence[Tensor], us: Sequence[Tensor], variances: Sequence[Tensor],
    lr_ratios: Sequence[Tensor], lr, *, weight_decay: float, cautious_wd: bool, beta2: float,
    split_sizes=None, shape=None,
) -> None:
    """NorMuon's normalization and apply for explicit updates ``us`` (one tensor per
    param, the elements in the param's order), per row block with ``split_sizes``."""
    shape = list(params[0].shape if shape is None else shape)
    args = (list(params), list(us), list(variances), list(lr_ratios), _as_tensor(lr),
            float(weight_decay), bool(cautious_wd), float(beta2),
            None if split_sizes is None else [int(v) for v in split_sizes], shape)
    if _compiling():
        torch.ops.muonium_amd.normuon_postpass(*args)
    else:
        _normuon_postpass_impl(*args)


def _fused_lp_impl(params: list[Tensor], grads: list[Tensor], codes: list[Tensor],
                   scales: list[Tensor], qmap: Optional[Tensor], qformat: int, block: int,
                   lr_ratios: list[Tensor], lr: Tensor, momentum: float, nesterov: bool,
                   maximize: bool, weight_decay: float, cautious_wd: bool, coeffs: list[float],
                   prescale: float, eps: float) -> None:
    lib = _lib.load()
    g0 = grads[0]
    device = g0.device
    _lib.ensure_device(device)
    _check_cuda_contig(list(params) + list(grads), "MuonLP step tensors")
    lrs = adjusted_lrs(lr_ratios, lr)
    nb, rows, cols = matrix_view(g0)
    count = len(grads)
    ws, cap = workspace(device, torch.bfloat16, count * nb, rows, cols)
    s = _lib.stream(device)
    steps = len(coeffs) // 3
    _lib.check(
        lib.muon_lp_prepass(
            count, _lib.ptr_array(grads), _lib.dtype_code(g0.dtype), _lib.ptr_array(codes),
            _lib.ptr_array(scales), qmap.data_ptr() if qmap is not None else None, qformat,
            block, nb, rows, cols, momentum, int(nesterov), int(maximize), ws.data_ptr(),
            _lib.DT_BF16, cap, s,
        ),
        "muon_lp_prepass",
    )
    # the iteration and the apply (fused into the last B X where the shapes allow)
    _lib.check(
        lib.muon_orth_run_apply(ws.data_ptr(), _lib.DT_BF16, cap, count * nb, rows, cols,
                                _flat_coeffs(coeffs), steps, prescale, eps, count,
                                _lib.ptr_array(params), _lib.dtype_code(params[0].dtype), nb,
                                _lib.f32_array(lrs), float(weight_decay), int(cautious_wd), s),
        "muon_orth_run_apply",
    )


def fused_lp_step(
    params: Sequence[Tensor],
    grads: Sequence[Tensor],
    states: Sequence,  # QuantizedState objects
    lr_ratios: Sequence[Tensor],
    lr,
    *,
    momentum: float,
    nesterov: bool,
    maximize: bool,
    weight_decay: float,
    cautious_wd: bool,
    coeffs: Sequence[tuple[float, float, float]],
    prescale: float,
    eps: float = 1e-7,
) -> None:
    """fused_step with quantized momentum: dequant -> momentum -> requant pre-pass."""
    st0 = states[0]
    args = (list(params), list(grads), [st.codes for st in states], [st.scale for st in states],
            st0.qmap, int(st0.qformat), int(st0.block_size), list(lr_ratios), _as_tensor(lr),
            float(momentum), bool(nesterov), bool(maximize), float(weight_decay),
            bool(cautious_wd), _flatten_coeffs(coeffs), float(prescale), float(eps))
    if _compiling():
        torch.ops.muonium_amd.fused_lp_step(*args)
    else:
        _fused_lp_impl(*args)


def _lp_quantize_impl(src: Tensor, codes: Tensor, scale: Tensor, qmap: Optional[Tensor],
                      qformat: int, block: int) -> None:
    lib = _lib.load()
    _lib.ensure_device(src.device)
    src = src.contiguous().float()
    _lib.check(
        lib.muon_lp_quantize(src.data_ptr(), codes.data_ptr(), scale.data_ptr(),
                             qmap.data_ptr() if qmap is not None else None, qformat, src.numel(),
                             block, _lib.stream(src.device)),
        "muon_lp_quantize",
    )


def lp_quantize(src: Tensor, codes: Tensor, scale: Tensor, qmap: Tensor | None, qformat: int,
                block: int) -> None:
    args = (src, codes, scale, qmap, int(qformat), int(block))
    if _compiling():
        torch.ops.muonium_amd.lp_quantize(*args)
    else:
        _lp_quantize_impl(*args)


def _lp_dequantize_impl(codes: Tensor, scale: Tensor, qmap: Optional[Tensor], qformat: int,
                        block: int, numel: int, out: Tensor) -> None:
    lib = _lib.load()
    _lib.ensure_device(codes.device)
    _lib.check(
        lib.muon_lp_dequantize(codes.data_ptr(), scale.data_ptr(),
                               qmap.data_ptr() if qmap is not None else None, qformat, numel,
                               block, out.data_ptr(), _lib.stream(codes.device)),
        "muon_lp_dequantize",
    )


def lp_dequantize(codes: Tensor, scale: Tensor, qmap: Tensor | None, qformat: int, block: int,
                  numel: int, out: Tensor) -> None:
    args = (codes, scale, qmap, int(qformat), int(block), int(numel), out)
    if _compiling():
        torch.ops.muonium_amd.lp_dequantize(*args)
    else:
        _lp_dequantize_impl(*args)


# ---------------------------------------------------------------------------------
# torch.library registration: the ops above, their written arguments and fake impls


def _register_ops() -> None:
    def op(name, impl, mutates, fake=None):
        o = torch.library.custom_op(f"muonium_amd::{name}", impl, mutates_args=mutates)
        o.register_fake(fake or (lambda *args, **kwargs: None))

    op("gram_", _gram_impl, ("y",))
    op("orthogonalize", _orthogonalize_impl, (),
       lambda tensors, coeffs, prescale, eps, iter_dtype, out_dtype: tensors[0].new_empty(
           (len(tensors), *tensors[0].shape), dtype=out_dtype))
    op("momentum_only", _momentum_impl, ("grads", "bufs"))
    op("postpass", _postpass_impl, ("params",))
    op("fused_step", _fused_step_impl, ("params", "grads", "bufs"))
    op("fused_normuon_step", _fused_normuon_impl, ("params", "grads", "bufs", "variances"))
    op("normuon_postpass", _normuon_postpass_impl, ("params", "variances"))
    op("fused_lp_step", _fused_lp_impl, ("params", "grads", "codes", "scales"))
    op("lp_quantize", _lp_quantize_impl, ("codes", "scale"))
    op("lp_dequantize", _lp_dequantize_impl, ("out",))


_register_ops()
