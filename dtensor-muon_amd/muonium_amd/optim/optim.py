"""Unified Muon + Adam optimizer (drop-in for muonium/optim/optim.py).

Same constructor, group keys, defaults, validation messages, state layout and
checkpoint (``__setstate__``) behaviour as the reference. What changes is below the
algorithm seam: Muon-family groups run this library's HIP kernels (see
``algorithms/muon.py``), and the per-algorithm implementation cache holds the plain
driver — there is no tracing compiler on this path.
"""

from __future__ import annotations

import contextlib
import functools
import math
from typing import cast

import torch
from torch import Tensor
from torch.optim.adam import adam
from torch.optim.optimizer import (
    _device_dtype_check_for_fused,
    _get_scalar_dtype,
    _use_grad_for_differentiable,
)

from muonium_amd.orthogonalize import OrthogonalizationStrategy
from muonium_amd.utils import group_tensors_by_shape, move_tensors_to_device
from muonium_amd.utils.offload import pipeline_supported, run_offloaded

from .algorithms import BufferSpec, MuonAlgorithm, get_algorithm
from .algorithms.base import ADAM_ALGORITHMS
from .lp_state import QuantizedState


def _group_muon_tensors(
    params: list[Tensor],
    grads: list[Tensor],
    state_lists: dict[str, list],
    lr_ratios: list[Tensor],
):
    """Buckets of (device, params, grads, state lists, lr_ratios) with one device,
    dtype and gradient shape each, in first-seen order (optim.py:51-78)."""
    by_dev_dtype: dict[tuple[torch.device, torch.dtype], list[int]] = {}
    for i, p in enumerate(params):
        by_dev_dtype.setdefault((p.device, p.dtype), []).append(i)
    buckets = []
    for (device, _), idx in by_dev_dtype.items():
        for _, (_, local) in group_tensors_by_shape([grads[i] for i in idx]).items():
            sel = [idx[j] for j in local]
            buckets.append(
                (
                    device,
                    [params[i] for i in sel],
                    [grads[i] for i in sel],
                    {k: [v[i] for i in sel] for k, v in state_lists.items()},
                    [lr_ratios[i] for i in sel],
                )
            )
    return buckets


def _per_tensor_runs(algorithm: MuonAlgorithm, params, grads, state, split_sizes):
    """Index lists for the per-parameter driver: singletons (one `update` call each, the
    reference's loop, optim.py:511-531), except that same-shape device tensors of a
    built-in algorithm whose per-tensor update runs entirely in this library's fused
    kernels are grouped and handed to `update_same_shape` in one launch sequence. Each
    tensor keeps the per-tensor semantics (its gradient is not rewritten) and gets bit
    for bit the result of its own `update` call: the kernels treat every matrix of a
    batch independently. Groups keep first-seen order; the updates are independent."""
    if not getattr(algorithm, "batches_per_tensor", lambda s: False)(split_sizes) or \
            torch.compiler.is_compiling():
        return [[i] for i in range(len(params))]
    keyed: dict[tuple, list[int]] = {}
    for i, (p, g) in enumerate(zip(params, grads)):
        if not p.is_cuda:
            keyed[("single", i)] = [i]
            continue
        bufs = tuple((type(b[i]), b[i].dtype, getattr(b[i], "block_size", None),
                      getattr(b[i], "signed", None)) for b in state.values())
        keyed.setdefault((p.device, p.dtype, tuple(g.shape), g.dtype, bufs), []).append(i)
    return list(keyed.values())


# GPU_MAX_HW_QUEUES is 4 by default: with the caller's stream, one hardware queue each (a
# fourth side stream shared a queue with the third, which serialized their buckets)
_MAX_SIDE_STREAMS = 3
_side_streams: dict[tuple[int, int], torch.cuda.Stream] = {}


def _side_stream(device: torch.device, slot: int) -> torch.cuda.Stream:
    """Side stream `slot` of `device` (default priority), created once per process."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, slot)
    stream = _side_streams.get(key)
    if stream is None:
        stream = _side_streams[key] = torch.cuda.Stream(device=index)
    return stream


_sync_events: dict[tuple, torch.cuda.Event] = {}


def _wait(waiter: torch.cuda.Stream, producer: torch.cuda.Stream, key: tuple) -> None:
    """``waiter.wait_stream(producer)`` with an event kept per (device, slot, direction):
    recording an event again is legal (a wait already issued keeps the state it saw), and
    it saves creating one per fork and join."""
    ev = _sync_events.get(key)
    if ev is None:
        ev = _sync_events[key] = torch.cuda.Event()
    ev.record(producer)
    waiter.wait_event(ev)


def _concurrent_plan(buckets, algorithm: MuonAlgorithm,
                     batch_size: int | None) -> tuple[dict[int, int], list[int]]:
    """Side-stream slot per bucket index for buckets too small to fill the device, and the
    order in which to enqueue the buckets.

    A bucket whose Gram products (upper-triangle 256-row tiles x matrices) launch fewer
    workgroups than the device has compute units leaves most of it idle (the GPT-2 set:
    72 workgroups per product on 256 CUs); such buckets run concurrently. When every bucket
    is small, the smallest stays on the caller's stream and the others take side streams,
    largest first; otherwise all small buckets take side streams and the large ones stay on
    the caller's stream. Buckets on side streams are enqueued first, so each forks from the
    caller's stream as the step starts and the largest is not held back by the host time of
    enqueueing the others (about 15 us per launch, 17 launches per bucket). Workspaces are
    cached per stream, so a side stream never touches the buffer of the current stream or of
    another side stream, also when two buckets pad to the same workspace shape (the GPT-2
    mlp c_fc and the transposed c_proj: on one stream they ran one after the other and made
    the step's critical path). Built-in algorithms only."""
    natural = list(range(len(buckets)))
    if not type(algorithm).__module__.startswith("muonium_amd.") or torch.compiler.is_compiling():
        return {}, natural  # (under an outer torch.compile the buckets run in the traced order)

    cus: dict[torch.device, int] = {}
    work: dict[int, int] = {}
    for bi, (device, _, dev_g, _, _) in enumerate(buckets):
        if device.type != "cuda" or dev_g[0].dim() < 2:
            continue
        if device not in cus:
            cus[device] = torch.cuda.get_device_properties(device).multi_processor_count
        rows, cols = dev_g[0].shape[-2:]
        nmat = math.prod(dev_g[0].shape[:-2]) * min(len(dev_g), batch_size or len(dev_g))
        tiles = -(-min(rows, cols) // 256)
        if tiles * (tiles + 1) // 2 * nmat < cus[device]:
            work[bi] = min(rows, cols) ** 2 * max(rows, cols) * nmat
    if len(work) < 2:
        return {}, natural
    ranked = sorted(work, key=lambda bi: -work[bi])
    side = ranked[:-1] if len(work) == len(buckets) else ranked
    slots = {bi: k % _MAX_SIDE_STREAMS for k, bi in enumerate(side)}
    return slots, side + [bi for bi in natural if bi not in slots]


class Muon(torch.optim.Optimizer):
    def __init__(
        self,
        params,
        lr: float = 1e-3,
        wd: float = 0.1,
        use_cautious_wd: bool = True,
        maximize: bool = False,
        # Muon defaults
        momentum: float = 0.95,
        nesterov: bool = True,
        ns_steps: int = 5,
        orthogonalization_strategy: OrthogonalizationStrategy = "polar_express",
        # Adam defaults
        amsgrad: bool = False,
        adam_betas: tuple[float, float] = (0.9, 0.95),
        adam_eps: float = 1e-8,
        is_adamw: bool = True,
        fused_adam: bool | None = None,
        foreach_adam: bool | None = None,
        # Execution strategy
        foreach: bool | None = None,
        batch_size: int | None = None,
    ):
        """Muon for 2D+ parameters plus Adam/AdamW groups, in one optimizer.

        Param-group keys and defaults are those of muonium's ``Muon``
        (optim.py:82-209): ``algorithm`` ("muon" default, any registered variant, or
        "adam"/"adamw"), ``lr``, ``wd``, ``use_cautious_wd``, ``momentum``,
        ``nesterov``, ``ns_steps``, ``orthogonalization_strategy``, ``maximize``,
        ``flatten``, ``split_sizes``, ``foreach`` and the algorithm's own options.
        ``foreach`` batches same-(device, dtype, shape) tensors into one kernel launch
        sequence; None enables it when every param of the group is on a HIP device.
        ``batch_size`` caps the tensors per batch.
        """
        self.lr = lr
        self.wd = wd
        self.use_cautious_wd = use_cautious_wd
        self.momentum = momentum
        self.nesterov = nesterov
        self.ns_steps = ns_steps
        self.orthogonalization_strategy = orthogonalization_strategy
        self.amsgrad = amsgrad
        self.adam_betas = adam_betas
        self.adam_eps = adam_eps
        self.is_adamw = is_adamw
        self.fused_adam = fused_adam
        self.foreach_adam = foreach_adam
        self.maximize = maximize
        self.foreach = foreach
        self.batch_size = batch_size

        if not 0.0 <= lr:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= adam_eps:
            raise ValueError(f"Invalid epsilon value: {adam_eps}")
        if not 0.0 <= adam_betas[0] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 0: {adam_betas[0]}")
        if not 0.0 <= adam_betas[1] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 1: {adam_betas[1]}")
        if isinstance(params, dict):
            raise TypeError(
                "params must be an iterable of parameters or "
                "an iterable of param-group dicts, not a single dict."
            )
        params = list(params)
        if len(params) == 0:
            raise ValueError("optimizer got an empty parameter list")
        if not isinstance(params[0], dict):
            params = [{"params": params}]

        groups: list[dict] = []
        for group in params:
            algorithm = cast(str, group.get("algorithm", "muon")).lower()
            if "params" not in group:
                raise ValueError("Param group dict must have a 'params' key")
            group["params"] = list(group["params"])
            if len(group["params"]) == 0:
                continue
            if algorithm in ADAM_ALGORITHMS:
                groups.append(self._build_adam_group(group))
            else:
                groups.append(self._build_muon_group(group, get_algorithm(algorithm)))

        super().__init__(groups, {"differentiable": False})
        self._init_muon_impl()

    # -- implementation cache (tests and subclasses use these private seams) --------

    def _init_muon_impl(self) -> None:
        """Reset the per-algorithm implementation cache (filled lazily per name)."""
        self._muon_impls: dict[str, object] = {}

    def _raw_muon_impl(self, algorithm: MuonAlgorithm):
        return functools.partial(self.muon, algorithm)

    def _get_muon_impl(self, algorithm: MuonAlgorithm):
        impl = self._muon_impls.get(algorithm.name)
        if impl is None:
            impl = self._raw_muon_impl(algorithm)
            self._muon_impls[algorithm.name] = impl
        return impl

    # -- group construction ---------------------------------------------------------

    @staticmethod
    def _validate_split_sizes(group: dict) -> tuple[int, ...] | None:
        """optim.py:231-257."""
        split_sizes = group.get("split_sizes")
        if split_sizes is None:
            return None
        if not isinstance(split_sizes, (tuple, list)) or len(split_sizes) < 2:
            raise ValueError(
                f"split_sizes must be a tuple or list of at least 2 block sizes, "
                f"got {split_sizes!r}."
            )
        if not all(isinstance(s, int) and not isinstance(s, bool) and s > 0 for s in split_sizes):
            raise ValueError(
                f"split_sizes entries must be positive integers, got {split_sizes!r}."
            )
        for p in group["params"]:
            if p.ndim != 2:
                raise ValueError(
                    f"split_sizes is only supported for 2D parameters, got shape "
                    f"{tuple(p.shape)}."
                )
            if sum(split_sizes) != p.shape[0]:
                raise ValueError(
                    f"split_sizes {tuple(split_sizes)} must sum to dim 0 of the "
                    f"parameter shape {tuple(p.shape)}."
                )
        return tuple(split_sizes)

    def _build_muon_group(self, group: dict, algorithm: MuonAlgorithm):
        """optim.py:259-295."""
        for p in group["params"]:
            algorithm.validate_param(p)
        foreach = group.get("foreach", self.foreach)
        if foreach is None:
            foreach = all(p.is_cuda for p in group["params"])
        built = {
            "params": group["params"],
            "algorithm": algorithm.name,
            "use_muon": True,
            "lr": torch.tensor(group.get("lr", self.lr)),
            "wd": group.get("wd", self.wd),
            "use_cautious_wd": group.get("use_cautious_wd", self.use_cautious_wd),
            "momentum": group.get("momentum", self.momentum),
            "nesterov": group.get("nesterov", self.nesterov),
            "ns_steps": group.get("ns_steps", self.ns_steps),
            "orthogonalization_strategy": group.get(
                "orthogonalization_strategy", self.orthogonalization_strategy
            ),
            "maximize": group.get("maximize", self.maximize),
            "flatten": group.get("flatten", False),
            "split_sizes": self._validate_split_sizes(group),
            "foreach": foreach,
        }
        for key, default in algorithm.options.items():
            built[key] = group.get(key, default)
        return built

    def _build_adam_group(self, group: dict):
        """optim.py:297-315."""
        algorithm = cast(str, group.get("algorithm", "adamw")).lower()
        return {
            "params": group["params"],
            "algorithm": algorithm,
            "use_muon": False,
            "lr": group.get("lr", self.lr),
            "wd": group.get("wd", self.wd),
            "amsgrad": group.get("amsgrad", self.amsgrad),
            "betas": group.get("betas", self.adam_betas),
            "eps": group.get("eps", self.adam_eps),
            "decoupled_weight_decay": group.get(
                "decoupled_weight_decay", self.is_adamw and algorithm == "adamw"
            ),
            "fused": group.get("fused", self.fused_adam),
            "foreach": group.get("foreach", self.foreach_adam),
            "maximize": group.get("maximize", self.maximize),
            "has_complex": any(torch.is_complex(p) for p in group["params"]),
        }

    def __setstate__(self, state):
        """Checkpoint load: legacy defaults and tensor coercion (optim.py:317-368)."""
        super().__setstate__(state)
        for group in self.param_groups:
            if group["use_muon"]:
                group.setdefault("algorithm", "muon")
                algorithm = get_algorithm(group["algorithm"])
                group.setdefault("ns_steps", 5)
                group.setdefault("nesterov", True)
                group.setdefault("flatten", False)
                group.setdefault("use_cautious_wd", True)
                group.setdefault("orthogonalization_strategy", "polar_express")
                group.setdefault("split_sizes", None)
                if "foreach" not in group:
                    group["foreach"] = all(p.is_cuda for p in group["params"])
                for key, default in algorithm.options.items():
                    group.setdefault(key, default)
                if not torch.is_tensor(group["lr"]):
                    group["lr"] = torch.tensor(float(group["lr"]))
                for p in group["params"]:
                    p_state = self.state.get(p, [])
                    if len(p_state) != 0 and not torch.is_tensor(p_state["step"]):
                        p_state["step"] = torch.tensor(float(p_state["step"]))
                    # load_state_dict moves tensor state to the param's device; quantized
                    # momentum (not a tensor) is moved here, as torchao's subclasses are
                    for key, val in (p_state.items() if len(p_state) != 0 else ()):
                        if isinstance(val, QuantizedState) and val.device != p.device:
                            p_state[key] = val.to(p.device)
            else:
                group.setdefault("amsgrad", False)
                group.setdefault("maximize", False)
                group.setdefault("foreach", None)
                group.setdefault("decoupled_weight_decay", False)
                if torch.is_tensor(group["wd"]):
                    group["wd"] = float(group["wd"])
                fused = group.setdefault("fused", None)
                for p in group["params"]:
                    p_state = self.state.get(p, [])
                    if len(p_state) != 0 and not torch.is_tensor(p_state["step"]):
                        step_val = float(p_state["step"])
                        p_state["step"] = (
                            torch.tensor(step_val, dtype=_get_scalar_dtype(is_fused=fused),
                                         device=p.device)
                            if group["fused"]
                            else torch.tensor(step_val, dtype=_get_scalar_dtype())
                        )
        self._init_muon_impl()

    # -- state ------------------------------------------------------------------------

    def _new_state_buffer(self, p: Tensor, grad: Tensor, spec: BufferSpec):
        """fp32 zeros shaped like the transformed grad (``like="grad"``) or one value
        per row (``"grad_rows"``) (optim.py:370-376). Overridden to quantize."""
        reference = grad if spec.like == "grad" else grad[..., :1]
        return torch.zeros_like(reference, dtype=torch.float32, memory_format=torch.preserve_format)

    def _init_muon_group(self, group, algorithm, params_with_grad, grads, state_lists,
                         lr_ratios, state_steps) -> None:
        """optim.py:378-419."""
        for p in group["params"]:
            grad = p.grad
            if grad is None:
                continue
            params_with_grad.append(p)
            assert not grad.is_sparse, "Muon does not support sparse gradients"
            if grad.ndim > 2:
                if group["flatten"]:
                    grad = grad.view(grad.size(0), -1)
                elif grad.ndim > 3:
                    grad = grad.flatten(end_dim=-3)
            grads.append(grad)
            state = self.state[p]
            if len(state) == 0:
                state["step"] = torch.tensor(0.0, dtype=_get_scalar_dtype())
                for key, spec in algorithm.state_spec.items():
                    state[key] = self._new_state_buffer(p, grad, spec)
                state["lr_ratio"] = torch.tensor(
                    math.sqrt(max(1.0, grad.shape[-2] / grad.shape[-1]))
                )
            for key in algorithm.state_spec:
                state_lists[key].append(state[key])
            lr_ratios.append(state["lr_ratio"])
            state_steps.append(state["step"])
        # state["step"] += 1 for every parameter with a gradient, in one call (one dispatch
        # instead of one per parameter: about 3 us each on the host, before the first launch)
        if state_steps:
            torch._foreach_add_(state_steps, 1)

    def _init_adam_group(self, group, params_with_grad, grads, exp_avgs, exp_avg_sqs,
                         max_exp_avg_sqs, state_steps, capturable):
        """optim.py:421-477."""
        for p in group["params"]:
            if p.grad is None:
                continue
            params_with_grad.append(p)
            assert not p.grad.is_sparse, (
                "Adam does not support sparse gradients, please consider SparseAdam instead"
            )
            grads.append(p.grad)
            state = self.state[p]
            if len(state) == 0:
                if group["fused"]:
                    _device_dtype_check_for_fused(p)
                state["step"] = (
                    torch.zeros((), dtype=_get_scalar_dtype(is_fused=group["fused"]),
                                device=p.device)
                    if capturable or group["fused"]
                    else torch.tensor(0.0, dtype=_get_scalar_dtype())
                )
                state["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                if group["amsgrad"]:
                    state["max_exp_avg_sq"] = torch.zeros_like(
                        p, memory_format=torch.preserve_format
                    )
            elif capturable and state["step"].device != p.device:
                state["step"] = state["step"].to(p.device)
            exp_avgs.append(state["exp_avg"])
            exp_avg_sqs.append(state["exp_avg_sq"])
            if group["amsgrad"]:
                max_exp_avg_sqs.append(state["max_exp_avg_sq"])
            state_steps.append(state["step"])

    # -- drivers ----------------------------------------------------------------------

    def muon(
        self,
        algorithm: MuonAlgorithm,
        params: list[Tensor],
        grads: list[Tensor],
        state: dict[str, list],
        lr_ratios: list[Tensor],
        *,
        foreach: bool = False,
        nesterov: bool,
        lr: Tensor,
        weight_decay: float,
        cautious_wd: bool,
        momentum: float,
        ns_steps: int,
        orthogonalization_strategy: OrthogonalizationStrategy,
        maximize: bool,
        split_sizes: tuple[int, ...] | None = None,
        **opts,
    ) -> None:
        """Muon-family update for a list of parameters (optim.py:479-595).

        ``foreach=False``: ``algorithm.update`` per tensor. ``foreach=True``: bucket by
        (device, dtype, shape), chunk by ``batch_size``, round-trip host-resident
        batches through the HIP device, and call ``algorithm.foreach_update``."""
        if len(params) == 0:
            return
        hp = dict(
            lr=lr, weight_decay=weight_decay, cautious_wd=cautious_wd, momentum=momentum,
            nesterov=nesterov, maximize=maximize, ns_steps=ns_steps,
            orthogonalization_strategy=orthogonalization_strategy, split_sizes=split_sizes,
            **opts,
        )
        if not foreach:
            for idx in _per_tensor_runs(algorithm, params, grads, state, split_sizes):
                if len(idx) == 1:
                    i = idx[0]
                    algorithm.update(params[i], grads[i], {k: b[i] for k, b in state.items()},
                                     lr_ratios[i], **hp)
                else:
                    algorithm.update_same_shape(
                        [params[i] for i in idx], [grads[i] for i in idx],
                        {k: [b[i] for i in idx] for k, b in state.items()},
                        [lr_ratios[i] for i in idx], **hp)
            return

        buckets = _group_muon_tensors(params, grads, state, lr_ratios)
        slots, order = _concurrent_plan(buckets, algorithm, self.batch_size)
        forked: dict[tuple[torch.device, int], torch.cuda.Stream] = {}
        for bi in order:
            device, dev_p, dev_g, dev_state, dev_lr = buckets[bi]
            if bi in slots:
                side = _side_stream(device, slots[bi])
                if (device, slots[bi]) not in forked:
                    _wait(side, torch.cuda.current_stream(device), (device, slots[bi], 0))
                    forked[(device, slots[bi])] = side
                ctx = torch.cuda.stream(side)
            else:
                ctx = contextlib.nullcontext()
            with ctx:
                self._muon_bucket(algorithm, hp, nesterov, maximize, device, dev_p, dev_g,
                                  dev_state, dev_lr)
        for (device, slot), side in forked.items():
            _wait(torch.cuda.current_stream(device), side, (device, slot, 1))

    def _muon_bucket(self, algorithm, hp, nesterov, maximize, device, dev_p, dev_g, dev_state,
                     dev_lr) -> None:
        """One (device, dtype, shape) bucket of the foreach driver, chunked by batch_size."""
        idx = list(range(len(dev_g)))
        if self.batch_size and len(idx) > self.batch_size:
            batches = [idx[i : i + self.batch_size] for i in range(0, len(idx), self.batch_size)]
        else:
            batches = [idx]
        if device.type != "cuda":
            host = [
                ([dev_p[i] for i in sel], [dev_g[i] for i in sel],
                 {k: [v[i] for i in sel] for k, v in dev_state.items()},
                 [dev_lr[i] for i in sel])
                for sel in batches
            ]
            if (torch.cuda.is_available() and not torch.compiler.is_compiling()
                    and all(pipeline_supported(b) for b in host)):
                # pinned-memory round trip, copies overlapped with the updates
                run_offloaded(
                    host,
                    lambda p, g, st, lr: algorithm.foreach_update(p, g, st, lr, **hp),
                    # the built-in algorithms rewrite the grads only under Nesterov
                    # without maximize (muon.py:117-118); copy them back for any other
                    grads_modified=(nesterov and not maximize)
                    or not type(algorithm).__module__.startswith("muonium_amd."),
                )
                return
        for sel in batches:
            p_orig = [dev_p[i] for i in sel]
            g_orig = [dev_g[i] for i in sel]
            s_orig = {k: [v[i] for i in sel] for k, v in dev_state.items()}
            lr_orig = [dev_lr[i] for i in sel]
            cuda = torch.device("cuda")
            p_b = move_tensors_to_device(p_orig, device, cuda)
            g_b = move_tensors_to_device(g_orig, device, cuda)
            s_b = {k: move_tensors_to_device(v, device, cuda) for k, v in s_orig.items()}
            lr_b = move_tensors_to_device(lr_orig, device, cuda)
            algorithm.foreach_update(
                cast(list[Tensor], p_b), cast(list[Tensor], g_b), cast(dict, s_b),
                cast(list[Tensor], lr_b), **hp,
            )
            pairs = [(p_orig, p_b), (g_orig, g_b), (lr_orig, lr_b)]
            pairs.extend((s_orig[k], s_b[k]) for k in s_orig)
            for originals, moved in pairs:
                if originals is not moved:
                    for o, v in zip(originals, moved, strict=True):
                        if o is not None and v is not None:
                            o.copy_(v.to(o.device))

    def _step_muon_group(self, group: dict) -> None:
        """optim.py:597-640."""
        algorithm = get_algorithm(group.get("algorithm", "muon"))
        params_with_grad: list[Tensor] = []
        grads: list[Tensor] = []
        state_steps: list[Tensor] = []
        state_lists: dict[str, list] = {key: [] for key in algorithm.state_spec}
        lr_ratios: list[Tensor] = []
        self._init_muon_group(group, algorithm, params_with_grad, grads, state_lists, lr_ratios,
                              state_steps)
        impl = (
            self._raw_muon_impl(algorithm)
            if torch.compiler.is_compiling()
            else self._get_muon_impl(algorithm)
        )
        impl(
            params_with_grad,
            grads,
            state_lists,
            lr_ratios,
            foreach=group["foreach"],
            nesterov=group["nesterov"],
            lr=group["lr"],
            weight_decay=group["wd"],
            cautious_wd=group["use_cautious_wd"],
            momentum=group["momentum"],
            ns_steps=group["ns_steps"],
            orthogonalization_strategy=group["orthogonalization_strategy"],
            maximize=group["maximize"],
            split_sizes=group["split_sizes"],
            **{key: group[key] for key in algorithm.options},
        )

    def _step_adam_group(self, group: dict) -> None:
        """Adam/AdamW groups delegate to torch's functional adam (optim.py:642-694)."""
        params_with_grad: list[Tensor] = []
        grads: list[Tensor] = []
        state_steps: list[Tensor] = []
        exp_avgs: list[Tensor] = []
        exp_avg_sqs: list[Tensor] = []
        max_exp_avg_sqs: list[Tensor] = []
        beta1, beta2 = group["betas"]
        capturable = torch.compiler.is_compiling()
        self._init_adam_group(group, params_with_grad, grads, exp_avgs, exp_avg_sqs,
                              max_exp_avg_sqs, state_steps, capturable)
        lr = group["lr"]
        weight_decay = group["wd"]
        if not group["fused"] and not torch.compiler.is_compiling():
            lr = float(lr) if torch.is_tensor(lr) else lr
            weight_decay = float(weight_decay) if torch.is_tensor(weight_decay) else weight_decay
        adam(
            params_with_grad,
            grads,
            exp_avgs,
            exp_avg_sqs,
            max_exp_avg_sqs,
            state_steps,
            amsgrad=group["amsgrad"],
            has_complex=group["has_complex"],
            beta1=beta1,
            beta2=beta2,
            lr=lr,
            weight_decay=weight_decay,
            eps=group["eps"],
            maximize=group["maximize"],
            capturable=capturable,
            differentiable=False,
            fused=group["fused"],
            foreach=group["foreach"],
            grad_scale=getattr(self, "grad_scale", None),
            found_inf=getattr(self, "found_inf", None),
            decoupled_weight_decay=group["decoupled_weight_decay"],
        )

    @_use_grad_for_differentiable
    def step(self, closure=None):
        """One optimization step over every group; returns the closure's loss."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            if group["use_muon"]:
                self._step_muon_group(group)
            else:
                self._step_adam_group(group)
        return loss
