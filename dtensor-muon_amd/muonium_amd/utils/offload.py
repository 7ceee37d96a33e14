"""Host-offloaded foreach batches through the HIP device, with the copies overlapped.

The reference's foreach driver (optim.py:546-595) copies each batch of host-resident
tensors to the device, runs the update, and copies every tensor back, one batch after
the other. Here the same round trip is pipelined over two copy streams of default
priority: while batch k's update runs on the current stream, batch k+1 is staged into
pinned host memory and uploaded on one stream, batch k's results are downloaded on the
other as soon as its update ends, and batch k-1's results are written back into the
host tensors. Values are those of the sequential round trip; tensors the update does not
modify (the lr ratios, and the gradients unless Nesterov rewrote them) are not copied
back, which leaves them unchanged as the reference's copy-back of an unmodified value
does.
"""

from __future__ import annotations

from typing import Callable, Sequence

import torch
from torch import Tensor

Batch = tuple[list[Tensor], list[Tensor], dict[str, list[Tensor]], list[Tensor]]


def pipeline_supported(batch: Batch) -> bool:
    """Plain host tensors only (quantized state objects take the sequential path)."""
    p, g, s, _ = batch
    tensors = [*p, *g, *(t for ts in s.values() for t in ts)]
    return all(isinstance(t, Tensor) and t.device.type == "cpu" for t in tensors)


class _Staged:
    def __init__(self, batch: Batch, stream: torch.cuda.Stream):
        p, g, s, lr = batch
        self.keys = list(s)
        self.host = [*p, *g, *(t for k in self.keys for t in s[k])]
        self.counts = (len(p), len(g), [len(s[k]) for k in self.keys])
        self.lr = lr
        # pageable -> pinned on the host, pinned -> device on the upload stream
        self.pinned = [torch.empty_like(t, device="cpu", pin_memory=True) for t in self.host]
        for dst, src in zip(self.pinned, self.host):
            dst.copy_(src)
        with torch.cuda.stream(stream):
            self.dev = [torch.empty_like(t, device="cuda") for t in self.host]
            for d, h in zip(self.dev, self.pinned):
                d.copy_(h, non_blocking=True)
        self.uploaded = torch.cuda.Event()
        self.uploaded.record(stream)
        self.downloaded: torch.cuda.Event | None = None
        self.back: list[int] = []

    def split(self):
        np_, ng, ns = self.counts
        p = self.dev[:np_]
        g = self.dev[np_:np_ + ng]
        s, o = {}, np_ + ng
        for k, n in zip(self.keys, ns):
            s[k] = self.dev[o:o + n]
            o += n
        return p, g, s

    def download(self, stream: torch.cuda.Stream, after: torch.cuda.Event, grads_modified: bool):
        np_, ng, _ = self.counts
        self.back = [i for i in range(len(self.dev)) if not (np_ <= i < np_ + ng) or grads_modified]
        with torch.cuda.stream(stream):
            stream.wait_event(after)
            for i in self.back:
                # the pinned buffer's upload finished before the update began
                self.pinned[i].copy_(self.dev[i], non_blocking=True)
                self.dev[i].record_stream(stream)
        self.downloaded = torch.cuda.Event()
        self.downloaded.record(stream)

    def write_back(self) -> None:
        assert self.downloaded is not None
        self.downloaded.synchronize()
        for i in self.back:
            self.host[i].copy_(self.pinned[i])
        self.dev = []
        self.pinned = []


def run_offloaded(
    batches: Sequence[Batch],
    update: Callable[[list[Tensor], list[Tensor], dict[str, list[Tensor]], list[Tensor]], None],
    *,
    grads_modified: bool,
) -> None:
    """Run ``update(params, grads, state, lr_ratios)`` on device copies of each host batch,
    writing the results back into the host tensors, with uploads, updates and downloads
    of neighbouring batches overlapped."""
    if not batches:
        return
    compute = torch.cuda.current_stream()
    up = torch.cuda.Stream()
    down = torch.cuda.Stream()
    staged = _Staged(batches[0], up)
    previous: _Staged | None = None
    for k in range(len(batches)):
        compute.wait_event(staged.uploaded)
        for d in staged.dev:
            d.record_stream(compute)
        p, g, s = staged.split()
        update(p, g, s, staged.lr)
        done = torch.cuda.Event()
        done.record(compute)
        staged.download(down, done, grads_modified)
        current = staged
        if k + 1 < len(batches):
            staged = _Staged(batches[k + 1], up)
        if previous is not None:
            previous.write_back()
        previous = current
    assert previous is not None
    previous.write_back()
