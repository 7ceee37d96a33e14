"""The allocation-free entry point muon_normuon_postpass_noalloc against the entry point
it varies, muon_normuon_postpass with an explicit update and a caller workspace: the same
params and variance states, bit for bit, on two calls in a row (the second smaller, so
it reads only what it wrote into the shared static scratch), through the C ABI. Sizes
beyond the scratch are refused before anything is launched."""

import pytest
import torch

from muonium_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _case(ntensors, nb, rows, cols, seed):
    gen = torch.Generator().manual_seed(seed)
    shape = (nb, rows, cols) if nb > 1 else (rows, cols)
    ps = [torch.randn(shape, generator=gen).bfloat16() for _ in range(ntensors)]
    # updates of orthogonalized scale, with rows of different magnitudes
    us = torch.stack([(torch.randn(shape, generator=gen)
                       * torch.exp(torch.randn(*shape[:-1], 1, generator=gen)) / cols**0.5)
                      for _ in range(ntensors)]).bfloat16()
    vs = [torch.rand(*shape[:-1], 1, generator=gen) * 1e-3 for _ in range(ntensors)]
    lrs = [0.01 * (1 + i % 3) for i in range(ntensors)]
    return ps, us, vs, lrs


def _run(noalloc, ps, us, vs, lrs, nb, rows, cols, splits, uscales=None):
    lib = _lib.load()
    dev = torch.device(DEV)
    _lib.ensure_device(dev)
    p = [t.clone().to(DEV) for t in ps]
    v = [t.clone().to(DEV) for t in vs]
    u = us.to(DEV)
    sp = _lib.i64_array(list(splits)) if splits else None
    nsp = len(splits) if splits else 0
    s = _lib.stream(dev)
    args = (len(p), _lib.ptr_array(p), _lib.DT_BF16, _lib.ptr_array(v), _lib.DT_F32,
            u.data_ptr(), _lib.DT_BF16)
    usc = None if uscales is None else _lib.f32_array(uscales)
    tail = (nb, rows, cols, sp, nsp, _lib.f32_array(lrs), usc, 0.1, 1, 0.95, s)
    if noalloc:
        rc = lib.muon_normuon_postpass_noalloc(*args, *tail)
    else:
        nbytes = lib.muon_orth_workspace_bytes(_lib.DT_BF16, len(p) * nb, rows, cols)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        rc = lib.muon_normuon_postpass(*args, ws.data_ptr(), _lib.DT_BF16, len(p) * nb, 0,
                                       *tail)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return [t.cpu() for t in p], [t.cpu() for t in v]


def test_noalloc_matches_workspace_entry_point_twice():
    # first call: 40 tensors (two chunks of the multi-tensor launch), 2 matrices each,
    # with row blocks and per-tensor update scales; second call smaller in every extent
    for ntensors, nb, rows, cols, splits, seed in ((40, 2, 384, 256, (128, 256), 1),
                                                   (3, 1, 100, 64, None, 2)):
        ps, us, vs, lrs = _case(ntensors, nb, rows, cols, seed)
        usc = [0.75 + 0.1 * (i % 4) for i in range(ntensors)] if splits else None
        ref_p, ref_v = _run(False, ps, us, vs, lrs, nb, rows, cols, splits, usc)
        got_p, got_v = _run(True, ps, us, vs, lrs, nb, rows, cols, splits, usc)
        for a, b, p0 in zip(got_p, ref_p, ps):
            assert torch.equal(a, b)
            assert not torch.equal(a, p0)  # the step did move the params
        for a, b in zip(got_v, ref_v):
            assert torch.equal(a, b)


def test_noalloc_refuses_sizes_beyond_the_scratch():
    lib = _lib.load()
    # 1 tensor of 5e6 rows needs 20 MB of row statistics > 16 MiB: refused before any
    # launch (no pointer is touched)
    rc = lib.muon_normuon_postpass_noalloc(1, _lib.ptr_array([None]), _lib.DT_BF16,
                                           _lib.ptr_array([None]), _lib.DT_F32, 16,
                                           _lib.DT_BF16, 1, 5_000_000, 8, None, 0,
                                           _lib.f32_array([0.01]), None, 0.1, 1, 0.95, None)
    assert rc == 1  # MUON_ERR_SHAPE
    assert "scratch" in _lib.last_error()
