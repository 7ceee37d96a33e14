"""optimizer.step() under an outer torch.compile (the reference: optim.py:616-623 runs the
raw update when a caller's compile traces step(); tests/optim/test_optim.py:30-69, :139 and
test_optim_foreach.py:140-222 pin it).

The library's calls are torch.library custom ops ("muonium_amd::*", with fake impls), so
the tracer captures them in the caller's graph. Checked here: the nested implementation
cache is not used; a recording backend sees graphs holding the library's ops; the compiled
step gives, bit for bit, the eager step's params and state (same kernels on the same
inputs), through the recording backend and through AOTAutograd's functionalization
("aot_eager"); the plain per-parameter, foreach, heterogeneous-bucket, NorMuon and MuonLP
paths all run."""

import pytest
import torch
import torch.nn as nn

import muonium_amd.optim.algorithms.base as algo_base
from muonium_amd import Muon
from muonium_amd.optim import Muon8bit
from muonium_amd.optim.algorithms import get_algorithm

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True)
def _fresh_dynamo(monkeypatch):
    """Each test compiles step() of new optimizer objects: start from an empty Dynamo
    cache with room for the recompiles (the reference's tests raise the same limits,
    benchmark/harness.py:21-23)."""
    monkeypatch.setattr(torch._dynamo.config, "recompile_limit", 256)
    monkeypatch.setattr(torch._dynamo.config, "accumulated_recompile_limit", 256)
    torch._dynamo.reset()
    yield
    torch._dynamo.reset()


def _fail_nested(*args, **kwargs):
    raise AssertionError("external compilation must use the raw Muon kernel")


def _backend(kind, graphs):
    if kind == "aot_eager":
        return "aot_eager"

    def recording_backend(graph_module, _example_inputs):
        graphs.append(graph_module)
        return graph_module.forward

    return recording_backend


def _ops_in(graphs):
    return sum(gm.code.count("muonium_amd") for gm in graphs)


@pytest.mark.parametrize("backend", ["recording", "aot_eager"])
def test_external_torch_compile_captures_muon_update(monkeypatch, backend):
    """test_optim.py:30-69 on the device: identity orthogonalizer, two steps."""
    monkeypatch.setattr(algo_base, "zeropower", lambda g, **_: g)
    p = nn.Parameter(torch.ones(4, 2, device=DEV))
    ref = nn.Parameter(p.detach().clone())
    kw = dict(lr=0.1, wd=0.0, momentum=0.0, nesterov=False)
    optimizer = Muon([p], **kw)
    ref_optimizer = Muon([ref], **kw)
    ref_optimizer._muon_impls["muon"] = ref_optimizer._raw_muon_impl(get_algorithm("muon"))
    optimizer._muon_impls["muon"] = _fail_nested
    graphs = []

    @torch.compile(backend=_backend(backend, graphs))
    def compiled_step():
        optimizer.step()

    for value in (0.5, 0.25):
        p.grad = torch.full_like(p, value)
        ref.grad = torch.full_like(ref, value)
        compiled_step()
        ref_optimizer.step()
    if backend == "recording":
        assert graphs and _ops_in(graphs) > 0
    torch.testing.assert_close(p, ref)
    for key in ("momentum_buffer", "step"):
        torch.testing.assert_close(optimizer.state[p][key], ref_optimizer.state[ref][key])


@pytest.mark.parametrize("backend", ["recording", "aot_eager"])
@pytest.mark.parametrize("foreach", [False, True])
@pytest.mark.parametrize("strategy", ["newton_schulz", "polar_express"])
def test_external_torch_compile_runs_real_kernels_bit_exact(backend, foreach, strategy):
    """test_optim.py:139 / test_optim_foreach.py:197-222 with the real kernels, checked
    against an eager step: several buckets (two shapes, two dtypes), cautious wd,
    Nesterov, two steps."""
    gen = torch.Generator().manual_seed(7)
    specs = [((8, 4), torch.float32), ((8, 4), torch.float32), ((64, 96), torch.bfloat16),
             ((3, 32, 16), torch.float32)]
    init = [torch.randn(s, generator=gen).to(dt) for s, dt in specs]
    grads = [[torch.randn(s, generator=gen).to(dt) for s, dt in specs] for _ in range(2)]
    kw = dict(lr=0.01, wd=0.1, momentum=0.9, nesterov=True, foreach=foreach,
              orthogonalization_strategy=strategy)
    a = [nn.Parameter(t.clone().to(DEV)) for t in init]
    b = [nn.Parameter(t.clone().to(DEV)) for t in init]
    opt_c, opt_e = Muon(a, **kw), Muon(b, **kw)
    opt_c._muon_impls["muon"] = _fail_nested
    graphs = []

    @torch.compile(backend=_backend(backend, graphs))
    def compiled_step():
        opt_c.step()

    for gs in grads:
        for pa, pb, g in zip(a, b, gs):
            pa.grad = g.clone().to(DEV)
            pb.grad = g.clone().to(DEV)
        compiled_step()
        opt_e.step()
    torch.cuda.synchronize()
    if backend == "recording":
        assert graphs and _ops_in(graphs) > 0
    for pa, pb, t0 in zip(a, b, init):
        assert torch.equal(pa.detach(), pb.detach())
        assert not torch.equal(pa.detach().cpu(), t0)
        assert torch.equal(opt_c.state[pa]["momentum_buffer"], opt_e.state[pb]["momentum_buffer"])
        assert torch.equal(opt_c.state[pa]["step"], opt_e.state[pb]["step"])


@pytest.mark.parametrize("algo", ["normuon", "muon8bit"])
def test_external_torch_compile_runs_normuon_and_quantized_state(algo):
    """NorMuon (extra row-variance state) and MuonLP (quantized momentum objects) under a
    compiled step, bit-exact against eager."""
    gen = torch.Generator().manual_seed(9)
    shapes = [(128, 256), (256, 128)]
    init = [torch.randn(s, generator=gen) for s in shapes]
    grads = [[torch.randn(s, generator=gen) for s in shapes] for _ in range(2)]

    def make(ps):
        if algo == "normuon":
            return Muon([{"params": ps, "algorithm": "normuon"}], lr=0.01, foreach=True)
        return Muon8bit(ps, lr=0.01, block_size=256)

    a = [nn.Parameter(t.clone().to(DEV)) for t in init]
    b = [nn.Parameter(t.clone().to(DEV)) for t in init]
    opt_c, opt_e = make(a), make(b)
    opt_c._muon_impls[opt_c.param_groups[0]["algorithm"]] = _fail_nested
    graphs = []

    @torch.compile(backend=_backend("recording", graphs))
    def compiled_step():
        opt_c.step()

    for gs in grads:
        for pa, pb, g in zip(a, b, gs):
            pa.grad = g.clone().to(DEV)
            pb.grad = g.clone().to(DEV)
        compiled_step()
        opt_e.step()
    torch.cuda.synchronize()
    assert graphs and _ops_in(graphs) > 0
    for pa, pb in zip(a, b):
        assert torch.equal(pa.detach(), pb.detach())
        for key, vb in opt_e.state[pb].items():
            va = opt_c.state[pa][key]
            if hasattr(vb, "codes"):
                assert torch.equal(va.codes, vb.codes) and torch.equal(va.scale, vb.scale)
            else:
                assert torch.equal(va, vb), key
