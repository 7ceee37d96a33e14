"""The Muon step on the HIP path vs the oracle (muonium's Muon/MuonBaseline semantics).

* Known answers of the reference tests (test_optim.py:392-584) with the orthogonalizer
  replaced by identity, run on the device (momentum, Nesterov, cautious / plain wd,
  maximize, flatten, lr_ratio).
* Bit-exactness of the fused pre/post passes: given the same U, the fused step equals
  the oracle's fp32 update arithmetic exactly, and its momentum buffer is exact.
* foreach == per-parameter, grad mutation semantics, multi-step trajectories,
  checkpoint continuity, host-offloaded parameters, NorMuon and split_sizes.
"""

import math

import pytest
import torch
import torch.nn as nn

import muonium_amd.optim.algorithms.base as algo_base
from helpers import assert_close_pct, rel_fro
from muonium_amd import Muon
from muonium_amd.orthogonalize import zeropower
from oracle import muon_ref

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _identity(monkeypatch):
    monkeypatch.setattr(algo_base, "zeropower", lambda g, **_: g)
    monkeypatch.setattr(algo_base, "foreach_zeropower", lambda gs, **_: [g for g in gs])


# ---- known answers (identity orthogonalizer) ------------------------------------------


@pytest.mark.parametrize("foreach", [False, True])
def test_direct_update_initializes_state_and_uses_lr_ratio(monkeypatch, foreach):
    _identity(monkeypatch)
    p = nn.Parameter(torch.ones(4, 2, device=DEV))
    p.grad = torch.full_like(p, 0.5)
    opt = Muon([p], lr=0.1, wd=0.0, momentum=0.0, nesterov=False, foreach=foreach)
    opt.step()
    st = opt.state[p]
    assert torch.equal(st["step"], torch.tensor(1.0))
    assert torch.equal(st["lr_ratio"], torch.tensor(math.sqrt(2.0)))
    torch.testing.assert_close(st["momentum_buffer"], torch.full_like(p, 0.5))
    torch.testing.assert_close(p, torch.ones_like(p) - math.sqrt(2.0) * 0.1 * 0.5)


@pytest.mark.parametrize("foreach", [False, True])
def test_nesterov_uses_updated_buffer(monkeypatch, foreach):
    _identity(monkeypatch)
    p = nn.Parameter(torch.ones(2, 2, device=DEV))
    p.grad = torch.full_like(p, 0.5)
    opt = Muon([p], lr=0.1, wd=0.0, momentum=0.5, nesterov=True, foreach=foreach)
    opt.step()
    torch.testing.assert_close(opt.state[p]["momentum_buffer"], torch.full_like(p, 0.5))
    torch.testing.assert_close(p, torch.ones_like(p) - 0.1 * 0.75)


@pytest.mark.parametrize("foreach", [False, True])
@pytest.mark.parametrize("cautious,expected", [(True, [[-1.0, -2.0], [2.0, 1.0]]),
                                                (False, [[-1.0, -1.0], [1.0, 1.0]])])
def test_weight_decay_known_answers(monkeypatch, foreach, cautious, expected):
    _identity(monkeypatch)
    p = nn.Parameter(torch.tensor([[1.0, -1.0], [1.0, -1.0]], device=DEV))
    p.grad = torch.tensor([[1.0, 1.0], [-1.0, -1.0]], device=DEV)
    opt = Muon([p], lr=1.0, wd=1.0, momentum=0.0, nesterov=False, use_cautious_wd=cautious,
               foreach=foreach)
    opt.step()
    torch.testing.assert_close(p, torch.tensor(expected, device=DEV))


@pytest.mark.parametrize("foreach", [False, True])
def test_maximize_keeps_grad_and_direction(monkeypatch, foreach):
    _identity(monkeypatch)
    p = nn.Parameter(torch.ones(2, 2, device=DEV))
    grad = torch.full_like(p, 0.5)
    p.grad = grad
    opt = Muon([p], lr=0.1, wd=0.0, momentum=0.0, nesterov=False, maximize=True,
               foreach=foreach)
    opt.step()
    first = p.detach().clone()
    opt.step()
    torch.testing.assert_close(grad, torch.full_like(grad, 0.5))
    torch.testing.assert_close(first, torch.full_like(first, 1.05))
    torch.testing.assert_close(p, torch.full_like(p, 1.10))


def test_bf16_params_keep_fp32_momentum(monkeypatch):
    _identity(monkeypatch)
    p = nn.Parameter(torch.ones(2, 2, dtype=torch.bfloat16, device=DEV))
    p.grad = torch.full_like(p, 0.5)
    opt = Muon([p], lr=0.1, wd=0.0, momentum=0.9, nesterov=False)
    opt.step()
    assert opt.state[p]["momentum_buffer"].dtype is torch.float32


def test_skips_params_without_grad(monkeypatch):
    _identity(monkeypatch)
    a = nn.Parameter(torch.ones(2, 2, device=DEV))
    b = nn.Parameter(torch.ones(2, 2, device=DEV))
    a.grad = torch.full_like(a, 0.5)
    opt = Muon([a, b], lr=0.1, wd=0.0, momentum=0.0)
    opt.step()
    assert a in opt.state and b not in opt.state
    torch.testing.assert_close(b, torch.ones_like(b))


@pytest.mark.parametrize(
    "shape,flatten,seen,ratio",
    [((2, 2, 2, 2), True, (2, 8), 1.0), ((2, 2, 2, 2), False, (4, 2, 2), 1.0),
     ((2, 4, 2), False, (2, 4, 2), math.sqrt(2.0)), ((2, 2, 2), False, (2, 2, 2), 1.0)],
)
def test_flatten_shapes(monkeypatch, shape, flatten, seen, ratio):
    seen_shapes = []

    def fake(g, **_):
        seen_shapes.append(tuple(g.shape))
        return g

    monkeypatch.setattr(algo_base, "zeropower", fake)
    p = nn.Parameter(torch.ones(*shape, device=DEV))
    p.grad = torch.full_like(p, 0.5)
    opt = Muon([{"params": [p], "flatten": flatten}], lr=0.1, wd=0.0, momentum=0.0,
               foreach=False)
    opt.step()
    assert seen_shapes == [seen]
    assert torch.equal(opt.state[p]["lr_ratio"], torch.tensor(ratio))
    torch.testing.assert_close(p, torch.ones_like(p) - ratio * 0.1 * 0.5)


# ---- the fused step vs the oracle --------------------------------------------------------

CASES = [
    # shape, param dtype, grad dtype
    ((64, 48), torch.float32, torch.float32),
    ((48, 64), torch.float32, torch.float32),
    ((256, 512), torch.float32, torch.float32),
    ((300, 130), torch.bfloat16, torch.bfloat16),
    ((3, 40, 72), torch.bfloat16, torch.bfloat16),
    ((130, 70), torch.float16, torch.float16),
]
HP = [
    dict(wd=0.1, use_cautious_wd=True, momentum=0.95, nesterov=True, maximize=False,
         orthogonalization_strategy="polar_express"),
    dict(wd=0.3, use_cautious_wd=False, momentum=0.9, nesterov=False, maximize=False,
         orthogonalization_strategy="newton_schulz"),
    dict(wd=0.0, use_cautious_wd=True, momentum=0.95, nesterov=True, maximize=True,
         orthogonalization_strategy="polar_express"),
]


def _make(shape, pdt, gdt, seed):
    gen = torch.Generator().manual_seed(seed)
    p0 = torch.randn(shape, generator=gen).to(pdt)
    g0 = torch.randn(shape, generator=gen).to(gdt)
    buf0 = torch.randn(shape, generator=gen) * 0.1
    return p0, g0, buf0


def _oracle_step(p0, g0, buf0, hp, orth, lr=0.02):
    strategy = hp["orthogonalization_strategy"]
    return muon_ref.muon_update(
        p0, g0, buf0, muon_ref.lr_ratio(g0.shape), lr=lr, weight_decay=hp["wd"],
        cautious_wd=hp["use_cautious_wd"], momentum=hp["momentum"], nesterov=hp["nesterov"],
        maximize=hp["maximize"], ns_steps=5, strategy=strategy, orth_single=orth,
    )


def _run_step(p0, g0, buf0, hp, foreach, lr=0.02):
    p = nn.Parameter(p0.clone().to(DEV))
    p.grad = g0.clone().to(DEV)
    opt = Muon([p], lr=lr, foreach=foreach, **hp)
    opt._init_muon_group  # noqa: B018
    # seed the momentum buffer with buf0 through a first state init
    st = opt.state[p]
    st["step"] = torch.tensor(0.0)
    st["momentum_buffer"] = buf0.clone().to(DEV)
    st["lr_ratio"] = torch.tensor(math.sqrt(max(1.0, g0.shape[-2] / g0.shape[-1])))
    opt.step()
    torch.cuda.synchronize()
    return p, opt


@pytest.mark.parametrize("hp", HP, ids=["pe-cautious-nesterov", "ns-plain-wd", "pe-maximize-nowd"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{str(c[1])[6:]}")
@pytest.mark.parametrize("foreach", [False, True])
def test_fused_step_bit_exact_given_u(case, hp, foreach):
    shape, pdt, gdt = case
    p0, g0, buf0 = _make(shape, pdt, gdt, seed=7)
    p, opt = _run_step(p0, g0, buf0, hp, foreach)
    # g' exactly as the kernel computes it, then U from the HIP orthogonalizer
    gt = muon_ref.transform_grad(g0, False)
    _, ref_buf, gq, _ = _oracle_step(p0, g0, buf0, hp, orth=lambda g: g)
    strategy = hp["orthogonalization_strategy"]
    U = zeropower(gq.to(DEV), steps=5, strategy=strategy).cpu()
    ref_p, _, _, _ = _oracle_step(p0, g0, buf0, hp, orth=lambda g: U)
    assert torch.equal(opt.state[p]["momentum_buffer"].cpu(), ref_buf), "momentum buffer"
    got = p.detach().cpu()
    assert torch.equal(got, ref_p), (
        f"param mismatch: {(got.float() - ref_p.float()).abs().max().item():.3e}"
    )
    assert gt.shape == g0.shape


@pytest.mark.parametrize("hp", HP[:2], ids=["pe", "ns"])
@pytest.mark.parametrize("case", CASES[:4], ids=lambda c: f"{c[0]}")
def test_fused_step_matches_oracle_update(case, hp):
    shape, pdt, gdt = case
    p0, g0, buf0 = _make(shape, pdt, gdt, seed=11)
    p, _ = _run_step(p0, g0, buf0, hp, foreach=True)
    coeffs, prescale = muon_ref.strategy_coeffs(hp["orthogonalization_strategy"], 5)
    orth = lambda g: muon_ref.polar_iteration_bf16(g, coeffs, prescale=prescale, eps=1e-7)
    ref_p, _, _, _ = _oracle_step(p0, g0, buf0, hp, orth=orth)
    d_got = p.detach().cpu().double() - p0.double()
    d_ref = ref_p.double() - p0.double()
    if hp["use_cautious_wd"] and hp["wd"] != 0:
        # the cautious mask [u*p > 0] is discrete: elements with u near 0 may flip, so
        # compare elementwise with a mismatch budget (the reference's foreach-vs-per-param
        # bar, test_optim_foreach.py:64-66)
        assert_close_pct(d_got, d_ref, rtol=1e-2, atol=3e-2 * d_ref.abs().max().item(),
                         max_mismatch_pct=5.0)
    else:
        assert rel_fro(d_got, d_ref) <= 2e-2


def test_foreach_equals_per_param_and_mutates_grads_under_nesterov():
    shapes = [(32, 16), (32, 16), (16, 32), (24, 24), (3, 8, 12)]
    gen = torch.Generator().manual_seed(0)
    init = [torch.randn(s, generator=gen) for s in shapes]
    kwargs = dict(lr=0.2, wd=0.3, nesterov=True, use_cautious_wd=True,
                  orthogonalization_strategy="polar_express")
    ref_p = [nn.Parameter(t.clone().to(DEV)) for t in init]
    fe_p = [nn.Parameter(t.clone().to(DEV)) for t in init]
    ref = Muon(ref_p, foreach=False, **kwargs)
    fe = Muon(fe_p, foreach=True, **kwargs)
    for step in range(3):
        grads = [torch.randn(s, generator=gen).to(DEV) for s in shapes]
        for p, g in zip(ref_p, grads):
            p.grad = g.clone()
        for p, g in zip(fe_p, grads):
            p.grad = g.clone()
        ref.step()
        fe.step()
        for p, g in zip(ref_p, grads):
            assert torch.equal(p.grad, g), "per-param driver must not touch the grad"
        for p, g in zip(fe_p, grads):
            buf = fe.state[p]["momentum_buffer"]
            assert torch.equal(p.grad, g + buf * 0.95) or rel_fro(p.grad, g + 0.95 * buf) < 1e-6
    for r, f in zip(ref_p, fe_p):
        assert torch.equal(r, f)


def test_multi_step_trajectory_matches_oracle():
    shapes = [(64, 32), (32, 96), (2, 48, 40)]
    gen = torch.Generator().manual_seed(3)
    init = [torch.randn(s, generator=gen) for s in shapes]
    params = [nn.Parameter(t.clone().to(DEV)) for t in init]
    opt = Muon(params, lr=0.05, wd=0.1, foreach=True)
    ref = muon_ref.MuonRef([t.clone() for t in init], lr=0.05, wd=0.1)
    coeffs, prescale = muon_ref.strategy_coeffs("polar_express", 5)

    for _ in range(3):
        grads = [torch.randn(s, generator=gen) for s in shapes]
        for p, g in zip(params, grads):
            p.grad = g.to(DEV)
        opt.step()
        # oracle: same arithmetic, orthogonalization at the HIP storage points
        for i, (rp, g) in enumerate(zip(ref.params, grads)):
            st = ref.state.setdefault(i, {
                "step": torch.tensor(0.0), "momentum_buffer": torch.zeros_like(g),
                "lr_ratio": torch.tensor(math.sqrt(max(1.0, g.shape[-2] / g.shape[-1])))})
            st["step"] += 1
            new_p, new_buf, _, _ = muon_ref.muon_update(
                rp, g, st["momentum_buffer"], float(st["lr_ratio"]), lr=0.05, weight_decay=0.1,
                cautious_wd=True, momentum=0.95, nesterov=True, maximize=False,
                orth_single=lambda x: muon_ref.polar_iteration_bf16(x, coeffs, prescale=prescale,
                                                                    eps=1e-7),
            )
            rp.copy_(new_p)
            st["momentum_buffer"] = new_buf
    for i, (p, rp, p0) in enumerate(zip(params, ref.params, init)):
        assert rel_fro(p.detach().cpu() - p0, rp - p0) < 2e-2
        assert torch.equal(opt.state[p]["momentum_buffer"].cpu(), ref.state[i]["momentum_buffer"])


def test_state_dict_round_trip_continuity():
    gen = torch.Generator().manual_seed(5)
    init = torch.randn(48, 32, generator=gen)
    a = nn.Parameter(init.clone().to(DEV))
    b = nn.Parameter(init.clone().to(DEV))
    c = nn.Parameter(init.clone().to(DEV))
    kw = dict(lr=0.1, wd=0.1, momentum=0.5, nesterov=False)
    oa, ob, oc = Muon([a], **kw), Muon([b], **kw), Muon([c], **kw)
    g1 = torch.randn(48, 32, generator=gen).to(DEV)
    a.grad, b.grad = g1.clone(), g1.clone()
    oa.step()
    ob.step()
    c.data.copy_(b.data)
    oc.load_state_dict(ob.state_dict())
    g2 = torch.randn(48, 32, generator=gen).to(DEV)
    a.grad, c.grad = g2.clone(), g2.clone()
    oa.step()
    oc.step()
    assert torch.equal(a, c)
    for key in ["step", "momentum_buffer", "lr_ratio"]:
        # torch's load_state_dict moves non-"step" state to the param's device
        assert torch.equal(oa.state[a][key].cpu(), oc.state[c][key].cpu())


@pytest.mark.parametrize("foreach", [True, False])
def test_host_resident_params_round_trip_through_device(foreach):
    gen = torch.Generator().manual_seed(6)
    init = torch.randn(32, 16, generator=gen)
    g = torch.randn(32, 16, generator=gen)
    cpu_p = nn.Parameter(init.clone())
    dev_p = nn.Parameter(init.clone().to(DEV))
    cpu_p.grad = g.clone()
    dev_p.grad = g.clone().to(DEV)
    kw = dict(lr=0.1, wd=0.0, orthogonalization_strategy="newton_schulz")
    Muon([cpu_p], foreach=foreach, **kw).step()
    Muon([dev_p], foreach=foreach, **kw).step()
    assert cpu_p.device.type == "cpu" and cpu_p.grad.device.type == "cpu"
    assert torch.equal(cpu_p.detach(), dev_p.detach().cpu())


def test_mixed_muon_and_adam_groups(monkeypatch):
    _identity(monkeypatch)
    mp = nn.Parameter(torch.ones(2, 2, device=DEV))
    ap = nn.Parameter(torch.randn(3, device=DEV))
    aref = nn.Parameter(ap.detach().clone())
    opt = Muon([{"params": [mp], "lr": 0.1, "wd": 0.0, "momentum": 0.0},
                {"params": [ap], "algorithm": "adamw", "lr": 0.01, "wd": 0.1, "fused": False}])
    ref = torch.optim.AdamW([aref], lr=0.01, weight_decay=0.1)
    mp.grad = torch.full_like(mp, 0.5)
    ag = torch.randn_like(ap)
    ap.grad, aref.grad = ag.clone(), ag.clone()
    opt.step()
    ref.step()
    torch.testing.assert_close(mp, torch.full_like(mp, 0.95))
    torch.testing.assert_close(ap, aref)


# ---- NorMuon and split_sizes --------------------------------------------------------------


@pytest.mark.parametrize("shape", [(40, 24), (24, 40), (2, 24, 40)])
def test_normuon_matches_oracle(shape):
    gen = torch.Generator().manual_seed(8)
    p0 = torch.randn(shape, generator=gen)
    p = nn.Parameter(p0.clone().to(DEV))
    opt = Muon([{"params": [p], "algorithm": "normuon", "muon_beta2": 0.9}], lr=0.1, wd=0.1,
               momentum=0.5, nesterov=True)
    ref_p, ref_buf = p0.clone(), torch.zeros(shape)
    ref_v = torch.zeros(*shape[:-1], 1)
    for step in range(2):
        g = torch.randn(shape, generator=gen)
        p.grad = g.clone().to(DEV)
        opt.step()
        gq_buf = ref_buf * 0.5 + g
        gq = g + gq_buf * 0.5
        U = zeropower(gq.to(DEV), strategy="polar_express").cpu()
        ref_p, ref_buf, ref_v, _ = muon_ref.normuon_update(
            ref_p, g, ref_buf, ref_v, muon_ref.lr_ratio(shape), lr=0.1, weight_decay=0.1,
            cautious_wd=True, momentum=0.5, nesterov=True, maximize=False, beta2=0.9,
            orth_single=lambda x: U,
        )
    assert rel_fro(p.detach().cpu() - p0, ref_p - p0) < 1e-4
    torch.testing.assert_close(opt.state[p]["variance_neuron"].cpu(), ref_v, rtol=1e-4, atol=1e-7)


def test_split_sizes_match_oracle():
    from muonium_amd.orthogonalize import foreach_zeropower

    gen = torch.Generator().manual_seed(9)
    p0 = torch.randn(96, 32, generator=gen)
    g = torch.randn(96, 32, generator=gen)
    p = nn.Parameter(p0.clone().to(DEV))
    p.grad = g.clone().to(DEV)
    opt = Muon([{"params": [p], "split_sizes": (64, 16, 16)}], lr=0.1, wd=0.0, momentum=0.0,
               nesterov=False)
    opt.step()
    # oracle: base.py:73-99 block split/scale/cat with the HIP orthogonalizer per height
    hip_batch = lambda blocks: [u.cpu() for u in foreach_zeropower([b.to(DEV) for b in blocks],
                                                                  strategy="polar_express")]
    ref_p, _, _, _ = muon_ref.muon_update(
        p0, g, torch.zeros(96, 32), muon_ref.lr_ratio((96, 32)), lr=0.1, weight_decay=0.0,
        cautious_wd=True, momentum=0.0, nesterov=False, maximize=False,
        split_sizes=(64, 16, 16), orth_batch=hip_batch,
    )
    assert torch.equal(p.detach().cpu(), ref_p)


@pytest.mark.parametrize("foreach", [True, False])
@pytest.mark.parametrize(
    "shape,split,dtype,hp",
    [((300, 128), (128, 172), torch.float32, (0.9, True, 0.1, True)),
     ((192, 96), (96, 64, 32), torch.bfloat16, (0.95, True, 0.1, True)),
     ((64, 256), (16, 48), torch.float32, (0.9, False, 0.0, False)),
     ((160, 64), (32, 64, 32, 32), torch.bfloat16, (0.5, True, 0.05, False))],
    ids=["tall-block", "qkv-bf16", "wide-blocks-nowd", "repeat-heights-bf16"],
)
def test_split_sizes_fused_blocks_exact(shape, split, dtype, hp, foreach):
    """split_sizes row blocks through the fused kernels (equal heights batched, per-block
    rescale) equal the oracle's base.py:73-99 split/scale/cat plus muon.py update exactly,
    given the HIP orthogonalizer per block height, over two steps and two params."""
    from muonium_amd.orthogonalize import foreach_zeropower

    mom, nesterov, wd, cautious = hp
    gen = torch.Generator().manual_seed(21)
    p0 = [torch.randn(shape, generator=gen).to(dtype) for _ in range(2)]
    params = [nn.Parameter(p.clone().to(DEV)) for p in p0]
    opt = Muon([{"params": params, "split_sizes": split}], lr=0.05, wd=wd, momentum=mom,
               nesterov=nesterov, use_cautious_wd=cautious, foreach=foreach)
    hip_batch = lambda blocks: [u.cpu() for u in foreach_zeropower([b.to(DEV) for b in blocks],
                                                                  strategy="polar_express")]
    ref_p = [p.clone() for p in p0]
    ref_buf = [torch.zeros(shape) for _ in p0]
    for _ in range(2):
        gs = [torch.randn(shape, generator=gen).to(dtype) for _ in p0]
        for p, g in zip(params, gs):
            p.grad = g.clone().to(DEV)
        opt.step()
        for i, g in enumerate(gs):
            ref_p[i], ref_buf[i], _, _ = muon_ref.muon_update(
                ref_p[i], g, ref_buf[i], muon_ref.lr_ratio(shape), lr=0.05, weight_decay=wd,
                cautious_wd=cautious, momentum=mom, nesterov=nesterov, maximize=False,
                split_sizes=split, orth_batch=hip_batch,
            )
    for p, rp, rb in zip(params, ref_p, ref_buf):
        assert torch.equal(p.detach().cpu(), rp)
        assert torch.equal(opt.state[p]["momentum_buffer"].cpu(), rb)


@pytest.mark.parametrize(
    "algo,nesterov,maximize,dtype",
    [("muon", True, False, torch.float32), ("muon", True, True, torch.bfloat16),
     ("muon", False, False, torch.float32), ("normuon", True, False, torch.float32)],
)
def test_offloaded_batches_pipeline_matches_device_run(algo, nesterov, maximize, dtype):
    """Host-resident params, foreach with batch_size=2 (three batches, two shapes): the
    pinned-memory pipelined round trip gives exactly the device-resident run's params,
    grads and state, and leaves every tensor on the host."""
    gen = torch.Generator().manual_seed(31)
    shapes = [(64, 48)] * 3 + [(32, 96)] * 2
    init = [torch.randn(s, generator=gen).to(dtype) for s in shapes]
    host = [nn.Parameter(t.clone()) for t in init]
    dev = [nn.Parameter(t.clone().to(DEV)) for t in init]
    kw = dict(lr=0.05, wd=0.1, momentum=0.9, nesterov=nesterov, maximize=maximize,
              foreach=True, batch_size=2)
    opt_h = Muon([{"params": host, "algorithm": algo}], **kw)
    opt_d = Muon([{"params": dev, "algorithm": algo}], **kw)
    for _ in range(2):
        gs = [torch.randn(s, generator=gen).to(dtype) for s in shapes]
        for h, d, g in zip(host, dev, gs):
            h.grad = g.clone()
            d.grad = g.clone().to(DEV)
        opt_h.step()
        opt_d.step()
    torch.cuda.synchronize()
    for h, d in zip(host, dev):
        assert h.device.type == "cpu" and h.grad.device.type == "cpu"
        assert torch.equal(h.detach(), d.detach().cpu())
        assert torch.equal(h.grad, d.grad.cpu())
        for key, val in opt_d.state[d].items():
            assert opt_h.state[h][key].device.type == "cpu"
            assert torch.equal(opt_h.state[h][key], val.cpu()), key


def test_plumbing_config_is_bit_repeatable():
    """The plumbing configuration: one fp32 256 x 512 parameter (p ~ N(0,1) seed 1, g ~ N(0,1) seed 0),
    Newton-Schulz 5, cautious wd 0.1, Nesterov 0.95, foreach=False: two runs of the step from
    the same state give bit-identical parameters and momentum."""
    p0 = torch.randn(256, 512, generator=torch.Generator().manual_seed(1))
    g0 = torch.randn(256, 512, generator=torch.Generator().manual_seed(0))
    outs = []
    for _ in range(2):
        p = nn.Parameter(p0.clone().to(DEV))
        p.grad = g0.clone().to(DEV)
        opt = Muon([p], lr=1e-3, wd=0.1, use_cautious_wd=True, momentum=0.95, nesterov=True,
                   ns_steps=5, orthogonalization_strategy="newton_schulz", foreach=False)
        for _ in range(3):
            opt.step()
        torch.cuda.synchronize()
        outs.append((p.detach().cpu(), opt.state[p]["momentum_buffer"].cpu()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])
    assert not torch.equal(outs[0][0], p0)


def test_small_buckets_on_side_streams_match_sequential_buckets():
    """Buckets too small to fill the device run concurrently (the smallest on the caller's
    stream, the others on side streams, two of them with the same workspace shape); the
    result is the same, bit for bit, as one bucket at a time, and the step is ordered after
    earlier work on the caller's stream and before later work."""
    from muonium_amd.optim import optim as optim_mod

    # workspace shapes (m_pad, n_pad): (256, 512), (256, 256), (256, 768) twice, (256, 512)
    shapes = [(96, 288), (96, 96), (96, 600), (600, 96), (96, 288)]
    gen = torch.Generator().manual_seed(31)
    p0 = [torch.randn(s, generator=gen).bfloat16() for s in shapes]
    gs = [[torch.randn(s, generator=gen).bfloat16() for s in shapes] for _ in range(2)]
    runs = []
    for split_groups in (False, True):
        params = [nn.Parameter(p.clone().to(DEV)) for p in p0]
        groups = [{"params": [p]} for p in params] if split_groups else [{"params": params}]
        opt = Muon(groups, lr=0.05, wd=0.1, momentum=0.9, foreach=True)
        optim_mod._side_streams.clear()
        for step in range(2):
            for p, g in zip(params, gs[step]):
                # written on the caller's stream right before the step
                p.grad = torch.empty_like(p).copy_(g.to(DEV))
            opt.step()
            if not split_groups:
                assert len(optim_mod._side_streams) == 3
            else:
                assert len(optim_mod._side_streams) == 0
        runs.append(([p.detach().clone() for p in params],
                     [opt.state[p]["momentum_buffer"].clone() for p in params]))
    (pa, ba), (pb, bb) = runs
    for x, y in zip(pa + ba, pb + bb):
        assert torch.equal(x, y)


def test_side_stream_bucket_sharing_padded_extents_with_large_bucket():
    """A small bucket on a side stream and a large bucket on the caller's stream whose
    matrices pad to the same workspace extents (96 x 288 -> 256 x 512) run at the same
    time: each stream has its own workspace, so three steps give bit for bit the
    parameters and momentum of one bucket per step call."""
    from muonium_amd.optim import optim as optim_mod

    # large: 4 x (64, 96, 288) = 256 matrices (fills the device, stays on the caller's
    # stream, listed first so it allocates first); small: (96, 288) x 2 and (96, 96) x 2
    shapes = [(64, 96, 288)] * 4 + [(96, 288)] * 2 + [(96, 96)] * 2
    gen = torch.Generator().manual_seed(47)
    p0 = [torch.randn(s, generator=gen).bfloat16() for s in shapes]
    gs = [[torch.randn(s, generator=gen).bfloat16() for s in shapes] for _ in range(3)]
    runs = []
    for split_groups in (False, True):
        params = [nn.Parameter(p.clone().to(DEV)) for p in p0]
        groups = [{"params": [p]} for p in params] if split_groups else [{"params": params}]
        opt = Muon(groups, lr=0.05, wd=0.1, momentum=0.9, foreach=True)
        optim_mod._side_streams.clear()
        for step in range(3):
            for p, g in zip(params, gs[step]):
                p.grad = g.to(DEV)
            opt.step()
            assert len(optim_mod._side_streams) == (0 if split_groups else 2)
        torch.cuda.synchronize()
        runs.append(([p.detach().clone() for p in params],
                     [opt.state[p]["momentum_buffer"].clone() for p in params]))
    (pa, ba), (pb, bb) = runs
    for x, y in zip(pa + ba, pb + bb):
        assert torch.equal(x, y)


@pytest.mark.parametrize("algo", ["muon", "normuon"])
def test_host_params_per_parameter_driver_matches_device_run(algo):
    """Host-resident params default to the per-parameter driver (foreach=False); each
    step runs on device copies and copies the results back: params, grads and state
    equal the device-resident run exactly and stay on the host (the reference steps
    host-resident muon / normuon groups, test_algorithms.py:140)."""
    gen = torch.Generator().manual_seed(5)
    shapes = [(64, 48), (32, 96), (3, 16, 24)]
    init = [torch.randn(s, generator=gen) for s in shapes]
    host = [nn.Parameter(t.clone()) for t in init]
    dev = [nn.Parameter(t.clone().to(DEV)) for t in init]
    kw = dict(lr=0.05, wd=0.1, momentum=0.9)
    opt_h = Muon([{"params": host, "algorithm": algo}], **kw)
    opt_d = Muon([{"params": dev, "algorithm": algo, "foreach": False}], **kw)
    assert opt_h.param_groups[0]["foreach"] is False
    for _ in range(2):
        gs = [torch.randn(s, generator=gen) for s in shapes]
        for h, d, g in zip(host, dev, gs):
            h.grad = g.clone()
            d.grad = g.clone().to(DEV)
        opt_h.step()
        opt_d.step()
    torch.cuda.synchronize()
    for h, d in zip(host, dev):
        assert h.device.type == "cpu"
        assert torch.equal(h.detach(), d.detach().cpu())
        assert torch.equal(h.grad, d.grad.cpu())
        for key, val in opt_d.state[d].items():
            assert opt_h.state[h][key].device.type == "cpu", key
            assert torch.equal(opt_h.state[h][key], val.cpu()), key


@pytest.mark.parametrize("kind", ["muon-fp32", "muon-bf16", "normuon", "muon8bit"])
def test_per_parameter_driver_groups_same_shapes_bit_exact(kind):
    """foreach=False runs same-shape device tensors of a built-in algorithm as one fused
    launch sequence with per-tensor semantics: params and state equal, bit for bit, one
    `update` call per tensor (forced here by wrapping `update` on the instance, which
    turns the grouping off), and the gradients are left untouched."""
    from muonium_amd.optim import Muon8bit
    from muonium_amd.optim.algorithms import get_algorithm

    dtype = torch.bfloat16 if kind == "muon-bf16" else torch.float32
    shapes = [(96, 64), (64, 160), (96, 64), (2, 64, 160), (64, 160), (96, 64)]
    gen = torch.Generator().manual_seed(13)
    init = [torch.randn(s, generator=gen).to(dtype) for s in shapes]
    grads = [[torch.randn(s, generator=gen).to(dtype) for s in shapes] for _ in range(2)]

    def run(split_calls):
        ps = [nn.Parameter(t.clone().to(DEV)) for t in init]
        kw = dict(lr=0.02, wd=0.1, momentum=0.9, foreach=False)
        if kind == "muon8bit":
            opt = Muon8bit(ps, block_size=64, **kw)
        else:
            opt = Muon([{"params": ps, "algorithm": "normuon" if kind == "normuon" else "muon"}],
                       **kw)
        algo = get_algorithm(opt.param_groups[0]["algorithm"])
        calls = []
        if split_calls:
            orig = type(algo).update

            def one(*args, **kwargs):
                calls.append(1)
                return orig(algo, *args, **kwargs)

            algo.update = one
        try:
            for gs in grads:
                for p, g in zip(ps, gs):
                    p.grad = g.clone().to(DEV)
                opt.step()
                for p, g in zip(ps, gs):
                    assert torch.equal(p.grad.cpu(), g)  # per-tensor semantics
        finally:
            if split_calls:
                del algo.update
        torch.cuda.synchronize()
        if split_calls:
            assert len(calls) == 2 * len(shapes)
        return ps, opt

    pa, oa = run(False)
    pb, ob = run(True)
    for a, b in zip(pa, pb):
        assert torch.equal(a.detach(), b.detach())
        for key, vb in ob.state[b].items():
            va = oa.state[a][key]
            if hasattr(vb, "codes"):
                assert torch.equal(va.codes, vb.codes) and torch.equal(va.scale, vb.scale)
            else:
                assert torch.equal(va, vb), key
