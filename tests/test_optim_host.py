"""Host-side logic of the optimizer on the CPU (no kernels): constructor validation,
group normalization, the algorithm registry, checkpoint legacy defaults, foreach
bucketing and chunking, Adam pass-through, MuonLP buffer eligibility, and the rule
that a Muon step needs a HIP device. Mirrors the CPU tests of the reference's
tests/optim/test_optim.py, test_optim_foreach.py, test_algorithms.py,
test_optim_lp.py and tests/utils/test_foreach.py.
"""

import math

import pytest
import torch
import torch.nn as nn

import muonium_amd.optim.optim as optim_module
from muonium_amd import (
    Muon,
    MuonAlgorithm,
    get_algorithm,
    register_muon_algorithm,
    registered_algorithms,
)
from muonium_amd.optim import Muon4bit, Muon8bit, MuonFp8
from muonium_amd.optim.algorithms import split_lr_scales
from muonium_amd.optim.lp_state import OptimState4bit, OptimState8bit, OptimStateFp8
from muonium_amd.utils import group_tensors_by_shape, move_tensors_to_device


@pytest.mark.parametrize(
    ("kwargs", "match"),
    [({"lr": -1.0}, "Invalid learning rate"), ({"adam_eps": -1.0}, "Invalid epsilon"),
     ({"adam_betas": (1.0, 0.9)}, "index 0"), ({"adam_betas": (0.9, -0.1)}, "index 1")],
)
def test_constructor_validates_scalars(kwargs, match):
    with pytest.raises(ValueError, match=match):
        Muon([nn.Parameter(torch.randn(2, 2))], **kwargs)


def test_constructor_rejections():
    p = nn.Parameter(torch.randn(2, 2))
    with pytest.raises(TypeError, match="not a single dict"):
        Muon({"params": [p]})
    with pytest.raises(ValueError, match="empty parameter list"):
        Muon([])
    with pytest.raises(ValueError, match="'params' key"):
        Muon([{"algorithm": "muon"}])
    with pytest.raises(ValueError, match="Unknown algorithm"):
        Muon([{"params": [p], "algorithm": "rmsprop"}])
    with pytest.raises(ValueError, match="2D\\+"):
        Muon([nn.Parameter(torch.randn(4))])
    with pytest.raises(NotImplementedError, match="Complex parameters"):
        Muon([nn.Parameter(torch.randn(2, 2, dtype=torch.cfloat))])


def test_group_normalization_and_defaults():
    mp, ap = nn.Parameter(torch.randn(2, 2)), nn.Parameter(torch.randn(4))
    opt = Muon([{"params": []}, {"params": [mp], "lr": 0.5, "wd": 0.25},
                {"params": [ap], "algorithm": "adamw", "lr": 0.3, "wd": 0.1}], lr=0.01, wd=0.9)
    mg, ag = opt.param_groups
    assert mg["use_muon"] is True and torch.equal(mg["lr"], torch.tensor(0.5)) and mg["wd"] == 0.25
    assert mg["orthogonalization_strategy"] == "polar_express" and mg["ns_steps"] == 5
    assert mg["nesterov"] is True and mg["use_cautious_wd"] is True and mg["flatten"] is False
    assert mg["foreach"] is False  # host params: auto foreach is off
    assert ag["use_muon"] is False and ag["lr"] == 0.3 and ag["decoupled_weight_decay"] is True


def test_registry_rules():
    assert {"muon", "normuon"} <= set(registered_algorithms())
    with pytest.raises(ValueError, match="Unknown algorithm 'nope'"):
        get_algorithm("nope")

    class Reserved(MuonAlgorithm):
        name = "adam"

        def update(self, *a, **k):
            pass

    class Dup(MuonAlgorithm):
        name = "muon"

        def update(self, *a, **k):
            pass

    class Shadow(MuonAlgorithm):
        name = "test-shadow"
        options = {"momentum": 0.5}

        def update(self, *a, **k):
            pass

    with pytest.raises(ValueError, match="reserved for the Adam path"):
        register_muon_algorithm(Reserved)
    with pytest.raises(ValueError, match="already registered"):
        register_muon_algorithm(Dup)
    with pytest.raises(ValueError, match="reserved group keys"):
        register_muon_algorithm(Shadow)


@register_muon_algorithm
class _SignDescent(MuonAlgorithm):
    name = "test-signsgd"
    options = {"scale": 1.0}

    def update(self, param, grad, state, lr_ratio, *, lr, scale, **kwargs):
        state["momentum_buffer"].copy_(grad)
        param.copy_(param - lr * scale * grad.sign())


def test_custom_algorithm_steps_end_to_end_on_host():
    p = nn.Parameter(torch.ones(2, 3))
    g = torch.tensor([[1.0, -2.0, 0.5], [-0.25, 3.0, -1.0]])
    p.grad = g.clone()
    opt = Muon([{"params": [p], "algorithm": "test-signsgd", "scale": 2.0}], lr=0.1)
    assert opt.param_groups[0]["scale"] == 2.0
    opt.step()
    torch.testing.assert_close(p, torch.ones(2, 3) - 0.1 * 2.0 * g.sign())
    torch.testing.assert_close(opt.state[p]["momentum_buffer"], g)
    assert Muon([{"params": [nn.Parameter(torch.ones(2, 2))], "algorithm": "test-signsgd"}]
                ).param_groups[0]["scale"] == 1.0


def test_split_sizes_validation():
    p2, p3 = nn.Parameter(torch.randn(6, 4)), nn.Parameter(torch.randn(2, 3, 4))
    with pytest.raises(ValueError, match="at least 2 block sizes"):
        Muon([{"params": [p2], "split_sizes": (6,)}])
    with pytest.raises(ValueError, match="positive integers"):
        Muon([{"params": [p2], "split_sizes": (4, -2)}])
    with pytest.raises(ValueError, match="only supported for 2D"):
        Muon([{"params": [p3], "split_sizes": (1, 1)}])
    with pytest.raises(ValueError, match="must sum to dim 0"):
        Muon([{"params": [p2], "split_sizes": (2, 2)}])
    assert Muon([{"params": [p2], "split_sizes": [2, 4]}]).param_groups[0]["split_sizes"] == (2, 4)
    full = math.sqrt(6 / 4)
    assert split_lr_scales((6, 4), (2, 4)) == pytest.approx((1 / full, 1 / full))


def test_load_state_dict_legacy_defaults():
    p = nn.Parameter(torch.randn(2, 2))
    opt = Muon([p])
    g = opt.param_groups[0]
    for key in ["ns_steps", "nesterov", "flatten", "use_cautious_wd",
                "orthogonalization_strategy", "algorithm", "split_sizes"]:
        del g[key]
    g["lr"] = 0.1
    opt.state[p]["step"] = 3.0
    opt._muon_impls["muon"] = "stale"
    opt.__setstate__({"state": opt.state, "param_groups": opt.param_groups})
    assert g["ns_steps"] == 5 and g["nesterov"] is True and g["flatten"] is False
    assert g["use_cautious_wd"] is True and g["orthogonalization_strategy"] == "polar_express"
    assert g["algorithm"] == "muon" and g["split_sizes"] is None
    assert torch.equal(g["lr"], torch.tensor(0.1))
    assert torch.equal(opt.state[p]["step"], torch.tensor(3.0))
    assert opt._muon_impls == {}


def test_adam_legacy_defaults():
    p = nn.Parameter(torch.randn(2, 2))
    opt = Muon([{"params": [p], "algorithm": "adamw", "fused": False}])
    g = opt.param_groups[0]
    for key in ["amsgrad", "maximize", "foreach", "decoupled_weight_decay", "fused"]:
        g.pop(key, None)
    opt.state[p]["step"] = 4.0
    opt.__setstate__({"state": opt.state, "param_groups": opt.param_groups})
    assert g["amsgrad"] is False and g["maximize"] is False and g["foreach"] is None
    assert g["decoupled_weight_decay"] is False and g["fused"] is None
    assert torch.equal(opt.state[p]["step"], torch.tensor(4.0))


@pytest.mark.parametrize("algorithm,ref_cls", [("adamw", torch.optim.AdamW), ("adam", torch.optim.Adam)])
@pytest.mark.parametrize("amsgrad", [False, True])
def test_adam_groups_match_torch(algorithm, ref_cls, amsgrad):
    p = nn.Parameter(torch.randn(3, 4))
    ref = nn.Parameter(p.detach().clone())
    opt = Muon([{"params": [p], "algorithm": algorithm, "lr": 0.01, "wd": 0.1,
                 "betas": (0.9, 0.95), "eps": 1e-8, "fused": False, "amsgrad": amsgrad}])
    ref_opt = ref_cls([ref], lr=0.01, weight_decay=0.1, betas=(0.9, 0.95), eps=1e-8,
                      amsgrad=amsgrad)
    for _ in range(3):
        g = torch.randn_like(p)
        p.grad, ref.grad = g.clone(), g.clone()
        opt.step()
        ref_opt.step()
    torch.testing.assert_close(p, ref)


def test_step_returns_closure_loss():
    p = nn.Parameter(torch.randn(3, 4))
    opt = Muon([{"params": [p], "algorithm": "adamw", "fused": False}])
    assert opt.step(lambda: p.square().sum()) == p.square().sum()


def test_standalone_step_uses_impl_cache():
    p = nn.Parameter(torch.randn(2, 2))
    p.grad = torch.randn_like(p)
    opt = Muon([p])
    calls = []
    opt._muon_impls["muon"] = lambda *a, **k: calls.append((a, k))
    opt.step()
    assert len(calls) == 1 and calls[0][0][0] == [p]


def test_foreach_batch_size_chunks(monkeypatch):
    calls = []
    monkeypatch.setattr(optim_module, "move_tensors_to_device", lambda ts, _s, _d: ts)
    monkeypatch.setattr(get_algorithm("muon"), "foreach_update",
                        lambda p, g, st, ratios, **kw: calls.append((len(p), [tuple(t.shape) for t in g])))
    params = [nn.Parameter(torch.ones(2, 2)) for _ in range(5)]
    for p in params:
        p.grad = torch.full_like(p, 0.5)
    Muon(params, foreach=True, batch_size=2).step()
    assert calls == [(2, [(2, 2)] * 2), (2, [(2, 2)] * 2), (1, [(2, 2)])]


def test_foreach_groups_by_dtype_and_skips_none(monkeypatch):
    calls = []
    monkeypatch.setattr(optim_module, "move_tensors_to_device", lambda ts, _s, _d: ts)
    monkeypatch.setattr(get_algorithm("muon"), "foreach_update",
                        lambda p, g, st, ratios, **kw: calls.append((p[0].dtype, st["momentum_buffer"][0].dtype, len(p))))
    a = nn.Parameter(torch.ones(2, 2))
    b = nn.Parameter(torch.ones(2, 2, dtype=torch.bfloat16))
    c = nn.Parameter(torch.ones(2, 2))
    a.grad, b.grad = torch.full_like(a, 0.5), torch.full_like(b, 0.5)
    opt = Muon([a, b, c], foreach=True)
    opt.step()
    assert sorted(calls, key=str) == sorted(
        [(torch.float32, torch.float32, 1), (torch.bfloat16, torch.float32, 1)], key=str)
    assert c not in opt.state


def test_muon_step_on_host_without_device_raises():
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present: host params take the offload round trip")
    p = nn.Parameter(torch.randn(4, 4))
    p.grad = torch.randn_like(p)
    with pytest.raises(RuntimeError, match="HIP device"):
        Muon([p], foreach=False).step()


@pytest.mark.parametrize("opt_cls,state_cls", [(Muon8bit, OptimState8bit), (Muon4bit, OptimState4bit),
                                               (MuonFp8, OptimStateFp8)])
@pytest.mark.parametrize("shape,block,quantized", [((64, 64), 2048, True), ((32, 32), 2048, False),
                                                   ((64, 64), 3000, False), ((64, 64), 4096, True),
                                                   ((64, 64), 8192, False)])
def test_lp_buffer_eligibility(opt_cls, state_cls, shape, block, quantized):
    p = nn.Parameter(torch.randn(*shape))
    buf = opt_cls([p], block_size=block)._new_buffer(p, signed=True)
    if quantized:
        assert isinstance(buf, state_cls)
        assert buf.codes.dtype is torch.uint8 and buf.scale.numel() == p.numel() // block
    else:
        assert type(buf) is torch.Tensor and buf.dtype == p.dtype
    assert buf.shape == p.shape and buf.device == p.device
    dense = buf.dequantize() if quantized else buf
    assert torch.count_nonzero(dense) == 0


@pytest.mark.parametrize("opt_cls,state_cls", [(Muon8bit, OptimState8bit), (MuonFp8, OptimStateFp8)])
def test_lp_block_size_none_gives_one_block_per_tensor(opt_cls, state_cls):
    """block_size=None: every quantized buffer is a single block (one scale per tensor),
    whatever its size; buffers under 4096 values stay dense in the param's dtype."""
    ps = [nn.Parameter(torch.randn(*s)) for s in ((64, 96), (128, 64), (3, 64, 32), (32, 32))]
    opt = opt_cls(ps, block_size=None)
    for p in ps:
        buf = opt._new_buffer(p, signed=True)
        if p.numel() >= 4096:
            assert isinstance(buf, state_cls)
            assert buf.block_size == p.numel() and buf.scale.numel() == 1
        else:
            assert type(buf) is torch.Tensor and buf.dtype == p.dtype


def test_lp_stochastic_round_flag_is_stored():
    assert Muon8bit([nn.Parameter(torch.randn(32, 32))], bf16_stochastic_round=True).bf16_stochastic_round


def test_group_tensors_by_shape_and_move_helpers():
    a, b, c = torch.randn(2, 3), torch.randn(4, 5), torch.randn(2, 3, dtype=torch.bfloat16)
    groups = group_tensors_by_shape([a, b, c])
    assert list(groups) == [(2, 3), (4, 5)]
    assert groups[(2, 3)][1] == [0, 2] and groups[(2, 3)][0][1] is c
    assert group_tensors_by_shape([]) == {}
    s = torch.tensor(1.0)
    assert group_tensors_by_shape([s]) == {(): ([s], [0])}
    ts = [a, None]
    assert move_tensors_to_device(ts, torch.device("cpu"), torch.device("cpu")) is ts
    assert move_tensors_to_device([], torch.device("cpu"), torch.device("cuda")) == []


@pytest.mark.parametrize("state_cls,args", [(OptimState8bit, (True, 256)),
                                            (OptimState4bit, (False, 128)),
                                            (OptimStateFp8, (512,))])
def test_quantized_state_loads_with_weights_only(state_cls, args):
    """A quantized momentum state inside an optimizer state dict survives torch.save and
    torch.load with the default weights_only=True: same class, shape, block size,
    signedness, codes, scales and map."""
    import io

    st = state_cls.zeros((32, 64), *args, device="cpu")
    st.codes.copy_(torch.arange(st.codes.numel(), dtype=torch.int64).remainder(251).to(torch.uint8))
    st.scale.copy_(torch.linspace(0.5, 2.0, st.scale.numel()))
    blob = io.BytesIO()
    torch.save({"state": {0: {"step": torch.tensor(2.0), "momentum_buffer": st}}}, blob)
    blob.seek(0)
    got = torch.load(blob, weights_only=True)["state"][0]["momentum_buffer"]
    assert type(got) is state_cls
    assert (got.shape, got.block_size, got.signed) == (st.shape, st.block_size, st.signed)
    assert torch.equal(got.codes, st.codes) and torch.equal(got.scale, st.scale)
    assert (got.qmap is None) == (st.qmap is None)
    if st.qmap is not None:
        assert torch.equal(got.qmap, st.qmap)
