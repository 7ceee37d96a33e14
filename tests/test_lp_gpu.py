"""Quantized momentum (MuonLP) on the HIP path vs the quantizer oracle.

Codes and scales must be bit-exact given identical fp32 inputs (standalone quantize,
and through the fused dequant -> momentum -> requant pre-pass); dequantization is
exact; the full MuonLP step matches the oracle's arithmetic given the same U.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn as nn

from muonium_amd.optim import Muon4bit, Muon8bit, MuonFp8, MuonLP
from muonium_amd.optim.lp_state import OptimState4bit, OptimState8bit, OptimStateFp8
from muonium_amd.orthogonalize import zeropower
from oracle import muon_ref, quant_ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
FORMATS = [("8bit", OptimState8bit), ("4bit", OptimState4bit), ("fp8", OptimStateFp8)]


def _qmap(fmt, signed=True):
    if fmt == "8bit":
        return quant_ref.qmap_8bit(signed)
    if fmt == "4bit":
        return quant_ref.qmap_4bit(signed)
    return None


def _state(cls, shape, block):
    if cls is OptimStateFp8:
        return cls.zeros(shape, block, DEV)
    return cls.zeros(shape, True, block, DEV)


@pytest.mark.parametrize("fmt,cls", FORMATS)
@pytest.mark.parametrize("block", [128, 256, 2048])
def test_quantize_bit_exact(fmt, cls, block):
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(64, 128, generator=gen) * torch.exp(torch.randn(64, 1, generator=gen))
    x[3, :] = 0.0  # an all-zero block exercises the 1e-12 clip
    st = _state(cls, x.shape, block)
    st.copy_(x.to(DEV))
    codes, scale = quant_ref.quantize(x.numpy(), block, fmt, _qmap(fmt))
    assert np.array_equal(st.codes.cpu().numpy(), codes)
    assert np.array_equal(st.scale.cpu().numpy().view(np.uint32), scale.view(np.uint32))
    deq = quant_ref.dequantize(codes, scale, block, fmt, _qmap(fmt))
    got = st.dequantize().cpu().numpy().reshape(-1)
    assert np.array_equal(got.view(np.uint32), deq.view(np.uint32))


def test_qmap_matches_oracle():
    assert np.array_equal(
        OptimState8bit.zeros((64, 64), True, 256, DEV).qmap.cpu().numpy(), quant_ref.qmap_8bit()
    )
    assert np.array_equal(
        OptimState4bit.zeros((64, 64), True, 256, DEV).qmap.cpu().numpy(), quant_ref.qmap_4bit()
    )


@pytest.mark.parametrize("fmt,cls", FORMATS)
@pytest.mark.parametrize("nesterov,maximize", [(True, False), (False, False), (True, True)])
@pytest.mark.parametrize("shape", [(128, 96), (96, 128)])  # tall and wide workspace paths
def test_lp_prepass_codes_bit_exact_and_step(fmt, cls, nesterov, maximize, shape):
    opt_cls = {"8bit": Muon8bit, "4bit": Muon4bit, "fp8": MuonFp8}[fmt]
    block = 256
    gen = torch.Generator().manual_seed(1)
    p0 = torch.randn(shape, generator=gen)
    p = nn.Parameter(p0.clone().to(DEV))
    opt = opt_cls([p], lr=0.05, wd=0.1, momentum=0.9, nesterov=nesterov, maximize=maximize,
                  block_size=block)
    codes = None
    scales = None
    ref_p = p0.clone()
    for step in range(2):
        g = torch.randn(shape, generator=gen)
        p.grad = g.clone().to(DEV)
        opt.step()
        st = opt.state[p]["momentum_buffer"]
        assert isinstance(st, cls)
        if codes is None:
            codes = np.zeros(st.codes.numel(), np.uint8)
            scales = np.zeros(st.scale.numel(), np.float32)
        codes, scales, gq = quant_ref.lp_momentum_step(
            codes, scales, g.numpy(), block=block, fmt=fmt, qmap=_qmap(fmt), momentum=0.9,
            nesterov=nesterov, maximize=maximize,
        )
        assert np.array_equal(st.codes.cpu().numpy(), codes), f"codes differ at step {step}"
        assert np.array_equal(st.scale.cpu().numpy().view(np.uint32), scales.view(np.uint32))
        # the parameter: oracle post-pass arithmetic on the HIP U of the same g'
        U = zeropower(torch.from_numpy(gq).view(shape).to(DEV), strategy="polar_express").cpu()
        u = U.float() + 0.1 * ref_p * ((U.float() * ref_p) > 0)
        adj = torch.tensor(muon_ref.lr_ratio(shape)) * torch.tensor(0.05)
        ref_p = ref_p - adj * u
        assert torch.equal(p.detach().cpu(), ref_p), f"param differs at step {step}"


@pytest.mark.parametrize("opt_cls", [Muon8bit, Muon4bit, MuonFp8])
def test_small_buffers_stay_dense_in_param_dtype(opt_cls):
    p = nn.Parameter(torch.randn(32, 32, device=DEV, dtype=torch.bfloat16))
    p.grad = torch.randn_like(p)
    opt = opt_cls([p], block_size=2048)
    opt.step()
    buf = opt.state[p]["momentum_buffer"]
    assert type(buf) is torch.Tensor and buf.dtype is torch.bfloat16


def test_base_muon_lp_matches_muon():
    from muonium_amd import Muon

    gen = torch.Generator().manual_seed(0)
    init = torch.randn(32, 16, generator=gen)
    a = nn.Parameter(init.clone().to(DEV))
    b = nn.Parameter(init.clone().to(DEV))
    kw = dict(lr=0.1, wd=0.0, orthogonalization_strategy="newton_schulz")
    lp, ref = MuonLP([a], **kw), Muon([b], **kw)
    for _ in range(2):
        g = torch.randn(32, 16, generator=gen).to(DEV)
        a.grad, b.grad = g.clone(), g.clone()
        lp.step()
        ref.step()
    # MuonLP's plain buffers are in the param's dtype (fp32 here): identical arithmetic
    assert torch.equal(a, b)
    assert math.isfinite(a.sum().item())
