"""The explicit-U (seam) path for quantized momentum: MuonLP with ``split_sizes`` and NorMuon
on quantized momentum.

Both run the momentum step on the dequantized state (muon.py:45-56 through the quantized
state: m' = m mu + g, the state stores quant(m'), Nesterov's input is the unquantized m'),
call the module-level orthogonalizer exactly as the reference does (base.py:56-168), and
apply its output with the post-pass (muon.py:58-77) or the NorMuon post-pass
(normuon.py:118-134). Checked over two steps against the oracle: codes and scales bit-exact
(quant_ref.lp_momentum_step); parameters bit-exact given the step's own U for Muon; for
NorMuon, the normalization at the tolerances of tests/test_normuon_gpu.py (fp32 row sums in
another order), the variance state to rtol 1e-4.
"""

import numpy as np
import pytest
import torch
import torch.nn as nn

from helpers import rel_fro
from muonium_amd.optim import Muon4bit, Muon8bit, MuonFp8
from muonium_amd.optim.algorithms.base import orthogonalize_single
from oracle import muon_ref, quant_ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
OPTS = {"8bit": Muon8bit, "4bit": Muon4bit, "fp8": MuonFp8}


def _qmap(fmt):
    return {"8bit": quant_ref.qmap_8bit(), "4bit": quant_ref.qmap_4bit(), "fp8": None}[fmt]


@pytest.mark.parametrize("fmt", ["8bit", "4bit", "fp8"])
@pytest.mark.parametrize("foreach", [False, True])
@pytest.mark.parametrize("shape,split,block,dtype", [
    ((384, 256), (128, 256), 256, torch.float32),
    ((384, 256), (128, 128, 128), 2048, torch.bfloat16),
    ((96, 512), (32, 64), 512, torch.float32),
], ids=["tall-mixed-b256-fp32", "tall-equal-b2048-bf16", "wide-b512-fp32"])
def test_lp_split_sizes_matches_oracle(fmt, foreach, shape, split, block, dtype):
    gen = torch.Generator().manual_seed(31)
    p0 = torch.randn(shape, generator=gen).to(dtype)
    ps = [nn.Parameter(p0.clone().to(DEV)) for _ in range(2)]
    opt = OPTS[fmt]([{"params": ps, "split_sizes": split}], lr=0.05, wd=0.1, momentum=0.9,
                    nesterov=True, foreach=foreach, block_size=block)
    state = [None, None]
    ref_p = [p0.clone(), p0.clone()]
    for step in range(2):
        gs = [torch.randn(shape, generator=gen).to(dtype) for _ in ps]
        for p, g in zip(ps, gs):
            p.grad = g.clone().to(DEV)
        opt.step()
        for i, (p, g) in enumerate(zip(ps, gs)):
            st = opt.state[p]["momentum_buffer"]
            assert type(st).__name__.startswith("OptimState")
            if state[i] is None:
                state[i] = (np.zeros(st.codes.numel(), np.uint8), np.zeros(st.scale.numel(), np.float32))
            c, s, gq = quant_ref.lp_momentum_step(
                *state[i], g.float().numpy(), block=block, fmt=fmt, qmap=_qmap(fmt),
                momentum=0.9, nesterov=True, maximize=False)
            state[i] = (c, s)
            assert np.array_equal(st.codes.cpu().numpy(), c), f"param {i}: codes, step {step}"
            assert np.array_equal(st.scale.cpu().numpy().view(np.uint32), s.view(np.uint32))
            # the update the step applied: this library's split orthogonalizer on the same g'
            U = orthogonalize_single(torch.from_numpy(gq).view(shape).to(DEV), ns_steps=5,
                                     strategy="polar_express", split_sizes=split).cpu()
            ref_p[i], _, _, _ = muon_ref.muon_update(
                ref_p[i], g, torch.zeros(shape), muon_ref.lr_ratio(shape), lr=0.05,
                weight_decay=0.1, cautious_wd=True, momentum=0.9, nesterov=True,
                maximize=False, orth_single=lambda x, U=U: U)
            assert torch.equal(p.detach().cpu(), ref_p[i]), f"param {i} differs at step {step}"


@pytest.mark.parametrize("fmt", ["8bit", "4bit", "fp8"])
@pytest.mark.parametrize("foreach", [False, True])
@pytest.mark.parametrize("shape,split,dtype", [
    ((384, 256), None, torch.float32),
    ((256, 640), None, torch.bfloat16),
    ((384, 256), (128, 256), torch.float32),
], ids=["tall-fp32", "wide-bf16", "tall-split-fp32"])
def test_normuon_quantized_momentum_matches_oracle(fmt, foreach, shape, split, dtype):
    beta2 = 0.9
    gen = torch.Generator().manual_seed(37)
    p0 = torch.randn(shape, generator=gen).to(dtype)
    ps = [nn.Parameter(p0.clone().to(DEV)) for _ in range(2)]
    group = {"params": ps, "algorithm": "normuon", "muon_beta2": beta2}
    if split is not None:
        group["split_sizes"] = split
    opt = OPTS[fmt]([group], lr=0.1, wd=0.1, momentum=0.5, nesterov=True, foreach=foreach,
                    block_size=256)
    state = [None, None]
    ref_p = [p0.clone(), p0.clone()]
    ref_v = [torch.zeros(shape[0], 1), torch.zeros(shape[0], 1)]
    for step in range(2):
        gs = [torch.randn(shape, generator=gen).to(dtype) for _ in ps]
        for p, g in zip(ps, gs):
            p.grad = g.clone().to(DEV)
        opt.step()
        for i, (p, g) in enumerate(zip(ps, gs)):
            st = opt.state[p]["momentum_buffer"]
            assert type(st).__name__.startswith("OptimState")
            if state[i] is None:
                state[i] = (np.zeros(st.codes.numel(), np.uint8), np.zeros(st.scale.numel(), np.float32))
            # the momentum the step starts from, so the oracle's own g' is this step's
            m_prev = torch.from_numpy(
                quant_ref.dequantize(*state[i], 256, fmt, _qmap(fmt)).copy()).view(shape)
            c, s, gq = quant_ref.lp_momentum_step(
                *state[i], g.float().numpy(), block=256, fmt=fmt, qmap=_qmap(fmt),
                momentum=0.5, nesterov=True, maximize=False)
            state[i] = (c, s)
            assert np.array_equal(st.codes.cpu().numpy(), c), f"param {i}: codes, step {step}"
            assert np.array_equal(st.scale.cpu().numpy().view(np.uint32), s.view(np.uint32))
            U = orthogonalize_single(torch.from_numpy(gq).view(shape).to(DEV), ns_steps=5,
                                     strategy="polar_express").cpu()
            if split is None:
                orth = dict(orth_single=lambda x, U=U: U)
            else:
                # row blocks orthogonalized on the device, then scaled by the oracle
                orth = dict(orth_batch=lambda blocks: [
                    orthogonalize_single(b.to(DEV), ns_steps=5, strategy="polar_express").cpu()
                    for b in blocks])
            new_p, _, ref_v[i], _ = muon_ref.normuon_update(
                ref_p[i], g, m_prev, ref_v[i], muon_ref.lr_ratio(shape), lr=0.1,
                weight_decay=0.1, cautious_wd=True, momentum=0.5, nesterov=True, maximize=False,
                beta2=beta2, split_sizes=split, **orth)
            got = p.detach().cpu().float()
            tol = 2e-2 if dtype == torch.bfloat16 else 1e-4
            r = rel_fro(got - ref_p[i].float(), new_p.float() - ref_p[i].float())
            assert r < tol, f"param {i}, step {step}: {r:.3e}"
            torch.testing.assert_close(opt.state[p]["variance_neuron"].cpu(), ref_v[i],
                                       rtol=1e-4, atol=1e-7)
            ref_p[i] = p.detach().cpu().clone()
