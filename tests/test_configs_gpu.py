"""Whole benchmark configurations stepped through the optimizer, against the oracle.

Config 4 (MoE experts) in its per-expert form, at two layers of 8
experts: the test at the end of this file.

Config 2 (the GPT-2-small-shaped set): 12 layers x {768x2304,
768x768, 768x3072, 3072x768} bf16 params with fp32 momentum, gradients with per-row
log-normal scales, Polar Express 5, the optimizer's defaults, foreach. Its buckets are too
small to fill the device, so the foreach driver runs them concurrently on side streams;
the test steps the whole set in one optimizer, as the benchmark does, and checks every
matrix:

* momentum buffers bit-exact against the oracle;
* parameters bit-exact against the oracle's update arithmetic given the orthogonalized
  update U of the same g' (zeropower on the device, the same kernels as the fused step;
  a batch equals its members run alone);
* on layer 0 and layer 11, U within the bf16 bar (1e-2 rel-Frobenius) of the oracle's
  bf16 Polar Express iteration.
"""

import pytest
import torch
import torch.nn as nn

from helpers import rel_fro
from muonium_amd import Muon
from muonium_amd.optim import optim as optim_mod
from muonium_amd.orthogonalize import foreach_zeropower
from oracle import muon_ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
GPT2 = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]


def test_gpt2_set_one_optimizer_matches_oracle():
    layers = 12
    shapes = [s for _ in range(layers) for s in GPT2]
    gen = torch.Generator().manual_seed(2024)
    p0 = [(0.02 * torch.randn(s, generator=gen)).bfloat16() for s in shapes]
    g0 = [(torch.randn(s, generator=gen) * torch.exp(torch.randn(s[0], 1, generator=gen))).bfloat16()
          for s in shapes]
    params = [nn.Parameter(p.clone().to(DEV)) for p in p0]
    for p, g in zip(params, g0):
        p.grad = g.clone().to(DEV)
    opt = Muon(params, foreach=True)  # defaults: lr 1e-3, wd 0.1 cautious, mu 0.95 Nesterov, PE 5
    optim_mod._side_streams.clear()
    opt.step()
    torch.cuda.synchronize()
    # four small buckets: the three largest on side streams (768 x 3072 and 3072 x 768, which
    # pad alike, on two of them, each with its own workspace), the 768 x 768 bucket on the
    # caller's stream
    assert len(optim_mod._side_streams) == 3

    coeffs, prescale = muon_ref.strategy_coeffs("polar_express", 5)
    hp = dict(lr=1e-3, weight_decay=0.1, cautious_wd=True, momentum=0.95, nesterov=True,
              maximize=False, ns_steps=5, strategy="polar_express")
    gqs = []
    for i, s in enumerate(shapes):
        zero = torch.zeros(s, dtype=torch.float32)
        _, ref_buf, gq, _ = muon_ref.muon_update(p0[i], g0[i], zero, muon_ref.lr_ratio(s),
                                                 orth_single=lambda g: g, **hp)
        assert torch.equal(opt.state[params[i]]["momentum_buffer"].cpu(), ref_buf), f"buf {i} {s}"
        gqs.append(gq)
    for k, s in enumerate(GPT2):
        idx = list(range(k, len(shapes), len(GPT2)))
        Us = foreach_zeropower([gqs[i].to(DEV) for i in idx], steps=5, strategy="polar_express")
        for i, U in zip(idx, Us):
            U = U.cpu()
            zero = torch.zeros(s, dtype=torch.float32)
            ref_p, _, _, _ = muon_ref.muon_update(p0[i], g0[i], zero, muon_ref.lr_ratio(s),
                                                  orth_single=lambda g: U, **hp)
            got = params[i].detach().cpu()
            assert torch.equal(got, ref_p), f"param {i} {s} differs given U"
            if i // len(GPT2) in (0, layers - 1):
                U_ref = muon_ref.polar_iteration_bf16(gqs[i], coeffs, prescale=prescale, eps=1e-7)
                r = rel_fro(U, U_ref)
                print(f"layer {i // len(GPT2)} {s}: U vs oracle rel-Frobenius {r:.3e}")
                assert r <= 1e-2, f"layer {i // len(GPT2)} {s}: {r:.3e}"


MOE = [(8, 1408, 2048), (8, 1408, 2048), (8, 2048, 1408)]


def test_moe_experts_one_optimizer_matches_oracle():
    """Config 4's per-expert form (flatten=False: each expert of a (E, rows, cols) tensor is
    one matrix of the batch), two layers of gate, up and down with 8 experts each, Newton-
    Schulz 5, foreach, per-expert log-normal gradient scales. m = 1408 pads to 1536 rows: the
    Gram products take packed tiles and the last B X of each bucket carries the apply on the
    3-D parameters (the down experts, 2048 x 1408, in their transposed form). Momentum bit-exact,
    parameters bit-exact given U, and U within the bf16 bar for two experts per bucket."""
    layers = 2
    shapes = [s for _ in range(layers) for s in MOE]
    gen = torch.Generator().manual_seed(77)
    p0 = [(0.02 * torch.randn(s, generator=gen)).bfloat16() for s in shapes]
    g0 = [(torch.randn(s, generator=gen) * torch.exp(torch.randn(s[0], 1, 1, generator=gen)))
          .bfloat16() for s in shapes]
    params = [nn.Parameter(p.clone().to(DEV)) for p in p0]
    for p, g in zip(params, g0):
        p.grad = g.clone().to(DEV)
    opt = Muon(params, foreach=True, orthogonalization_strategy="newton_schulz")
    opt.step()
    torch.cuda.synchronize()

    coeffs, prescale = muon_ref.strategy_coeffs("newton_schulz", 5)
    hp = dict(lr=1e-3, weight_decay=0.1, cautious_wd=True, momentum=0.95, nesterov=True,
              maximize=False, ns_steps=5, strategy="newton_schulz")
    gqs = []
    for i, s in enumerate(shapes):
        zero = torch.zeros(s, dtype=torch.float32)
        _, ref_buf, gq, _ = muon_ref.muon_update(p0[i], g0[i], zero, muon_ref.lr_ratio(s),
                                                 orth_single=lambda g: g, **hp)
        assert torch.equal(opt.state[params[i]]["momentum_buffer"].cpu(), ref_buf), f"buf {i} {s}"
        gqs.append(gq)
    for k, s in enumerate(MOE):
        idx = list(range(k, len(shapes), len(MOE)))
        Us = foreach_zeropower([gqs[i].to(DEV) for i in idx], steps=5, strategy="newton_schulz")
        for i, U in zip(idx, Us):
            U = U.cpu()
            zero = torch.zeros(s, dtype=torch.float32)
            ref_p, _, _, _ = muon_ref.muon_update(p0[i], g0[i], zero, muon_ref.lr_ratio(s),
                                                  orth_single=lambda g: U, **hp)
            got = params[i].detach().cpu()
            assert torch.equal(got, ref_p), f"param {i} {s} differs given U"
            if i < len(MOE):
                for e in (0, s[0] - 1):
                    U_ref = muon_ref.polar_iteration_bf16(gqs[i][e], coeffs, prescale=prescale,
                                                          eps=1e-7)
                    r = rel_fro(U[e], U_ref)
                    print(f"{s} expert {e}: U vs oracle rel-Frobenius {r:.3e}")
                    assert r <= 1e-2, f"{s} expert {e}: {r:.3e}"
