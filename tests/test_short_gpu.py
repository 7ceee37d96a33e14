"""Iterates with at most 64 rows on the short side (the 64-row workspace of short.hip):
stacked experts under flatten=True, e.g. the MoE tensors (64, 1408, 2048) -> (64, 2883584).

The small shapes are compared with the CPU oracle in test_orth_gpu.py; here:
* the full flatten=True MoE shape against the oracle's bf16 iteration (a few seconds of
  CPU work at this size) and through the spectral identity of the iteration (the
  singular values of U are the composed polynomial of the normalized singular values of
  X; fp64 eigenvalues of the 64 x 64 Gram matrix);
* the Gram partials are summed in a fixed order: a batch equals its members run alone,
  a tall input gives exactly the transpose of its transpose's result, and repeated runs
  are bit-identical;
* a Muon step with flatten=True on a 3D tensor against the oracle's per-parameter step.
"""

import math

import pytest
import torch
import torch.nn as nn

from helpers import rel_fro
from muonium_amd import Muon
from muonium_amd.orthogonalize import foreach_zeropower, zeropower
from oracle import muon_ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
SPECTRUM_TOL = 1e-2


def _g(shape, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(shape, generator=gen, device=DEV)


def _svals(M):
    M = M.double()
    G = M @ M.T if M.shape[0] <= M.shape[1] else M.T @ M
    return torch.linalg.eigvalsh(G).clamp_min(0).sqrt()


def _spectrum_err(X, U, strategy):
    coeffs, prescale = muon_ref.strategy_coeffs(strategy, 5)
    s = _svals(X) / (X.double().norm() * prescale)
    for a, b, c in coeffs:
        s = a * s + b * s ** 3 + c * s ** 5
    su = _svals(U)
    return (su.sort().values - s.sort().values).abs().max().item(), su


@pytest.mark.parametrize("strategy", ["newton_schulz", "polar_express"])
def test_moe_flatten_shape_matches_oracle(strategy):
    """The full (64, 2883584) matrix with per-row log-normal scales (the benchmark's
    gradient model): U within the bf16 bar of the oracle's iteration at the same storage
    points (about 5 s of CPU work), and its spectrum as close to the polynomial image as
    the oracle's own (bf16 rounding of a 64-row Gram over 2.9M columns leaves about 2e-2)."""
    gen = torch.Generator().manual_seed(4)
    z = torch.randn(64, 1, generator=torch.Generator().manual_seed(5))
    X = (torch.randn(64, 1408 * 2048, generator=gen) * torch.exp(z)).bfloat16()
    U = zeropower(X.to(DEV), strategy=strategy)
    coeffs, prescale = muon_ref.strategy_coeffs(strategy, 5)
    ref = muon_ref.polar_iteration_bf16(X.float(), coeffs, prescale=prescale, eps=1e-7)
    d = rel_fro(U.cpu(), ref)
    err, su = _spectrum_err(X.to(DEV), U, strategy)
    err_ref, _ = _spectrum_err(X.to(DEV), ref.to(DEV), strategy)
    print(f"{strategy}: rel-Frobenius vs oracle {d:.3e}; max |sigma(U) - p(sigma(X))| = "
          f"{err:.4e} (oracle {err_ref:.4e}), sigma(U) in [{su.min():.4f}, {su.max():.4f}]")
    assert d <= 1e-2
    assert err <= max(SPECTRUM_TOL, 1.5 * err_ref)


def test_short_batch_transpose_and_repeat_are_exact():
    X = _g((64, 70000), 6)
    a = zeropower(X, strategy="polar_express")
    assert torch.equal(zeropower(X, strategy="polar_express"), a)
    ys = [_g((64, 70000), 7 + i) for i in range(2)]
    both = foreach_zeropower([X] + ys, strategy="polar_express")
    assert torch.equal(both[0], a)
    for y, u in zip(ys, both[1:]):
        assert torch.equal(u, zeropower(y, strategy="polar_express"))
    T = _g((50000, 40), 9)
    assert torch.equal(zeropower(T, strategy="newton_schulz"),
                       zeropower(T.T.contiguous(), strategy="newton_schulz").T)


def test_flatten_true_step_matches_oracle():
    """A 3D tensor under flatten=True is one (8, 15360) matrix (optim.py:396-398): momentum
    and parameters bit-exact against the oracle's update arithmetic given the same U, and U
    within the bf16 bar of the oracle's iteration."""
    shape, flat = (8, 48, 320), (8, 15360)
    hp = dict(wd=0.1, use_cautious_wd=True, momentum=0.95, nesterov=True, maximize=False)
    gen = torch.Generator().manual_seed(21)
    p0 = torch.randn(shape, generator=gen).bfloat16()
    g0 = torch.randn(shape, generator=gen).bfloat16()
    p = nn.Parameter(p0.clone().to(DEV))
    p.grad = g0.clone().to(DEV)
    opt = Muon([{"params": [p], "flatten": True}], lr=0.02, foreach=True,
               orthogonalization_strategy="newton_schulz", **hp)
    opt.step()
    torch.cuda.synchronize()
    st = opt.state[p]
    assert st["momentum_buffer"].shape == flat
    assert math.isclose(float(st["lr_ratio"]), 1.0)

    def oracle(orth):
        return muon_ref.muon_update(
            p0.view(flat), g0.view(flat), torch.zeros(flat), muon_ref.lr_ratio(flat), lr=0.02,
            weight_decay=hp["wd"], cautious_wd=hp["use_cautious_wd"], momentum=hp["momentum"],
            nesterov=hp["nesterov"], maximize=hp["maximize"], ns_steps=5,
            strategy="newton_schulz", orth_single=orth)

    _, ref_buf, gq, _ = oracle(lambda g: g)
    U = zeropower(gq.to(DEV), steps=5, strategy="newton_schulz").cpu()
    ref_p, _, _, _ = oracle(lambda g: U)
    assert torch.equal(st["momentum_buffer"].cpu(), ref_buf)
    assert torch.equal(p.detach().cpu().view(flat), ref_p)
    coeffs, prescale = muon_ref.strategy_coeffs("newton_schulz", 5)
    ref_u = muon_ref.polar_iteration_bf16(gq, coeffs, prescale=prescale, eps=1e-7)
    assert rel_fro(U, ref_u) <= 1e-2, f"{rel_fro(U, ref_u):.3e}"
