"""NorMuon on the HIP path (muon_normuon_postpass) vs the oracle's NorMuon.update.

The oracle (oracle/muon_ref.normuon_update, a restatement of normuon.py:74-134 and
_normuon_normalize, normuon.py:16-55) is given the same orthogonalized update U the HIP
path computes (zeropower / foreach_zeropower on the device), so the comparison isolates
the normalization, the variance EMA and the apply. Tolerances: the row normalization is
fp32 arithmetic in a different order (row sums, a row multiplier instead of a division),
so fp32 parameters agree to 1e-4 in relative Frobenius norm of the update, bf16 parameters
to 2e-2 (one bf16 rounding of p can flip), and the variance state to rtol 1e-4.
"""

import pytest
import torch
import torch.nn as nn

from helpers import rel_fro
from muonium_amd import Muon
from muonium_amd.orthogonalize import foreach_zeropower, zeropower
from oracle import muon_ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
HP = dict(lr=0.1, weight_decay=0.1, cautious_wd=True, momentum=0.5, nesterov=True,
          maximize=False)


def _run(shapes, dtype, foreach, beta2=0.9, steps=2, seed=11, split_sizes=None):
    gen = torch.Generator().manual_seed(seed)
    p0 = [torch.randn(s, generator=gen).to(dtype) for s in shapes]
    params = [nn.Parameter(p.clone().to(DEV)) for p in p0]
    group = {"params": params, "algorithm": "normuon", "muon_beta2": beta2}
    if split_sizes is not None:
        group["split_sizes"] = split_sizes
    opt = Muon([group], lr=HP["lr"], wd=HP["weight_decay"], momentum=HP["momentum"],
               nesterov=HP["nesterov"], foreach=foreach)
    ref_p = [p.clone() for p in p0]
    ref_buf = [torch.zeros(s) for s in shapes]
    ref_v = [torch.zeros(*s[:-1], 1) for s in shapes]
    for _ in range(steps):
        gs = [torch.randn(s, generator=gen).to(dtype) for s in shapes]
        for p, g in zip(params, gs):
            p.grad = g.clone().to(DEV)
        opt.step()
        for i, (s, g) in enumerate(zip(shapes, gs)):
            g32 = g.float()
            buf = ref_buf[i] * HP["momentum"] + g32
            gq = g32 + buf * HP["momentum"]
            if split_sizes is None:
                U = zeropower(gq.to(DEV), strategy="polar_express").cpu()
                orth = dict(orth_single=lambda x, U=U: U)
            else:
                orth = dict(orth_batch=lambda blocks: [
                    u.cpu() for u in foreach_zeropower([b.to(DEV) for b in blocks],
                                                       strategy="polar_express")])
            ref_p[i], ref_buf[i], ref_v[i], _ = muon_ref.normuon_update(
                ref_p[i], g, ref_buf[i], ref_v[i], muon_ref.lr_ratio(s), beta2=beta2,
                split_sizes=split_sizes, **HP, **orth,
            )
    return opt, params, p0, ref_p, ref_v


@pytest.mark.parametrize("foreach", [True, False])
@pytest.mark.parametrize(
    "shapes,dtype",
    [([(300, 130)] * 3, torch.bfloat16), ([(2, 70, 200)] * 2, torch.float32),
     ([(64, 512)], torch.float32), ([(520, 260)] * 2, torch.float32),
     ([(512, 48)] * 2, torch.bfloat16), ([(40, 768)], torch.float32)],
    ids=["tall-bf16-x3", "stacked-fp32-x2", "wide-fp32", "tall-fp32-x2",
         "short-tall-bf16-x2", "short-wide-fp32"],
)
def test_normuon_matches_oracle_buckets(shapes, dtype, foreach):
    opt, params, p0, ref_p, ref_v = _run(shapes, dtype, foreach)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-4
    for p, p_init, rp, rv in zip(params, p0, ref_p, ref_v):
        got = p.detach().cpu().float() - p_init.float()
        want = rp.float() - p_init.float()
        assert rel_fro(got, want) < tol, f"{rel_fro(got, want):.3e}"
        torch.testing.assert_close(opt.state[p]["variance_neuron"].cpu(), rv, rtol=1e-4,
                                   atol=1e-7)


@pytest.mark.parametrize("foreach", [True, False])
@pytest.mark.parametrize(
    "shapes,dtype,split",
    [([(96, 32)], torch.float32, (64, 16, 16)),
     ([(384, 256)] * 3, torch.bfloat16, (128, 128, 128)),
     ([(320, 128)] * 2, torch.float32, (64, 256)),
     ([(520, 96)], torch.bfloat16, (8, 512))],
    ids=["small-fp32", "equal-blocks-bf16-x3", "mixed-fp32-x2", "tiny-block-bf16"],
)
def test_normuon_split_sizes_matches_oracle(shapes, dtype, split, foreach):
    """Row blocks normalized independently (normuon.py:30-42) after their split_lr_scales
    rescale: each block runs as its own matrix through the fused pre-pass, iteration and
    NorMuon post-pass, with its slice of the variance state."""
    opt, params, p0, ref_p, ref_v = _run(shapes, dtype, foreach, split_sizes=split)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-4
    for p, p_init, rp, rv in zip(params, p0, ref_p, ref_v):
        got = p.detach().cpu().float() - p_init.float()
        assert rel_fro(got, rp.float() - p_init.float()) < tol
        torch.testing.assert_close(opt.state[p]["variance_neuron"].cpu(), rv, rtol=1e-4,
                                   atol=1e-7)


def test_normuon_beta2_weight_is_exact():
    # lerp weight 1 - beta2 is formed in double from the Python float, as torch does: with
    # beta2 = 0.95 the variance after one step from zero is exactly 0.05 * mean(U^2) (fp32).
    opt, params, p0, ref_p, ref_v = _run([(64, 128)], torch.float32, True, beta2=0.95, steps=1)
    torch.testing.assert_close(opt.state[params[0]]["variance_neuron"].cpu(), ref_v[0],
                               rtol=2e-6, atol=0)
