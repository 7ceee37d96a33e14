"""Writes the golden fixtures used by the oracle and GPU tests.

known_answers.json: the closed-form answers of the reference's own update tests
(muonium tests/optim/test_optim.py:392-482), written out as numbers.
vectors.npz: seeded inputs and the oracle's outputs for them (quantization maps,
blockwise codes/scales, a bf16 iteration), so later changes to the oracle show up.

Run: python tests/golden/make_golden.py
"""

import json
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import muon_ref as R  # noqa: E402
from oracle import quant_ref as Q  # noqa: E402


def known_answers():
    base = dict(lr=0.1, weight_decay=0.0, cautious_wd=True, momentum=0.0, nesterov=False,
                maximize=False)
    cases = [
        # test_optim.py:392-404: lr_ratio sqrt(2) on a 4x2
        dict(param=[[1.0] * 2] * 4, grad=[[0.5] * 2] * 4, hp={},
             expected=[[1.0 - math.sqrt(2.0) * 0.1 * 0.5] * 2] * 4),
        # :407-417 Nesterov: update 0.75
        dict(param=[[1.0] * 2] * 2, grad=[[0.5] * 2] * 2, hp=dict(momentum=0.5, nesterov=True),
             expected=[[1.0 - 0.1 * 0.75] * 2] * 2),
        # :420-435 cautious weight decay
        dict(param=[[1.0, -1.0], [1.0, -1.0]], grad=[[1.0, 1.0], [-1.0, -1.0]],
             hp=dict(lr=1.0, weight_decay=1.0, cautious_wd=True),
             expected=[[-1.0, -2.0], [2.0, 1.0]]),
        # :438-453 plain weight decay
        dict(param=[[1.0, -1.0], [1.0, -1.0]], grad=[[1.0, 1.0], [-1.0, -1.0]],
             hp=dict(lr=1.0, weight_decay=1.0, cautious_wd=False),
             expected=[[-1.0, -1.0], [1.0, 1.0]]),
        # :456-467 maximize
        dict(param=[[1.0] * 2] * 2, grad=[[0.5] * 2] * 2, hp=dict(maximize=True),
             expected=[[1.05] * 2] * 2),
    ]
    for c in cases:
        hp = dict(base)
        hp.update(c["hp"])
        c["hp"] = hp
    return {"updates": cases}


def vectors():
    gen = torch.Generator().manual_seed(1234)
    lp_x = (torch.randn(4096, generator=gen) * torch.exp(torch.randn(16, generator=gen)).repeat_interleave(256)).numpy()
    out = {"qmap8": Q.qmap_8bit(), "qmap4": Q.qmap_4bit(), "lp_x": lp_x.astype(np.float32)}
    for fmt, qmap in (("8bit", Q.qmap_8bit()), ("4bit", Q.qmap_4bit()), ("fp8", None)):
        codes, scale = Q.quantize(lp_x, 256, fmt, qmap)
        out[f"codes_{fmt}"] = codes
        out[f"scale_{fmt}"] = scale
    X = torch.randn(48, 80, generator=gen)
    out["orth_x"] = X.numpy()
    for strat in ("polar_express", "newton_schulz"):
        coeffs, prescale = R.strategy_coeffs(strat, 5)
        out[f"orth_{strat}"] = R.polar_iteration_bf16(X, coeffs, prescale=prescale,
                                                      eps=1e-7).float().numpy()
    return out


if __name__ == "__main__":
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(known_answers(), f, indent=1)
    np.savez_compressed(os.path.join(HERE, "vectors.npz"), **vectors())
    print("wrote", os.listdir(HERE))
