"""Run-to-run determinism of the orthogonalization with batched launches that give every
workgroup of the persistent products several tiles: each product kernel (B X for K below
and above 2048, the SYRK with full, packed and 128-row tiles) runs twice more on the same
inputs, and every result is bit-identical to the first. (A single matrix of one bucket did not expose
the race an earlier B X kernel had: its beta step's register moves read MFMA results early,
a one-ulp difference in about 0.003% of the outputs of a batched launch.)"""
import pytest
import torch

from muonium_amd.orthogonalize import foreach_zeropower

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.mark.parametrize("shape,count", [((2048, 2048), 16), ((4096, 4096), 8), ((1024, 4096), 16),
                                         ((1408, 2048), 16), ((4096, 14336), 4), ((768, 3072), 12)],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_orthogonalization_is_deterministic(shape, count):
    gen = torch.Generator(device=DEV).manual_seed(11)
    gs = [torch.randn(shape, generator=gen, device=DEV).bfloat16() for _ in range(count)]
    first = foreach_zeropower(gs, strategy="polar_express")
    for _ in range(2):
        again = foreach_zeropower(gs, strategy="polar_express")
        for i, (a, b) in enumerate(zip(first, again)):
            assert torch.equal(a, b), f"matrix {i} differs between runs"
