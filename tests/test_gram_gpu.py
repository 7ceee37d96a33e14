"""Gram kernel (bf16 / fp32 SYRK) parity against the oracle's x @ x^T.

Mirrors the reference's tests/kernels/test_gram.py:50-188 (shapes, symmetry,
determinism, zero rows, contract violations) with the HIP kernel as the subject.
"""

import pytest
import torch

from muonium_amd.kernels.gram import gram, gram_
from oracle import muon_ref

pytestmark = pytest.mark.gpu

SHAPES = [
    (128, 64),
    (32, 128, 64),
    (2, 32, 128, 64),
    (32, 128, 256),
    (32, 256, 64),
    (4, 300, 70),
    (3, 130, 70),
    (1, 1, 8),
    (4, 1, 1),
    (4, 64, 1024),
    (2, 520, 300),
    # whole 256-row tiles, K a multiple of 64: the SYRK reads the caller's tensors in place
    (3, 512, 320),
    (2, 2048, 1024),
    # m_pad - m = 128: packed tiles for the last tile column (bf16), diagonal tiles remapped
    # (K <= 4096) or whole (K > 4096)
    (2, 1408, 2048),
    (1, 1408, 4160),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", SHAPES)
def test_gram_matches_oracle(shape, dtype):
    gen = torch.Generator().manual_seed(42)
    x = torch.randn(*shape, generator=gen).to(dtype)
    y = gram(x.cuda()).cpu()
    ref = muon_ref.gram(x)  # fp32 accumulation, rounded to dtype
    assert y.dtype == dtype and y.shape == ref.shape
    if dtype is torch.float32:
        # fp32 MFMA vs CPU fp32: only summation order differs, whose error grows about as
        # sqrt(K) (K = 2048: up to 1.7e-4 on sums of magnitude 45)
        atol = 1e-4 * max(1.0, (shape[-1] / 256) ** 0.5)
        torch.testing.assert_close(y, ref, rtol=1e-4, atol=atol)
    else:
        # both round the fp32 accumulator once to bf16: at most one bf16 ulp apart
        torch.testing.assert_close(y.float(), ref.float(), rtol=8e-3, atol=1e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(4, 300, 70), (2, 512, 320)])
def test_gram_output_is_exactly_symmetric(dtype, shape):
    gen = torch.Generator().manual_seed(42)
    x = torch.randn(*shape, generator=gen).to(dtype).cuda()
    y = gram(x)
    assert torch.equal(y, y.mT)


def test_gram_inplace_accepts_non_contiguous_input():
    base = torch.randn(4, 70, 130, device="cuda")
    x = base.transpose(-2, -1)
    assert not x.is_contiguous()
    out = torch.empty(4, 130, 130, device="cuda")
    gram_(x, out)
    torch.testing.assert_close(out.cpu(), muon_ref.gram(x.cpu()), rtol=1e-4, atol=1e-4)


def test_gram_inplace_rejects_non_contiguous_output():
    x = torch.randn(32, 16, device="cuda")
    out = torch.empty(32, 32, device="cuda").T
    with pytest.raises(AssertionError, match="d_out must be contiguous"):
        gram_(x, out)


def test_gram_inplace_rejects_contract_violations():
    x = torch.randn(4, 8, 16, device="cuda")
    out = torch.empty(4, 8, 8, device="cuda")
    with pytest.raises(AssertionError):
        gram_(x.cpu(), out.cpu())
    with pytest.raises(AssertionError):
        gram_(x, out.cpu())
    with pytest.raises(AssertionError):
        gram_(x, out.to(torch.bfloat16))
    with pytest.raises(AssertionError):
        gram_(x, torch.empty(3, 8, 8, device="cuda"))
    with pytest.raises(AssertionError):
        gram_(x, torch.empty(4, 8, 7, device="cuda"))
    with pytest.raises(AssertionError):
        gram_(torch.randn(8, device="cuda"), torch.empty(8, 8, device="cuda"))


def test_gram_is_deterministic():
    x = torch.randn(4, 130, 70, device="cuda")
    assert torch.equal(gram(x), gram(x))


def test_gram_zero_rows_give_zero_rows_and_columns():
    x = torch.randn(4, 8, 16, device="cuda")
    x[2].zero_()
    x[:, 3].zero_()
    y = gram(x)
    assert torch.count_nonzero(y[2]) == 0
    assert torch.count_nonzero(y[:, 3]) == 0
    assert torch.count_nonzero(y[:, :, 3]) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gram_abi_empty_contraction_writes_zeros(dtype):
    """muon_gram with K == 0 through the C ABI: y is all zeros (x is never read, so a
    null x is fine), whatever y held before."""
    from muonium_amd import _lib

    lib = _lib.load()
    _lib.ensure_device(torch.device("cuda"))
    y = torch.full((3, 17, 17), float("nan"), dtype=dtype, device="cuda")
    rc = lib.muon_gram(None, y.data_ptr(), _lib.dtype_code(dtype), 3, 17, 0,
                       _lib.stream(y.device))
    assert rc == 0, _lib.last_error()
    assert torch.equal(y.cpu(), torch.zeros(3, 17, 17, dtype=dtype))
