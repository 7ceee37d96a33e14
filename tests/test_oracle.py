"""Pins the CPU oracle independently of its own formulas.

Iteration: the reference's property tests (tests/orthogonalize/test_newton_schulz.py
and test_polar_express.py: orthogonality, SVD closeness, steps=0, manual one-step
expansion, transpose symmetry, zero / rank-1, orthogonal fixed point, scale invariance,
batched == unbatched), plus fp32 vs fp64 agreement and the two bf16 storage schemes
against fp64. Update rules: the closed-form answers of the reference's tests.
Quantizers: brute-force nearest code, map structure, round-trip bounds, torch's fp8
cast.
"""

import json
import math
import os

import numpy as np
import pytest
import torch

from helpers import rel_fro
from oracle import muon_ref as R
from oracle import quant_ref as Q

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _orth_gram(x):
    return x @ x.T if x.size(-2) <= x.size(-1) else x.T @ x


# ---- iteration ----------------------------------------------------------------------------


def _spectrum_input(shape, smin, seed=0):
    """U diag(s) V^T with s log-spaced in [smin, 1]: a seed-independent condition."""
    gen = torch.Generator().manual_seed(seed)
    m, n = shape
    k = min(m, n)
    u, _ = torch.linalg.qr(torch.randn(m, k, generator=gen))
    v, _ = torch.linalg.qr(torch.randn(n, k, generator=gen))
    s = torch.logspace(math.log10(smin), 0, k)
    return (u * s) @ v.T


@pytest.mark.parametrize("shape", [(64, 32), (32, 64), (48, 48)])
@pytest.mark.parametrize("loop,atol,sv", [(R.ns_loop, 0.45, 0.35), (R.pe_loop, 0.16, 0.16)])
def test_output_is_approximately_orthogonal(shape, loop, atol, sv):
    # The reference's bounds (0.45 / 0.35 NS, 0.13 / 0.16 PE) are tuned to its own
    # Gaussian draw; a fixed log-spaced spectrum keeps the check independent of the
    # torch RNG stream (PE's Gram bound widened to 0.16 for it).
    X = _spectrum_input(shape, smin=0.2).bfloat16()
    out = loop(X, 5).float()
    torch.testing.assert_close(_orth_gram(out), torch.eye(min(shape)), rtol=0.0, atol=atol)
    assert (torch.linalg.svdvals(out) - 1).abs().max() < sv


@pytest.mark.parametrize("loop,prescale,eps", [(R.ns_loop, 1.0, 1e-7), (R.pe_loop, 1.02, 1e-6)])
def test_steps_zero_returns_prescaled_input(loop, prescale, eps):
    torch.manual_seed(0)
    X = torch.randn(64, 32, dtype=torch.bfloat16)
    expected = X / (X.norm(dim=(-2, -1), keepdim=True) * prescale + eps)
    assert torch.equal(loop(X, 0), expected)


@pytest.mark.parametrize("loop,atol", [(R.ns_loop, 0.12), (R.pe_loop, 0.05)])
def test_approximates_matrix_sign(loop, atol):
    torch.manual_seed(1)
    X = torch.randn(64, 32, dtype=torch.bfloat16)
    u, _, vh = torch.linalg.svd(X.float(), full_matrices=False)
    torch.testing.assert_close(loop(X, 5).float(), u @ vh, rtol=0, atol=atol)


def test_coefficient_overrides_match_manual_expansion():
    torch.manual_seed(3)
    X = torch.randn(16, 8)
    a, b, c = 2.0, -1.5, 0.25
    n = X / (X.norm() + 1e-7)
    G = n @ n.T
    expected = n * a + (G * b + (G @ G) * c) @ n
    torch.testing.assert_close(R.ns_loop(X, 1, a=a, b=b, c=c), expected, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("loop", [R.ns_loop, R.pe_loop])
def test_transpose_symmetry_zero_and_rank1(loop):
    torch.manual_seed(2)
    X = torch.randn(64, 32, dtype=torch.bfloat16)
    assert torch.equal(loop(X, 5), loop(X.T.contiguous(), 5).T)
    z = torch.zeros(32, 16, dtype=torch.bfloat16)
    assert torch.count_nonzero(loop(z, 5)) == 0
    torch.manual_seed(4)
    r1 = torch.outer(torch.randn(32), torch.randn(16)).bfloat16()
    assert torch.isfinite(loop(r1, 5)).all()


@pytest.mark.parametrize("loop,tol", [(R.ns_loop, 0.03), (R.pe_loop, 0.07)])
def test_orthogonal_input_is_near_fixed_point(loop, tol):
    torch.manual_seed(5)
    q, _ = torch.linalg.qr(torch.randn(64, 32))
    torch.testing.assert_close(loop(q.bfloat16(), 5).float(), q, rtol=0, atol=tol)


@pytest.mark.parametrize("loop,tol", [(R.ns_loop, 0.05), (R.pe_loop, 0.06)])
def test_scale_invariance_and_batching(loop, tol):
    torch.manual_seed(6)
    Y = torch.randn(32, 16, dtype=torch.bfloat16)
    base = loop(Y, 5).float()
    for s in (1e-2, 1e2, 1e4):
        torch.testing.assert_close(loop((Y.float() * s).bfloat16(), 5).float(), base, rtol=0,
                                   atol=tol)
    assert torch.equal(loop(Y.unsqueeze(0), 5)[0], loop(Y, 5))


def test_polar_express_coefficient_table():
    assert len(R.POLAR_EXPRESS_COEFFS) == 5
    assert R.POLAR_EXPRESS_COEFFS[0] == (8.156554524902461, -22.48329292557795, 15.878769915207462)


@pytest.mark.parametrize("strategy", ["polar_express", "newton_schulz"])
@pytest.mark.parametrize("shape", [(256, 128), (3, 130, 70), (2, 512, 512)])
def test_precision_ladder(strategy, shape):
    """fp32 iteration within 1e-5 of fp64; the HIP ("fused") bf16 storage scheme within
    2e-2 of fp64 and tighter than the reference's compiled-Triton scheme, which is in
    turn tighter than the eager bf16 iteration."""
    X = torch.randn(*shape, generator=torch.Generator().manual_seed(0))
    coeffs, prescale = R.strategy_coeffs(strategy, 5)
    u64 = R.polar_iteration(X.bfloat16().double(), coeffs, prescale=prescale, eps=1e-7)
    u32 = R.polar_iteration(X.bfloat16().float(), coeffs, prescale=prescale, eps=1e-7)
    fused = R.polar_iteration_bf16(X, coeffs, prescale=prescale, eps=1e-7)
    triton = R.polar_iteration_bf16(X, coeffs, prescale=prescale, eps=1e-7, rounding="triton")
    eager = R.polar_iteration(X.bfloat16(), coeffs, prescale=prescale, eps=1e-7)
    # square Gaussian inputs carry tiny singular values that the first Polar Express
    # step amplifies: the fp32 iteration itself lands ~1.3e-5 from fp64 there
    square = shape[-1] == shape[-2]
    assert rel_fro(u32, u64) < (3e-5 if square else 1e-5)
    assert rel_fro(fused, u64) < 2e-2
    assert rel_fro(fused, u64) < rel_fro(triton, u64) < rel_fro(eager, u64)


def test_bf16_schemes_reduce_to_exact_iteration_structure():
    """With a diagonal input every product is elementwise, so each scheme must equal
    the scalar polynomial recursion on the singular values (rounded per scheme)."""
    d = torch.tensor([3.0, 1.0, 0.5, 0.25])
    X = torch.diag(d)
    coeffs, prescale = R.strategy_coeffs("polar_express", 5)
    s = d / (d.norm() * prescale + 1e-7)
    for a, b, c in coeffs:
        s = a * s + (b * s**2 + c * s**4) * s
    out = R.polar_iteration(X.double(), coeffs, prescale=prescale, eps=1e-7)
    torch.testing.assert_close(torch.diagonal(out).float(), s, rtol=1e-5, atol=1e-6)
    fused = R.polar_iteration_bf16(X, coeffs, prescale=prescale, eps=1e-7)
    torch.testing.assert_close(torch.diagonal(fused).float(), s, rtol=2e-2, atol=1e-2)


def test_gram_is_library_matmul():
    x = torch.randn(3, 7, 5)
    torch.testing.assert_close(R.gram(x), torch.einsum("bik,bjk->bij", x, x))


# ---- update rules (closed forms of the reference tests) -------------------------------------

_ID = dict(orth_single=lambda g: g)


def _upd(p, g, buf=None, **kw):
    buf = torch.zeros_like(g) if buf is None else buf
    base = dict(lr=0.1, weight_decay=0.0, cautious_wd=True, momentum=0.0, nesterov=False,
                maximize=False)
    base.update(kw)
    return R.muon_update(p, g, buf, R.lr_ratio(g.shape), **base, **_ID)


def test_update_lr_ratio_known_answer():
    p = torch.ones(4, 2)
    new_p, buf, _, _ = _upd(p, torch.full((4, 2), 0.5))
    assert R.lr_ratio((4, 2)) == float(torch.tensor(math.sqrt(2.0)))
    torch.testing.assert_close(buf, torch.full((4, 2), 0.5))
    torch.testing.assert_close(new_p, torch.ones(4, 2) - math.sqrt(2.0) * 0.1 * 0.5)


def test_update_nesterov_known_answer():
    new_p, _, _, _ = _upd(torch.ones(2, 2), torch.full((2, 2), 0.5), momentum=0.5, nesterov=True)
    torch.testing.assert_close(new_p, torch.ones(2, 2) - 0.1 * 0.75)


@pytest.mark.parametrize("cautious,expected", [(True, [[-1.0, -2.0], [2.0, 1.0]]),
                                                (False, [[-1.0, -1.0], [1.0, 1.0]])])
def test_update_weight_decay_known_answers(cautious, expected):
    p = torch.tensor([[1.0, -1.0], [1.0, -1.0]])
    g = torch.tensor([[1.0, 1.0], [-1.0, -1.0]])
    new_p, _, _, _ = _upd(p, g, lr=1.0, weight_decay=1.0, cautious_wd=cautious)
    torch.testing.assert_close(new_p, torch.tensor(expected))


def test_update_maximize_known_answer():
    new_p, _, _, _ = _upd(torch.ones(2, 2), torch.full((2, 2), 0.5), maximize=True)
    torch.testing.assert_close(new_p, torch.full((2, 2), 1.05))


def test_transform_grad_shapes():
    g = torch.ones(2, 2, 2, 2)
    assert R.transform_grad(g, True).shape == (2, 8)
    assert R.transform_grad(g, False).shape == (4, 2, 2)
    assert R.transform_grad(torch.ones(2, 4, 2), False).shape == (2, 4, 2)


def test_split_orthogonalize_known_answer():
    g = torch.randn(6, 4, generator=torch.Generator().manual_seed(3))
    u = R.split_orthogonalize(g, (2, 4), ns_steps=5, strategy="polar_express",
                              orth=lambda gs: [x / x.norm() for x in gs])
    scales = R.split_lr_scales((6, 4), (2, 4))
    expected = torch.cat([s * b / b.norm() for b, s in zip(g.split([2, 4]), scales)])
    torch.testing.assert_close(u, expected)
    full = math.sqrt(6 / 4)
    assert scales == pytest.approx((1.0 / full, 1.0 / full))


def test_normuon_invariants():
    """NorMuon's normalization pinned by what the method fixes, not by its formula:
    the Frobenius norm of u is preserved; from v = 0 every row ends with the same norm
    (the division by sqrt of the row mean square equalizes them), i.e. ||u||_F /
    sqrt(rows); v' = (1 - beta2) * mean_j u_ij^2 from v = 0; a v that already equals the
    row mean squares is a fixed point of the EMA and then leaves u's direction
    row-scaled only; with split_sizes the same holds per row block."""
    gen = torch.Generator().manual_seed(0)
    # rows with very different scales, so equal row norms are not an accident
    u = torch.randn(6, 5, generator=gen, dtype=torch.float64) * torch.tensor(
        [[0.1], [0.3], [1.0], [3.0], [10.0], [100.0]], dtype=torch.float64)
    rows, cols = u.shape
    un, vn = R.normuon_normalize(u, torch.zeros(rows, 1, dtype=torch.float64), 0.9)
    torch.testing.assert_close(un.norm(), u.norm(), rtol=1e-12, atol=0)
    torch.testing.assert_close(un.norm(dim=1), torch.full((rows,), u.norm().item() / rows**0.5,
                                                          dtype=torch.float64), rtol=1e-5, atol=0)
    ms = torch.tensor([[(u[i] ** 2).sum().item() / cols] for i in range(rows)], dtype=torch.float64)
    torch.testing.assert_close(vn, 0.1 * ms, rtol=1e-12, atol=0)
    # fixed point of the EMA: v' = v; u is only row-scaled, by 1 / (sqrt(v_i) + 1e-8)
    un2, vn2 = R.normuon_normalize(u, ms.clone(), 0.5)
    torch.testing.assert_close(vn2, ms, rtol=1e-12, atol=0)
    ratio = un2 / u
    torch.testing.assert_close(ratio, ratio[:, :1].expand_as(ratio), rtol=1e-10, atol=0)
    # per row block with split_sizes
    ub, vb = R.normuon_normalize(u, torch.zeros(rows, 1, dtype=torch.float64), 0.9,
                                 split_sizes=(2, 4))
    for lo, hi in ((0, 2), (2, 6)):
        blk = u[lo:hi]
        torch.testing.assert_close(ub[lo:hi].norm(), blk.norm(), rtol=1e-12, atol=0)
        torch.testing.assert_close(
            ub[lo:hi].norm(dim=1),
            torch.full((hi - lo,), blk.norm().item() / (hi - lo) ** 0.5, dtype=torch.float64),
            rtol=1e-5, atol=0)
    torch.testing.assert_close(vb, vn, rtol=1e-12, atol=0)


def test_normuon_update_known_answer():
    """NorMuon.update (normuon.py:74-134) on a 3 x 2 case with an identity orthogonalizer,
    numbers worked by hand. Order fixed by the reference: normalize u, then cautious wd on
    the normalized u (mask u * p > 0), then p - lr * lr_ratio * u.

    g rows (0.6, 0.8), (3, -4), (7, 0) have norms 1, 5, 7 (||g||_F = sqrt(75)). With
    momentum 0.5, no Nesterov and a zero buffer, u = buf' = g. beta2 = 0.75 from v = 0:
    v' = 0.25 * (row mean of u^2) = r^2 / 8 = (0.125, 3.125, 6.125). Dividing by sqrt(v')
    gives every row norm 2 sqrt(2); rescaling to ||g||_F gives every row norm
    sqrt(75 / 3) = 5: u_n = (3, 4), (3, -4), (5, 0). With p = (1, -1), (-1, 1), (2, 2)
    the mask u_n * p > 0 keeps (0, 0) and (2, 0) only: u = (3.1, 4), (3, -4), (5.2, 0);
    lr_ratio = sqrt(3 / 2), lr 0.1."""
    g = torch.tensor([[0.6, 0.8], [3.0, -4.0], [7.0, 0.0]])
    p = torch.tensor([[1.0, -1.0], [-1.0, 1.0], [2.0, 2.0]])
    hp = dict(lr=0.1, weight_decay=0.1, cautious_wd=True, momentum=0.5, nesterov=False,
              maximize=False, beta2=0.75)
    new_p, new_buf, v_new, u = R.normuon_update(
        p, g, torch.zeros(3, 2), torch.zeros(3, 1), R.lr_ratio((3, 2)), **hp, **_ID)
    u_expected = torch.tensor([[3.1, 4.0], [3.0, -4.0], [5.2, 0.0]])
    torch.testing.assert_close(u, u_expected, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(v_new, torch.tensor([[0.125], [3.125], [6.125]]), rtol=1e-7, atol=0)
    torch.testing.assert_close(new_buf, g, rtol=0, atol=0)
    p_expected = p - 0.1 * math.sqrt(1.5) * u_expected
    torch.testing.assert_close(new_p, p_expected, rtol=1e-6, atol=1e-6)
    # the other composition order (wd on the raw update, then normalize) lands elsewhere
    raw = g + 0.1 * p * (g * p > 0)
    wrong, _ = R.normuon_normalize(raw, torch.zeros(3, 1), 0.75)
    assert (wrong - u_expected).abs().max() > 1e-2


def _lp_case(fmt):
    qmap = {"8bit": Q.qmap_8bit(), "4bit": Q.qmap_4bit(), "fp8": None}[fmt]
    block = 4
    # c and c / 3 in one block: c / 3 divided by the block scale c is 1/3, which no map
    # entry and no e4m3 value holds, so requantization is lossy there
    c = np.float32(1.5)
    g = np.array([c, c / np.float32(3.0), -0.25, 0.0625, c / np.float32(3.0), -c, 0.75, 0.1],
                 dtype=np.float32)
    ncodes = g.size // 2 if fmt == "4bit" else g.size
    codes0 = np.zeros(ncodes, np.uint8)     # torchao zeros(): codes 0, scales 0 -> m = 0
    scales0 = np.zeros(g.size // block, np.float32)
    return qmap, block, g, codes0, scales0


def _lookup(codes, fmt, qmap):
    """Code -> value by the format's definition, independently of quant_ref.dequantize."""
    if fmt == "fp8":
        return torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    if fmt == "4bit":
        codes = np.stack([codes >> 4, codes & 0xF], axis=-1).reshape(-1)
    return np.array([qmap[int(k)] for k in codes], np.float32)


@pytest.mark.parametrize("fmt", ["8bit", "4bit", "fp8"])
def test_lp_momentum_step_known_answer(fmt):
    """MuonLP's momentum on a quantized buffer (muon.py:45-56 through the quantized
    state): m = dequant(state); m' = m mu + g; the state stores quant(m'); Nesterov's g'
    is built from the unquantized fp32 m'; the next step starts from dequant(quant(m')).
    Expected values are worked out here by hand and by brute-force nearest code, not by
    calling quant_ref.quantize / dequantize."""
    qmap, block, g, codes0, scales0 = _lp_case(fmt)
    mu = 0.9
    c1, s1, gq = Q.lp_momentum_step(codes0, scales0, g, block=block, fmt=fmt, qmap=qmap,
                                    momentum=mu, nesterov=True, maximize=False)
    # from m = 0, m' = g exactly; g' = g + mu g, in fp32
    m1 = g
    expect_gq = (g + (m1 * np.float32(mu)).astype(np.float32)).astype(np.float32)
    assert np.array_equal(gq, expect_gq)
    # block scales: absmax (divided by 448 for fp8)
    amax = np.abs(m1.reshape(-1, block)).max(1).astype(np.float32)
    assert np.array_equal(s1, amax / np.float32(448.0) if fmt == "fp8" else amax)
    # codes: the nearest representable value of m' / scale, ties up (brute force)
    y = (m1.reshape(-1, block) / s1[:, None]).astype(np.float32).reshape(-1)
    if fmt == "fp8":
        expect_vals = torch.from_numpy(y.copy()).to(torch.float8_e4m3fn).float().numpy()
    else:
        d = np.abs(qmap[None, :].astype(np.float64) - y[:, None].astype(np.float64))
        best = d.min(1, keepdims=True)
        expect_vals = np.array([qmap[np.nonzero(row == b)[0].max()] for row, b in zip(d, best[:, 0])],
                               np.float32)
    assert np.array_equal(_lookup(c1, fmt, qmap), expect_vals)
    # the stored momentum is lossy at c / 3: a g' built from it would differ from the
    # one above, so the test tells the two Nesterov inputs apart
    stored = (_lookup(c1, fmt, qmap).reshape(-1, block) * s1[:, None]).astype(np.float32).reshape(-1)
    assert stored[1] != m1[1]
    wrong_gq = (g + (stored * np.float32(mu)).astype(np.float32)).astype(np.float32)
    assert not np.array_equal(gq, wrong_gq)
    # step 2 starts from the dequantized state: with g = 0 and no Nesterov, g' = m mu
    _, _, gq2 = Q.lp_momentum_step(c1, s1, np.zeros_like(g), block=block, fmt=fmt, qmap=qmap,
                                   momentum=mu, nesterov=False, maximize=False)
    assert np.array_equal(gq2, ((stored * np.float32(mu)).astype(np.float32) + np.float32(0)).astype(np.float32))
    assert not np.array_equal(gq2, (m1 * np.float32(mu)).astype(np.float32))


# ---- quantizers -----------------------------------------------------------------------------


@pytest.mark.parametrize("signed", [True, False])
def test_dynamic_map_structure(signed):
    q = Q.qmap_8bit(signed)
    assert q.shape == (256,) and q.dtype == np.float32
    assert np.all(np.diff(q) >= 0) and q[-1] == 1.0 and 0.0 in q
    if signed:
        pos = q[q > 0][:-1]  # all positives except the appended 1.0
        assert np.array_equal(np.sort(-q[q < 0]), pos)
        assert q.min() == -q[-2]
    # ten-fold magnitude ladder: smallest positive entry is 1e-6 * midpoint of [0.1, ...]
    assert abs(q[q > 0].min() - 1e-6 * 0.55) < 1e-9 if signed else True
    q4 = Q.qmap_4bit(True)
    assert q4.shape == (16,) and np.all(np.diff(q4) > 0) and q4[-1] == 1.0 and 0.0 in q4


@pytest.mark.parametrize("fmt", ["8bit", "4bit"])
def test_codes_are_nearest_with_ties_up(fmt):
    qmap = Q.qmap_8bit() if fmt == "8bit" else Q.qmap_4bit()
    rng = np.random.default_rng(0)
    y = np.concatenate([rng.uniform(-1, 1, 20000).astype(np.float32),
                        ((qmap[:-1] + qmap[1:]) * np.float32(0.5)).astype(np.float32), qmap])
    codes = Q.quantize_codes(y, qmap).astype(np.int64)
    dist = np.abs(y[:, None].astype(np.float64) - qmap[None, :].astype(np.float64))
    best = dist.min(axis=1)
    got = dist[np.arange(y.size), codes]
    # the chosen entry is a nearest one (fp32 midpoint arithmetic may tie-break either
    # way within one fp32 ulp of the exact midpoint)
    assert np.all(got <= best + 1e-7)
    # exact midpoints go up
    mids = ((qmap[:-1] + qmap[1:]) * np.float32(0.5)).astype(np.float32)
    mcodes = Q.quantize_codes(mids, qmap).astype(np.int64)
    ok_up = mcodes == np.arange(1, len(qmap))
    half = ((qmap[1:] - qmap[:-1]) * np.float32(0.5)).astype(np.float32)
    res = (mids - qmap[:-1]).astype(np.float32)
    assert np.all(ok_up == (res >= half))


@pytest.mark.parametrize("fmt,block", [("8bit", 256), ("4bit", 128), ("fp8", 256), ("8bit", 2048)])
def test_quantize_round_trip_bounds(fmt, block):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(8192) * np.exp(rng.standard_normal(8192 // block).repeat(block))).astype(np.float32)
    qmap = Q.qmap_8bit() if fmt == "8bit" else (Q.qmap_4bit() if fmt == "4bit" else None)
    codes, scale = Q.quantize(x, block, fmt, qmap)
    assert np.allclose(scale, np.maximum(np.abs(x.reshape(-1, block)).max(1) / (448 if fmt == "fp8" else 1), 1e-12 / (448 if fmt == "fp8" else 1)), rtol=1e-7)
    y = Q.dequantize(codes, scale, block, fmt, qmap)
    err = np.abs(y - x).reshape(-1, block) / scale[:, None]
    if fmt == "fp8":
        # relative spacing of e4m3 normals is 2^-3: half-ulp bound relative to the value
        assert np.all(np.abs(y - x) <= np.abs(x) * 2**-4 + scale.repeat(block) * 2**-10)
    else:
        gaps = np.diff(qmap).max()
        assert err.max() <= gaps / 2 + 1e-6
    # the block absmax element is reproduced exactly (it maps to +-1 or 448)
    if fmt != "4bit":
        idx = np.abs(x.reshape(-1, block)).argmax(1)
        xm = x.reshape(-1, block)[np.arange(x.size // block), idx]
        ym = y.reshape(-1, block)[np.arange(x.size // block), idx]
        pos = xm > 0
        assert np.allclose(ym[pos], xm[pos], rtol=1e-6)


def test_four_bit_packing_high_nibble_first():
    qmap = Q.qmap_4bit()
    x = np.array([1.0, -1.0] * 64, dtype=np.float32)
    codes, scale = Q.quantize(x, 128, "4bit", qmap)
    assert codes.size == 64 and np.all(codes == (15 << 4 | 0))
    assert np.array_equal(Q.dequantize(codes, scale, 128, "4bit", qmap)[:2],
                          np.array([1.0, qmap[0]], np.float32))


def test_fp8_matches_torch_cast():
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = np.concatenate([x[np.isfinite(x)], np.linspace(-470, 470, 100001, dtype=np.float32),
                        np.array([464.0, -464.0, 448.0, 2**-9, 2**-10, 3 * 2**-11], np.float32)])
    with np.errstate(invalid="ignore"):
        mine = Q.f32_to_e4m3fn(x)
    ref = torch.from_numpy(x.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    both_nan = ((mine & 0x7F) == 0x7F) & ((ref & 0x7F) == 0x7F)
    assert np.all((mine == ref) | both_nan)
    back = Q.e4m3fn_to_f32(ref)
    tb = torch.from_numpy(ref.copy()).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(back), np.isnan(tb))
    assert np.array_equal(back[~np.isnan(back)], tb[~np.isnan(tb)])


def test_golden_fixtures_reproduce():
    """Committed vectors (tests/golden/make_golden.py) still come out of the oracle."""
    with open(os.path.join(GOLDEN, "known_answers.json")) as f:
        known = json.load(f)
    for case in known["updates"]:
        p = torch.tensor(case["param"])
        g = torch.tensor(case["grad"])
        new_p, _, _, _ = _upd(p, g, **case["hp"])
        torch.testing.assert_close(new_p, torch.tensor(case["expected"]), rtol=0, atol=1e-7)
    data = np.load(os.path.join(GOLDEN, "vectors.npz"))
    assert np.array_equal(Q.qmap_8bit(), data["qmap8"])
    assert np.array_equal(Q.qmap_4bit(), data["qmap4"])
    for fmt in ("8bit", "4bit", "fp8"):
        qmap = {"8bit": Q.qmap_8bit(), "4bit": Q.qmap_4bit(), "fp8": None}[fmt]
        codes, scale = Q.quantize(data["lp_x"], 256, fmt, qmap)
        assert np.array_equal(codes, data[f"codes_{fmt}"])
        assert np.array_equal(scale, data[f"scale_{fmt}"])
    X = torch.from_numpy(data["orth_x"])
    for strat in ("polar_express", "newton_schulz"):
        coeffs, prescale = R.strategy_coeffs(strat, 5)
        u = R.polar_iteration_bf16(X, coeffs, prescale=prescale, eps=1e-7).float().numpy()
        assert np.array_equal(u, data[f"orth_{strat}"])
