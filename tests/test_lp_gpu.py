"""Quantized momentum (MuonLP) on the HIP path vs the quantizer oracle.

Codes and scales must be bit-exact given identical fp32 inputs (standalone quantize,
and through the fused dequant -> momentum -> requant pre-pass); dequantization is
exact; the full MuonLP step matches the oracle's arithmetic given the same U.
"""

import ctypes
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
# tall and wide workspace paths; at most 64 rows on the short side: the 64-row iterate
@pytest.mark.parametrize("shape", [(128, 96), (96, 128), (512, 48), (48, 512)])
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



def _rel(a, b):
    return float((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-30))


TILED = [("8bit", OptimState8bit, 256), ("4bit", OptimState4bit, 128), ("fp8", OptimStateFp8, 256),
         ("8bit", OptimState8bit, 64)]
TILED_SHAPES = [(512, 256), (256, 768), (300, 256), (2, 256, 512), (4, 96, 512)]


# wide rows of a multiple of 2048 values: the row-segment kernel serves these blocks too
TILED_SHAPES += [(128, 2048), (40, 4096), (3, 96, 2048)]


@pytest.mark.parametrize("fmt,cls,block", TILED)
@pytest.mark.parametrize("shape", TILED_SHAPES)
@pytest.mark.parametrize("gdtype", [torch.float32, torch.bfloat16])
def test_lp_tiled_prepass_outputs_exact(fmt, cls, block, shape, gdtype):
    """Shapes whose column count is a multiple of 256 take the one-pass tiled prepass
    (wide ones with rows of a multiple of 2048: the row-segment kernel),
    which writes X straight into the iteration's wide buffer X0 (transposed through LDS
    for tall matrices, zero padding included) and the norm partials. Called through
    the C ABI: codes and scales bit-exact against the quantizer oracle, X0 equal to
    bf16(g') in the wide layout, the partials summing to sum(x^2)."""
    _check_tiled_prepass(fmt, cls, block, shape, gdtype)


@pytest.mark.parametrize("fmt,cls,block", [("8bit", OptimState8bit, 256), ("4bit", OptimState4bit, 128),
                                           ("fp8", OptimStateFp8, 256), ("8bit", OptimState8bit, 2048),
                                           ("fp8", OptimStateFp8, 2048)])
@pytest.mark.parametrize("shape", [(256, 512), (64, 2048)])
def test_lp_extreme_values_exact(fmt, cls, block, shape):
    """Blocks at the edges of fp32 through the tiled pre-pass (one-pass and deferred
    scales): a 1e38 absmax (a scale above 2^125, whose reciprocal is subnormal); values of
    1e-35 and subnormals beside an absmax of 1; a block clipped at 1e-12 holding 1e-31;
    signed zeros and all-zero blocks. Codes and scales bit-exact against the oracle's IEEE
    quotients, X0 equal to bf16(g'). 512 columns: the tile kernel (and deferred scales at
    2048); 2048 columns: the row-segment kernel. (The norm partials of values near 1e38
    overflow fp32; not checked.)"""
    rows, cols = shape
    gen = torch.Generator().manual_seed(17)
    g = torch.randn(rows, cols, generator=gen)
    special = [
        [1e38, -3e37, 1e30, 1.0, 1e-10, -2.5e36],
        [1.0, 1e-35, -2e-38, 3e-39, -1e-40, 1e-45, 0.0, -0.0],
        [1e-20, 1e-40, -1e-25, 0.0],
        [5e-31, -1e-31, 7e-31, 8e-31, 1e-32],
        [0.0, -0.0],
    ]
    for r, vals in enumerate(special):
        row = torch.tensor(vals, dtype=torch.float32)
        reps = -(-cols // len(vals))
        g[2 * r] = row.repeat(reps)[:cols] * (torch.rand(cols, generator=gen) < 0.97)
        g[2 * r + 1] = row.flip(0).repeat(reps)[:cols]
    g[10, 300:] = 0.0
    _check_tiled_prepass(fmt, cls, block, shape, torch.float32, g=g, check_partials=False)


# blocks of more than 256 values: the reference's default 2048 (optim_lp.py:49), other
# multiples of 256, and one block per tensor (an fp8 per-tensor scale)
DEFERRED = [("8bit", OptimState8bit, 2048), ("4bit", OptimState4bit, 2048),
            ("fp8", OptimStateFp8, 2048), ("8bit", OptimState8bit, 512),
            ("4bit", OptimState4bit, 768), ("fp8", OptimStateFp8, "numel"),
            ("8bit", OptimState8bit, "numel")]
DEFERRED_SHAPES = [(512, 256), (256, 768), (2048, 256), (2, 256, 512), (4, 96, 512)]


@pytest.mark.parametrize("fmt,cls,block", DEFERRED)
@pytest.mark.parametrize("shape", DEFERRED_SHAPES)
@pytest.mark.parametrize("gdtype", [torch.float32, torch.bfloat16])
def test_lp_deferred_scale_prepass_outputs_exact(fmt, cls, block, shape, gdtype):
    """Blocks larger than a tile row (multiples of 256, up to the whole tensor) take the
    tiled pass with the scale deferred: absmax partials per 256 values, a per-block
    reduction, and a requant pass that recomputes the same momentum. Codes, scales, X0
    and the norm partials exactly as for the one-pass blocks, wide and tall."""
    numel = math.prod(shape)
    block = numel if block == "numel" else block
    if numel % block:
        pytest.skip(f"{numel} values do not split into blocks of {block}")
    _check_tiled_prepass(fmt, cls, block, shape, gdtype)


ROWSEG = [("8bit", OptimState8bit), ("4bit", OptimState4bit), ("fp8", OptimStateFp8)]
ROWSEG_CASES = [(2048, (128, 2048)), (2048, (3000, 2048)), (2048, (192, 4096)), (512, (1024, 512)),
                (1024, (200, 1024)), (8192, (64, 8192)), (2048, (2, 256, 2048)), (2048, (4096, 6144)),
                (512, (256, 2048)), (1024, (2560, 2048)), (512, (2100, 2048)), (2048, (64, 4096)),
                (1024, (3, 40, 6144))]


@pytest.mark.parametrize("fmt,cls", ROWSEG)
@pytest.mark.parametrize("block,shape", ROWSEG_CASES)
@pytest.mark.parametrize("gdtype", [torch.float32, torch.bfloat16])
def test_lp_row_segment_blocks_exact(fmt, cls, block, shape, gdtype):
    """Blocks of 512 to 8192 values whose width divides the column count (the reference's
    default 2048 on every Llama shape: each block a whole row segment). Blocks of 512-2048
    in rows of a multiple of 2048 take the one-pass row-segment kernel (wide, and tall
    through its LDS transpose: 2100, 2560 and 3000 rows, partial row groups included),
    the others the deferred-scale path. Codes, scales, X0 and the norm partials exactly as
    the oracle, stacked, 64-row and shorter iterates, two steps."""
    _check_tiled_prepass(fmt, cls, block, shape, gdtype)


@pytest.mark.parametrize("fmt,cls,block,shape", [
    ("8bit", OptimState8bit, 2048, (256, 768)), ("4bit", OptimState4bit, 2048, (768, 256)),
    ("fp8", OptimStateFp8, 2048, (256, 768)), ("fp8", OptimStateFp8, "numel", (768, 256)),
    ("8bit", OptimState8bit, 256, (768, 256)), ("8bit", OptimState8bit, 2048, (256, 2048)),
    ("4bit", OptimState4bit, 1024, (128, 4096))])
def test_lp_prepass_bucket_spanning_two_chunks(fmt, cls, block, shape):
    """A foreach bucket of 34 same-shape tensors in one muon_lp_prepass call: more than
    MUON_MAX_TENSORS (32), so the library launches two chunks (32 + 2), each with its own
    per-tensor block-max slots, old-scale slots and requant grid on the deferred-scale path
    (blocks of 2048 and one per tensor), and its own tensor table on the row-segment path
    (rows of 2048 and 4096). Every tensor's codes, scales and X0 bit-exact against the
    oracle over two steps, wide and tall."""
    from muonium_amd import _lib

    lib = _lib.load()
    dev = torch.device(DEV)
    _lib.ensure_device(dev)
    nt = 34
    rows, cols = shape
    numel = rows * cols
    block = numel if block == "numel" else block
    gen = torch.Generator().manual_seed(21)
    # per-tensor scales spread over 2^-20 .. 2^20, so a tensor's codes depend on using its
    # own block maxima, and per-row log-normal scales inside each tensor
    gs = [(torch.randn(shape, generator=gen) * torch.exp(torch.randn(rows, 1, generator=gen))
           * 2.0 ** (t * 40 / (nt - 1) - 20)).bfloat16() for t in range(nt)]
    sts = [_state(cls, shape, block) for _ in range(nt)]
    ref = [(np.zeros(st.codes.numel(), np.uint8), np.zeros(st.scale.numel(), np.float32))
           for st in sts]
    nbytes = lib.muon_orth_workspace_bytes(_lib.DT_BF16, nt, rows, cols)
    ws = torch.full((nbytes,), 0x7F, dtype=torch.uint8, device=dev)
    gds = [g.to(dev) for g in gs]
    qmap = sts[0].qmap
    for step in range(2):
        rc = lib.muon_lp_prepass(nt, _lib.ptr_array(gds), _lib.DT_BF16,
                                 _lib.ptr_array([st.codes for st in sts]),
                                 _lib.ptr_array([st.scale for st in sts]),
                                 qmap.data_ptr() if qmap is not None else None, sts[0].qformat,
                                 block, 1, rows, cols, 0.9, 1, 0, ws.data_ptr(), _lib.DT_BF16, nt,
                                 _lib.stream(dev))
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        gqs = []
        for t in range(nt):
            c, s, gq = quant_ref.lp_momentum_step(
                ref[t][0], ref[t][1], gs[t].float().numpy(), block=block, fmt=fmt,
                qmap=_qmap(fmt), momentum=0.9, nesterov=True, maximize=False)
            ref[t] = (c, s)
            gqs.append(gq)
            assert np.array_equal(sts[t].codes.cpu().numpy(), c), f"tensor {t} codes, step {step}"
            assert np.array_equal(sts[t].scale.cpu().numpy().view(np.uint32), s.view(np.uint32)), \
                f"tensor {t} scales, step {step}"
    m, n = min(rows, cols), max(rows, cols)
    mp, npad = -(-m // 256) * 256, -(-n // 256) * 256
    off0, pitch, mst = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    trans = ctypes.c_int()
    assert lib.muon_orth_result(_lib.DT_BF16, nt, rows, cols, 0, off0, pitch, mst, trans) == 0
    X0 = ws[: nt * mst.value * 2].view(torch.bfloat16).view(nt, mp, pitch.value)[:, :, :npad]
    X0 = X0.float().cpu()
    for t in range(nt):
        x = torch.from_numpy(gqs[t]).view(rows, cols).bfloat16().float()
        exp = torch.zeros(mp, npad)
        exp[:m, :n] = x.T if rows > cols else x
        assert torch.equal(X0[t], exp), f"tensor {t}: X0 differs"


def _check_tiled_prepass(fmt, cls, block, shape, gdtype, g=None, check_partials=True):
    from muonium_amd import _lib

    lib = _lib.load()
    dev = torch.device(DEV)
    _lib.ensure_device(dev)
    nb = 1
    for d in shape[:-2]:
        nb *= d
    rows, cols = shape[-2:]
    if g is None:
        gen = torch.Generator().manual_seed(5)
        g = torch.randn(shape, generator=gen) * torch.exp(torch.randn(*shape[:-1], 1, generator=gen))
    g = g.to(gdtype)
    st = _state(cls, shape, block)
    codes = np.zeros(st.codes.numel(), np.uint8)
    scales = np.zeros(st.scale.numel(), np.float32)
    nbytes = lib.muon_orth_workspace_bytes(_lib.DT_BF16, nb, rows, cols)
    ws = torch.full((nbytes,), 0x7F, dtype=torch.uint8, device=dev)  # garbage: padding must be rewritten
    gd = g.to(dev)
    for step in range(2):
        rc = lib.muon_lp_prepass(1, _lib.ptr_array([gd]), _lib.dtype_code(gdtype), _lib.ptr_array([st.codes]),
                                 _lib.ptr_array([st.scale]),
                                 st.qmap.data_ptr() if st.qmap is not None else None, st.qformat, block,
                                 nb, rows, cols, 0.9, 1, 0, ws.data_ptr(), _lib.DT_BF16, nb,
                                 _lib.stream(dev))
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        codes, scales, gq = quant_ref.lp_momentum_step(
            codes, scales, g.float().numpy(), block=block, fmt=fmt, qmap=_qmap(fmt), momentum=0.9,
            nesterov=True, maximize=False,
        )
        assert np.array_equal(st.codes.cpu().numpy(), codes), f"codes differ at step {step}"
        assert np.array_equal(st.scale.cpu().numpy().view(np.uint32), scales.view(np.uint32))
    m, n = min(rows, cols), max(rows, cols)
    # iterates of at most 64 rows pad their rows to 64 only (the short path)
    mp, npad = (64 if m <= 64 else -(-m // 256) * 256), -(-n // 256) * 256
    # X0 (the iterate before any step) in rows of `pitch` elements: the padding columns
    # up to n_pad are rewritten to zero, the rest of each row is never read
    off0, pitch, mst = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    trans = ctypes.c_int()
    assert lib.muon_orth_result(_lib.DT_BF16, nb, rows, cols, 0, off0, pitch, mst, trans) == 0
    assert off0.value == 0 and mst.value == mp * pitch.value and pitch.value >= npad
    X0 = ws[: nb * mst.value * 2].view(torch.bfloat16).view(nb, mp, pitch.value)[:, :, :npad]
    X0 = X0.float().cpu()
    exp = torch.zeros(nb, mp, npad)
    x = torch.from_numpy(gq).view(nb, rows, cols).bfloat16().float()
    exp[:, :m, :n] = x.transpose(1, 2) if rows > cols else x
    assert torch.equal(X0, exp)
    if not check_partials:
        return
    rup = lambda v: -(-v // 256) * 256
    off = 2 * rup(nb * mst.value * 2) + 2 * rup(nb * mp * mp * 2)
    parts = (mp // 64) * (npad // 64)
    P = ws[off: off + nb * parts * 4].view(torch.float32).view(nb, parts).double().cpu()
    want = (x.double() ** 2).sum(dim=(1, 2))
    torch.testing.assert_close(P.sum(dim=1), want, rtol=1e-6, atol=0)


@pytest.mark.parametrize("fmt,cls,block", TILED[:3] + [("8bit", OptimState8bit, 2048),
                                                      ("fp8", OptimStateFp8, 2048),
                                                      ("fp8", OptimStateFp8, None)])
@pytest.mark.parametrize("shape", [(512, 256), (256, 768)])
def test_lp_tiled_step_matches_oracle(fmt, cls, block, shape):
    """The full MuonLP step on a tiled shape: codes bit-exact; the update within the
    bf16 bar (1e-2 rel-Frobenius) of the fused-bf16 oracle iteration of the same g'.
    wd = 0 here: the cautious mask (U * p > 0) flips discontinuously on bf16-level
    differences in U, so the wd term is covered by the bit-exact small-shape test."""
    opt_cls = {"8bit": Muon8bit, "4bit": Muon4bit, "fp8": MuonFp8}[fmt]
    gen = torch.Generator().manual_seed(3)
    p0 = torch.randn(shape, generator=gen)
    p = nn.Parameter(p0.clone().to(DEV))
    opt = opt_cls([p], lr=0.05, wd=0.0, momentum=0.9, nesterov=True, block_size=block)
    codes = scales = None
    ref_p = p0.clone()
    coeffs, prescale = muon_ref.strategy_coeffs("polar_express", 5)
    for step in range(2):
        g = torch.randn(shape, generator=gen)
        p.grad = g.clone().to(DEV)
        opt.step()
        st = opt.state[p]["momentum_buffer"]
        assert isinstance(st, cls)
        if codes is None:
            codes = np.zeros(st.codes.numel(), np.uint8)
            scales = np.zeros(st.scale.numel(), np.float32)
        assert st.block_size == (block or math.prod(shape))  # None: one block per tensor
        codes, scales, gq = quant_ref.lp_momentum_step(
            codes, scales, g.numpy(), block=st.block_size, fmt=fmt, qmap=_qmap(fmt),
            momentum=0.9, nesterov=True, maximize=False,
        )
        assert np.array_equal(st.codes.cpu().numpy(), codes), f"codes differ at step {step}"
        assert np.array_equal(st.scale.cpu().numpy().view(np.uint32), scales.view(np.uint32))
        U = muon_ref.polar_iteration_bf16(torch.from_numpy(gq).view(shape), coeffs,
                                          prescale=prescale, eps=1e-7)
        adj = muon_ref.lr_ratio(shape) * 0.05
        got = p.detach().cpu()
        r = _rel(got - ref_p, -adj * U.float())
        assert r < 1e-2, f"step {step}: {r:.3e}"
        ref_p = got.clone()


def _same_scales(got, want):
    """Scales bit-exact where finite; NaN exactly where the oracle has NaN."""
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn)
    assert np.array_equal(got[~gn].view(np.uint32), want[~wn].view(np.uint32))


@pytest.mark.filterwarnings("ignore:invalid value encountered:RuntimeWarning")
@pytest.mark.parametrize("fmt,cls,block", TILED[:3])
@pytest.mark.parametrize("path", ["quantize", "general", "tiled-wide", "tiled-tall",
                                  "deferred-wide", "deferred-tall", "rowseg-wide", "rowseg-tall",
                                  "rowseg-small-blocks"])
def test_lp_nan_and_inf_blocks_match_oracle(fmt, cls, block, path):
    """A NaN in a block makes the block's scale NaN and codes every value of it as a NaN
    quotient (0 for the maps, 0x7f for fp8), as torch's amax / clamp do in the reference;
    an infinite value makes the scale infinite (its own quotient NaN, the others 0).
    Covered for the standalone quantizer, the general pre-pass (columns not a multiple
    of 256), the tiled pre-pass in both orientations and its deferred-scale form (blocks
    of 2048 across 256-column tiles), and the row-segment kernel (rows of a multiple of
    2048: blocks of 2048 wide and tall, and the one-pass blocks on a wide matrix), two steps
    each."""
    from muonium_amd import _lib

    shape = {"quantize": (64, 256), "general": (128, 96), "tiled-wide": (256, 768),
             "tiled-tall": (512, 256), "deferred-wide": (256, 768),
             "deferred-tall": (512, 256), "rowseg-wide": (64, 4096), "rowseg-tall": (2304, 2048),
             "rowseg-small-blocks": (64, 2048)}[path]
    if path.startswith("deferred") or path in ("rowseg-wide", "rowseg-tall"):
        block = 2048  # a block longer than a tile row
    gen = torch.Generator().manual_seed(9)
    g = torch.randn(shape, generator=gen)
    g[0, 5] = float("nan")
    g[7, 60] = float("inf")
    g[9, 1] = float("-inf")
    st = _state(cls, shape, block)
    if path == "quantize":
        st.copy_(g.to(DEV))
        codes, scales = quant_ref.quantize(g.numpy(), block, fmt, _qmap(fmt))
        assert np.array_equal(st.codes.cpu().numpy(), codes)
        _same_scales(st.scale.cpu().numpy(), scales)
        assert np.isnan(scales).sum() >= 1 and np.isinf(scales).sum() >= 2
        return
    lib = _lib.load()
    dev = torch.device(DEV)
    _lib.ensure_device(dev)
    rows, cols = shape
    codes = np.zeros(st.codes.numel(), np.uint8)
    scales = np.zeros(st.scale.numel(), np.float32)
    ws = torch.zeros(lib.muon_orth_workspace_bytes(_lib.DT_BF16, 1, rows, cols), dtype=torch.uint8,
                     device=dev)
    gd = g.to(dev)
    for step in range(2):
        rc = lib.muon_lp_prepass(1, _lib.ptr_array([gd]), _lib.DT_F32, _lib.ptr_array([st.codes]),
                                 _lib.ptr_array([st.scale]),
                                 st.qmap.data_ptr() if st.qmap is not None else None, st.qformat, block,
                                 1, rows, cols, 0.9, 1, 0, ws.data_ptr(), _lib.DT_BF16, 1,
                                 _lib.stream(dev))
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        codes, scales, _ = quant_ref.lp_momentum_step(
            codes, scales, g.numpy(), block=block, fmt=fmt, qmap=_qmap(fmt), momentum=0.9,
            nesterov=True, maximize=False,
        )
        assert np.array_equal(st.codes.cpu().numpy(), codes), f"codes differ at step {step}"
        _same_scales(st.scale.cpu().numpy(), scales)
    # every block holding a non-finite value has a NaN scale at the second step (an inf
    # block's own quotient inf / inf is NaN, so its momentum is NaN from then on)
    bad_blocks = {(r * cols + c) // block for r, c in ((0, 5), (7, 60), (9, 1))}
    assert np.isnan(scales).sum() == len(bad_blocks)


def test_fp8_codes_exact_at_every_rounding_boundary():
    """The fp8 quantizer codes y with the hardware e4m3 conversion; against the oracle's
    restatement of the format at every rounding decision: each midpoint between adjacent
    e4m3 values and 3 ulps either side, each grid point +-1 ulp, fp32 denormals, the 448
    edge, both signs, and 4M random values. Every block holds 448 (its absmax), so the
    block scale is exactly 1 and y = x."""
    grid = quant_ref.e4m3fn_to_f32(np.arange(0x7f, dtype=np.uint8))  # 0 .. 448
    vals = []
    u = lambda x: np.asarray(x, np.float32).view(np.uint32).astype(np.int64)
    f = lambda b: np.asarray(b, np.uint32).view(np.float32)
    mids = ((grid[:-1].astype(np.float64) + grid[1:]) / 2).astype(np.float32)
    for k in range(-3, 4):
        vals.append(f(np.maximum(u(mids) + k, 0)))
        vals.append(f(np.maximum(u(grid) + k // 3, 0)))
    vals.append(f(np.arange(0, 4096, dtype=np.uint32)))                    # fp32 denormals
    vals.append(np.array([448.0, np.nextafter(np.float32(448), np.float32(0))], np.float32))
    gen = np.random.default_rng(3)
    vals.append(gen.uniform(-448, 448, 4 << 20).astype(np.float32))
    x = np.concatenate([np.concatenate(vals[:-1]), -np.concatenate(vals[:-1]), vals[-1]])
    x = np.clip(x, -448, 448).astype(np.float32)
    block = 256
    per = block - 1
    nb = -(-x.size // per)
    xb = np.zeros((nb, block), np.float32)
    xb[:, 0] = 448.0
    flat = np.zeros(nb * per, np.float32)
    flat[: x.size] = x
    xb[:, 1:] = flat.reshape(nb, per)
    xt = torch.from_numpy(xb.reshape(-1))
    st = OptimStateFp8.zeros(xt.shape, block, DEV)
    st.copy_(xt.to(DEV))
    codes, scale = quant_ref.quantize(xb.reshape(-1), block, "fp8", None)
    assert np.all(scale == 1.0)
    assert np.array_equal(st.codes.cpu().numpy(), codes)


@pytest.mark.parametrize("dense", [False, True], ids=["standard-map", "dense-map"])
def test_lp_custom_map_codes_exact_and_flag(dense):
    """A quantization map with 200 of its 256 entries inside one key bucket (key >> 18) has
    more than two thresholds per bucket: the table flag marks it and the tiled pre-pass
    takes the full threshold count for it. Codes and scales bit-exact against the oracle's
    quantizer with the same map; the standard map keeps the flag clear."""
    from muonium_amd import _lib

    lib = _lib.load()
    dev = torch.device(DEV)
    _lib.ensure_device(dev)
    if dense:
        qmap = np.unique(np.concatenate([np.linspace(-1.0, 1.0, 56, dtype=np.float32),
                                         np.float32(0.5) + np.arange(200, dtype=np.float32) * np.float32(4e-7)]))
        assert qmap.size == 256
    else:
        qmap = quant_ref.qmap_8bit(True)
    qmap = qmap.astype(np.float32)
    rows, cols, block = 256, 512, 256
    gen = torch.Generator().manual_seed(9)
    # fp32 gradients with a block maximum of 1 and every third value within 1e-4 of 0.5, so
    # y = m / scale falls among the clustered entries
    g = (0.25 * torch.randn(rows, cols, generator=gen)).clamp(-0.9, 0.9)
    g[:, 1::3] = 0.5 + 2e-5 * torch.randn(rows, (cols + 1) // 3, generator=gen)
    g[:, 0] = 1.0
    g[:, block] = 1.0
    codes_d = torch.zeros(rows * cols, dtype=torch.uint8, device=dev)
    scales_d = torch.zeros(rows * cols // block, dtype=torch.float32, device=dev)
    qmap_d = torch.from_numpy(qmap).to(dev)
    nbytes = lib.muon_orth_workspace_bytes(_lib.DT_BF16, 1, rows, cols)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    gd = g.to(dev)
    codes = np.zeros(rows * cols, np.uint8)
    scales = np.zeros(rows * cols // block, np.float32)
    for step in range(2):
        rc = lib.muon_lp_prepass(1, _lib.ptr_array([gd]), _lib.DT_F32, _lib.ptr_array([codes_d]),
                                 _lib.ptr_array([scales_d]), qmap_d.data_ptr(), 8, block, 1, rows,
                                 cols, 0.9, 1, 0, ws.data_ptr(), _lib.DT_BF16, 1, _lib.stream(dev))
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        codes, scales, _ = quant_ref.lp_momentum_step(
            codes, scales, g.numpy(), block=block, fmt="8bit", qmap=qmap, momentum=0.9,
            nesterov=True, maximize=False)
        assert np.array_equal(codes_d.cpu().numpy(), codes), f"codes differ at step {step}"
        assert np.array_equal(scales_d.cpu().numpy().view(np.uint32), scales.view(np.uint32))
    # flag word: last threshold pad slot, after the 16 KB bucket table in the qtab region
    rup = lambda v: -(-v // 256) * 256
    x, a = 256 * 512 * 2, 256 * 256 * 2
    off_qtab = 2 * rup(x) + 2 * rup(a) + rup((256 // 64) * (512 // 64) * 4) + rup(4)
    thr = ws[off_qtab + 16384: off_qtab + 16384 + 260 * 4].cpu().view(torch.int32).numpy().view(np.uint32)
    assert thr[259] == (1 if dense else 0)
    assert thr[256] == 0xFFFFFFFF and thr[257] == 0xFFFFFFFF


@pytest.mark.parametrize("opt_cls", [Muon8bit, Muon4bit, MuonFp8])
@pytest.mark.parametrize("map_location", [None, "cpu"])
def test_lp_checkpoint_round_trip_with_weights_only(opt_cls, map_location):
    """state_dict -> torch.save -> torch.load(weights_only=True) -> load_state_dict keeps
    training continuous (test_optim.py:660-686 for Muon, here for the quantized states):
    two more steps from the loaded checkpoint give bit for bit the params, codes and
    scales of an uninterrupted run. Loaded onto the CPU (map_location="cpu"), the
    quantized state moves back to its param's device on load_state_dict."""
    import io

    gen = torch.Generator().manual_seed(3)
    # tiled wide, tiled tall, general (cols not a multiple of 256) and dense (numel < 4096).
    # lr_ratio is 1 or 2 here: load_state_dict casts every state tensor but `step` to the
    # param's dtype (torch.optim.Optimizer, as in the reference), so a bf16 param's
    # lr_ratio = sqrt(2) would come back rounded to bf16 and the trajectory would differ
    shapes = [(128, 256), (1024, 256), (256, 64), (8, 16)]
    init = [torch.randn(s, generator=gen).bfloat16() for s in shapes]
    grads = [[torch.randn(s, generator=gen).bfloat16() for s in shapes] for _ in range(4)]
    kw = dict(lr=0.05, wd=0.1, momentum=0.9, block_size=256)

    def run(params, opt, steps):
        for k in steps:
            for p, g in zip(params, grads[k]):
                p.grad = g.to(DEV)
            opt.step()

    ref_p = [nn.Parameter(t.clone().to(DEV)) for t in init]
    ref = opt_cls(ref_p, **kw)
    run(ref_p, ref, range(4))

    src_p = [nn.Parameter(t.clone().to(DEV)) for t in init]
    src = opt_cls(src_p, **kw)
    run(src_p, src, range(2))
    blob = io.BytesIO()
    torch.save(src.state_dict(), blob)
    blob.seek(0)
    sd = torch.load(blob, weights_only=True, map_location=map_location)
    dst_p = [nn.Parameter(p.detach().clone()) for p in src_p]
    dst = opt_cls(dst_p, **kw)
    dst.load_state_dict(sd)
    mb = dst.state[dst_p[0]]["momentum_buffer"]
    assert type(mb).__name__.startswith("OptimState") and mb.device.type == "cuda"
    run(dst_p, dst, range(2, 4))
    torch.cuda.synchronize()
    for a, b in zip(dst_p, ref_p):
        assert torch.equal(a.detach(), b.detach())
    for a, b in zip(dst_p, ref_p):
        sa, sb = dst.state[a]["momentum_buffer"], ref.state[b]["momentum_buffer"]
        if hasattr(sb, "codes"):
            assert torch.equal(sa.codes, sb.codes) and torch.equal(sa.scale, sb.scale)
        else:
            assert torch.equal(sa, sb)
