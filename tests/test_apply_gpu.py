"""The apply fused into the last X' = a X + B X (muon_orth_run_apply) against the iteration
followed by the post-pass (muon_orth_run + muon_postpass), through the C ABI.

Both sides start from the same pre-pass output; the parameters must come out bit for bit
equal: the fused epilogue applies muon.py:58-77 (cautious weight decay, the shape-scaled
step; with wd = 0 the bf16-rounded step) to each bf16 element of the last iterate exactly as
the post-pass does from the stored U. Wide matrices, tall ones (whose last product runs
with swapped MFMA operands so its accumulators hold parameter rows), partial edge tiles,
stacked 3D tensors, iterates of at most 64 rows (the short path's last product, wide
parameters), and the shapes that fall back to the two calls (fp32 parameters, a short side
from 65 to below 768 after padding to 128 rows, fp16 parameters, tall short parameters).
"""

import pytest
import torch

from muonium_amd import _lib
from muonium_amd._ops import _flat_coeffs, adjusted_lrs, matrix_view
from oracle import muon_ref

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")


def _run(params, grads, bufs, *, fused, wd, cautious, steps=5):
    lib = _lib.load()
    _lib.ensure_device(DEV)
    nb, rows, cols = matrix_view(grads[0])
    count = len(grads)
    cap = count * nb
    ws = torch.zeros(lib.muon_orth_workspace_bytes(_lib.DT_BF16, cap, rows, cols),
                     dtype=torch.uint8, device=DEV)
    s = _lib.stream(DEV)
    coeffs, prescale = muon_ref.strategy_coeffs("polar_express", steps)
    flat = [c for t in coeffs for c in t]
    lrs = adjusted_lrs([torch.tensor(muon_ref.lr_ratio((rows, cols)))] * count, torch.tensor(0.02))
    _lib.check(lib.muon_prepass(count, _lib.ptr_array(grads), _lib.ptr_array(bufs),
                                _lib.dtype_code(grads[0].dtype), _lib.dtype_code(bufs[0].dtype),
                                nb, rows, cols, 0.9, 1, 0, 1, ws.data_ptr(), _lib.DT_BF16, cap, s),
               "muon_prepass")
    pdt = _lib.dtype_code(params[0].dtype)
    if fused:
        _lib.check(lib.muon_orth_run_apply(ws.data_ptr(), _lib.DT_BF16, cap, cap, rows, cols,
                                           _flat_coeffs(flat), steps, prescale, 1e-7, count,
                                           _lib.ptr_array(params), pdt, nb, _lib.f32_array(lrs),
                                           wd, int(cautious), s), "muon_orth_run_apply")
    else:
        _lib.check(lib.muon_orth_run(ws.data_ptr(), _lib.DT_BF16, cap, cap, rows, cols,
                                     _flat_coeffs(flat), steps, prescale, 1e-7, s), "muon_orth_run")
        _lib.check(lib.muon_postpass(count, _lib.ptr_array(params), pdt, None, 0, ws.data_ptr(),
                                     _lib.DT_BF16, cap, steps, nb, rows, cols, _lib.f32_array(lrs),
                                     None, wd, int(cautious), s), "muon_postpass")
    torch.cuda.synchronize()


def _case(shape, count, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    p = [torch.randn(shape, generator=gen).to(dtype) for _ in range(count)]
    rows_scale = torch.exp(torch.randn(*shape[:-1], 1, generator=gen))
    g = [(torch.randn(shape, generator=gen) * rows_scale).to(dtype) for _ in range(count)]
    b = [torch.randn(shape, generator=gen) * 0.1 for _ in range(count)]
    return p, g, b


@pytest.mark.parametrize("shape,count", [
    ((1024, 2048), 3),     # wide
    ((2048, 1024), 2),     # tall: swapped operands in the last product
    ((1100, 1536), 2),     # wide, partial last tile row (1100 of 1280 rows)
    ((1800, 1032), 2),     # tall, partial tiles both ways
    ((2, 1024, 1280), 2),  # stacked: two matrices per tensor
    ((3, 1280, 1032), 2),  # stacked tall, partial tiles
    ((64, 8192), 3),       # iterate of at most 64 rows: the short path's last B X
    ((48, 5000), 2),       # short, padding rows 48-63 and a partial last column panel
    ((3, 32, 4096), 2),    # short, stacked
    ((64, 1408 * 2048), 1),  # a flattened MoE expert stack
    ((768, 2304), 2),      # K = 768 (the GPT-2 shapes), wide
    ((3072, 768), 2),      # K = 768, tall
])
@pytest.mark.parametrize("wd,cautious", [(0.1, True), (0.1, False), (0.0, True)])
def test_fused_apply_matches_postpass_bit_for_bit(shape, count, wd, cautious):
    p, g, b = _case(shape, count, torch.bfloat16, seed=sum(shape) + count)
    pa = [t.clone().to(DEV) for t in p]
    pb = [t.clone().to(DEV) for t in p]
    ga, gb = [t.clone().to(DEV) for t in g], [t.clone().to(DEV) for t in g]
    ba, bb = [t.clone().to(DEV) for t in b], [t.clone().to(DEV) for t in b]
    _run(pa, ga, ba, fused=True, wd=wd, cautious=cautious)
    _run(pb, gb, bb, fused=False, wd=wd, cautious=cautious)
    for i, (x, y, p0) in enumerate(zip(pa, pb, p)):
        assert not torch.equal(x.cpu(), p0), f"tensor {i} not updated"
        assert torch.equal(x, y), (
            f"tensor {i}: {(x.float() - y.float()).ne(0).sum().item()} elements differ")
    for x, y in zip(ga + ba, gb + bb):
        assert torch.equal(x, y)


@pytest.mark.parametrize("shape,dtype", [
    ((1024, 2048), torch.float32),   # fp32 parameters: the separate post-pass
    ((512, 2048), torch.bfloat16),   # short side 512 < 768: the separate post-pass
    ((2048, 1024), torch.float16),
    ((4096, 64), torch.bfloat16),    # tall with at most 64 columns: the separate post-pass
    ((64, 4096), torch.float32),     # short, fp32 parameters
])
def test_fallback_shapes_match_postpass(shape, dtype):
    p, g, b = _case(shape, 2, dtype, seed=5)
    pa = [t.clone().to(DEV) for t in p]
    pb = [t.clone().to(DEV) for t in p]
    ga, gb = [t.clone().to(DEV) for t in g], [t.clone().to(DEV) for t in g]
    ba, bb = [t.clone().to(DEV) for t in b], [t.clone().to(DEV) for t in b]
    _run(pa, ga, ba, fused=True, wd=0.1, cautious=True)
    _run(pb, gb, bb, fused=False, wd=0.1, cautious=True)
    for x, y in zip(pa, pb):
        assert torch.equal(x, y)


def test_optimizer_step_uses_fused_apply_and_matches_given_u():
    """A foreach Muon step on a Llama-like gate shape goes through the fused apply (the
    timing kind of the fused launch records it) and equals the oracle's update arithmetic
    given the U that muon_orth_run computes for the same g' (bit for bit)."""
    from muonium_amd import Muon
    from muonium_amd.orthogonalize import foreach_zeropower

    gen = torch.Generator().manual_seed(11)
    shape = (3072, 1024)
    p0 = [torch.randn(shape, generator=gen).bfloat16() for _ in range(2)]
    g0 = [torch.randn(shape, generator=gen).bfloat16() for _ in range(2)]
    params = [torch.nn.Parameter(t.clone().to(DEV)) for t in p0]
    for p, g in zip(params, g0):
        p.grad = g.clone().to(DEV)
    opt = Muon(params, lr=0.02, wd=0.1, momentum=0.9, nesterov=True, foreach=True)
    _lib.timing_enable(True)
    opt.step()
    kern = _lib.timing_read()
    _lib.timing_enable(False)
    assert kern["gemm_bx_apply"][1] == 1 and kern["postpass"][1] == 0
    # g' = g + mu * (0 * mu + g), as the pre-pass writes it back into the gradients
    gq = [(g.float() + (g.float() * 0.9)).bfloat16() for g in g0]
    assert all(torch.equal(p.grad.cpu(), q) for p, q in zip(params, gq))
    us = [u.cpu() for u in foreach_zeropower([q.float().to(DEV) for q in
                                              [g.float() + g.float() * 0.9 for g in g0]],
                                             strategy="polar_express")]
    for p, p_init, u in zip(params, p0, us):
        ref, _, _, _ = muon_ref.muon_update(
            p_init, torch.zeros(shape), torch.zeros(shape), muon_ref.lr_ratio(shape), lr=0.02,
            weight_decay=0.1, cautious_wd=True, momentum=0.0, nesterov=False, maximize=False,
            orth_single=lambda x, u=u: u)
        assert torch.equal(p.detach().cpu(), ref)


@pytest.mark.parametrize("shape", [(1024, 2048), (2048, 1024)])
@pytest.mark.parametrize("wd,cautious", [(0.1, True), (0.1, False), (0.0, True)])
def test_fused_apply_nonfinite_matches_postpass_bitwise(shape, wd, cautious):
    """Non-finite and signed-zero parameters, and a NaN gradient element (which makes the
    whole update of its matrix NaN): the fused epilogue rounds, masks and propagates them
    exactly as the post-pass does, NaN payloads included (compared as bit patterns)."""
    p, g, b = _case(shape, 2, torch.bfloat16, seed=sum(shape) + 7)
    special = torch.tensor([float("nan"), float("inf"), float("-inf"), 0.0, -0.0, 1e-40,
                            -3e38, 3e38], dtype=torch.bfloat16)
    p[0][0, : special.numel()] = special
    p[0][-1, -special.numel():] = special
    p[1][5, 100] = float("nan")
    g[1][3, 7] = float("nan")
    pa = [t.clone().to(DEV) for t in p]
    pb = [t.clone().to(DEV) for t in p]
    ga, gb = [t.clone().to(DEV) for t in g], [t.clone().to(DEV) for t in g]
    ba, bb = [t.clone().to(DEV) for t in b], [t.clone().to(DEV) for t in b]
    _run(pa, ga, ba, fused=True, wd=wd, cautious=cautious)
    _run(pb, gb, bb, fused=False, wd=wd, cautious=cautious)
    assert pa[1].isnan().all(), "a NaN gradient element makes its matrix's update NaN"
    for i, (x, y) in enumerate(zip(pa, pb)):
        xi, yi = x.view(torch.int16), y.view(torch.int16)
        assert torch.equal(xi, yi), f"tensor {i}: {(xi != yi).sum().item()} bit patterns differ"


def test_flattened_stack_step_takes_the_short_fused_apply():
    """flatten=True makes a (16, 48, 320) tensor one (16, 15360) matrix: an iterate of at
    most 64 rows, whose last B X carries the apply (its timing kind records the launch and no
    post-pass runs); parameters against the oracle are pinned by test_short_gpu.py."""
    from muonium_amd import Muon

    gen = torch.Generator().manual_seed(13)
    p = torch.nn.Parameter(torch.randn(16, 48, 320, generator=gen).bfloat16().to(DEV))
    p.grad = torch.randn(16, 48, 320, generator=gen).bfloat16().to(DEV)
    p_init = p.detach().clone()
    opt = Muon([{"params": [p], "flatten": True}], lr=0.02, foreach=True)
    _lib.timing_enable(True)
    opt.step()
    kern = _lib.timing_read()
    _lib.timing_enable(False)
    assert kern["gemm_bx_apply"][1] == 1 and kern["postpass"][1] == 0
    assert not torch.equal(p.detach(), p_init)


@pytest.mark.parametrize("shape", [(1024, 1024), (48, 4096)])
def test_more_tensors_than_one_apply_table(shape):
    """A bucket of 130 tensors (more than the 128 one launch's table holds): the last product
    runs as two launches (128 tensors, then 2) on the tiled and on the short path, with
    parameters bit for bit those of the iteration followed by the post-pass."""
    p, g, b = _case(shape, 130, torch.bfloat16, seed=130)
    pa = [t.clone().to(DEV) for t in p]
    pb = [t.clone().to(DEV) for t in p]
    ga, gb = [t.clone().to(DEV) for t in g], [t.clone().to(DEV) for t in g]
    ba, bb = [t.clone().to(DEV) for t in b], [t.clone().to(DEV) for t in b]
    _run(pa, ga, ba, fused=True, wd=0.1, cautious=True)
    _run(pb, gb, bb, fused=False, wd=0.1, cautious=True)
    for i, (x, y) in enumerate(zip(pa, pb)):
        assert torch.equal(x, y), f"tensor {i}"
