"""The C ABI library on the CPU: it loads, exports every entry point include/muon_amd.h
declares, and validates arguments (returning an error, never touching the device)
before any launch."""

import ctypes
import os
import re

import pytest

from muonium_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "muon_amd.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(muon_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared()
    assert len(declared) >= 12
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    assert sorted(_lib.EXPORTED_SYMBOLS) == declared


def test_abi_version_and_error_text():
    lib = _lib.load()
    assert lib.muon_amd_abi_version() == 5
    assert isinstance(_lib.last_error(), str)


def test_workspace_size_formula():
    lib = _lib.load()
    # bf16, 2 matrices of 300 x 130 -> m_pad 256, n_pad 512
    nbytes = lib.muon_orth_workspace_bytes(_lib.DT_BF16, 2, 300, 130)
    x = 2 * 256 * 512 * 2
    a = 2 * 256 * 256 * 2
    parts = 2 * (256 // 64) * (512 // 64) * 4
    # two ping-pong copies of the wide iterate, A, B, norm partials, per-matrix scale,
    # the quantized-state search tables (16 KB bucket table + 260 thresholds, padded), and
    # one fp32 per stored row (n_pad) per matrix for NorMuon's row statistics
    assert nbytes == 2 * x + 2 * a + parts + 256 + 16384 + 1280 + 2 * 512 * 4
    assert lib.muon_orth_workspace_bytes(_lib.DT_BF16, 1, 300, 130) < nbytes
    assert lib.muon_orth_workspace_bytes(7, 1, 4, 4) == -1
    assert lib.muon_orth_workspace_bytes(_lib.DT_F32, 1, 0, 4) == -1


def test_short_workspace_pads_rows_to_64():
    lib = _lib.load()
    # bf16 with at most 64 rows on the short side: 64-row iterate, plus per-matrix Gram
    # partials (12 KB each) over min(256, max(1, panels / 4)) column ranges of 256 columns
    rows, cols = 48, 70000                 # n_pad 70144: 274 panels -> 68 ranges
    nbytes = lib.muon_orth_workspace_bytes(_lib.DT_BF16, 3, rows, cols)
    rup = lambda v: -(-v // 256) * 256
    x = 3 * 64 * 70144 * 2
    a = 3 * 64 * 64 * 2
    parts = 3 * 1 * (70144 // 64) * 4
    want = (2 * rup(x) + 2 * rup(a) + rup(parts) + 256 + rup(16384 + 1280) + rup(3 * 70144 * 4)
            + 3 * 68 * 3 * 1024 * 4)
    assert nbytes == want
    off, pitch, mst = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    trans = ctypes.c_int()
    for r, c, t in ((rows, cols, 0), (cols, rows, 1)):
        assert lib.muon_orth_result(_lib.DT_BF16, 3, r, c, 1, off, pitch, mst, trans) == 0
        assert (off.value, pitch.value, mst.value, trans.value) == (rup(x), 70144, 64 * 70144, t)
    # 65 rows, or an fp32 iteration, keep the 256-row tiles
    assert lib.muon_orth_result(_lib.DT_BF16, 1, 65, 512, 1, off, pitch, mst, trans) == 0
    assert (pitch.value, mst.value) == (512, 256 * 512)
    assert lib.muon_orth_result(_lib.DT_F32, 1, 64, 512, 1, off, pitch, mst, trans) == 0
    assert (pitch.value, mst.value) == (512, 256 * 512)


def test_result_location_follows_orientation():
    lib = _lib.load()
    off, pitch, mst = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    trans = ctypes.c_int()
    x1 = 4 * 256 * 512 * 2  # byte offset of the second iterate buffer
    # the result is X[steps % 2] in the wide layout (pitch n_pad) for both orientations;
    # a tall matrix's result is flagged as transposed
    for rows, cols, t in ((100, 300, 0), (300, 100, 1)):
        assert lib.muon_orth_result(_lib.DT_BF16, 4, rows, cols, 5, off, pitch, mst, trans) == 0
        assert (off.value, pitch.value, mst.value, trans.value) == (x1, 512, 256 * 512, t)
        assert lib.muon_orth_result(_lib.DT_BF16, 4, rows, cols, 4, off, pitch, mst, trans) == 0
        assert (off.value, pitch.value, trans.value) == (0, 512, t)
        assert lib.muon_orth_result(_lib.DT_BF16, 4, rows, cols, 0, off, pitch, mst, trans) == 0
        assert (off.value, trans.value) == (0, t)
    # iterates wider than 4096 columns get rows of n_pad + 64 elements (128 more bytes in
    # bf16), in both orientations and in the workspace size
    for rows, cols in ((300, 14336), (14336, 300)):  # m_pad 512, n_pad 14336
        assert lib.muon_orth_result(_lib.DT_BF16, 2, rows, cols, 1, off, pitch, mst, trans) == 0
        assert (off.value, pitch.value, mst.value) == (2 * 512 * 14400 * 2, 14400, 512 * 14400)
    nb = lib.muon_orth_workspace_bytes(_lib.DT_BF16, 2, 300, 14336)
    # X0, X1 with the wider rows, A, B, partials over n_pad (not the pitch), ...
    assert nb == (2 * (2 * 512 * 14400 * 2) + 2 * (2 * 512 * 512 * 2) + 2 * (512 // 64) * (14336 // 64) * 4
                  + 256 + 16384 + 1280 + 2 * 14336 * 4)


@pytest.mark.parametrize(
    "call,code",
    [
        (lambda L: L.muon_gram(None, None, 9, 1, 4, 4, None), 2),
        (lambda L: L.muon_gram(None, None, 1, -1, 4, 4, None), 1),
        # K == 0 never reads x; y must hold whole elements (an odd address is refused)
        (lambda L: L.muon_gram(None, 1, 1, 1, 4, 0, None), 3),
        (lambda L: L.muon_prepass(1, None, None, 1, 0, 0, 4, 4, 0.9, 1, 0, 0, None, 1, 1, None), 1),
        (lambda L: L.muon_prepass(1, None, None, 1, 0, 1, 4, 4, 0.9, 1, 0, 0, None, 1, 1, None), 5),
        (lambda L: L.muon_orth_run(None, 1, 1, 2, 4, 4, None, 1, 1.0, 1e-7, None), 5),
        (lambda L: L.muon_orth_run(None, 5, 1, 1, 4, 4, None, 1, 1.0, 1e-7, None), 2),
        (lambda L: L.muon_postpass(1, None, 9, None, 1, None, 1, 1, 1, 1, 4, 4, None, None, 0.0, 0, None), 2),
        (lambda L: L.muon_lp_quantize(None, None, None, None, 3, 256, 256, None), 5),
        (lambda L: L.muon_lp_quantize(None, None, None, None, 8, 300, 256, None), 1),
        (lambda L: L.muon_lp_dequantize(None, None, None, 4, 254, 127, None, None), 1),
    ],
)
def test_argument_errors_return_codes_without_launching(call, code):
    lib = _lib.load()
    assert call(lib) == code
    assert _lib.last_error() != ""


def test_library_calls_are_registered_torch_ops_with_fake_impls():
    """Every library call of the package is a torch.library custom op (namespace
    muonium_amd) that declares the tensors it writes, and its fake implementation runs
    on fake tensors without a device: what lets an outer torch.compile trace step()."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode

    import muonium_amd  # noqa: F401  (registers the ops)

    writes = {
        "gram_": ["y"], "orthogonalize": [], "momentum_only": ["grads", "bufs"],
        "postpass": ["params"], "fused_step": ["params", "grads", "bufs"],
        "fused_normuon_step": ["params", "grads", "bufs", "variances"],
        "normuon_postpass": ["params", "variances"],
        "fused_lp_step": ["params", "grads", "codes", "scales"],
        "lp_quantize": ["codes", "scale"], "lp_dequantize": ["out"],
    }
    for name, mutated in writes.items():
        schema = getattr(torch.ops.muonium_amd, name).default._schema
        got = [a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write]
        assert got == mutated, (name, got)
    with FakeTensorMode():
        x = torch.empty(3, 64, 32, device="cuda")
        u = torch.ops.muonium_amd.orthogonalize([x, x], [3.4445, -4.775, 2.0315], 1.0, 1e-7,
                                                torch.bfloat16, torch.bfloat16)
        assert u.shape == (2, 3, 64, 32) and u.dtype == torch.bfloat16
        assert torch.ops.muonium_amd.fused_step(
            [x], [x], [x], [torch.empty(())], torch.empty(()), 0.9, True, False, True, 0.1,
            True, [3.4445, -4.775, 2.0315], 1.0, 1e-7, None) is None
