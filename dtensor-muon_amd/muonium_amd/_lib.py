"""ctypes binding of libmuon_amd.so (the C ABI declared in include/muon_amd.h).

The library is the only compute path of this package: every Muon-family step on a
HIP device runs its kernels. If the shared object is missing or fails to load, the
first call raises — there is no fallback implementation.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Sequence

import torch

_LIB_PATH = os.path.join(os.path.dirname(__file__), "_lib", "libmuon_amd.so")

# dtype codes (MUON_DT_*)
DT_F32, DT_BF16, DT_F16 = 0, 1, 2
_DTYPE_CODE = {torch.float32: DT_F32, torch.bfloat16: DT_BF16, torch.float16: DT_F16}

# quantized-state formats (MUON_Q_*)
Q_8BIT, Q_4BIT, Q_FP8 = 8, 4, 0

MAX_TENSORS = 32

_c_int, _c_i64, _c_f32, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
_pp = ctypes.POINTER(ctypes.c_void_p)
_SIGNATURES = {
    "muon_amd_abi_version": (_c_int, []),
    "muon_amd_last_error": (ctypes.c_char_p, []),
    "muon_amd_init": (_c_int, []),
    "muon_gram": (_c_int, [_vp, _vp, _c_int, _c_i64, _c_i64, _c_i64, _vp]),
    "muon_orth_workspace_bytes": (_c_i64, [_c_int, _c_i64, _c_i64, _c_i64]),
    "muon_orth_result": (
        _c_int,
        [_c_int, _c_i64, _c_i64, _c_i64, _c_int, ctypes.POINTER(_c_i64),
         ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), ctypes.POINTER(_c_int)],
    ),
    "muon_prepass": (
        _c_int,
        [_c_int, _pp, _pp, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_f32, _c_int, _c_int,
         _c_int, _vp, _c_int, _c_i64, _vp],
    ),
    "muon_orth_run": (
        _c_int,
        [_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.POINTER(ctypes.c_double), _c_int,
         _c_f32, _c_f32, _vp],
    ),
    "muon_orth_run_apply": (
        _c_int,
        [_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.POINTER(ctypes.c_double), _c_int,
         _c_f32, _c_f32, _c_int, _pp, _c_int, _c_i64, ctypes.POINTER(_c_f32), _c_f32, _c_int,
         _vp],
    ),
    "muon_orth_extract": (
        _c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _vp, _c_int, _vp]
    ),
    "muon_postpass": (
        _c_int,
        [_c_int, _pp, _c_int, _vp, _c_int, _vp, _c_int, _c_i64, _c_int, _c_i64, _c_i64, _c_i64,
         ctypes.POINTER(_c_f32), ctypes.POINTER(_c_f32), _c_f32, _c_int, _vp],
    ),
    "muon_normuon_postpass": (
        _c_int,
        [_c_int, _pp, _c_int, _pp, _c_int, _vp, _c_int, _vp, _c_int, _c_i64, _c_int, _c_i64,
         _c_i64, _c_i64, ctypes.POINTER(_c_i64), _c_int, ctypes.POINTER(_c_f32),
         ctypes.POINTER(_c_f32), _c_f32, _c_int, ctypes.c_double, _vp],
    ),
    "muon_normuon_postpass_noalloc": (
        _c_int,
        [_c_int, _pp, _c_int, _pp, _c_int, _vp, _c_int, _c_i64, _c_i64, _c_i64,
         ctypes.POINTER(_c_i64), _c_int, ctypes.POINTER(_c_f32), ctypes.POINTER(_c_f32), _c_f32,
         _c_int, ctypes.c_double, _vp],
    ),
    "muon_lp_quantize": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_i64, _c_i64, _vp]),
    "muon_lp_dequantize": (_c_int, [_vp, _vp, _vp, _c_int, _c_i64, _c_i64, _vp, _vp]),
    "muon_timing_enable": (_c_int, [_c_int]),
    "muon_timing_read": (
        _c_int,
        [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_c_i64), ctypes.POINTER(ctypes.c_double)],
    ),
    "muon_lp_prepass": (
        _c_int,
        [_c_int, _pp, _c_int, _pp, _pp, _vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_f32,
         _c_int, _c_int, _vp, _c_int, _c_i64, _vp],
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_initialized_devices: set[int] = set()


class MuonKernelError(RuntimeError):
    """A libmuon_amd entry point returned an error status."""


def library_path() -> str:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load libmuon_amd.so once (after torch, so the HIP runtime torch already
    loaded is the one the library binds to) and declare every signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise ImportError(
                    f"muonium_amd: {_LIB_PATH} is missing; build it with "
                    "`python -c 'import __graft_entry__ as g; g.build()'` "
                    "or `make -C dtensor-muon_amd/csrc`"
                )
            lib = ctypes.CDLL(_LIB_PATH)
            for name, (restype, argtypes) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = lib
    return _lib


def last_error() -> str:
    return (load().muon_amd_last_error() or b"").decode()


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise MuonKernelError(f"{what} failed (status {rc}): {last_error()}")


def ensure_device(device: torch.device) -> None:
    """First use on a device: verify it is a gfx950 and the code objects load."""
    if device.type != "cuda":
        raise RuntimeError(f"muonium_amd kernels run on a HIP device; got a {device.type} tensor")
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx in _initialized_devices:
        return
    lib = load()
    with torch.cuda.device(idx):
        check(lib.muon_amd_init(), "muon_amd_init")
    _initialized_devices.add(idx)


KERNEL_KINDS = ("syrk_xx", "syrk_aa", "gemm_bx", "prepass", "postpass", "lp_prepass", "other",
                "gemm_bx_apply")


def timing_enable(on: bool) -> None:
    """Bracket every launch of the step entry points with hipEvents (or stop)."""
    check(load().muon_timing_enable(int(on)), "muon_timing_enable")


def timing_read() -> dict[str, tuple[float, int, float]]:
    """{kind: (total ms, launches, algorithmic work)} since timing was enabled."""
    n = len(KERNEL_KINDS)
    ms = (ctypes.c_double * n)()
    cnt = (ctypes.c_int64 * n)()
    work = (ctypes.c_double * n)()
    check(load().muon_timing_read(ms, cnt, work), "muon_timing_read")
    return {k: (ms[i], cnt[i], work[i]) for i, k in enumerate(KERNEL_KINDS)}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"muonium_amd: unsupported dtype {dtype}") from None


def stream(device: torch.device) -> int:
    """The current stream of ``device`` as the raw handle the C ABI takes (the same value as
    ``torch.cuda.current_stream(device).cuda_stream``, without building a Stream object:
    a step makes a few calls per bucket and the host time adds up for small buckets)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


def ptr_array(tensors: Sequence[torch.Tensor | None]):
    arr = (ctypes.c_void_p * max(len(tensors), 1))()
    for i, t in enumerate(tensors):
        arr[i] = None if t is None else t.data_ptr()
    return arr


def f32_array(values: Sequence[float]):
    arr = (ctypes.c_float * max(len(values), 1))()
    for i, v in enumerate(values):
        arr[i] = v
    return arr


def i64_array(values: Sequence[int]):
    arr = (ctypes.c_int64 * max(len(values), 1))()
    for i, v in enumerate(values):
        arr[i] = v
    return arr


def f64_array(values: Sequence[float]):
    arr = (ctypes.c_double * max(len(values), 1))()
    for i, v in enumerate(values):
        arr[i] = v
    return arr
