"""CPU restatement of the blockwise quantized momentum state (test infrastructure only).

MuonLP (muonium/optim/optim_lp.py:118-133) stores momentum through torchao 0.17.0's
``OptimState8bit`` / ``OptimState4bit`` / ``OptimStateFp8`` (uv.lock:533-534). torchao
is not installed in this environment, so this module restates torchao's published
algorithm (itself following bitsandbytes' dynamic quantization map):

* 8-bit: codes index a 256-entry "dynamic" map (signed: 7 exponent levels of
  10^-6..10^0 times evenly spaced fractions, plus 0 and 1); one fp32 absmax scale per
  block of ``block_size`` consecutive values of the flattened tensor.
* 4-bit: the same construction with 3 exponent levels and 4 total bits (16 entries,
  signed); two codes per byte, element 2i in the high nibble.
* fp8: float8_e4m3fn codes of x / scale with scale = absmax / 448 per block.

Quantizing a value y = x / scale: binary search for the largest code with
map[code] <= y, then step up one code when y - map[code] >= (map[code+1] - map[code]) / 2.
A NaN anywhere in a block makes its absmax, and so its scale, NaN (torch's amax and clamp
propagate NaN, as np.max and np.maximum do here); every value of such a block then
quantizes a NaN quotient: code 0 for the maps (every comparison fails), 0x7f for fp8.

Parity of these codes with torchao itself is UNPINNED (torchao is absent); the tests
pin the restatement with brute-force nearest-code search, the map's structure,
round-trip error bounds and torch's own float8_e4m3fn cast.
"""

from __future__ import annotations

import numpy as np
import torch


def create_dynamic_map(signed: bool = True, max_exponent_bits: int = 7, total_bits: int = 8) -> list[float]:
    """Sorted dynamic map with exactly 2**total_bits entries (fp32 values).

    Built with torch fp32 arithmetic so every entry is the fp32 value torchao's map
    holds: for exponent level i the entries are 10^(i - (E-1)) times the midpoints of
    torch.linspace(0.1, 1, k + 1) (k fractions, k doubling per level), mirrored for
    the signed map, plus 0 and 1.
    """
    data: list[float] = []
    non_sign_bits = total_bits - 1
    additional = 2 ** (non_sign_bits - max_exponent_bits) - 1
    i = 0
    for i in range(max_exponent_bits):
        n = int(2 ** (i + non_sign_bits - max_exponent_bits) + 1 if signed
                else 2 ** (i + non_sign_bits - max_exponent_bits + 1) + 1)
        edges = torch.linspace(0.1, 1, n)
        mids = (edges[:-1] + edges[1:]) / 2.0
        scale = 10 ** (-(max_exponent_bits - 1) + i)
        data += (scale * mids).tolist()
        if signed:
            data += (-scale * mids).tolist()
    if additional > 0:
        edges = torch.linspace(0.1, 1, additional + 1)
        mids = (edges[:-1] + edges[1:]) / 2.0
        scale = 10 ** (-(max_exponent_bits - 1) + i)
        data += (scale * mids).tolist()
        if signed:
            data += (-scale * mids).tolist()
    data.append(0.0)
    data.append(1.0)
    assert len(data) == 2**total_bits
    data.sort()
    return data


def qmap_8bit(signed: bool = True) -> np.ndarray:
    return np.asarray(create_dynamic_map(signed), dtype=np.float32)


def qmap_4bit(signed: bool = True) -> np.ndarray:
    if signed:
        return np.asarray(create_dynamic_map(True, 3, 4), dtype=np.float32)
    # unsigned 4-bit map is linear without zero: linspace(0, 1, 17)[1:]
    return torch.linspace(0, 1, 17)[1:].numpy().astype(np.float32)


def _block_scale(x: np.ndarray, block: int, fp8: bool) -> np.ndarray:
    xb = x.reshape(-1, block)
    amax = np.abs(xb).max(axis=1).astype(np.float32)
    amax = np.maximum(amax, np.float32(1e-12))
    if fp8:
        amax = (amax / np.float32(448.0)).astype(np.float32)
    return amax


def quantize_codes(y: np.ndarray, qmap: np.ndarray) -> np.ndarray:
    """Binary search + round-half-up between neighbours, all in fp32."""
    y = y.astype(np.float32)
    n = len(qmap)
    bits = int(np.log2(n))
    c = np.zeros(y.shape, dtype=np.int64)
    step = n // 2
    c = np.where(y >= qmap[step], step, 0)
    for k in range(bits - 2, -1, -1):
        s = 1 << k
        c = c + np.where(y >= qmap[c + s], s, 0)
    up = np.minimum(c + 1, n - 1)
    lo, hi = qmap[c], qmap[up]
    res = (y - lo).astype(np.float32)
    half = ((hi - lo).astype(np.float32) * np.float32(0.5)).astype(np.float32)
    return np.where(res >= half, up, c).astype(np.uint8)


def f32_to_e4m3fn(x: np.ndarray) -> np.ndarray:
    """fp32 -> float8_e4m3fn bits, round-to-nearest-even; magnitudes that round past
    448 (i.e. > 464, or NaN/inf) become NaN (0x7f | sign), as torch's cast does."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    sign = ((u >> 24) & 0x80).astype(np.uint8)
    a = u & 0x7FFFFFFF
    out = np.zeros(x.shape, dtype=np.uint8)
    nan = a > 0x43E80000
    sub = a < 0x3C800000
    # subnormal: round |x| * 2^9 to an integer, ties to even
    s = np.abs(x).astype(np.float64) * 512.0
    r = np.rint(s).astype(np.uint64)  # numpy rint is ties-to-even; exact for these values
    out = np.where(sub, r.astype(np.uint8), out)
    # normal: keep 3 mantissa bits with RNE on the dropped 20 bits
    exp = (a >> 23).astype(np.int64) - 127 + 7
    mant = a & 0x7FFFFF
    q = (exp << 3).astype(np.uint64) | (mant >> 20)
    rem = mant & 0xFFFFF
    rnd = (rem > 0x80000) | ((rem == 0x80000) & ((q & 1) == 1))
    q = q + rnd.astype(np.uint64)
    norm = (~sub) & (~nan)
    out = np.where(norm, (q & 0xFF).astype(np.uint8), out)
    out = np.where(nan, np.uint8(0x7F), out)
    return (out | sign).astype(np.uint8)


def e4m3fn_to_f32(c: np.ndarray) -> np.ndarray:
    c = np.asarray(c, dtype=np.uint8).astype(np.uint32)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m * 2.0**-9, (1.0 + m / 8.0) * 2.0 ** (e.astype(np.int64) - 7))
    val = np.where((e == 0xF) & (m == 0x7), np.nan, val)
    return (sign * val).astype(np.float32)


def quantize(x: np.ndarray, block: int, fmt: str, qmap: np.ndarray | None = None):
    """Quantize an fp32 array (flattened) -> (codes, scales).

    fmt in {"8bit", "4bit", "fp8"}; 4-bit codes are packed two per byte (element 2i
    in the high nibble)."""
    x = np.asarray(x, dtype=np.float32).reshape(-1)
    assert x.size % block == 0
    scale = _block_scale(x, block, fmt == "fp8")
    y = (x.reshape(-1, block) / scale[:, None]).astype(np.float32).reshape(-1)
    if fmt == "fp8":
        # the reference divides on the GPU, whose NaN results are the positive canonical
        # NaN (x86 gives inf / inf a negative one): NaN quotients code as 0x7f
        y = np.where(np.isnan(y), np.float32(np.nan), y)
        return f32_to_e4m3fn(y), scale
    codes = quantize_codes(y, qmap)
    if fmt == "4bit":
        codes = ((codes[0::2] << 4) | codes[1::2]).astype(np.uint8)
    return codes, scale


def dequantize(codes: np.ndarray, scales: np.ndarray, block: int, fmt: str, qmap=None) -> np.ndarray:
    if fmt == "fp8":
        vals = e4m3fn_to_f32(codes)
    else:
        if fmt == "4bit":
            codes = np.stack([codes >> 4, codes & 0xF], axis=-1).reshape(-1)
        vals = qmap[codes.astype(np.int64)]
    return (vals.reshape(-1, block).astype(np.float32) * scales[:, None].astype(np.float32)).reshape(-1).astype(np.float32)


def lp_momentum_step(codes, scales, grad: np.ndarray, *, block: int, fmt: str, qmap,
                     momentum: float, nesterov: bool, maximize: bool):
    """One MuonLP momentum update on a quantized buffer (muon.py:39-56 through the
    quantized state): m = dequant; m' = m * mu + g; store quant(m'); the Nesterov
    input uses the unquantized m'. Returns (codes', scales', g_prime fp32)."""
    g = np.asarray(grad, dtype=np.float32).reshape(-1)
    if maximize:
        g = -g
    m = dequantize(codes, scales, block, fmt, qmap)
    mu = np.float32(momentum)
    m1 = (m * mu).astype(np.float32)
    m1 = (m1 + g).astype(np.float32)
    c2, s2 = quantize(m1, block, fmt, qmap)
    if nesterov:
        gq = (g + (m1 * mu).astype(np.float32)).astype(np.float32)
    else:
        gq = m1
    return c2, s2, gq
