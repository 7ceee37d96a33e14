// Shared device helpers for the MI355X (gfx950) Muon kernels.
//
// Numeric conventions follow PyTorch's CPU/GPU semantics so the kernels can be
// compared bit-for-bit with the CPU oracle where the reference is elementwise:
//  * fp32 -> bf16 is round-to-nearest-even, NaN -> 0x7FC0 (torch's BFloat16 cast).
//  * fp32 -> fp8 e4m3fn is round-to-nearest-even with magnitudes that round past
//    448 mapped to NaN (torch's Float8_e4m3fn cast).
//  * No FMA contraction in elementwise math (see the pragmas in each kernel).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/muon_amd.h"

#define MUON_DEVICE __device__ __forceinline__

typedef uint16_t bf16_t;  // raw bfloat16 bits

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_mfma;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;

MUON_DEVICE float bf16_to_f32(bf16_t v) { return __uint_as_float(((uint32_t)v) << 16); }

MUON_DEVICE bf16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)0x7fc0;  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
}

// fp16 (IEEE binary16) <-> fp32 via the hardware conversion (exact / RNE).
MUON_DEVICE float f16_to_f32(uint16_t v) {
  _Float16 h;
  __builtin_memcpy(&h, &v, 2);
  return (float)h;
}
MUON_DEVICE uint16_t f32_to_f16(float f) {
  _Float16 h = (_Float16)f;
  uint16_t v;
  __builtin_memcpy(&v, &h, 2);
  return v;
}

// Element load/store by dtype code (MUON_DT_*).
template <int DT>
struct Elem;
template <>
struct Elem<MUON_DT_F32> {
  typedef float T;
  static MUON_DEVICE float load(const void* p, int64_t i) { return ((const float*)p)[i]; }
  static MUON_DEVICE void store(void* p, int64_t i, float v) { ((float*)p)[i] = v; }
  static MUON_DEVICE float round(float v) { return v; }
};
template <>
struct Elem<MUON_DT_BF16> {
  typedef bf16_t T;
  static MUON_DEVICE float load(const void* p, int64_t i) { return bf16_to_f32(((const bf16_t*)p)[i]); }
  static MUON_DEVICE void store(void* p, int64_t i, float v) { ((bf16_t*)p)[i] = f32_to_bf16(v); }
  static MUON_DEVICE float round(float v) { return bf16_to_f32(f32_to_bf16(v)); }
};
template <>
struct Elem<MUON_DT_F16> {
  typedef uint16_t T;
  static MUON_DEVICE float load(const void* p, int64_t i) { return f16_to_f32(((const uint16_t*)p)[i]); }
  static MUON_DEVICE void store(void* p, int64_t i, float v) { ((uint16_t*)p)[i] = f32_to_f16(v); }
  static MUON_DEVICE float round(float v) { return f16_to_f32(f32_to_f16(v)); }
};

// Eight consecutive elements as floats through one or two 16-byte accesses. The
// caller guarantees 16-byte alignment of element i.
template <int DT>
struct Vec8;
template <>
struct Vec8<MUON_DT_F32> {
  static MUON_DEVICE void load(const void* p, int64_t i, float (&v)[8]) {
    const float4 a = ((const float4*)((const float*)p + i))[0];
    const float4 b = ((const float4*)((const float*)p + i))[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static MUON_DEVICE void store(void* p, int64_t i, const float (&v)[8]) {
    ((float4*)((float*)p + i))[0] = make_float4(v[0], v[1], v[2], v[3]);
    ((float4*)((float*)p + i))[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
};
template <>
struct Vec8<MUON_DT_BF16> {
  static MUON_DEVICE void load(const void* p, int64_t i, float (&v)[8]) {
    const uint4 w = *(const uint4*)((const bf16_t*)p + i);
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = bf16_to_f32((bf16_t)(u[k] & 0xffffu));
      v[2 * k + 1] = bf16_to_f32((bf16_t)(u[k] >> 16));
    }
  }
  static MUON_DEVICE void store(void* p, int64_t i, const float (&v)[8]) {
    uint32_t u[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      u[k] = (uint32_t)f32_to_bf16(v[2 * k]) | ((uint32_t)f32_to_bf16(v[2 * k + 1]) << 16);
    *(uint4*)((bf16_t*)p + i) = make_uint4(u[0], u[1], u[2], u[3]);
  }
};
template <>
struct Vec8<MUON_DT_F16> {
  static MUON_DEVICE void load(const void* p, int64_t i, float (&v)[8]) {
    const uint4 w = *(const uint4*)((const uint16_t*)p + i);
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = f16_to_f32((uint16_t)(u[k] & 0xffffu));
      v[2 * k + 1] = f16_to_f32((uint16_t)(u[k] >> 16));
    }
  }
  static MUON_DEVICE void store(void* p, int64_t i, const float (&v)[8]) {
    uint32_t u[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      u[k] = (uint32_t)f32_to_f16(v[2 * k]) | ((uint32_t)f32_to_f16(v[2 * k + 1]) << 16);
    *(uint4*)((uint16_t*)p + i) = make_uint4(u[0], u[1], u[2], u[3]);
  }
};

// Non-temporal 16-byte global access (streamed data that no kernel re-reads soon: the
// elementwise passes move every byte once).
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_nt;
MUON_DEVICE uint4 ld_nt(const void* p) {
  const u32x4_nt v = __builtin_nontemporal_load((const u32x4_nt*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
MUON_DEVICE void st_nt(void* p, uint4 w) {
  const u32x4_nt v = {w.x, w.y, w.z, w.w};
  __builtin_nontemporal_store(v, (u32x4_nt*)p);
}

// Eight consecutive elements kept as raw bits (16 B for 2-byte types, 32 B for fp32),
// loaded and stored non-temporally; unpack()/pack() convert as Vec8 does.
template <int DT>
struct Raw8 {
  static constexpr int N = DT == MUON_DT_F32 ? 2 : 1;
  uint4 w[N];
  MUON_DEVICE void load(const void* p, int64_t i) {
    const char* b = (const char*)p + i * (DT == MUON_DT_F32 ? 4 : 2);
#pragma unroll
    for (int k = 0; k < N; ++k) w[k] = ld_nt(b + 16 * k);
  }
  MUON_DEVICE void store(void* p, int64_t i) const {
    char* b = (char*)p + i * (DT == MUON_DT_F32 ? 4 : 2);
#pragma unroll
    for (int k = 0; k < N; ++k) st_nt(b + 16 * k, w[k]);
  }
  MUON_DEVICE void unpack(float (&v)[8]) const {
    if constexpr (DT == MUON_DT_F32) {
      const uint32_t u[8] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = __uint_as_float(u[e]);
    } else {
      const uint32_t u[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if constexpr (DT == MUON_DT_BF16) {
          v[2 * k] = bf16_to_f32((bf16_t)(u[k] & 0xffffu));
          v[2 * k + 1] = bf16_to_f32((bf16_t)(u[k] >> 16));
        } else {
          v[2 * k] = f16_to_f32((uint16_t)(u[k] & 0xffffu));
          v[2 * k + 1] = f16_to_f32((uint16_t)(u[k] >> 16));
        }
      }
    }
  }
  MUON_DEVICE void pack(const float (&v)[8]) {
    if constexpr (DT == MUON_DT_F32) {
      w[0] = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                        __float_as_uint(v[3]));
      w[1] = make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                        __float_as_uint(v[7]));
    } else {
      uint32_t u[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if constexpr (DT == MUON_DT_BF16)
          u[k] = (uint32_t)f32_to_bf16(v[2 * k]) | ((uint32_t)f32_to_bf16(v[2 * k + 1]) << 16);
        else
          u[k] = (uint32_t)f32_to_f16(v[2 * k]) | ((uint32_t)f32_to_f16(v[2 * k + 1]) << 16);
      }
      w[0] = make_uint4(u[0], u[1], u[2], u[3]);
    }
  }
};

// fp32 -> float8_e4m3fn (bias 7, no infinities, 0x7f/0xff are NaN, max 448).
// Written from the format definition: exact round-to-nearest-even onto the e4m3fn
// grid; a magnitude that rounds above 448 becomes NaN (matching torch's cast).
// Branch-free (both the subnormal and the normal rounding are formed, one selected).
MUON_DEVICE uint8_t f32_to_e4m3fn(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  // |f| < 2^-6: subnormal range of e4m3 (step 2^-9). |f| * 2^9 rounded to an integer with
  // ties-to-even is exact in fp32 (power-of-two scaling); 8 is the smallest normal 0x08.
  const uint32_t sub = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
  // normal range: keep 3 mantissa bits, round to nearest even on the dropped 20 bits
  uint32_t q = ((((a >> 23) - 120u) << 3) | ((a >> 20) & 7u)) & 0xffu;
  const uint32_t rem = a & 0xfffffu;
  q += (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) ? 1u : 0u;
  uint32_t r = a < 0x3c800000u ? sub : q;
  // values >= 464 (the midpoint between 448 and the next, unrepresentable, grid point
  // 480) round above the largest finite value; 464 itself ties to even (448). NaN and
  // infinity land here too.
  r = a > 0x43e80000u ? 0x7fu : r;
  return (uint8_t)(sign | r);
}

MUON_DEVICE float e4m3fn_to_f32(uint8_t v) {
  const uint32_t sign = ((uint32_t)v & 0x80u) << 24;
  const uint32_t e = (v >> 3) & 0xfu;
  const uint32_t m = v & 0x7u;
  const float sub = (float)m * 0.001953125f;  // m * 2^-9, exact
  uint32_t bits = e == 0 ? __float_as_uint(sub) : (((e + 120u) << 23) | (m << 20));
  bits = (e == 0xf && m == 0x7) ? 0x7fc00000u : bits;
  return __uint_as_float(sign | bits);
}

MUON_DEVICE float warp_sum(float v) {
  // Fixed butterfly order over the 64-lane wavefront: deterministic.
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

MUON_DEVICE float warp_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

static inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Thread-local last-error text for muon_amd_last_error().
void muon_set_error(const char* fmt, ...);

#define MUON_CHECK_LAUNCH(what)                                          \
  do {                                                                   \
    hipError_t _e = hipGetLastError();                                   \
    if (_e != hipSuccess) {                                              \
      muon_set_error("%s: launch failed: %s", what, hipGetErrorString(_e)); \
      return MUON_ERR_LAUNCH;                                            \
    }                                                                    \
  } while (0)

// Workspace layout shared by the prepass, iteration and postpass entry points.
// X0/X1: the wide iterate (m_pad x n_pad, row-major), ping-ponged by the GEMM; the
// result of a tall matrix is written transposed (n_pad x m_pad) into one of them.
struct OrthLayout {
  int64_t rows, cols;  // stored (param) matrix shape
  int64_t m, n;        // m = min, n = max: the iteration runs on the wide m x n matrix
  int64_t m_pad, n_pad;
  int tall;            // rows > cols: stored layout is the transpose of X
  int es;              // element size of the iteration dtype
  int64_t batch;       // capacity in matrices
  int64_t parts;       // norm partials per matrix
  size_t off_x0, off_x1, off_a, off_b, off_part, off_scale, off_qtab, off_rows, total;
};

// Code-search tables of the 8/4-bit quantized state (lp.hip): one byte per bucket of the
// order-preserving key of an fp32 value (key >> 18), then 256 + MUON_QTHR_PAD uint32
// thresholds.
constexpr int MUON_QTAB_SHIFT = 18;
constexpr int MUON_QTAB_SIZE = 1 << (32 - MUON_QTAB_SHIFT);
constexpr int MUON_QTHR_PAD = 4;
constexpr int MUON_QTAB_BYTES = MUON_QTAB_SIZE + (256 + MUON_QTHR_PAD) * 4;

OrthLayout muon_orth_layout(int dtype, int64_t batch, int64_t rows, int64_t cols);
