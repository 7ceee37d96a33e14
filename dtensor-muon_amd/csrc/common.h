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

// fp32 -> float8_e4m3fn (bias 7, no infinities, 0x7f/0xff are NaN, max 448) by the
// hardware conversion (v_cvt_pk_fp8_f32: OCP e4m3, round to nearest even; a magnitude that
// rounds above 448 becomes NaN, as torch's cast does). Compared on the GPU with a direct
// restatement of the format (exact RNE onto the e4m3fn grid) for all 2^32 inputs: identical
// except for NaN inputs, which the hardware codes 0xff whatever their sign; torch codes a
// NaN as 0x7f | sign, and so does this function.
MUON_DEVICE uint8_t f32_to_e4m3fn(float f) {
  const uint32_t h = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(f, 0.0f, 0, false) & 0xffu;
  return f != f ? (uint8_t)(0x7fu | ((__float_as_uint(f) >> 24) & 0x80u)) : (uint8_t)h;
}

// float8_e4m3fn -> fp32 by the hardware conversion (v_cvt_f32_fp8); equal to the format's
// definition on all 256 codes (the two NaN codes give a NaN).
MUON_DEVICE float e4m3fn_to_f32(uint8_t v) { return __builtin_amdgcn_cvt_f32_fp8((int)v, 0); }

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

// The apply of one element (weight decay, cautious mask, shape-scaled step), shared by the
// post-pass and the B X epilogue that fuses it.
// muon.py:62-77 for one element, eager op order, no contraction.
template <int PDT, int UDT>
MUON_DEVICE float apply_elem(float p, float u, float wd, int cautious, float adj) {
#pragma clang fp contract(off)
  if (wd != 0.0f) {
    float t = wd * p;
    if (cautious) {
      float prod = u * p;
      float mask = prod > 0.0f ? 1.0f : 0.0f;
      t = t * mask;
    }
    float v = u + t;
    float step = adj * v;
    return p - step;
  }
  // 0-dim fp32 tensor * u: type promotion keeps u's dtype, so the scalar is cast to
  // it first and the product is rounded to it (eager torch semantics).
  float step = Elem<UDT>::round(Elem<UDT>::round(adj) * u);
  return p - step;
}

// apply_elem<bf16, bf16> on 8 packed bf16 values: the update u (q4) and the parameter p
// (pq), 16 bytes each, in one of three straight forms (wd and cautious are uniform over a
// launch): AM 1 cautious weight decay, 2 plain weight decay, 0 no weight decay (the
// bf16-rounded step, adjr = bf16(adj)). The same operations in the same order as
// apply_elem, and the same rounding as f32_to_bf16: v_cvt_pk_bf16_f32 rounds two values to
// nearest even (IEEE, denormals kept), and a NaN result becomes 0x7fc0 whatever its sign
// and payload. So a fused apply writes the post-pass's parameters bit for bit.
typedef __attribute__((ext_vector_type(4))) unsigned int muon_u32x4;
typedef __attribute__((ext_vector_type(2))) float muon_f2x;
typedef __attribute__((ext_vector_type(2))) __bf16 muon_bf2x;
template <int AM>
MUON_DEVICE muon_u32x4 apply_bf16x8(muon_u32x4 q4, muon_u32x4 pq, float adj, float adjr,
                                    float wd) {
  uint32_t ow[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float o[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const float u = __uint_as_float(hh ? q4[e] & 0xffff0000u : q4[e] << 16);
      const float pp = __uint_as_float(hh ? pq[e] & 0xffff0000u : pq[e] << 16);
      {
#pragma clang fp contract(off)
        if constexpr (AM == 1) {
          const float prod = u * pp;
          const float m = prod > 0.0f ? 1.0f : 0.0f;
          const float tt = (wd * pp) * m;
          o[hh] = pp - adj * (u + tt);
        } else if constexpr (AM == 2) {
          o[hh] = pp - adj * (u + wd * pp);
        } else {
          o[hh] = pp - bf16_to_f32(f32_to_bf16(adjr * u));
        }
      }
    }
    uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(muon_f2x{o[0], o[1]}, muon_bf2x));
    w = o[0] != o[0] ? (w & 0xffff0000u) | 0x7fc0u : w;
    w = o[1] != o[1] ? (w & 0x0000ffffu) | 0x7fc00000u : w;
    ow[e] = w;
  }
  return muon_u32x4{ow[0], ow[1], ow[2], ow[3]};
}

// The apply fused into the last B X of a bucket of bf16 parameters: one entry per tensor
// (matrices bidx = t nb .. t nb + nb - 1 of the launch are tensor t's), the stored extents of
// one matrix, and the post-pass's scalars.
constexpr int MUON_APPLY_MAX = 128;
struct MuonApply {
  void* params[MUON_APPLY_MAX];
  float adj[MUON_APPLY_MAX];  // lr * lr_ratio per tensor
  int64_t nb, prows, pcols;
  float wd;
  int cautious;
};

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
// X0/X1: the wide iterate (m_pad x n_pad in rows of x_pitch elements), ping-ponged by
// the GEMM; the
// result of a tall matrix is written transposed (n_pad x m_pad) into one of them.
// A bf16 iterate with at most 64 rows (short) is padded to 64 rows, not 256, and its
// iterations run in short.hip with Gram partials per column range (off_gpart).
struct OrthLayout {
  int64_t rows, cols;  // stored (param) matrix shape
  int64_t m, n;        // m = min, n = max: the iteration runs on the wide m x n matrix
  int64_t m_pad, n_pad;
  int64_t x_pitch;     // row pitch of X0/X1 in elements: n_pad (+ 64 beyond 4096 columns)
  int tall;            // rows > cols: stored layout is the transpose of X
  int short_m;         // bf16 and m <= 64: short.hip iterations
  int es;              // element size of the iteration dtype
  int64_t batch;       // capacity in matrices
  int64_t parts;       // norm partials per matrix
  int64_t gparts;      // short: Gram partials (column ranges) per matrix
  size_t off_x0, off_x1, off_a, off_b, off_part, off_scale, off_qtab, off_rows, off_gpart,
      total;
};

// Code-search tables of the 8/4-bit quantized state (lp.hip): one byte per bucket of the
// order-preserving key of an fp32 value (key >> 18), then 256 + MUON_QTHR_PAD uint32
// thresholds.
constexpr int MUON_QTAB_SHIFT = 18;
constexpr int MUON_QTAB_SIZE = 1 << (32 - MUON_QTAB_SHIFT);
constexpr int MUON_QTHR_PAD = 4;
// The last pad slot (never compared: lookups read thresholds 0 .. 257) holds 0 when no key
// bucket holds more than two thresholds (every standard map), else 1.
constexpr int MUON_QTHR_FLAG = 256 + MUON_QTHR_PAD - 1;
constexpr int MUON_QTAB_BYTES = MUON_QTAB_SIZE + (256 + MUON_QTHR_PAD) * 4;

OrthLayout muon_orth_layout(int dtype, int64_t batch, int64_t rows, int64_t cols);
