// Quantized momentum state for MuonLP (8-bit / 4-bit dynamic-map codes and fp8
// e4m3fn codes, one fp32 absmax scale per block of consecutive values).
//
// The format and rounding follow the blockwise scheme MuonLP gets from torchao 0.17.0
// (optim_lp.py:118-133): scale = max(|x|) over the block clipped at 1e-12 (divided by
// 448 for fp8), y = x / scale, and for the map formats the code is found by a
// fixed-depth binary search over the sorted map followed by a round-half-up step
// between the two neighbouring entries. The general kernel: one wavefront owns one
// block, read twice (absmax, then quantize) with the second read served from cache; the
// tiled kernel (below) keeps each block in registers and finds 8-bit codes through a
// bucket table that gives the same result as the search.
#include <algorithm>
#include <type_traits>

#include "common.h"

namespace {

typedef __attribute__((ext_vector_type(2))) float f2x;
typedef __attribute__((ext_vector_type(2))) __bf16 bf2x;  // v_cvt_pk_bf16_f32 (RNE)

struct LpArgs {
  void* grads[MUON_MAX_TENSORS];
  void* codes[MUON_MAX_TENSORS];
  float* scales[MUON_MAX_TENSORS];
  const float* qmap;
  int64_t nb, rows, cols, numel, block;
  int64_t blocks_per_tensor;
  void* direct;  // workspace stored-layout X, matrix 0 of this launch
  int64_t d_pitch, d_mstride;
  float momentum;
  int nesterov, maximize;
};

// Largest i with q[i] <= y over a sorted 256-entry map (0 if none, or y NaN).
MUON_DEVICE int quant_search8(float y, const float* q) {
  int c = (y >= q[128]) ? 128 : 0;
  c += (y >= q[c + 64]) ? 64 : 0;
  c += (y >= q[c + 32]) ? 32 : 0;
  c += (y >= q[c + 16]) ? 16 : 0;
  c += (y >= q[c + 8]) ? 8 : 0;
  c += (y >= q[c + 4]) ? 4 : 0;
  c += (y >= q[c + 2]) ? 2 : 0;
  c += (y >= q[c + 1]) ? 1 : 0;
  return c;
}

template <int QF>
MUON_DEVICE int quant_code(float y, const float* q) {
  if (QF == MUON_Q_8BIT) {
    const int c = quant_search8(y, q);
    const int up = c + 1 > 255 ? 255 : c + 1;
    const float lo = q[c], hi = q[up];
    const float res = y - lo;
    const float half = (hi - lo) * 0.5f;
    return res >= half ? up : c;
  } else if (QF == MUON_Q_4BIT) {
    int c = (y >= q[8]) ? 8 : 0;
    c += (y >= q[c + 4]) ? 4 : 0;
    c += (y >= q[c + 2]) ? 2 : 0;
    c += (y >= q[c + 1]) ? 1 : 0;
    const int up = c + 1 > 15 ? 15 : c + 1;
    const float lo = q[c], hi = q[up];
    const float res = y - lo;
    const float half = (hi - lo) * 0.5f;
    return res >= half ? up : c;
  } else {
    // a NaN quotient codes as the positive NaN 0x7f (the canonical NaN a GPU division
    // returns; its sign is not defined by IEEE 754)
    return y != y ? 0x7f : f32_to_e4m3fn(y);
  }
}

// Value of element e (index within the tensor) from the stored codes.
template <int QF>
MUON_DEVICE float dequant(const uint8_t* codes, int64_t e, const float* q, float scale) {
  if (QF == MUON_Q_8BIT) return q[codes[e]] * scale;
  if (QF == MUON_Q_4BIT) {
    const uint8_t b = codes[e >> 1];
    const int c = (e & 1) ? (b & 15) : (b >> 4);
    return q[c] * scale;
  }
  return e4m3fn_to_f32(codes[e]) * scale;
}

// Unit = the values that share one code byte: 1 for 8-bit / fp8, 2 for 4-bit.
template <int QF>
constexpr int unit_size() {
  return QF == MUON_Q_4BIT ? 2 : 1;
}

// Block absmax as the bit patterns of |v|: for non-negative floats the unsigned order is
// the numeric order, and NaN patterns sort above infinity, so a NaN in the block wins as
// it does in torch's amax (and the oracle's np.max).
MUON_DEVICE uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7fffffffu; }
MUON_DEVICE uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off, 64));
  return v;
}
// Block scale from the absmax: clipped below at 1e-12 (a NaN absmax stays NaN, as
// torch's clamp keeps it), divided by 448 for fp8.
template <int QF>
MUON_DEVICE float block_scale(uint32_t amax_bits) {
  const float amax = __uint_as_float(amax_bits);
  float sc = amax < 1e-12f ? 1e-12f : amax;
  if (QF == MUON_Q_FP8) sc = sc / 448.0f;
  return sc;
}

template <int GDT, int QF>
__global__ __launch_bounds__(256) void lp_prepass_kernel(LpArgs a) {
#pragma clang fp contract(off)
  __shared__ float q[256];
  const int tid = threadIdx.x;
  if (QF != MUON_Q_FP8) q[tid] = a.qmap[tid < (QF == MUON_Q_8BIT ? 256 : 16) ? tid : 0];
  __syncthreads();
  const int lane = tid & 63;
  const int64_t blk = (int64_t)blockIdx.x * 4 + (tid >> 6);
  if (blk >= a.blocks_per_tensor) return;
  const int t = blockIdx.y;
  const void* gp = a.grads[t];
  uint8_t* codes = (uint8_t*)a.codes[t];
  float* scales = a.scales[t];
  const float old_scale = scales[blk];
  const int64_t e0 = blk * a.block;
  constexpr int US = unit_size<QF>();
  const int64_t units = a.block / US;

  // pass 1: momentum in fp32 and the block absmax of the new buffer
  uint32_t ab = 0;
  for (int64_t u = lane; u < units; u += 64) {
#pragma unroll
    for (int k = 0; k < US; ++k) {
      const int64_t e = e0 + u * US + k;
      float g = Elem<GDT>::load(gp, e);
      if (a.maximize) g = -g;
      float m = dequant<QF>(codes, e, q, old_scale) * a.momentum;
      m = m + g;
      ab = max(ab, abs_bits(m));
    }
  }
  const float sc = block_scale<QF>(wave_max_u32(ab));

  // pass 2: recompute, quantize with the new scale, emit X = cast(g') in the stored layout
  const int64_t mat_elems = a.rows * a.cols;
  for (int64_t u = lane; u < units; u += 64) {
    int cq[US];
    float xs[US];
#pragma unroll
    for (int k = 0; k < US; ++k) {
      const int64_t e = e0 + u * US + k;
      float g = Elem<GDT>::load(gp, e);
      if (a.maximize) g = -g;
      float m = dequant<QF>(codes, e, q, old_scale) * a.momentum;
      m = m + g;
      cq[k] = quant_code<QF>(m / sc, q);
      float gq = m;
      if (a.nesterov) {
        float tt = m * a.momentum;
        gq = g + tt;
      }
      xs[k] = gq;
    }
    // every lane has read its own code bytes above; write the new ones
    if (QF == MUON_Q_4BIT)
      codes[(e0 >> 1) + u] = (uint8_t)((cq[0] << 4) | cq[US - 1]);
    else
      codes[e0 + u] = (uint8_t)cq[0];
#pragma unroll
    for (int k = 0; k < US; ++k) {
      const int64_t e = e0 + u * US + k;
      const int64_t mb = e / mat_elems, rem = e % mat_elems;
      const int64_t r = rem / a.cols, c = rem % a.cols;
      const int64_t o = ((int64_t)t * a.nb + mb) * a.d_mstride + r * a.d_pitch + c;
      Elem<MUON_DT_BF16>::store(a.direct, o, xs[k]);
    }
  }
  if (lane == 0) scales[blk] = sc;
}

// ---- tiled variant -------------------------------------------------------------------
// One workgroup owns 64 stored rows x 256 columns of one matrix, 8 rows per pass, each
// lane 8 consecutive values (16-byte loads of the gradient, 8/4-byte loads of the
// codes). A quantization block is block/8 consecutive lanes of one row, so its absmax
// is a shuffle reduction and the new momentum never leaves registers between the
// absmax and the requantization. The same workgroup writes X in the layout the
// iteration reads (the wide X0: the stored layout itself, or, for a tall matrix, its
// transpose staged through LDS) and the sum of squares of its X values as one norm
// partial, so no second pass over X is needed.
// Applies when cols % 256 == 0 and block is a power of two in [8, 256].
struct LpTileArgs {
  void* grads[MUON_MAX_TENSORS];
  void* codes[MUON_MAX_TENSORS];
  float* scales[MUON_MAX_TENSORS];
  const float* qmap;
  int64_t nb, rows, cols;
  int block_shift;          // log2(block)
  void* x0;                 // X0 of matrix 0 of this launch
  int64_t x_pitch, x_mstride;
  const uint8_t* qtab;      // 8/4-bit: bucket table (MUON_QTAB_SIZE bytes), then thresholds
  float* partials;          // partials of matrix 0 of this launch
  int64_t parts;            // partial slots per matrix
  int tiles_c, tiles_used;  // column tiles (cols / 256), tiles with data or padding
  float momentum;
  int nesterov, maximize;
  // deferred scales (blocks larger than 256 values): block / 256, blocks per tensor, and
  // the running absmax (as fp32 bit patterns) of every block of this launch's tensors,
  // zero before the launch
  uint32_t block256;
  int64_t nblocks;
  uint32_t* bmax;
};

constexpr int LPT_ROWS = 64, LPT_COLS = 256, LPT_PITCH = LPT_COLS + 8;

template <int QF>
struct LpCodes;  // code bytes of 8 consecutive values
template <>
struct LpCodes<MUON_Q_8BIT> {
  typedef uint2 T;
  static MUON_DEVICE T load(const uint8_t* c, int64_t e) { return *(const uint2*)(c + e); }
  static MUON_DEVICE int get(const T& v, int k) { return ((k < 4 ? v.x : v.y) >> (8 * (k & 3))) & 255; }
  static MUON_DEVICE void store(uint8_t* c, int64_t e, const int (&q)[8]) {
    uint2 v;
    v.x = (uint32_t)q[0] | ((uint32_t)q[1] << 8) | ((uint32_t)q[2] << 16) | ((uint32_t)q[3] << 24);
    v.y = (uint32_t)q[4] | ((uint32_t)q[5] << 8) | ((uint32_t)q[6] << 16) | ((uint32_t)q[7] << 24);
    *(uint2*)(c + e) = v;
  }
};
template <>
struct LpCodes<MUON_Q_FP8> : LpCodes<MUON_Q_8BIT> {};
template <>
struct LpCodes<MUON_Q_4BIT> {
  typedef uint32_t T;  // byte i holds values 2i (high nibble) and 2i + 1
  static MUON_DEVICE T load(const uint8_t* c, int64_t e) { return *(const uint32_t*)(c + (e >> 1)); }
  static MUON_DEVICE int get(const T& v, int k) {
    const uint32_t b = (v >> (8 * (k >> 1))) & 255;
    return (k & 1) ? (int)(b & 15) : (int)(b >> 4);
  }
  static MUON_DEVICE void store(uint8_t* c, int64_t e, const int (&q)[8]) {
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) v |= (uint32_t)((q[2 * i] << 4) | q[2 * i + 1]) << (8 * i);
    *(uint32_t*)(c + (e >> 1)) = v;
  }
};

template <int QF>
MUON_DEVICE float code_value(int code, const float* q) {
  if (QF == MUON_Q_FP8) return e4m3fn_to_f32((uint8_t)code);
  return q[code];
}

// ---- faster exact code search ------------------------------------------------------
// Order-preserving integer key of a non-NaN fp32 value (larger value, larger key), and
// the value of a key (the smallest value of bucket b is the value of key b << SHIFT).
MUON_DEVICE uint32_t f32_order_key(float v) {
  const uint32_t b = __float_as_uint(v);
  return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);  // negative: ~b; else b | sign
}
MUON_DEVICE float f32_from_order_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// The code as a function of y (search, then the half-step rule, in fp32) never
// decreases as y grows: within [q[c], q[c+1]) the rounded difference y - q[c] grows with
// y, and at q[c+1] the search moves up. So code(y) is the number of thresholds
// thr[k] <= key(y), thr[k] = the smallest order key whose value codes to at least k + 1
// (k < nq - 1; the entries from nq - 1 on are 0xffffffff). The thresholds are found by
// bisection over keys with quant_code itself, so the count reproduces it bit for bit.
// One thread per threshold; one workgroup.
template <int QF>
__global__ __launch_bounds__(256) void build_qthr_kernel(const float* qmap, uint32_t* thr) {
  constexpr int NQ = QF == MUON_Q_8BIT ? 256 : 16;
  __shared__ float q[256];
  __shared__ uint32_t ts[256];
  const int k = threadIdx.x;
  q[k] = qmap[k < NQ ? k : 0];
  __syncthreads();
  uint32_t t = 0xffffffffu;
  if (k < NQ - 1) {
    uint32_t lo = f32_order_key(-__builtin_inff()), hi = f32_order_key(__builtin_inff());
    while (lo < hi) {
      const uint32_t mid = lo + (hi - lo) / 2;
      if (quant_code<QF>(f32_from_order_key(mid), q) >= k + 1)
        hi = mid;
      else
        lo = mid + 1;
    }
    t = lo;
  }
  // the flag: three consecutive thresholds in one key bucket (sorted, so any bucket with
  // more than two has such a triple)
  ts[k] = t;
  __syncthreads();
  const int dense = k + 2 < NQ - 1 && (ts[k] >> MUON_QTAB_SHIFT) == (ts[k + 2] >> MUON_QTAB_SHIFT);
  const int any_dense = __syncthreads_or(dense);
  thr[k] = t;
  if (k < MUON_QTHR_PAD)
    thr[256 + k] = 256 + k == MUON_QTHR_FLAG ? (any_dense ? 1u : 0u) : 0xffffffffu;
}

// qtab[b] = the number of thresholds <= b << SHIFT (the code of the smallest value of
// key bucket b). For y in bucket b the code is qtab[b] plus the thresholds of bucket b
// up to key(y): at most 2 for the standard 8-bit map (1 for the 4-bit map), which the
// lookup steps over; a map with more takes the full count. One thread per bucket.
__global__ __launch_bounds__(256) void build_qtab_kernel(const uint32_t* thr, int nq,
                                                         uint8_t* qtab) {
  const uint32_t b = blockIdx.x * 256u + threadIdx.x;
  const uint32_t key = b << MUON_QTAB_SHIFT;
  int lo = 0, hi = nq - 1;  // thr[nq - 1] = 0xffffffff bounds the count
  while (lo < hi) {
    const int mid = (lo + hi) / 2;
    if (thr[mid] <= key)
      lo = mid + 1;
    else
      hi = mid;
  }
  qtab[b] = (uint8_t)lo;
}

// quant_code<QF> (8- or 4-bit) of a non-NaN y through the thresholds: a table read and
// two compares, branch-free so the compiler can overlap the lookups of many values. Sets
// `more` when the bucket holds more thresholds than that (then quant_code_thr_all gives
// the code). A NaN y gets an in-range code here; the caller routes it to
// quant_code_thr_all.
template <bool CHECK_MORE>
MUON_DEVICE int quant_code_thr(float y, const uint32_t* thr, const uint8_t* qtab, bool& more) {
  const uint32_t ky = f32_order_key(y);
  const int c0 = qtab[ky >> MUON_QTAB_SHIFT];
  const int c = c0 + (ky >= thr[c0] ? 1 : 0) + (ky >= thr[c0 + 1] ? 1 : 0);
  if (CHECK_MORE) more = more || ky >= thr[c0 + 2];
  return c;
}

// The code as the full count of thresholds <= key(y).
template <int NQ>
MUON_DEVICE int quant_code_thr_all(float y, const uint32_t* thr) {
  const uint32_t ky = f32_order_key(y);
  int lo = 0, hi = NQ - 1;
  while (lo < hi) {
    const int mid = (lo + hi) / 2;
    if (thr[mid] <= ky)
      lo = mid + 1;
    else
      hi = mid;
  }
  return (y != y) ? 0 : lo;
}

// Workgroup barrier for LDS data: release and acquire fences scoped to LDS around the
// barrier, so LDS accesses are ordered across it (lgkmcnt(0), s_barrier) while, unlike
// __syncthreads, outstanding global loads and stores are not waited for.
MUON_DEVICE void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Unsigned max over aligned groups of `lanes` consecutive lanes (a power of two, 1 to
// 32; wave-uniform, so each level is a scalar branch): DPP moves within rows of 16 (quad
// xor 1 and 2, then the 8- and 16-lane mirrors, which pair every lane with one of the
// other half) and a swizzle for xor 16.
MUON_DEVICE uint32_t group_max_u32(uint32_t v, int lanes) {
  if (lanes > 1) v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true));
  if (lanes > 2) v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true));
  if (lanes > 4) v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, true));
  if (lanes > 8) v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, true));
  // bitmask swizzle within 32 lanes: and 0x1f, or 0, xor 0x10
  if (lanes > 16) v = max(v, (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401F));
  return v;
}
typedef __attribute__((ext_vector_type(2))) __bf16 bf2v;
typedef __attribute__((ext_vector_type(4))) short lp_i16x4;

// New momentum of 8 consecutive values: m = g * gs + (dequant(code) * old_scale) * mu, in
// fp32 with one rounding per operation (the fma rounds once; g * gs is exact). Also the
// unsigned max of |m| as bit patterns. Shared by every LP kernel so a value recomputed
// by a second pass has the same bits as in the first.
template <int QF>
MUON_DEVICE void lp_momentum8(const float (&g)[8], const typename LpCodes<QF>::T& cw, float osc,
                              float mom, float gs, const float* q, float (&m)[8], uint32_t& ab) {
#pragma clang fp contract(off)
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float v;
    if constexpr (QF == MUON_Q_FP8) {
      // hardware e4m3 conversion straight from byte k of the loaded code word
      const int wd = (int)(k < 4 ? cw.x : cw.y);
      switch (k & 3) {  // the byte selector must be a constant; k is unrolled
        case 0: v = __builtin_amdgcn_cvt_f32_fp8(wd, 0); break;
        case 1: v = __builtin_amdgcn_cvt_f32_fp8(wd, 1); break;
        case 2: v = __builtin_amdgcn_cvt_f32_fp8(wd, 2); break;
        default: v = __builtin_amdgcn_cvt_f32_fp8(wd, 3); break;
      }
      v = v * osc;
    } else {
      v = code_value<QF>(LpCodes<QF>::get(cw, k), q) * osc;
    }
    v = v * mom;
    m[k] = __builtin_fmaf(g[k], gs, v);
    ab = max(ab, abs_bits(m[k]));
  }
}

// Codes of 8 values m / sc: for fp8 the packed code bytes (c8), for the map formats the
// 8 code indices (cq), through the threshold tables in LDS.
template <int QF>
MUON_DEVICE void lp_codes8(const float (&m)[8], float sc, bool sparse_map, const uint32_t* qthr,
                           const uint8_t* qtab, int (&cq)[8], uint2& c8) {
#pragma clang fp contract(off)
  // The quotients m / sc, correctly rounded, by Markstein's method from the correctly
  // rounded reciprocal r = 1 / sc (one IEEE division per 8 values): q0 = m r, then the
  // exact remainder e = m - sc q0 (fma) and y = q0 + e r (fma) is the rounded quotient
  // (P. Markstein, IBM J. Res. Dev. 34(1), 1990). It needs normal intermediates: r normal
  // (sc <= 2^125), e exact and normal (|m| >= 2^-78) and q0 normal (|m| >= sc 2^-100).
  // A lane with any value outside that range (zeros included) takes the IEEE division for
  // its 8 values; NaN or infinite scales fail the first test. Quotients above 1 (fp8:
  // sc = absmax / 448, so |m| / sc <= 448) reduce to |m| <= sc: m = 2^k m' with m' in
  // (sc / 2, sc] scales q0, e and y by exactly 2^k while they stay normal and finite, which
  // the range above and a finite m (|q0| <= 448, |e| <= ulp(m)) guarantee. Checked against the IEEE
  // division on the CPU over every |m| <= sc for eight scales and on random pairs with
  // |m| up to 448 sc.
  float ys[8];
  const float r = 1.0f / sc;
  const float lim = fmaxf(0x1p-78f, sc * 0x1p-100f);
  bool fast = sc <= 0x1p125f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float q0 = m[k] * r;
    const float e = __builtin_fmaf(-sc, q0, m[k]);
    ys[k] = __builtin_fmaf(e, r, q0);
    fast = fast && fabsf(m[k]) >= lim;
  }
  if (!fast) {
#pragma unroll
    for (int k = 0; k < 8; ++k) ys[k] = m[k] / sc;
  }
  if constexpr (QF == MUON_Q_FP8) {
    // v_cvt_pk_fp8_f32 writes two codes into the low or high half of the word
    uint32_t w0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ys[0], ys[1], 0, false);
    w0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ys[2], ys[3], (int)w0, true);
    uint32_t w1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ys[4], ys[5], 0, false);
    w1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ys[6], ys[7], (int)w1, true);
    if (!(sc <= 3.40282347e38f)) {
      // NaN or infinite scale: NaN quotients code as the positive NaN 0x7f
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (ys[k] != ys[k]) {
          uint32_t& w = k < 4 ? w0 : w1;
          w = (w & ~(0xffu << (8 * (k & 3)))) | (0x7fu << (8 * (k & 3)));
        }
      }
    }
    c8 = make_uint2(w0, w1);
  } else {
    bool more = false;
    if (sparse_map) {
      // no key bucket holds more than two thresholds: the third compare is never true
#pragma unroll
      for (int k = 0; k < 8; ++k) cq[k] = quant_code_thr<false>(ys[k], qthr, qtab, more);
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) cq[k] = quant_code_thr<true>(ys[k], qthr, qtab, more);
    }
    // y is NaN only when the scale is NaN or infinite: those blocks take the full
    // count, which codes NaN as 0
    if (more || !(sc <= 3.40282347e38f)) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        cq[k] = quant_code_thr_all<QF == MUON_Q_8BIT ? 256 : 16>(ys[k], qthr);
    }
  }
}

// Block index of element e (a multiple of 256 apart from the block start) for a block of
// block256 * 256 values: a 32-bit division (the launcher checks e / 256 < 2^32).
MUON_DEVICE int64_t lp_block_of(int64_t e, uint32_t block256) {
  return (int64_t)((uint32_t)(e >> 8) / block256);
}

template <int GDT, int QF, bool TALL, bool DEFER>
__global__ __launch_bounds__(256) void lp_prepass_tile_kernel(LpTileArgs a) {
#pragma clang fp contract(off)
  constexpr bool MAP = QF != MUON_Q_FP8;
  constexpr bool TABLES = MAP && !DEFER;  // code search here (not in a requant pass)
  __shared__ float q[256];
  __shared__ __align__(16) uint8_t qtab[TABLES ? MUON_QTAB_SIZE : 16];
  __shared__ __align__(16) uint32_t qthr[TABLES ? 256 + MUON_QTHR_PAD : 4];
  // the tall transpose tile: one 32-row half at a time when the code-search tables are
  // here (they take 18 KB of LDS, and four workgroups per CU need a quarter of the CU's
  // 160 KB), else the whole 64 rows
  constexpr int TROWS = TABLES ? LPT_ROWS / 2 : LPT_ROWS;
  __shared__ bf16_t tileT[TALL ? TROWS : 1][TALL ? LPT_PITCH : 1];
  __shared__ float wsum[4];
  __shared__ uint32_t wmaxs[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int mat = blockIdx.y;
  float* part = a.partials + (int64_t)mat * a.parts;
  if ((int)blockIdx.x >= a.tiles_used) {
    if (tid == 0) part[blockIdx.x] = 0.0f;
    return;
  }
  const int t = (int)(mat / a.nb);
  const int64_t mb = mat % a.nb;
  const int tr = blockIdx.x / a.tiles_c, tcol = blockIdx.x % a.tiles_c;
  const int64_t r0 = (int64_t)tr * LPT_ROWS, c0 = (int64_t)tcol * LPT_COLS;
  const void* gp = a.grads[t];
  uint8_t* codes = (uint8_t*)a.codes[t];
  float* scales = a.scales[t];
  const int chunk = lane & 31;              // 8-value chunk within the row
  const int rsub = wave * 2 + (lane >> 5);  // row within the 8-row pass
  const int64_t c = c0 + chunk * 8;
  const int block_lanes = DEFER ? 32 : 1 << (a.block_shift - 3);
  const float mom = a.momentum;
  constexpr int NP = LPT_ROWS / 8;

  // The table loads go first, then every data load of the tile (gradient, code bytes,
  // old scale per pass) from a clamped row (rows past the end re-read the last row and
  // are not used), with nothing consumed in between, so all of them are in flight at
  // once. The barrier that publishes the tables waits for this wave's table writes only
  // (a __syncthreads would wait for every outstanding load of the tile), and pass p
  // starts as soon as its own data has arrived.
  uint4 tq0 = {}, tq1 = {}, tq2 = {}, tq3 = {};
  float tqm = 0.0f;
  uint32_t tt0 = 0, tt1 = 0;
  bool sparse_map = false;
  if (MAP) {
    static_assert(MUON_QTAB_SIZE == 4 * 256 * 16, "one 16-byte table piece per thread and step");
    const uint4* gt = (const uint4*)a.qtab + tid;
    const uint32_t* gthr = (const uint32_t*)(a.qtab + MUON_QTAB_SIZE);
    tqm = a.qmap[tid < (QF == MUON_Q_8BIT ? 256 : 16) ? tid : 0];
    if (TABLES) {
      tq0 = gt[0];
      tq1 = gt[256];
      tq2 = gt[512];
      tq3 = gt[768];
      tt0 = gthr[tid];
      tt1 = gthr[256 + (tid & (MUON_QTHR_PAD - 1))];
      sparse_map = gthr[MUON_QTHR_FLAG] == 0u;  // the same address for every thread
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  Raw8<GDT> graw[NP];
  typename LpCodes<QF>::T cw[NP];
  float osc[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int64_t r = r0 + p * 8 + rsub;
    const int64_t rr = r < a.rows ? r : a.rows - 1;
    const int64_t e = (mb * a.rows + rr) * a.cols + c;  // element index in the tensor
    graw[p].load(gp, e);
    cw[p] = LpCodes<QF>::load(codes, e);
    osc[p] = scales[DEFER ? lp_block_of(e, a.block256) : (e >> a.block_shift)];
  }
  if (MAP) {
    q[tid] = tqm;
    if (TABLES) {
      ((uint4*)qtab)[tid] = tq0;
      ((uint4*)qtab)[256 + tid] = tq1;
      ((uint4*)qtab)[512 + tid] = tq2;
      ((uint4*)qtab)[768 + tid] = tq3;
      qthr[tid] = tt0;
      if (tid < MUON_QTHR_PAD) qthr[256 + tid] = tt1;
    }
    lds_sync();
  }

  bf16_t* x0 = (bf16_t*)a.x0 + (int64_t)mat * a.x_mstride;
  float ss = 0.0f;
  // DEFER: when every valid row of the tile lies in one block (always, for one block per
  // tensor) the tile's absmax goes out as one atomic max; else one per row (256 values)
  int64_t blk0 = 0;
  bool one_block = false;
  uint32_t tmax = 0;
  // tall tiles in 32-row halves: the first half's transposed X0 pieces (one per round)
  uint4 xkeep[TALL && TROWS < LPT_ROWS ? (LPT_COLS * (TROWS / 8)) / 256 : 1];
  if constexpr (DEFER) {
    // (a tile of padding rows only, r0 >= rows, has no block and sends nothing)
    if (r0 < a.rows) {
      const int64_t rl = min(r0 + LPT_ROWS - 1, a.rows - 1);
      blk0 = lp_block_of((mb * a.rows + r0) * a.cols + c0, a.block256);
      one_block = blk0 == lp_block_of((mb * a.rows + rl) * a.cols + c0, a.block256);
    }
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int rl = p * 8 + rsub;
    const int64_t r = r0 + rl;
    const bool valid = r < a.rows;
    uint32_t xw[4];  // X as bf16 pairs (RNE), element 2i in the low half
    if (valid) {
      const int64_t e = (mb * a.rows + r) * a.cols + c;
      float g[8];
      graw[p].unpack(g);
      const float gs = a.maximize ? -1.0f : 1.0f;  // g * gs is exact: the fma rounds once
      float m[8];
      uint32_t ab = 0;
      lp_momentum8<QF>(g, cw[p], osc[p], mom, gs, q, m, ab);
      int cq[8];
      uint2 c8 = {0u, 0u};  // fp8: the 8 code bytes, packed by the conversion itself
      float sc = 0.0f;
      if constexpr (DEFER) {
        // the block extends past this tile: its absmax over these 256 values (one row,
        // 32 lanes) joins the block's running max; codes come in the requant pass
        const uint32_t amax = group_max_u32(ab, 32);
        if (one_block)
          tmax = max(tmax, amax);
        else if (chunk == 0)
          atomicMax(a.bmax + (int64_t)t * a.nblocks + lp_block_of(e, a.block256), amax);
      } else {
        // absmax over the block_lanes consecutive lanes of this block (all in one row)
        sc = block_scale<QF>(group_max_u32(ab, block_lanes));
        lp_codes8<QF>(m, sc, sparse_map, qthr, qtab, cq, c8);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float gq0 = m[2 * i], gq1 = m[2 * i + 1];
        if (a.nesterov) {
          gq0 = __builtin_fmaf(g[2 * i], gs, m[2 * i] * mom);
          gq1 = __builtin_fmaf(g[2 * i + 1], gs, m[2 * i + 1] * mom);
        }
        const f2x v = {gq0, gq1};
        xw[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2x));
        // sum of squares of the two bf16 values (products exact in fp32)
        ss = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2v, xw[i]),
                                             __builtin_bit_cast(bf2v, xw[i]), ss, false);
      }
      if constexpr (!DEFER) {
        if constexpr (QF == MUON_Q_FP8)
          *(uint2*)(codes + e) = c8;
        else
          LpCodes<QF>::store(codes, e, cq);
        if ((chunk & (block_lanes - 1)) == 0) scales[e >> a.block_shift] = sc;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) xw[i] = 0u;
    }
    if (TALL) {
#pragma unroll
      for (int i = 0; i < 4; ++i) *(uint32_t*)&tileT[rl % TROWS][chunk * 8 + 2 * i] = xw[i];
      if ((p + 1) % (TROWS / 8) == 0) {
        // X0 row (c0 + cc) holds stored column cc: TROWS consecutive values, this tile's
        // rows r0 + p0 ..
        constexpr int SEGS = TROWS / 8;  // 16-byte pieces per X0 row
        const int p0 = (p + 1) * 8 - TROWS;
        lds_sync();
        // ds_read_b64_tr_b16: within 16 lanes, lane i points at 4 elements of row kb + i/4,
        // columns jb + 4 (i % 4) .. +3, and receives column jb + i of rows kb .. kb+3; two
        // such reads give the 8 rows of one X0 piece. Round `it`: column group
        // 4 wave + it % 4, lane group gg takes rows 32 (it / 4) + 8 gg, so the four lane
        // groups write 64 contiguous bytes of each X0 row. With 32-row halves the first
        // half's pieces stay in registers and go out beside the second half's, so each X0
        // row's 128 bytes are written together.
        const int tl = tid & 63, gg = tl >> 4, ti = tl & 15;
#pragma unroll
        for (int it = 0; it < (LPT_COLS * SEGS) / 256; ++it) {
          const int jb = 16 * (4 * (tid >> 6) + (it & 3));
          const int rr = 32 * (it >> 2) + 8 * gg;
          const lp_i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) lp_i16x4*)&tileT[rr + (ti >> 2)][jb + 4 * (ti & 3)]);
          const lp_i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) lp_i16x4*)&tileT[rr + 4 + (ti >> 2)][jb + 4 * (ti & 3)]);
          const uint4 w = __builtin_bit_cast(uint4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
          bf16_t* const xrow = x0 + (c0 + jb + ti) * a.x_pitch + r0;
          if constexpr (TROWS < LPT_ROWS) {
            if (p0 == 0) {
              xkeep[it] = w;
            } else {
              *(uint4*)(xrow + rr) = xkeep[it];
              *(uint4*)(xrow + p0 + rr) = w;
            }
          } else {
            *(uint4*)(xrow + p0 + rr) = w;
          }
        }
        if (p != NP - 1) lds_sync();  // the next rows reuse the tile
      }
    } else {
      *(uint4*)(x0 + r * a.x_pitch + c) = make_uint4(xw[0], xw[1], xw[2], xw[3]);
    }
  }
  ss = warp_sum(ss);
  if (lane == 0) wsum[wave] = ss;
  if constexpr (DEFER) {
    if (one_block) {
      const uint32_t wm = wave_max_u32(tmax);
      if (lane == 0) wmaxs[wave] = wm;
    }
  }
  __syncthreads();
  if (tid == 0) {
    part[blockIdx.x] = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
    if (DEFER && one_block)
      atomicMax(a.bmax + (int64_t)t * a.nblocks + blk0,
                max(max(wmaxs[0], wmaxs[1]), max(wmaxs[2], wmaxs[3])));
  }
}

template <int GDT, int QF, bool DEFER>
void launch_lp_tile_t(bool tall, const LpTileArgs& a, dim3 grid, hipStream_t s) {
  if (tall)
    hipLaunchKernelGGL((lp_prepass_tile_kernel<GDT, QF, true, DEFER>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((lp_prepass_tile_kernel<GDT, QF, false, DEFER>), grid, dim3(256), 0, s, a);
}

template <int GDT, bool DEFER>
void launch_lp_tile_q(int qf, bool tall, const LpTileArgs& a, dim3 grid, hipStream_t s) {
  if (qf == MUON_Q_8BIT) launch_lp_tile_t<GDT, MUON_Q_8BIT, DEFER>(tall, a, grid, s);
  else if (qf == MUON_Q_4BIT) launch_lp_tile_t<GDT, MUON_Q_4BIT, DEFER>(tall, a, grid, s);
  else launch_lp_tile_t<GDT, MUON_Q_FP8, DEFER>(tall, a, grid, s);
}

// ---- row-segment blocks: 512, 1024 or 2048 values --------------------------------
// Blocks of 512-2048 values in matrices whose width is a multiple of 2048 (the reference's
// default block, on every Llama-sized shape). A wavefront owns 2048 consecutive values of
// one stored row: lane l holds values 8 l .. 8 l + 7 of each 512-value quarter, so a block
// is one, two or four quarters of one wavefront and its absmax a wave reduction. The new
// momentum stays in registers between the absmax and the codes, as in the tile kernel, and
// every value is read and written once (6 bytes for 8-bit and fp8 codes, against 9 for the
// deferred-scale passes). A workgroup owns 8 rows x 2048 columns, two rows per wave with
// every load of both issued first, and writes one norm partial. X0: the stored layout, or
// for a tall matrix its transpose staged through LDS: 16 bytes of each of 2048 X0 rows per
// workgroup. Workgroup w takes unit (w % 8) (units / 8) + w / 8 (when 8 divides the unit
// count), so the eight row groups that fill one 128-byte piece of those X0 rows run on one
// XCD (workgroups are dispatched to the XCDs round robin) in neighbouring slots, and their
// pieces meet in that XCD's L2. Wide matrices take this kernel for blocks of 8-256 values
// as well (block / 8 lanes of one quarter, a shuffle reduction).
constexpr int LPS_ROWS = 8, LPS_COLS = 2048;
// LDS row pitch of the transpose stage: 32 mod 256 bytes, so the four rows a 16-lane
// transposing read covers fall in distinct banks. The fp8 kernel (no code tables in LDS)
// takes a longer pitch, 43 KB in all, so that at most three of its workgroups share a CU
// as with the map formats: with four, the partly written X0 lines of the concurrent row
// groups outgrow the XCD's L2 and are written back in pieces (a Llama step's fp8 pre-pass
// took 9.3 ms at four per CU, 8.6 at three, like the 8-bit one).
template <int QF>
constexpr int lps_pitch() {
  return QF == MUON_Q_FP8 ? LPS_COLS + 656 : LPS_COLS + 16;
}

template <int GDT, int QF, bool TALL>
__global__ __launch_bounds__(256) void lp_prepass_seg_kernel(LpTileArgs a) {
#pragma clang fp contract(off)
  constexpr bool MAP = QF != MUON_Q_FP8;
  __shared__ float q[256];
  __shared__ __align__(16) uint8_t qtab[MAP ? MUON_QTAB_SIZE : 16];
  __shared__ __align__(16) uint32_t qthr[MAP ? 256 + MUON_QTHR_PAD : 4];
  __shared__ __align__(16) bf16_t tileT[TALL ? LPS_ROWS : 1][TALL ? lps_pitch<QF>() : 8];
  __shared__ float wsum[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int mat = blockIdx.y;
  float* part = a.partials + (int64_t)mat * a.parts;
  const int units = a.tiles_used;  // row groups x column strips, = gridDim.x
  if (tid == 0) {
    // the partial slots past the units hold nothing
    for (int64_t sl = units + (int64_t)blockIdx.x; sl < a.parts; sl += units) part[sl] = 0.0f;
  }
  const int w = blockIdx.x;
  const int u = (units & 7) == 0 ? (w & 7) * (units >> 3) + (w >> 3) : w;
  const int rgroups = units / a.tiles_c;
  const int rg = u % rgroups, cs = u / rgroups;
  const int t = (int)(mat / a.nb);
  const int64_t mb = mat % a.nb;
  const int64_t r0 = (int64_t)rg * LPS_ROWS, c0 = (int64_t)cs * LPS_COLS;
  const void* gp = a.grads[t];
  uint8_t* codes = (uint8_t*)a.codes[t];
  float* scales = a.scales[t];
  const float mom = a.momentum;

  // table loads first, then every data load of both rows, nothing consumed in between
  uint4 tq0 = {}, tq1 = {}, tq2 = {}, tq3 = {};
  float tqm = 0.0f;
  uint32_t tt0 = 0, tt1 = 0;
  bool sparse_map = false;
  if (MAP) {
    const uint4* gt = (const uint4*)a.qtab + tid;
    const uint32_t* gthr = (const uint32_t*)(a.qtab + MUON_QTAB_SIZE);
    tqm = a.qmap[tid < (QF == MUON_Q_8BIT ? 256 : 16) ? tid : 0];
    tq0 = gt[0];
    tq1 = gt[256];
    tq2 = gt[512];
    tq3 = gt[768];
    tt0 = gthr[tid];
    tt1 = gthr[256 + (tid & (MUON_QTHR_PAD - 1))];
    sparse_map = gthr[MUON_QTHR_FLAG] == 0u;
    __builtin_amdgcn_sched_barrier(0);
  }
  Raw8<GDT> graw[2][4];
  typename LpCodes<QF>::T cw[2][4];
  float osc[2][4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t r = r0 + 2 * wave + h;
    const int64_t rr = r < a.rows ? r : a.rows - 1;  // rows past the end: not used
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int64_t e = (mb * a.rows + rr) * a.cols + c0 + k * 512 + lane * 8;
      graw[h][k].load(gp, e);
      cw[h][k] = LpCodes<QF>::load(codes, e);
      osc[h][k] = scales[e >> a.block_shift];
    }
  }
  if (MAP) {
    q[tid] = tqm;
    ((uint4*)qtab)[tid] = tq0;
    ((uint4*)qtab)[256 + tid] = tq1;
    ((uint4*)qtab)[512 + tid] = tq2;
    ((uint4*)qtab)[768 + tid] = tq3;
    qthr[tid] = tt0;
    if (tid < MUON_QTHR_PAD) qthr[256 + tid] = tt1;
    lds_sync();
  }

  bf16_t* x0 = (bf16_t*)a.x0 + (int64_t)mat * a.x_mstride;
  const float gs = a.maximize ? -1.0f : 1.0f;  // g * gs is exact: the fma rounds once
  float ss = 0.0f;
  // max over the wavefront: within each 32-lane half, then the two halves
  auto wmax = [&](uint32_t v) -> uint32_t {
    v = group_max_u32(v, 32);
    return max((uint32_t)__builtin_amdgcn_readlane((int)v, 0),
               (uint32_t)__builtin_amdgcn_readlane((int)v, 32));
  };
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int rl = 2 * wave + h;
    const int64_t r = r0 + rl;
    uint4 xw[4] = {};
    if (r < a.rows) {
      float m[4][8];
      uint32_t ab[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float g[8];
        graw[h][k].unpack(g);
        ab[k] = 0;
        lp_momentum8<QF>(g, cw[h][k], osc[h][k], mom, gs, q, m[k], ab[k]);
      }
      // the absmax of each block: quarters k of one block share it; a block of 8-256
      // values is block / 8 consecutive lanes of one quarter
      uint32_t bm[4];
      if (a.block_shift <= 8) {
#pragma unroll
        for (int k = 0; k < 4; ++k) bm[k] = group_max_u32(ab[k], 1 << (a.block_shift - 3));
      } else if (a.block_shift == 11) {
        bm[0] = bm[1] = bm[2] = bm[3] = wmax(max(max(ab[0], ab[1]), max(ab[2], ab[3])));
      } else if (a.block_shift == 10) {
        bm[0] = bm[1] = wmax(max(ab[0], ab[1]));
        bm[2] = bm[3] = wmax(max(ab[2], ab[3]));
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) bm[k] = wmax(ab[k]);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t e = (mb * a.rows + r) * a.cols + c0 + k * 512 + lane * 8;
        const float sc = block_scale<QF>(bm[k]);
        int cq[8];
        uint2 c8 = {0u, 0u};
        lp_codes8<QF>(m[k], sc, sparse_map, qthr, qtab, cq, c8);
        if constexpr (QF == MUON_Q_FP8)
          *(uint2*)(codes + e) = c8;
        else
          LpCodes<QF>::store(codes, e, cq);
        // the lane holding a block's first 8 values stores its scale
        if (((k * 512 + lane * 8) & ((1 << a.block_shift) - 1)) == 0) scales[e >> a.block_shift] = sc;
        float g[8];
        graw[h][k].unpack(g);
        uint32_t xv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float gq0 = m[k][2 * i], gq1 = m[k][2 * i + 1];
          if (a.nesterov) {
            gq0 = __builtin_fmaf(g[2 * i], gs, m[k][2 * i] * mom);
            gq1 = __builtin_fmaf(g[2 * i + 1], gs, m[k][2 * i + 1] * mom);
          }
          const f2x v = {gq0, gq1};
          xv[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2x));
          // sum of squares of the two bf16 values (products exact in fp32)
          ss = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2v, xv[i]),
                                               __builtin_bit_cast(bf2v, xv[i]), ss, false);
        }
        xw[k] = make_uint4(xv[0], xv[1], xv[2], xv[3]);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (TALL)
        *(uint4*)&tileT[rl][k * 512 + lane * 8] = xw[k];
      else
        *(uint4*)(x0 + r * a.x_pitch + c0 + k * 512 + lane * 8) = xw[k];
    }
  }
  if constexpr (TALL) {
    lds_sync();
    // X0 row c0 + j holds stored column j of rows r0 .. r0 + 7: ds_read_b64_tr_b16 over 16
    // lanes, lane i pointing at 4 elements of row kb + i/4, columns jb + 4 (i % 4) .. +3,
    // returns column jb + i of rows kb .. kb + 3; two reads give the 8 rows. Round it: lane
    // group gg of wave wv takes the 16 columns from jb = 16 (16 it + 4 wv + gg).
    const int gg = lane >> 4, ti = lane & 15;
#pragma unroll
    for (int it = 0; it < LPS_COLS / 256; ++it) {
      const int jb = 16 * (16 * it + 4 * wave + gg);
      const lp_i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) lp_i16x4*)&tileT[ti >> 2][jb + 4 * (ti & 3)]);
      const lp_i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) lp_i16x4*)&tileT[4 + (ti >> 2)][jb + 4 * (ti & 3)]);
      const uint4 wv = __builtin_bit_cast(uint4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      *(uint4*)(x0 + (c0 + jb + ti) * a.x_pitch + r0) = wv;
    }
  }
  ss = warp_sum(ss);
  if (lane == 0) wsum[wave] = ss;
  __syncthreads();
  if (tid == 0) part[u] = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
}

template <int GDT, int QF>
void launch_lp_seg_t(bool tall, const LpTileArgs& a, dim3 grid, hipStream_t s) {
  if (tall)
    hipLaunchKernelGGL((lp_prepass_seg_kernel<GDT, QF, true>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((lp_prepass_seg_kernel<GDT, QF, false>), grid, dim3(256), 0, s, a);
}

template <int GDT>
void launch_lp_seg_q(int qf, bool tall, const LpTileArgs& a, dim3 grid, hipStream_t s) {
  if (qf == MUON_Q_8BIT) launch_lp_seg_t<GDT, MUON_Q_8BIT>(tall, a, grid, s);
  else if (qf == MUON_Q_4BIT) launch_lp_seg_t<GDT, MUON_Q_4BIT>(tall, a, grid, s);
  else launch_lp_seg_t<GDT, MUON_Q_FP8>(tall, a, grid, s);
}

// ---- deferred scales: blocks of more than 256 values --------------------------------
// The tile kernel (DEFER) has left each block's absmax (unsigned max of the |m| bit
// patterns, so a NaN wins); this kernel keeps the old scale for the requant pass and
// stores the new one, one thread per block. Nothing else reads `scales` between the tile
// kernel and the requant pass.
struct LpReduceArgs {
  float* scales[MUON_MAX_TENSORS];
  const uint32_t* bmax;  // [tensor][nblocks] for the tensors of this launch
  float* oldsc;          // [tensor][nblocks]
  int64_t nblocks;       // per tensor
  int ntensors;
};

template <int QF>
__global__ __launch_bounds__(256) void lp_scale_reduce_kernel(LpReduceArgs a) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= a.nblocks * a.ntensors) return;
  const int64_t t = gid / a.nblocks, b = gid % a.nblocks;
  float* sc = a.scales[t];
  a.oldsc[gid] = sc[b];
  sc[b] = block_scale<QF>(a.bmax[gid]);
}

// Requantization of blocks whose scale was reduced across tiles: recompute the new
// momentum exactly as the tile kernel did (the same inputs, lp_momentum8) and code it
// with the new scale. Flat over each tensor's values, 8 per lane, 8 passes of 2048 per
// workgroup with every load issued before the first is used.
struct LpRequantArgs {
  void* grads[MUON_MAX_TENSORS];
  void* codes[MUON_MAX_TENSORS];
  float* scales[MUON_MAX_TENSORS];  // new scales
  const float* oldsc;               // [tensor][nblocks]
  const float* qmap;
  const uint8_t* qtab;              // bucket table, then thresholds
  int64_t numel, nblocks;           // per tensor
  uint32_t block256;
  float momentum;
  int maximize;
};

constexpr int LPR_PASSES = 8;

template <int GDT, int QF>
__global__ __launch_bounds__(256) void lp_requant_kernel(LpRequantArgs a) {
#pragma clang fp contract(off)
  constexpr bool MAP = QF != MUON_Q_FP8;
  __shared__ float q[256];
  __shared__ __align__(16) uint8_t qtab[MAP ? MUON_QTAB_SIZE : 16];
  __shared__ __align__(16) uint32_t qthr[MAP ? 256 + MUON_QTHR_PAD : 4];
  const int tid = threadIdx.x;
  const int t = blockIdx.y;
  uint4 tq0 = {}, tq1 = {}, tq2 = {}, tq3 = {};
  float tqm = 0.0f;
  uint32_t tt0 = 0, tt1 = 0;
  bool sparse_map = false;
  if (MAP) {
    const uint4* gt = (const uint4*)a.qtab + tid;
    const uint32_t* gthr = (const uint32_t*)(a.qtab + MUON_QTAB_SIZE);
    tqm = a.qmap[tid < (QF == MUON_Q_8BIT ? 256 : 16) ? tid : 0];
    tq0 = gt[0];
    tq1 = gt[256];
    tq2 = gt[512];
    tq3 = gt[768];
    tt0 = gthr[tid];
    tt1 = gthr[256 + (tid & (MUON_QTHR_PAD - 1))];
    sparse_map = gthr[MUON_QTHR_FLAG] == 0u;
    __builtin_amdgcn_sched_barrier(0);
  }
  const void* gp = a.grads[t];
  uint8_t* codes = (uint8_t*)a.codes[t];
  const float* nsc = a.scales[t];
  const float* osc_t = a.oldsc + (int64_t)t * a.nblocks;
  const int64_t base = (int64_t)blockIdx.x * LPR_PASSES * 2048 + tid * 8;
  Raw8<GDT> graw[LPR_PASSES];
  typename LpCodes<QF>::T cw[LPR_PASSES];
  float osc[LPR_PASSES], sc[LPR_PASSES];
#pragma unroll
  for (int p = 0; p < LPR_PASSES; ++p) {
    const int64_t e0 = base + p * 2048;
    const int64_t e = e0 < a.numel ? e0 : a.numel - 8;  // clamped, not used
    const int64_t b = lp_block_of(e, a.block256);
    graw[p].load(gp, e);
    cw[p] = LpCodes<QF>::load(codes, e);
    osc[p] = osc_t[b];
    sc[p] = nsc[b];
  }
  if (MAP) {
    q[tid] = tqm;
    ((uint4*)qtab)[tid] = tq0;
    ((uint4*)qtab)[256 + tid] = tq1;
    ((uint4*)qtab)[512 + tid] = tq2;
    ((uint4*)qtab)[768 + tid] = tq3;
    qthr[tid] = tt0;
    if (tid < MUON_QTHR_PAD) qthr[256 + tid] = tt1;
    lds_sync();
  }
  const float gs = a.maximize ? -1.0f : 1.0f;
#pragma unroll
  for (int p = 0; p < LPR_PASSES; ++p) {
    const int64_t e = base + p * 2048;
    if (e >= a.numel) continue;
    float g[8], m[8];
    graw[p].unpack(g);
    uint32_t ab = 0;
    lp_momentum8<QF>(g, cw[p], osc[p], a.momentum, gs, q, m, ab);
    int cq[8];
    uint2 c8 = {0u, 0u};
    lp_codes8<QF>(m, sc[p], sparse_map, qthr, qtab, cq, c8);
    if constexpr (QF == MUON_Q_FP8)
      *(uint2*)(codes + e) = c8;
    else
      LpCodes<QF>::store(codes, e, cq);
  }
}

template <int GDT>
void launch_lp_requant_q(int qf, const LpRequantArgs& a, dim3 grid, hipStream_t s) {
  if (qf == MUON_Q_8BIT)
    hipLaunchKernelGGL((lp_requant_kernel<GDT, MUON_Q_8BIT>), grid, dim3(256), 0, s, a);
  else if (qf == MUON_Q_4BIT)
    hipLaunchKernelGGL((lp_requant_kernel<GDT, MUON_Q_4BIT>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((lp_requant_kernel<GDT, MUON_Q_FP8>), grid, dim3(256), 0, s, a);
}

template <int QF>
__global__ __launch_bounds__(256) void quantize_kernel(const float* src, uint8_t* codes,
                                                       float* scales, const float* qmap,
                                                       int64_t block, int64_t nblocks) {
#pragma clang fp contract(off)
  __shared__ float q[256];
  const int tid = threadIdx.x;
  if (QF != MUON_Q_FP8) q[tid] = qmap[tid < (QF == MUON_Q_8BIT ? 256 : 16) ? tid : 0];
  __syncthreads();
  const int lane = tid & 63;
  const int64_t blk = (int64_t)blockIdx.x * 4 + (tid >> 6);
  if (blk >= nblocks) return;
  const int64_t e0 = blk * block;
  constexpr int US = unit_size<QF>();
  const int64_t units = block / US;
  uint32_t ab = 0;
  for (int64_t e = lane; e < block; e += 64) ab = max(ab, abs_bits(src[e0 + e]));
  const float sc = block_scale<QF>(wave_max_u32(ab));
  for (int64_t u = lane; u < units; u += 64) {
    int cq[US];
#pragma unroll
    for (int k = 0; k < US; ++k) cq[k] = quant_code<QF>(src[e0 + u * US + k] / sc, q);
    if (QF == MUON_Q_4BIT)
      codes[(e0 >> 1) + u] = (uint8_t)((cq[0] << 4) | cq[US - 1]);
    else
      codes[e0 + u] = (uint8_t)cq[0];
  }
  if (lane == 0) scales[blk] = sc;
}

template <int QF>
__global__ __launch_bounds__(256) void dequantize_kernel(const uint8_t* codes,
                                                         const float* scales,
                                                         const float* qmap, int64_t block,
                                                         int64_t numel, float* dst) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < numel;
       e += (int64_t)gridDim.x * 256)
    dst[e] = dequant<QF>(codes, e, qmap, scales[e / block]);
}

template <int GDT>
void launch_lp_q(int qf, const LpArgs& a, dim3 grid, hipStream_t s) {
  if (qf == MUON_Q_8BIT)
    hipLaunchKernelGGL((lp_prepass_kernel<GDT, MUON_Q_8BIT>), grid, dim3(256), 0, s, a);
  else if (qf == MUON_Q_4BIT)
    hipLaunchKernelGGL((lp_prepass_kernel<GDT, MUON_Q_4BIT>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((lp_prepass_kernel<GDT, MUON_Q_FP8>), grid, dim3(256), 0, s, a);
}

}  // namespace

int muon_launch_zero(void* dst, int64_t bytes, hipStream_t s);

int muon_check_lp_format(int qformat, int64_t numel, int64_t block) {
  if (qformat != MUON_Q_8BIT && qformat != MUON_Q_4BIT && qformat != MUON_Q_FP8) {
    muon_set_error("lp: unknown quantization format %d", qformat);
    return MUON_ERR_ARG;
  }
  if (block <= 0 || numel % block != 0) {
    muon_set_error("lp: numel %lld is not a multiple of block %lld", (long long)numel,
                   (long long)block);
    return MUON_ERR_SHAPE;
  }
  if (qformat == MUON_Q_4BIT && block % 2 != 0) {
    muon_set_error("lp: 4-bit blocks must hold an even number of values (block %lld)",
                   (long long)block);
    return MUON_ERR_SHAPE;
  }
  return MUON_OK;
}

int muon_launch_lp_prepass(int ntensors, void* const* grads, int gdt, void* const* codes,
                           void* const* scales, const float* qmap, int qf, int64_t block,
                           int64_t nb, int64_t rows, int64_t cols, float momentum,
                           int nesterov, int maximize, void* direct, int64_t d_pitch,
                           int64_t d_mstride, hipStream_t s) {
  LpArgs a;
  for (int i = 0; i < ntensors; ++i) {
    a.grads[i] = grads[i];
    a.codes[i] = codes[i];
    a.scales[i] = (float*)scales[i];
  }
  a.qmap = qmap;
  a.nb = nb;
  a.rows = rows;
  a.cols = cols;
  a.numel = nb * rows * cols;
  a.block = block;
  a.blocks_per_tensor = a.numel / block;
  a.direct = direct;
  a.d_pitch = d_pitch;
  a.d_mstride = d_mstride;
  a.momentum = momentum;
  a.nesterov = nesterov;
  a.maximize = maximize;
  dim3 grid((unsigned)((a.blocks_per_tensor + 3) / 4), (unsigned)ntensors);
  switch (gdt) {
    case MUON_DT_F32: launch_lp_q<MUON_DT_F32>(qf, a, grid, s); break;
    case MUON_DT_BF16: launch_lp_q<MUON_DT_BF16>(qf, a, grid, s); break;
    case MUON_DT_F16: launch_lp_q<MUON_DT_F16>(qf, a, grid, s); break;
    default:
      muon_set_error("lp_prepass: unsupported grad dtype %d", gdt);
      return MUON_ERR_DTYPE;
  }
  MUON_CHECK_LAUNCH("lp_prepass");
  return MUON_OK;
}

// Tiled LP prepass (see lp_prepass_tile_kernel) when the shape allows it; returns
// MUON_ERR_SHAPE without launching anything otherwise.
int muon_launch_lp_prepass_tiled(int ntensors, void* const* grads, int gdt, void* const* codes,
                                 void* const* scales, const float* qmap, int qf, int64_t block,
                                 int64_t nb, int64_t rows, int64_t cols, float momentum,
                                 int nesterov, int maximize, const OrthLayout& L, void* ws,
                                 int64_t mat0, hipStream_t s) {
  int shift = 0;
  while ((1LL << shift) < block) ++shift;
  // blocks of at most 256 values (a power of two) lie within one tile row: one pass;
  // blocks of 512, 1024 or 2048 values in rows of a multiple of 2048 lie within one
  // wavefront's row segment: one pass (lp_prepass_seg_kernel); other multiples of 256, up
  // to the whole tensor, defer their scale to a reduction over the tiles' absmax partials
  // and a requant pass
  const int64_t numel = nb * rows * cols;
  const bool fused = (1LL << shift) == block && block >= 8 && block <= LPT_COLS;
  // wide matrices with rows of a multiple of 2048 take the row-segment kernel for the
  // one-pass blocks too (each wave store there writes 1 KB of one X0 row: q/o 583 against
  // 670 us per launch at block 256); tall ones keep the tile kernel's 128-byte X0 pieces
  const bool seg = cols % LPS_COLS == 0 &&
                   (fused ? !L.tall : (block == 512 || block == 1024 || block == 2048));
  const bool defer = !fused && !seg && block % 256 == 0 && (numel >> 8) < (1LL << 32);
  if (cols % LPT_COLS || !(fused || seg || defer)) return MUON_ERR_SHAPE;
  for (int i = 0; i < ntensors; ++i) {
    if (((uintptr_t)grads[i] & 15) || ((uintptr_t)codes[i] & 7) || ((uintptr_t)scales[i] & 3))
      return MUON_ERR_SHAPE;
  }
  LpTileArgs a;
  for (int i = 0; i < ntensors; ++i) {
    a.grads[i] = grads[i];
    a.codes[i] = codes[i];
    a.scales[i] = (float*)scales[i];
  }
  a.qmap = qmap;
  a.nb = nb;
  a.rows = rows;
  a.cols = cols;
  a.block_shift = shift;
  const int64_t mst = L.m_pad * L.x_pitch;
  a.x0 = (char*)ws + L.off_x0 + mat0 * mst * 2;
  a.x_pitch = L.x_pitch;
  a.x_mstride = mst;
  a.partials = (float*)((char*)ws + L.off_part) + mat0 * L.parts;
  a.parts = L.parts;
  a.qtab = (const uint8_t*)ws + L.off_qtab;
  const int64_t rows_pad = L.tall ? L.n_pad : L.m_pad;
  a.tiles_c = (int)(cols / (seg ? LPS_COLS : LPT_COLS));
  a.tiles_used = (int)((rows_pad / (seg ? LPS_ROWS : LPT_ROWS)) * a.tiles_c);
  if (a.tiles_used > L.parts) return MUON_ERR_SHAPE;
  a.momentum = momentum;
  a.nesterov = nesterov;
  a.maximize = maximize;
  // deferred scales: the blocks' running absmax, then their old scales, for every tensor
  // of the call, in the X1 iterate buffer, which nothing reads before the first product
  // of the iteration writes it (at most 8 bytes per 256 values; X1 holds 2 per value)
  const int64_t nblocks = numel / block;
  const int64_t t_first = mat0 / nb;  // tensor index of this launch's first tensor
  const int64_t all_tensors = L.batch / nb;
  uint32_t* bmax_all = (uint32_t*)((char*)ws + L.off_x1);
  float* oldsc_all = (float*)((char*)bmax_all + round_up(all_tensors * nblocks * 4, 256));
  a.block256 = (uint32_t)(block / 256);
  a.nblocks = nblocks;
  a.bmax = bmax_all + t_first * nblocks;
  if (defer) {
    const int zrc = muon_launch_zero(a.bmax, (int64_t)ntensors * nblocks * 4, s);
    if (zrc != MUON_OK) return zrc;
  }
  if (qf != MUON_Q_FP8 && mat0 == 0) {
    // thresholds and bucket table of this map, rebuilt per call (a few microseconds)
    uint8_t* tab = (uint8_t*)ws + L.off_qtab;
    uint32_t* thr = (uint32_t*)(tab + MUON_QTAB_SIZE);
    if (qf == MUON_Q_8BIT)
      hipLaunchKernelGGL(build_qthr_kernel<MUON_Q_8BIT>, dim3(1), dim3(256), 0, s, qmap, thr);
    else
      hipLaunchKernelGGL(build_qthr_kernel<MUON_Q_4BIT>, dim3(1), dim3(256), 0, s, qmap, thr);
    hipLaunchKernelGGL(build_qtab_kernel, dim3(MUON_QTAB_SIZE / 256), dim3(256), 0, s,
                       (const uint32_t*)thr, qf == MUON_Q_8BIT ? 256 : 16, tab);
  }
  if (gdt != MUON_DT_F32 && gdt != MUON_DT_BF16 && gdt != MUON_DT_F16) {
    muon_set_error("lp_prepass: unsupported grad dtype %d", gdt);
    return MUON_ERR_DTYPE;
  }
  if (seg) {
    // one workgroup per unit; the units' workgroups zero the partial slots past them
    dim3 sgrid((unsigned)a.tiles_used, (unsigned)(ntensors * nb));
    switch (gdt) {
      case MUON_DT_F32: launch_lp_seg_q<MUON_DT_F32>(qf, L.tall, a, sgrid, s); break;
      case MUON_DT_BF16: launch_lp_seg_q<MUON_DT_BF16>(qf, L.tall, a, sgrid, s); break;
      default: launch_lp_seg_q<MUON_DT_F16>(qf, L.tall, a, sgrid, s); break;
    }
    MUON_CHECK_LAUNCH("lp_prepass_seg");
    return MUON_OK;
  }
  dim3 grid((unsigned)L.parts, (unsigned)(ntensors * nb));
  switch (gdt) {
    case MUON_DT_F32:
      defer ? launch_lp_tile_q<MUON_DT_F32, true>(qf, L.tall, a, grid, s)
            : launch_lp_tile_q<MUON_DT_F32, false>(qf, L.tall, a, grid, s);
      break;
    case MUON_DT_BF16:
      defer ? launch_lp_tile_q<MUON_DT_BF16, true>(qf, L.tall, a, grid, s)
            : launch_lp_tile_q<MUON_DT_BF16, false>(qf, L.tall, a, grid, s);
      break;
    default:
      defer ? launch_lp_tile_q<MUON_DT_F16, true>(qf, L.tall, a, grid, s)
            : launch_lp_tile_q<MUON_DT_F16, false>(qf, L.tall, a, grid, s);
      break;
  }
  MUON_CHECK_LAUNCH("lp_prepass_tiled");
  if (!defer) return MUON_OK;

  LpReduceArgs r;
  for (int i = 0; i < ntensors; ++i) r.scales[i] = (float*)scales[i];
  r.bmax = a.bmax;
  r.oldsc = oldsc_all + t_first * nblocks;
  r.nblocks = nblocks;
  r.ntensors = ntensors;
  dim3 rgrid((unsigned)((nblocks * ntensors + 255) / 256));
  if (qf == MUON_Q_FP8)
    hipLaunchKernelGGL(lp_scale_reduce_kernel<MUON_Q_FP8>, rgrid, dim3(256), 0, s, r);
  else
    hipLaunchKernelGGL(lp_scale_reduce_kernel<MUON_Q_8BIT>, rgrid, dim3(256), 0, s, r);
  MUON_CHECK_LAUNCH("lp_scale_reduce");

  LpRequantArgs q;
  for (int i = 0; i < ntensors; ++i) {
    q.grads[i] = grads[i];
    q.codes[i] = codes[i];
    q.scales[i] = (float*)scales[i];
  }
  q.oldsc = r.oldsc;
  q.qmap = qmap;
  q.qtab = a.qtab;
  q.numel = numel;
  q.nblocks = nblocks;
  q.block256 = a.block256;
  q.momentum = momentum;
  q.maximize = maximize;
  dim3 qgrid((unsigned)((numel + LPR_PASSES * 2048 - 1) / (LPR_PASSES * 2048)), (unsigned)ntensors);
  switch (gdt) {
    case MUON_DT_F32: launch_lp_requant_q<MUON_DT_F32>(qf, q, qgrid, s); break;
    case MUON_DT_BF16: launch_lp_requant_q<MUON_DT_BF16>(qf, q, qgrid, s); break;
    default: launch_lp_requant_q<MUON_DT_F16>(qf, q, qgrid, s); break;
  }
  MUON_CHECK_LAUNCH("lp_requant");
  return MUON_OK;
}

extern "C" int muon_lp_quantize(const float* src, void* codes, float* scales, const float* qmap,
                                int qformat, int64_t numel, int64_t block, void* stream) {
  int rc = muon_check_lp_format(qformat, numel, block);
  if (rc != MUON_OK) return rc;
  const int64_t nblocks = numel / block;
  if (nblocks == 0) return MUON_OK;
  dim3 grid((unsigned)((nblocks + 3) / 4));
  hipStream_t s = (hipStream_t)stream;
  if (qformat == MUON_Q_8BIT)
    hipLaunchKernelGGL((quantize_kernel<MUON_Q_8BIT>), grid, dim3(256), 0, s, src,
                       (uint8_t*)codes, scales, qmap, block, nblocks);
  else if (qformat == MUON_Q_4BIT)
    hipLaunchKernelGGL((quantize_kernel<MUON_Q_4BIT>), grid, dim3(256), 0, s, src,
                       (uint8_t*)codes, scales, qmap, block, nblocks);
  else
    hipLaunchKernelGGL((quantize_kernel<MUON_Q_FP8>), grid, dim3(256), 0, s, src,
                       (uint8_t*)codes, scales, qmap, block, nblocks);
  MUON_CHECK_LAUNCH("lp_quantize");
  return MUON_OK;
}

extern "C" int muon_lp_dequantize(const void* codes, const float* scales, const float* qmap,
                                  int qformat, int64_t numel, int64_t block, float* dst,
                                  void* stream) {
  int rc = muon_check_lp_format(qformat, numel, block);
  if (rc != MUON_OK) return rc;
  if (numel == 0) return MUON_OK;
  dim3 grid((unsigned)std::min<int64_t>((numel + 255) / 256, 8192));
  hipStream_t s = (hipStream_t)stream;
  const uint8_t* c = (const uint8_t*)codes;
  if (qformat == MUON_Q_8BIT)
    hipLaunchKernelGGL((dequantize_kernel<MUON_Q_8BIT>), grid, dim3(256), 0, s, c, scales, qmap,
                       block, numel, dst);
  else if (qformat == MUON_Q_4BIT)
    hipLaunchKernelGGL((dequantize_kernel<MUON_Q_4BIT>), grid, dim3(256), 0, s, c, scales, qmap,
                       block, numel, dst);
  else
    hipLaunchKernelGGL((dequantize_kernel<MUON_Q_FP8>), grid, dim3(256), 0, s, c, scales, qmap,
                       block, numel, dst);
  MUON_CHECK_LAUNCH("lp_dequantize");
  return MUON_OK;
}
