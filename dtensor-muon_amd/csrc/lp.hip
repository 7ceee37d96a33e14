// Quantized momentum state for MuonLP (8-bit / 4-bit dynamic-map codes and fp8
// e4m3fn codes, one fp32 absmax scale per block of consecutive values).
//
// The format and rounding follow the blockwise scheme MuonLP gets from torchao 0.17.0
// (optim_lp.py:118-133): scale = max(|x|) over the block clipped at 1e-12 (divided by
// 448 for fp8), y = x / scale, and for the map formats the code is found by a
// fixed-depth binary search over the sorted map followed by a round-half-up step
// between the two neighbouring entries. One wavefront owns one block; the block is
// read twice (absmax, then quantize) with the second read served from cache.
#include <algorithm>

#include "common.h"

namespace {

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

template <int QF>
MUON_DEVICE int quant_code(float y, const float* q) {
  if (QF == MUON_Q_8BIT) {
    int c = (y >= q[128]) ? 128 : 0;
    c += (y >= q[c + 64]) ? 64 : 0;
    c += (y >= q[c + 32]) ? 32 : 0;
    c += (y >= q[c + 16]) ? 16 : 0;
    c += (y >= q[c + 8]) ? 8 : 0;
    c += (y >= q[c + 4]) ? 4 : 0;
    c += (y >= q[c + 2]) ? 2 : 0;
    c += (y >= q[c + 1]) ? 1 : 0;
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
    return f32_to_e4m3fn(y);
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
  float amax = 0.0f;
  for (int64_t u = lane; u < units; u += 64) {
#pragma unroll
    for (int k = 0; k < US; ++k) {
      const int64_t e = e0 + u * US + k;
      float g = Elem<GDT>::load(gp, e);
      if (a.maximize) g = -g;
      float m = dequant<QF>(codes, e, q, old_scale) * a.momentum;
      m = m + g;
      amax = fmaxf(amax, fabsf(m));
    }
  }
  amax = warp_max(amax);
  float sc = amax > 1e-12f ? amax : 1e-12f;
  if (QF == MUON_Q_FP8) sc = sc / 448.0f;

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
  float* partials;          // partials of matrix 0 of this launch
  int64_t parts;            // partial slots per matrix
  int tiles_c, tiles_used;  // column tiles (cols / 256), tiles with data or padding
  float momentum;
  int nesterov, maximize;
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

template <int GDT, int QF, bool TALL>
__global__ __launch_bounds__(256) void lp_prepass_tile_kernel(LpTileArgs a) {
#pragma clang fp contract(off)
  __shared__ float q[256];
  __shared__ bf16_t tileT[TALL ? LPT_ROWS : 1][TALL ? LPT_PITCH : 1];
  __shared__ float wsum[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (QF != MUON_Q_FP8) q[tid] = a.qmap[tid < (QF == MUON_Q_8BIT ? 256 : 16) ? tid : 0];
  const int mat = blockIdx.y;
  const int t = (int)(mat / a.nb);
  const int64_t mb = mat % a.nb;
  float* part = a.partials + (int64_t)mat * a.parts;
  if ((int)blockIdx.x >= a.tiles_used) {
    if (tid == 0) part[blockIdx.x] = 0.0f;
    return;
  }
  __syncthreads();
  const int tr = blockIdx.x / a.tiles_c, tcol = blockIdx.x % a.tiles_c;
  const int64_t r0 = (int64_t)tr * LPT_ROWS, c0 = (int64_t)tcol * LPT_COLS;
  const void* gp = a.grads[t];
  uint8_t* codes = (uint8_t*)a.codes[t];
  float* scales = a.scales[t];
  const int chunk = lane & 31;              // 8-value chunk within the row
  const int rsub = wave * 2 + (lane >> 5);  // row within the 8-row pass
  const int64_t c = c0 + chunk * 8;
  const int block_lanes = 1 << (a.block_shift - 3);
  const float mom = a.momentum;
  bf16_t* x0 = (bf16_t*)a.x0 + (int64_t)mat * a.x_mstride;
  float ss = 0.0f;
#pragma unroll 2
  for (int p = 0; p < LPT_ROWS / 8; ++p) {
    const int rl = p * 8 + rsub;
    const int64_t r = r0 + rl;
    const bool valid = r < a.rows;
    float xv[8];
    if (valid) {
      const int64_t e = (mb * a.rows + r) * a.cols + c;  // element index in the tensor
      const int64_t blk = e >> a.block_shift;
      float g[8];
      Vec8<GDT>::load(gp, e, g);
      const typename LpCodes<QF>::T cw = LpCodes<QF>::load(codes, e);
      const float old_scale = scales[blk];
      float m[8];
      float amax = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (a.maximize) g[k] = -g[k];
        float v = code_value<QF>(LpCodes<QF>::get(cw, k), q) * old_scale;
        v = v * mom;
        m[k] = v + g[k];
        amax = fmaxf(amax, fabsf(m[k]));
      }
      // absmax over the block_lanes consecutive lanes of this block (all in one row)
      for (int off = 1; off < block_lanes; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
      float sc = amax > 1e-12f ? amax : 1e-12f;
      if (QF == MUON_Q_FP8) sc = sc / 448.0f;
      int cq[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        cq[k] = quant_code<QF>(m[k] / sc, q);
        float gq = m[k];
        if (a.nesterov) {
          const float tt = m[k] * mom;
          gq = g[k] + tt;
        }
        xv[k] = Elem<MUON_DT_BF16>::round(gq);
        ss += xv[k] * xv[k];
      }
      LpCodes<QF>::store(codes, e, cq);
      if ((chunk & (block_lanes - 1)) == 0) scales[blk] = sc;
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) xv[k] = 0.0f;
    }
    if (TALL) {
#pragma unroll
      for (int k = 0; k < 8; ++k) tileT[rl][chunk * 8 + k] = f32_to_bf16(xv[k]);
    } else {
      Vec8<MUON_DT_BF16>::store(x0, r * a.x_pitch + c, xv);
    }
  }
  if (TALL) {
    // X0 row (c0 + cc) holds stored column cc: 64 consecutive values from the 64 rows
    __syncthreads();
#pragma unroll 2
    for (int it = 0; it < (LPT_COLS * LPT_ROWS / 8) / 256; ++it) {
      const int id = it * 256 + tid;
      const int cc = id >> 3, rr = (id & 7) * 8;
      uint16_t ev[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) ev[k] = tileT[rr + k][cc];
      uint4 w;
      __builtin_memcpy(&w, ev, 16);
      *(uint4*)(x0 + (c0 + cc) * a.x_pitch + r0 + rr) = w;
    }
  }
  ss = warp_sum(ss);
  if (lane == 0) wsum[wave] = ss;
  __syncthreads();
  if (tid == 0) part[blockIdx.x] = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
}

template <int GDT, int QF>
void launch_lp_tile_t(bool tall, const LpTileArgs& a, dim3 grid, hipStream_t s) {
  if (tall)
    hipLaunchKernelGGL((lp_prepass_tile_kernel<GDT, QF, true>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((lp_prepass_tile_kernel<GDT, QF, false>), grid, dim3(256), 0, s, a);
}

template <int GDT>
void launch_lp_tile_q(int qf, bool tall, const LpTileArgs& a, dim3 grid, hipStream_t s) {
  if (qf == MUON_Q_8BIT) launch_lp_tile_t<GDT, MUON_Q_8BIT>(tall, a, grid, s);
  else if (qf == MUON_Q_4BIT) launch_lp_tile_t<GDT, MUON_Q_4BIT>(tall, a, grid, s);
  else launch_lp_tile_t<GDT, MUON_Q_FP8>(tall, a, grid, s);
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
  float amax = 0.0f;
  for (int64_t e = lane; e < block; e += 64) amax = fmaxf(amax, fabsf(src[e0 + e]));
  amax = warp_max(amax);
  float sc = amax > 1e-12f ? amax : 1e-12f;
  if (QF == MUON_Q_FP8) sc = sc / 448.0f;
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
  if (cols % LPT_COLS || (1LL << shift) != block || block < 8 || block > LPT_COLS) return MUON_ERR_SHAPE;
  const int64_t ges = gdt == MUON_DT_F32 ? 4 : 2;
  for (int i = 0; i < ntensors; ++i) {
    if (((uintptr_t)grads[i] & 15) || ((uintptr_t)codes[i] & 7) || ((uintptr_t)scales[i] & 3))
      return MUON_ERR_SHAPE;
  }
  (void)ges;
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
  const int64_t mst = L.m_pad * L.n_pad;
  a.x0 = (char*)ws + L.off_x0 + mat0 * mst * 2;
  a.x_pitch = L.n_pad;
  a.x_mstride = mst;
  a.partials = (float*)((char*)ws + L.off_part) + mat0 * L.parts;
  a.parts = L.parts;
  const int64_t rows_pad = L.tall ? L.n_pad : L.m_pad;
  a.tiles_c = (int)(cols / LPT_COLS);
  a.tiles_used = (int)((rows_pad / LPT_ROWS) * a.tiles_c);
  if (a.tiles_used > L.parts) return MUON_ERR_SHAPE;
  a.momentum = momentum;
  a.nesterov = nesterov;
  a.maximize = maximize;
  dim3 grid((unsigned)L.parts, (unsigned)(ntensors * nb));
  switch (gdt) {
    case MUON_DT_F32: launch_lp_tile_q<MUON_DT_F32>(qf, L.tall, a, grid, s); break;
    case MUON_DT_BF16: launch_lp_tile_q<MUON_DT_BF16>(qf, L.tall, a, grid, s); break;
    case MUON_DT_F16: launch_lp_tile_q<MUON_DT_F16>(qf, L.tall, a, grid, s); break;
    default:
      muon_set_error("lp_prepass: unsupported grad dtype %d", gdt);
      return MUON_ERR_DTYPE;
  }
  MUON_CHECK_LAUNCH("lp_prepass_tiled");
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
