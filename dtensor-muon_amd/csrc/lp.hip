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
