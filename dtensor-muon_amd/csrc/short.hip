// Orthogonalization iterations of short matrices: at most 64 rows in the wide
// orientation (m <= 64), as stacked experts flattened to (experts, rest) produce.
//
// The iterate X is stored 64 x n_pad (rows m..63 and columns n..n_pad-1 zero), so
// A = X X^T and B = b A + c A A are single 64 x 64 blocks, and every product of an
// iteration is bound by streaming X through HBM, not by the matrix cores (X X^T does
// 64 FLOP per byte of X). One iteration is:
//   short_gram_kernel  (first iteration only) partial Gram matrices of X over column
//                      ranges: [matrix][range][blocks (0,0), (0,1), (1,1) of 32 x 32] fp32;
//   short_poly_kernel  per matrix, the fixed-order sum of the partials -> A (bf16; the
//                      Frobenius prescale folds in as s^2 on the first iteration), then
//                      B = c (A A + (b / c) A) rounded to bf16;
//   short_bx_kernel    X' = alpha (B X + ratio X) over 64 x 256 column panels, plus the
//                      partial Gram matrices of the bf16 X' for the next iteration,
//                      formed from the registers that hold X' (X is read once per
//                      iteration, X' written once).
// The arithmetic is the one of the tiled path (gemm.hip) for the same iteration: fp32
// accumulation of bf16 products, A and B rounded to bf16 once, X' = alpha (acc + ratio X)
// rounded once; only the summation order of the Gram sums differs (column ranges).
#include <algorithm>
#include <cstring>

#include "common.h"

namespace {

constexpr int SG_ROWS = 64;          // stored rows of the iterate
constexpr int SG_PANEL = 256;        // columns per workgroup step: 4 waves x 64
constexpr int SG_PART = 3 * 1024;    // floats per Gram partial (three 32 x 32 blocks)
constexpr int SG_WAVE_LDS = 64 * 128;  // a wave's 64 x 64 bf16 sub-panel
constexpr int64_t SG_GRID_Y = 65535;   // matrices per launch (grid y extent)

typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
typedef __attribute__((ext_vector_type(2))) float f2x;
typedef __attribute__((ext_vector_type(2))) __bf16 bf2x;  // v_cvt_pk_bf16_f32 (RNE)

struct ShortArgs {
  const bf16_t* x;     // iterate of matrix 0 (64 rows of `pitch` elements)
  bf16_t* xo;          // next iterate (short_bx_kernel)
  bf16_t* bm;          // B: 64 x 64 bf16 per matrix, row-major
  float* part;         // Gram partials [matrix][P][SG_PART]
  int64_t pitch;       // n_pad
  int64_t mstride;     // 64 * n_pad
  int panels;          // n_pad / 256
  int P;               // column ranges (partials) per matrix
  float alpha, beta;   // short_bx_kernel: X' = alpha B X + beta X
  float pa, pb;        // short_poly_kernel: B = pa A A + pb A
  const float* scale;  // per-matrix Frobenius prescale s
  int first;           // fold s in (A *= s^2; alpha, beta *= s)
  int gram;            // short_bx_kernel: write the next iteration's partials
  int64_t b0;          // index of this launch's matrix 0 in the bucket (the apply's tensors)
};

// Column range [pb, pe) of panels for range p: balanced, non-empty when P <= panels.
MUON_DEVICE void short_range(const ShortArgs& a, int p, int& pb, int& pe) {
  pb = (int)((int64_t)p * a.panels / a.P);
  pe = (int)((int64_t)(p + 1) * a.panels / a.P);
}

MUON_DEVICE bf16x8_mfma as_frag(uint4 v) { return __builtin_bit_cast(bf16x8_mfma, v); }

// Sum of the four waves' Gram accumulators in a fixed order, written as partial p of
// matrix b. Accumulator element r of lane l in block q is at q * 1024 + r * 64 + l.
// Called by the whole workgroup after its last use of `red` for other data.
MUON_DEVICE void short_write_partial(const ShortArgs& a, float* red, const f32x16& g00,
                                     const f32x16& g01, const f32x16& g11, int b, int p) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __syncthreads();
  float* mine = red + wave * SG_PART;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    mine[r * 64 + lane] = g00[r];
    mine[1024 + r * 64 + lane] = g01[r];
    mine[2048 + r * 64 + lane] = g11[r];
  }
  __syncthreads();
  float* out = a.part + ((int64_t)b * a.P + p) * SG_PART;
#pragma unroll
  for (int k = 0; k < SG_PART / 256; ++k) {
    const int e = k * 256 + tid;
    out[e] = ((red[e] + red[SG_PART + e]) + red[2 * SG_PART + e]) + red[3 * SG_PART + e];
  }
}

// Partial Gram matrices of X over column ranges: grid (P, batch), 4 waves. Wave w takes
// columns 64 w .. +63 of every panel of the range; lane l loads rows l % 32 and
// l % 32 + 32, elements 32 (l / 32) .. +31 of those 64 columns, and its four 16-byte
// pieces per row are directly the MFMA fragments of both operands: a Gram sum may
// take its k in any order as long as both operands use the same one. One load
// instruction covers 32 bytes of each of 32 rows, so the loads are ordinary (cached):
// the four instructions that complete a 128-byte line then hit it in L2 (measured with
// non-temporal loads instead: 3.7 TB/s against 6.0 TB/s).
__global__ __launch_bounds__(256) void short_gram_kernel(ShortArgs a) {
  __shared__ __align__(16) float red[4 * SG_PART];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int p = blockIdx.x, b = blockIdx.y;
  int pb, pe;
  short_range(a, p, pb, pe);
  const bf16_t* x0 = a.x + (int64_t)b * a.mstride + (int64_t)(lane & 31) * a.pitch +
                     wave * 64 + (lane >> 5) * 32;
  const bf16_t* x1 = x0 + 32 * a.pitch;
  f32x16 g00 = {}, g01 = {}, g11 = {};
  uint4 f0[4], f1[4];
  auto load = [&](int pn) {
    const int64_t o = (int64_t)pn * SG_PANEL;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f0[q] = *(const uint4*)(x0 + o + 8 * q);
      f1[q] = *(const uint4*)(x1 + o + 8 * q);
    }
  };
  if (pb < pe) load(pb);
  for (int pn = pb; pn < pe; ++pn) {
    bf16x8_mfma h0[4], h1[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      h0[q] = as_frag(f0[q]);
      h1[q] = as_frag(f1[q]);
    }
    if (pn + 1 < pe) load(pn + 1);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      g00 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(h0[q], h0[q], g00, 0, 0, 0);
      g01 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(h0[q], h1[q], g01, 0, 0, 0);
      g11 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(h1[q], h1[q], g11, 0, 0, 0);
    }
  }
  short_write_partial(a, red, g00, g01, g11, b, p);
}

// A from the partials, then B: grid (batch), 1024 threads.
__global__ __launch_bounds__(1024) void short_poly_kernel(ShortArgs a) {
#pragma clang fp contract(off)
  __shared__ float G[SG_ROWS][SG_ROWS + 1];
  const int t = threadIdx.x, b = blockIdx.x;
  const float* part = a.part + (int64_t)b * a.P * SG_PART;
  // thread t owns element t of each block; partials summed in order p = 0, 1, ...
  float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f;
#pragma unroll 16
  for (int p = 0; p < a.P; ++p) {
    const float* pp = part + (int64_t)p * SG_PART;
    s0 += pp[t];
    s1 += pp[1024 + t];
    s2 += pp[2048 + t];
  }
  // element r * 64 + l of a block is (8 (r / 4) + 4 (l / 32) + r % 4, l % 32)
  const int r = t >> 6, l = t & 63;
  const int bi = 8 * (r >> 2) + 4 * (l >> 5) + (r & 3), bj = l & 31;
  float alpha = 1.0f;
  if (a.first) {
    const float s = a.scale[b];
    alpha *= s * s;
  }
  // exact symmetry: diagonal blocks keep their upper triangle, block (0,1) both halves
  if (bi <= bj) {
    const float v0 = bf16_to_f32(f32_to_bf16(alpha * s0));
    const float v2 = bf16_to_f32(f32_to_bf16(alpha * s2));
    G[bi][bj] = v0;
    G[bj][bi] = v0;
    G[32 + bi][32 + bj] = v2;
    G[32 + bj][32 + bi] = v2;
  }
  {
    const float v1 = bf16_to_f32(f32_to_bf16(alpha * s1));
    G[bi][32 + bj] = v1;
    G[32 + bj][bi] = v1;
  }
  __syncthreads();
  // B(i, j .. j+3) = pa (sum_k A(i, k) A(k, j) + (pb / pa) A(i, j)), k ascending
  const float ratio = a.pb != 0.0f ? a.pb / a.pa : 0.0f;
  const int i = t >> 4, j0 = (t & 15) * 4;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
  for (int k = 0; k < SG_ROWS; ++k) {
    const float aik = G[i][k];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = __builtin_fmaf(aik, G[k][j0 + q], acc[q]);
  }
  uint16_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    // c = 0 (a custom Newton-Schulz table): B = b A, as the tiled path computes it
    const float rv = ratio * G[i][j0 + q];
    o[q] = f32_to_bf16(a.pa != 0.0f ? a.pa * (acc[q] + rv) : a.pb * G[i][j0 + q]);
  }
  uint2 w;
  w.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
  w.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
  *(uint2*)(a.bm + (int64_t)b * SG_ROWS * SG_ROWS + i * SG_ROWS + j0) = w;
}

// 16-byte chunk position of logical chunk c in row `row` of a wave's sub-panel (rows of
// 128 bytes). Bit 2 (row bit 1) puts the four rows of one transposing read in four
// different 64-byte bank groups; bits 0-1 (row bits 2-3) spread the 32 rows of one
// 8-byte column access over the chunk positions.
MUON_DEVICE int sg_swz(int row) { return (((row >> 1) & 1) << 2) | ((row >> 2) & 3); }

// X' = alpha (B X + ratio X), and the next partial Gram matrices: grid (P, batch), 4
// waves. Wave w owns columns 64 w .. +63 of each panel of its range and an 8 KB LDS
// region holding that 64 x 64 sub-panel, so the waves never wait for each other inside
// the loop. Per sub-panel: 8 coalesced 16-byte loads per lane (rows 8 t + lane / 8,
// chunk lane % 8) into the region, the next sub-panel's loads issued right after; per
// 32-column block fn, the MFMA takes the X^T fragment (ds_read_b64_tr_b16: within 16
// lanes, lane r points at row kb + r / 4, columns jb + 4 (r % 4) .. +3 and receives
// column jb + r of rows kb .. kb+3) as its first operand and B(i, k .. k+7) as its
// second, so lane l's accumulator holds row i = 32 fm + l % 32, columns
// 32 fn + 8 rg + 4 (l / 32) + q (element 4 rg + q). The beta term reads those 8 bytes of
// row i from the region; X' goes back into the region (block fn's columns, already
// consumed) and leaves as whole 128-byte row pieces. The bf16 X' of rows i and i + 32
// in the same registers forms the Gram fragments of the next iteration (16 columns per
// fragment: lane l holds columns 16 h + 4 (l / 32) + {0..3, 8..11}).
// AM >= 0 (the last iteration of a wide bucket of bf16 parameters): X' is not stored; each
// 16-byte piece of it is the update of 8 parameter elements, applied as the post-pass does
// (apply_bf16x8, form AM) and the parameter written back. The parameter pieces of a panel
// load before the next panel's X, so waiting for them never waits for that prefetch.
template <int AM>
__global__ __launch_bounds__(256) void short_bx_kernel(ShortArgs a, MuonApply ap) {
  __shared__ __align__(16) float red[4 * SG_PART];  // sub-panels (32 KB), then partials
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int p = blockIdx.x, b = blockIdx.y;
  int pb, pe;
  short_range(a, p, pb, pe);
  float alpha = a.alpha, beta = a.beta;
  if (a.first) {
    const float s = a.scale[b];
    alpha *= s;
    beta *= s;
  }
  const float ratio = beta != 0.0f ? beta / alpha : 0.0f;

  // B fragments: lane l holds B(32 fm + l % 32, 16 ks + 8 (l / 32) .. +7)
  bf16x8_mfma bfr[2][4];
  {
    const bf16_t* bp = a.bm + (int64_t)b * SG_ROWS * SG_ROWS + (lane & 31) * SG_ROWS + (lane >> 5) * 8;
#pragma unroll
    for (int fm = 0; fm < 2; ++fm)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        bfr[fm][ks] = as_frag(*(const uint4*)(bp + fm * 32 * SG_ROWS + ks * 16));
  }

  uint8_t* reg = (uint8_t*)red + wave * SG_WAVE_LDS;
  // load / store lanes: row 8 t + lr, logical chunk lc
  const int lr = lane >> 3, lc = lane & 7;
  const int64_t loff = (int64_t)b * a.mstride + (int64_t)lr * a.pitch + wave * 64 + lc * 8;
  const bf16_t* xs = a.x + loff;
  bf16_t* xd = a.xo + loff;
  uint4 cur[8];
  // apply: parameter element (row, col) of this matrix at byte row * ldp_b + 2 col from prm;
  // a lane outside the parameter takes an offset past the descriptor's range (its loads read
  // zeros, its stores are dropped)
  bf16_t* prm = nullptr;
  int ldp_b = 0, vop = 0;
  float adj = 0.0f, adjr = 0.0f;
  muon_u32x4 pv[8];
  if constexpr (AM >= 0) {
    const int64_t bg = a.b0 + b;
    const int t = (int)(bg / ap.nb);
    const int64_t mb = bg - (int64_t)t * ap.nb;
    prm = (bf16_t*)ap.params[t] + mb * ap.prows * ap.pcols;
    ldp_b = (int)(ap.pcols * 2);
    vop = lr * ldp_b + (wave * 64 + lc * 8) * 2;
    adj = ap.adj[t];
    adjr = bf16_to_f32(f32_to_bf16(adj));
  }
  const __amdgpu_buffer_rsrc_t rsp =
      __builtin_amdgcn_make_buffer_rsrc((void*)prm, 0, AM >= 0 ? 0x7fffffff : 0, 0x00020000);
  auto pvoff = [&](int pn, int t) -> int {
    return 8 * t + lr < ap.prows && pn * SG_PANEL + wave * 64 + lc * 8 < ap.pcols ? vop
                                                                                  : (int)0x80000000;
  };
  auto load = [&](int pn) {
    const int64_t o = (int64_t)pn * SG_PANEL;
#pragma unroll
    for (int t = 0; t < 8; ++t) cur[t] = ld_nt(xs + o + 8 * t * a.pitch);
  };
  // transposing-read lanes: group g = lane / 16, r = lane % 16
  const int tg = lane >> 4, tr = lane & 15;
  const int fi = lane & 31, fh = lane >> 5;

  f32x16 g00 = {}, g01 = {}, g11 = {};
  if (pb < pe) load(pb);
  for (int pn = pb; pn < pe; ++pn) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int row = 8 * t + lr;
      *(uint4*)(reg + row * 128 + ((lc ^ sg_swz(row)) << 4)) = cur[t];
    }
    // the transposing reads return other lanes' data: keep every LDS access of the
    // wave in program order (LDS serves one wave's accesses in order)
    asm volatile("" ::: "memory");
    if constexpr (AM >= 0) {
#pragma unroll
      for (int t = 0; t < 8; ++t)
        pv[t] = __builtin_amdgcn_raw_buffer_load_b128(rsp, pvoff(pn, t), 8 * t * ldp_b + pn * 2 * SG_PANEL, 2);
    }
    if (pn + 1 < pe) load(pn + 1);
#pragma unroll
    for (int fn = 0; fn < 2; ++fn) {
      bf16x8_mfma xf[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int row = 16 * ks + 8 * (tg >> 1) + (tr >> 2);
        const int c = 4 * fn + 2 * (tg & 1) + ((tr & 3) >> 1);
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(reg + row * 128 + ((c ^ sg_swz(row)) << 4) + (tr & 1) * 8));
        const int row4 = row + 4;
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(reg + row4 * 128 + ((c ^ sg_swz(row4)) << 4) + (tr & 1) * 8));
        xf[ks] = __builtin_bit_cast(bf16x8_mfma, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
      f32x16 acc[2] = {{}, {}};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int fm = 0; fm < 2; ++fm)
          acc[fm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xf[ks], bfr[fm][ks], acc[fm], 0, 0, 0);
      u32x2 w[2][4];
#pragma unroll
      for (int fm = 0; fm < 2; ++fm) {
        const int row = 32 * fm + fi;
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          uint8_t* pos = reg + row * 128 + (((4 * fn + rg) ^ sg_swz(row)) << 4) + fh * 8;
          const u32x2 xw = *(const u32x2*)pos;
          const f2x v01 = {alpha * (acc[fm][rg * 4 + 0] + ratio * __uint_as_float(xw.x << 16)),
                           alpha * (acc[fm][rg * 4 + 1] + ratio * __uint_as_float(xw.x & 0xffff0000u))};
          const f2x v23 = {alpha * (acc[fm][rg * 4 + 2] + ratio * __uint_as_float(xw.y << 16)),
                           alpha * (acc[fm][rg * 4 + 3] + ratio * __uint_as_float(xw.y & 0xffff0000u))};
          w[fm][rg] = u32x2{__builtin_bit_cast(uint32_t, __builtin_convertvector(v01, bf2x)),
                            __builtin_bit_cast(uint32_t, __builtin_convertvector(v23, bf2x))};
          *(u32x2*)pos = w[fm][rg];
        }
      }
      if (AM < 0 && a.gram) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const bf16x8_mfma h0 = as_frag(uint4{w[0][2 * h].x, w[0][2 * h].y, w[0][2 * h + 1].x, w[0][2 * h + 1].y});
          const bf16x8_mfma h1 = as_frag(uint4{w[1][2 * h].x, w[1][2 * h].y, w[1][2 * h + 1].x, w[1][2 * h + 1].y});
          g00 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(h0, h0, g00, 0, 0, 0);
          g01 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(h0, h1, g01, 0, 0, 0);
          g11 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(h1, h1, g11, 0, 0, 0);
        }
      }
    }
    asm volatile("" ::: "memory");
    const int64_t o = (int64_t)pn * SG_PANEL;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int row = 8 * t + lr;
      const uint4 xw = *(const uint4*)(reg + row * 128 + ((lc ^ sg_swz(row)) << 4));
      if constexpr (AM >= 0) {
        const muon_u32x4 u4 = {xw.x, xw.y, xw.z, xw.w};
        __builtin_amdgcn_raw_buffer_store_b128(apply_bf16x8<AM>(u4, pv[t], adj, adjr, ap.wd), rsp,
                                               pvoff(pn, t), 8 * t * ldp_b + pn * 2 * SG_PANEL, 2);
      } else {
        st_nt(xd + o + 8 * t * a.pitch, xw);
      }
    }
    asm volatile("" ::: "memory");
  }
  if (AM < 0 && a.gram) short_write_partial(a, red, g00, g01, g11, b, p);
}

}  // namespace

// Column ranges (Gram partials) per matrix of a short iterate with n_pad columns:
// at least 4 panels per range where possible, at most 256 ranges.
int64_t muon_short_parts(int64_t n_pad) {
  const int64_t panels = n_pad / SG_PANEL;
  return std::max<int64_t>(1, std::min<int64_t>(256, panels / 4));
}

// Launch helpers for muon_orth_run (api.hip). X, X' and B point at matrix 0.
int muon_launch_short_gram(const OrthLayout& L, const void* x, float* part, int64_t batch,
                           hipStream_t s) {
  ShortArgs a = {};
  a.x = (const bf16_t*)x;
  a.part = part;
  a.pitch = L.n_pad;
  a.mstride = SG_ROWS * L.n_pad;
  a.panels = (int)(L.n_pad / SG_PANEL);
  a.P = (int)L.gparts;
  for (int64_t b0 = 0; b0 < batch; b0 += SG_GRID_Y) {
    ShortArgs c = a;
    c.x += b0 * c.mstride;
    c.part += b0 * c.P * SG_PART;
    const int64_t nb = std::min<int64_t>(SG_GRID_Y, batch - b0);
    hipLaunchKernelGGL(short_gram_kernel, dim3((unsigned)c.P, (unsigned)nb), dim3(256), 0, s, c);
  }
  MUON_CHECK_LAUNCH("short_gram");
  return MUON_OK;
}

int muon_launch_short_poly(const OrthLayout& L, float* part, void* bm, int64_t batch, float pa,
                           float pb, const float* scale, int first, hipStream_t s) {
  ShortArgs a = {};
  a.bm = (bf16_t*)bm;
  a.part = part;
  a.P = (int)L.gparts;
  a.pa = pa;
  a.pb = pb;
  a.scale = scale;
  a.first = first;
  hipLaunchKernelGGL(short_poly_kernel, dim3((unsigned)batch), dim3(1024), 0, s, a);
  MUON_CHECK_LAUNCH("short_poly");
  return MUON_OK;
}

// X' = alpha B X + beta X of a short iterate (ap == nullptr: into xo, with the next partials
// when gram), or the last iteration with the apply of a wide bucket of bf16 parameters
// (ap: X' is not stored, the parameters are updated in place; no partials).
static int launch_short_bx(const OrthLayout& L, const void* x, void* xo, const void* bm,
                           float* part, int64_t batch, float alpha, float beta,
                           const float* scale, int first, int gram, const MuonApply* ap,
                           hipStream_t s) {
  if (alpha == 0.0f) {
    muon_set_error("short_bx: alpha must be nonzero");
    return MUON_ERR_ARG;
  }
  int mode = -1;
  MuonApply none;
  memset(&none, 0, sizeof(none));
  none.nb = 1;
  if (ap) {
    if (L.tall || ap->prows > L.m || ap->pcols > L.n || ap->pcols % 8 || ap->nb <= 0 ||
        (batch + ap->nb - 1) / ap->nb > MUON_APPLY_MAX ||
        // every byte offset the kernel forms (rows up to 64, plus the out-of-range marker
        // 2^31 for lanes outside the parameter) stays below 2^32
        (int64_t)SG_ROWS * ap->pcols * 2 + SG_PANEL * 2 > (int64_t)0x7fffffff) {
      muon_set_error("short_bx: apply does not fit this layout");
      return MUON_ERR_ARG;
    }
    mode = ap->wd == 0.0f ? 0 : (ap->cautious ? 1 : 2);
    gram = 0;
  }
  const MuonApply& apv = ap ? *ap : none;
  ShortArgs a = {};
  a.x = (const bf16_t*)x;
  a.xo = (bf16_t*)xo;
  a.bm = (bf16_t*)bm;
  a.part = part;
  a.pitch = L.n_pad;
  a.mstride = SG_ROWS * L.n_pad;
  a.panels = (int)(L.n_pad / SG_PANEL);
  a.P = (int)L.gparts;
  a.alpha = alpha;
  a.beta = beta;
  a.scale = scale;
  a.first = first;
  a.gram = gram;
  for (int64_t b0 = 0; b0 < batch; b0 += SG_GRID_Y) {
    ShortArgs c = a;
    c.x += b0 * c.mstride;
    if (c.xo) c.xo += b0 * c.mstride;
    c.bm += b0 * SG_ROWS * SG_ROWS;
    if (c.part) c.part += b0 * c.P * SG_PART;
    c.scale = scale ? scale + b0 : nullptr;
    c.b0 = b0;
    const int64_t nb = std::min<int64_t>(SG_GRID_Y, batch - b0);
    const dim3 grid((unsigned)c.P, (unsigned)nb);
    switch (mode) {
      case 0: hipLaunchKernelGGL(short_bx_kernel<0>, grid, dim3(256), 0, s, c, apv); break;
      case 1: hipLaunchKernelGGL(short_bx_kernel<1>, grid, dim3(256), 0, s, c, apv); break;
      case 2: hipLaunchKernelGGL(short_bx_kernel<2>, grid, dim3(256), 0, s, c, apv); break;
      default: hipLaunchKernelGGL(short_bx_kernel<-1>, grid, dim3(256), 0, s, c, apv); break;
    }
  }
  MUON_CHECK_LAUNCH("short_bx");
  return MUON_OK;
}

int muon_launch_short_bx(const OrthLayout& L, const void* x, void* xo, const void* bm,
                         float* part, int64_t batch, float alpha, float beta, const float* scale,
                         int first, int gram, hipStream_t s) {
  return launch_short_bx(L, x, xo, bm, part, batch, alpha, beta, scale, first, gram, nullptr, s);
}

int muon_launch_short_bx_apply(const OrthLayout& L, const void* x, const void* bm,
                               int64_t batch, float alpha, float beta, const float* scale,
                               int first, const MuonApply& ap, hipStream_t s) {
  return launch_short_bx(L, x, nullptr, bm, nullptr, batch, alpha, beta, scale, first, 0, &ap, s);
}
