// Batched matrix products on CDNA4 MFMA for the Newton-Schulz / Polar Express
// iteration.
//
//  * SYRK mode ("NT": C(i, j) = alpha * sum_k A(i, k) A(j, k) + beta * Cin(i, j), both
//    operands K-contiguous rows, upper-triangle tiles only, mirrored store): the Gram
//    products X X^T and A A (A symmetric) of pe_loop_triton / ns_loop_triton
//    (polar_express.py:98-104, newton_schulz.py:105-112; Triton gram_nd,
//    gram.py:21-106). The polynomial combination B = b*A + c*A^2 rides in the
//    epilogue (beta*Cin with Cin = A).
//  * GEMM mode ("NN": C(i, j) = alpha * sum_k B(i, k) X(k, j) + beta * X(i, j)):
//    X' = a*X + B X (polar_express.py:109-110) with X in its own row-major layout
//    as the second operand; the epilogue writes X' row-major (into the other of two
//    ping-pong buffers) or, for the last iteration of a tall matrix, transposed.
//
// Operands live in workspaces whose extents are padded to the tile size and whose
// padding is rewritten as zeros by every producer, so the K loop and the stores
// need no masking (only the standalone gram_ path uses the masked variant). The one
// exception is the last 128 rows and columns of a SYRK output whose valid extent
// leaves them empty (packed tiles, below): what reads them lands only in output rows
// that are masked to zeros or not stored.
#include <algorithm>
#include <atomic>
#include <cstring>
#include <mutex>
#include <type_traits>

#include "common.h"

namespace {

enum { MODE_GEMM = 0, MODE_SYRK = 1 };

struct GemmArgs {
  const void* a;   // operand rows i, K contiguous
  const void* b;   // operand rows j, K contiguous
  const void* cin; // beta source, element (i, j) at cin[i * ldc + j]
  void* out;       // (i, j) at out[i * ldo + j]
  void* out_t;     // optional: (j, i) at out_t[j * ldt + i]
  int64_t lda, ldb, ldc, ldo, ldt;
  int64_t sa, sb, sc, so, st;  // batch strides in elements
  int64_t K;                   // multiple of BK (padded)
  int64_t Mv, Nv;              // valid extents; outside them zeros are stored
  int64_t Mt, Nt, Kt;          // masked variant only: true row counts of a / b and K
  float alpha, beta;
  const float* scale;          // per-batch prescale s (nullable)
  int scale_mode;              // 1: alpha *= s, beta *= s;  2: alpha *= s * s
  int tiles_m, tiles_n, tiles_per_batch;
  int tiles_total;             // tiles_per_batch * batch
  int store_out, store_out_t;
};

// Workgroup L of a one-tile-per-workgroup launch of `total` -> tile index. Dispatch
// hands consecutive workgroups to the 8 XCDs round-robin (L on XCD L % 8). When a matrix
// has at least XCD_STRIPE tiles, XCD x takes stripes x, x + 8, x + 16, ... of XCD_STRIPE
// consecutive tiles while whole rounds of 8 stripes remain, so all XCDs work on the same
// matrices at a time (the operand panels their L2s miss on then come from one matrix's
// worth of data, which the Infinity Cache holds: X X^T on the 4096 x 14336 bucket 5%
// faster than contiguous ranges); the rest, or every tile of launches of smaller
// matrices, is dealt as one contiguous range per XCD, so each XCD works through
// neighbouring tiles with its own L2.
constexpr int XCD_STRIPE = 64;
MUON_DEVICE int64_t xcd_tile(int64_t L, int64_t total, int tiles_per_batch) {
  const int64_t x = L & 7, i = L >> 3;
  const int64_t nfull = tiles_per_batch >= XCD_STRIPE ? total / (8 * XCD_STRIPE) * XCD_STRIPE : 0;
  const int64_t rq = (total - 8 * nfull) >> 3, rr = (total - 8 * nfull) & 7;
  return i < nfull ? ((i / XCD_STRIPE) * 8 + x) * XCD_STRIPE + i % XCD_STRIPE
                   : 8 * nfull + x * rq + std::min<int64_t>(x, rr) + (i - nfull);
}

MUON_DEVICE void map_tile(const GemmArgs& g, int mode, int& bidx, int& tm, int& tn) {
  const int64_t L = xcd_tile(blockIdx.x, (int64_t)gridDim.x, g.tiles_per_batch);
  bidx = (int)(L / g.tiles_per_batch);
  int t = (int)(L % g.tiles_per_batch);
  if (mode == MODE_SYRK) {
    int T = g.tiles_m, r = 0;
    while (t >= T - r) {
      t -= T - r;
      ++r;
    }
    tm = r;
    tn = r + t;
  } else {
    const int GM = 8;  // 8 tile rows per group: measured best for the GEMM stores (X^T rows stay adjacent)
    int TN = g.tiles_n, TM = g.tiles_m;
    int group = t / (GM * TN);
    int first = group * GM;
    int gsz = min(TM - first, GM);
    int local = t % (GM * TN);
    tm = first + local % gsz;
    tn = local / gsz;
  }
}

template <typename OutT>
MUON_DEVICE void store_elem(void* p, int64_t idx, float v);
template <>
MUON_DEVICE void store_elem<bf16_t>(void* p, int64_t idx, float v) {
  ((bf16_t*)p)[idx] = f32_to_bf16(v);
}
template <>
MUON_DEVICE void store_elem<float>(void* p, int64_t idx, float v) {
  ((float*)p)[idx] = v;
}
template <typename OutT>
MUON_DEVICE float load_elem(const void* p, int64_t idx);
template <>
MUON_DEVICE float load_elem<bf16_t>(const void* p, int64_t idx) {
  return bf16_to_f32(((const bf16_t*)p)[idx]);
}
template <>
MUON_DEVICE float load_elem<float>(const void* p, int64_t idx) {
  return ((const float*)p)[idx];
}

// Store 4 values at consecutive addresses (i0..i0+3 of row j in the transposed view).
template <typename OutT>
MUON_DEVICE void store4(void* p, int64_t idx, const float* v);
template <>
MUON_DEVICE void store4<bf16_t>(void* p, int64_t idx, const float* v) {
  uint2 w;
  w.x = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
  w.y = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
  *(uint2*)((bf16_t*)p + idx) = w;
}
template <>
MUON_DEVICE void store4<float>(void* p, int64_t idx, const float* v) {
  *(float4*)((float*)p + idx) = make_float4(v[0], v[1], v[2], v[3]);
}

// Epilogue over one wave's FM x FN grid of 32x32 MFMA accumulators.
// 32x32 accumulator layout: lane l, register r -> column j = l % 32,
// row i = 8 * (r / 4) + 4 * (l / 32) + r % 4.
// Unmasked (workspace) outputs are padded to the tile, and elements outside the
// valid Mv x Nv region are stored as zeros so the padding stays zero. Masked
// (caller-owned, unpadded) outputs skip every store outside the valid region and
// use element stores only, since their row pitch need not keep 4-element groups
// aligned.
template <typename OutT, int FM, int FN, bool MASKED>
MUON_DEVICE void epilogue(const GemmArgs& g, int mode, int bidx, int64_t row0, int64_t col0,
                          f32x16 (&acc)[FM][FN], int lane, bool diag) {
  float alpha = g.alpha, beta = g.beta;
  if (g.scale_mode != 0) {
    float s = g.scale[bidx];
    if (g.scale_mode == 1) {
      alpha *= s;
      beta *= s;
    } else {
      alpha *= s * s;
    }
  }
  const int64_t lc = lane & 31, lr = (lane >> 5) * 4;
  void* out = g.out ? (void*)((OutT*)g.out + (int64_t)bidx * g.so) : nullptr;
  void* out_t = g.out_t ? (void*)((OutT*)g.out_t + (int64_t)bidx * g.st) : nullptr;
  const void* cin = g.cin ? (const void*)((const OutT*)g.cin + (int64_t)bidx * g.sc) : nullptr;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int64_t j = col0 + fn * 32 + lc;
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        const int64_t i0 = row0 + fm * 32 + rb * 8 + lr;
        float v[4];
        bool ok[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t i = i0 + q;
          ok[q] = i < g.Mv && j < g.Nv;
          float x = alpha * acc[fm][fn][rb * 4 + q];
          if (beta != 0.0f && ok[q]) x += beta * load_elem<OutT>(cin, i * g.ldc + j);
          if (!ok[q]) x = 0.0f;
          v[q] = x;
        }
        if (mode == MODE_SYRK) {
          if (!diag) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (!MASKED || ok[q]) store_elem<OutT>(out, (i0 + q) * g.ldo + j, v[q]);
            if (!MASKED) {
              store4<OutT>(out, j * g.ldo + i0, v);
            } else {
#pragma unroll
              for (int q = 0; q < 4; ++q)
                if (ok[q]) store_elem<OutT>(out, j * g.ldo + i0 + q, v[q]);
            }
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int64_t i = i0 + q;
              if (MASKED && !ok[q]) continue;
              if (i <= j) store_elem<OutT>(out, i * g.ldo + j, v[q]);
              if (i < j) store_elem<OutT>(out, j * g.ldo + i, v[q]);
            }
          }
        } else {
          if (g.store_out) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (!MASKED || ok[q]) store_elem<OutT>(out, (i0 + q) * g.ldo + j, v[q]);
          }
          if (g.store_out_t) {
            if (!MASKED) {
              store4<OutT>(out_t, j * g.ldt + i0, v);
            } else {
#pragma unroll
              for (int q = 0; q < 4; ++q)
                if (ok[q]) store_elem<OutT>(out_t, j * g.ldt + i0 + q, v[q]);
            }
          }
        }
      }
    }
  }
}

// ----------------------------------------------------------------------------------
// bf16: 256 x 256 x 64 tile over a WGM x WGN grid of wavefronts, each owning a
// (256/WGM) x (256/WGN) block of 32x32x16 MFMA accumulators. With 4 wavefronts
// (2 x 2) each holds 128 x 128 (256 fp32 accumulators per lane, one wave per SIMD);
// with 8 (2 x 4) each holds 128 x 64 and two waves share a SIMD, hiding each
// other's LDS and memory latency. LDS: double-buffered operand panels with an
// 8-element row pad (row pitch 144 B) so the 16-byte fragment reads of consecutive
// rows hit distinct banks. Global loads for tile k+1 are issued before the MFMAs of
// tile k and parked in registers until the LDS slot frees up.
constexpr int BF_BM = 256, BF_BN = 256, BF_BK = 64, BF_LDSP = BF_BK + 8;
constexpr int BF_SMEM = 2 * (BF_BM + BF_BN) * BF_LDSP * 2;

template <int MODE, bool MASKED, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void gemm_bf16_kernel(GemmArgs g) {
  constexpr int NT = 64 * WGM * WGN;
  constexpr int WM = BF_BM / WGM, WN = BF_BN / WGN;
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int CPT = (BF_BM * BF_BK / 8) / NT;  // 16-byte chunks per thread per operand
  constexpr int RPQ = NT / 8;                      // rows covered by one chunk pass
  extern __shared__ __align__(16) uint8_t smem[];
  bf16_t* As = (bf16_t*)smem;
  bf16_t* Bs = As + 2 * BF_BM * BF_LDSP;

  int bidx, tm, tn;
  map_tile(g, MODE, bidx, tm, tn);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;

  const bf16_t* A = (const bf16_t*)g.a + (int64_t)bidx * g.sa;
  const bf16_t* B = (const bf16_t*)g.b + (int64_t)bidx * g.sb;
  const int64_t arow0 = (int64_t)tm * BF_BM, brow0 = (int64_t)tn * BF_BN;

  // Unmasked loads go through buffer descriptors (base in SGPRs, one VGPR offset per
  // thread, per-chunk offsets in SGPRs) to keep VGPR pressure off the main loop.
  const int64_t lda_b = g.lda * 2, ldb_b = g.ldb * 2;
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(A + arow0 * g.lda), 0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(B + brow0 * g.ldb), 0, 0x7fffffff, 0x00020000);
  const int voa = (int)((tid >> 3) * lda_b + (tid & 7) * 16);
  const int vob = (int)((tid >> 3) * ldb_b + (tid & 7) * 16);
  uint4 ra[CPT], rb[CPT];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      if (!MASKED) {
        typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
        u32x4 va = __builtin_amdgcn_raw_buffer_load_b128(rsa, voa, (int)(q * RPQ * lda_b + k0 * 2), 0);
        u32x4 vb = __builtin_amdgcn_raw_buffer_load_b128(rsb, vob, (int)(q * RPQ * ldb_b + k0 * 2), 0);
        ra[q] = make_uint4(va.x, va.y, va.z, va.w);
        rb[q] = make_uint4(vb.x, vb.y, vb.z, vb.w);
      } else {
        const int c = q * NT + tid;
        const int r = c >> 3, cc = (c & 7) * 8;
        uint16_t ta[8], tb[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int64_t k = k0 + cc + e;
          const int64_t ia = arow0 + r, ib = brow0 + r;
          ta[e] = (ia < g.Mt && k < g.Kt) ? A[ia * g.lda + k] : (uint16_t)0;
          tb[e] = (ib < g.Nt && k < g.Kt) ? B[ib * g.ldb + k] : (uint16_t)0;
        }
        __builtin_memcpy(&ra[q], ta, 16);
        __builtin_memcpy(&rb[q], tb, 16);
      }
    }
  };
  auto sstore = [&](int buf) {
    bf16_t* as = As + buf * BF_BM * BF_LDSP;
    bf16_t* bs = Bs + buf * BF_BN * BF_LDSP;
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      const int c = q * NT + tid;
      const int r = c >> 3, cc = (c & 7) * 8;
      *(uint4*)(as + r * BF_LDSP + cc) = ra[q];
      *(uint4*)(bs + r * BF_LDSP + cc) = rb[q];
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int KT = (int)(g.K / BF_BK);
  gload(0);
  sstore(0);
  __syncthreads();
  const int frow = lane & 31, fk = (lane >> 5) * 8;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload((int64_t)(kt + 1) * BF_BK);
    const bf16_t* as = As + cur * BF_BM * BF_LDSP + (wm * WM + frow) * BF_LDSP + fk;
    const bf16_t* bs = Bs + cur * BF_BN * BF_LDSP + (wn * WN + frow) * BF_LDSP + fk;
#pragma unroll
    for (int ks = 0; ks < BF_BK / 16; ++ks) {
      bf16x8_mfma af[FM], bfr[FN];
#pragma unroll
      for (int f = 0; f < FM; ++f)
        af[f] = __builtin_bit_cast(bf16x8_mfma, *(const uint4*)(as + f * 32 * BF_LDSP + ks * 16));
#pragma unroll
      for (int f = 0; f < FN; ++f)
        bfr[f] = __builtin_bit_cast(bf16x8_mfma, *(const uint4*)(bs + f * 32 * BF_LDSP + ks * 16));
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
          acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[fm], bfr[fn], acc[fm][fn], 0, 0, 0);
    }
    if (kt + 1 < KT) sstore(cur ^ 1);
    __syncthreads();
  }

  epilogue<bf16_t, FM, FN, MASKED>(g, MODE, bidx, arow0 + wm * WM, brow0 + wn * WN, acc, lane,
                                   MODE == MODE_SYRK && tm == tn);
}

// ----------------------------------------------------------------------------------
// fp32: 128 x 128 x 16 tile, 4 wavefronts in 2 x 2, each 64 x 64 (2 x 2 MFMA
// 32x32x2 f32 blocks). Used for the fp32 iteration mode and fp32 gram_. In GEMM (NN)
// mode the b panel is staged as rows k of X (pitch F_XP); the MFMA takes one value
// per lane, so no transpose is needed.
constexpr int F_BM = 128, F_BN = 128, F_BK = 16, F_LDSP = F_BK + 4, F_XP = F_BN + 4;
static_assert(F_BK * F_XP <= F_BN * F_LDSP, "fp32 X panel fits the b buffer");

template <int MODE, bool MASKED>
__global__ __launch_bounds__(256, 2) void gemm_f32_kernel(GemmArgs g) {
  __shared__ __align__(16) float As[2][F_BM * F_LDSP];
  __shared__ __align__(16) float Bs[2][F_BN * F_LDSP];

  int bidx, tm, tn;
  map_tile(g, MODE, bidx, tm, tn);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const float* A = (const float*)g.a + (int64_t)bidx * g.sa;
  const float* B = (const float*)g.b + (int64_t)bidx * g.sb;
  const int64_t arow0 = (int64_t)tm * F_BM, brow0 = (int64_t)tn * F_BN;

  float4 ra[2], rb[2];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int c = q * 256 + tid;
      const int r = c >> 2, cc = (c & 3) * 4;
      if (!MASKED) {
        ra[q] = *(const float4*)(A + (arow0 + r) * g.lda + k0 + cc);
        if (MODE == MODE_GEMM)
          rb[q] = *(const float4*)(B + (k0 + (c >> 5)) * g.ldb + brow0 + (c & 31) * 4);
        else
          rb[q] = *(const float4*)(B + (brow0 + r) * g.ldb + k0 + cc);
      } else {
        float ta[4], tb[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t k = k0 + cc + e;
          const int64_t ia = arow0 + r, ib = brow0 + r;
          ta[e] = (ia < g.Mt && k < g.Kt) ? A[ia * g.lda + k] : 0.0f;
          tb[e] = (ib < g.Nt && k < g.Kt) ? B[ib * g.ldb + k] : 0.0f;
        }
        ra[q] = make_float4(ta[0], ta[1], ta[2], ta[3]);
        rb[q] = make_float4(tb[0], tb[1], tb[2], tb[3]);
      }
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int c = q * 256 + tid;
      const int r = c >> 2, cc = (c & 3) * 4;
      *(float4*)(&As[buf][r * F_LDSP + cc]) = ra[q];
      if (MODE == MODE_GEMM)
        *(float4*)(&Bs[buf][(c >> 5) * F_XP + (c & 31) * 4]) = rb[q];
      else
        *(float4*)(&Bs[buf][r * F_LDSP + cc]) = rb[q];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int KT = (int)(g.K / F_BK);
  gload(0);
  sstore(0);
  __syncthreads();
  const int frow = lane & 31, fk = lane >> 5;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload((int64_t)(kt + 1) * F_BK);
#pragma unroll
    for (int ks = 0; ks < F_BK / 2; ++ks) {
      float af[2], bfr[2];
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        af[f] = As[cur][(wm * 64 + f * 32 + frow) * F_LDSP + ks * 2 + fk];
        bfr[f] = MODE == MODE_GEMM ? Bs[cur][(ks * 2 + fk) * F_XP + wn * 64 + f * 32 + frow]
                                   : Bs[cur][(wn * 64 + f * 32 + frow) * F_LDSP + ks * 2 + fk];
      }
#pragma unroll
      for (int fm = 0; fm < 2; ++fm)
#pragma unroll
        for (int fn = 0; fn < 2; ++fn)
          acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[fm], bfr[fn], acc[fm][fn], 0, 0, 0);
    }
    if (kt + 1 < KT) sstore(cur ^ 1);
    __syncthreads();
  }

  epilogue<float, 2, 2, MASKED>(g, MODE, bidx, arow0 + wm * 64, brow0 + wn * 64, acc, lane,
                        MODE == MODE_SYRK && tm == tn);
}

// ----------------------------------------------------------------------------------
// bf16, direct-to-LDS: the unmasked workhorse of the iteration.
//
// Main loop. 256 x 256 x 64 tile, 8 wavefronts in 4 x 2 (each 64 x 128, two waves per
// SIMD). Operands stream HBM/L2 -> LDS with `buffer_load_dwordx4 ... lds` (no VGPR
// staging, no ds_write), double-buffered: the loads of K-tile k+2 go out in two
// halves during K-tile k (a panel) and k+1 (b panel) and land while their MFMAs run. Each load
// instruction fills 1 KB of LDS (64 lanes x 16 B), i.e. 8 rows of 128 B; the lane ->
// global-address map stores 16-byte chunk c of row r at chunk position c ^ kswz(r).
// The LDS has 64 four-byte banks (256 B per cycle) and serves a 16-byte read 16 lanes
// at a time; a fragment read puts 16 consecutive rows (at one logical chunk) in those
// 16 lanes. With a 128-byte row pitch even rows start at bank 0 and odd rows at bank
// 32, so the swizzle must give the 8 even (and the 8 odd) rows of a 16-row group 8
// distinct chunk positions: kswz(r) = (r >> 1) & 7. (c ^ (r & 7) repeats every 8 rows
// and costs a 2-way conflict on every fragment read.)
// The barrier is an LDS-only wait plus s_barrier: a full __syncthreads would also
// wait for the in-flight prefetch.
//
// Software pipeline. Each k-substep (16 of the 64 k) is one inline-asm block: the 8
// MFMAs of the current fragments interleaved with the 6 LDS reads of the next
// substep's fragments, ending with those reads complete, so LDS latency hides behind
// MFMAs instead of stalling them (the compiler otherwise reorders the MFMAs of the
// next substep up against their own loads). Per K-tile k:
//   DMA of K-tile k+1's b panel into the other stage, substeps 0-2 (reading substeps
//   1-3 of this K-tile), [beta term], wait for K-tile k+1's DMA, barrier, DMA of K-tile
//   k+2's a panel into this K-tile's stage, substep 3 (reading substep 0 of K-tile k+1).
// The loop body has no branch around the MFMAs, which keeps the accumulators in one
// register assignment (a branch there made the allocator copy and spill them); the
// last tile's extra fragment reads hit a stale stage and are discarded.
//
// The beta term. Both uses of beta read the transpose of the b operand:
//   GEMM  X' = a X + B X      with b = X^T   (cin = X   = b^T)
//   SYRK  B  = c A A + b A    with b = A     (cin = A   = A^T, A symmetric)
// so cin(i, j) = b(j, i), and during the K-tile whose k range covers a wave's output
// rows i the needed values sit in the b panel in LDS. The wave adds (beta/alpha) *
// cin into its accumulators there and never reads cin from memory.
//
// Epilogue. The finished tile is staged through LDS (the operand buffers are dead by
// then) so every global store is a coalesced 16-byte row chunk:
//   * transposed stores (GEMM out_t, the mirror half of an off-diagonal SYRK tile):
//     the accumulators hold 4 consecutive rows of one column per lane, written to a
//     transposed LDS tile with 8-byte ds_writes and read back as rows;
//   * row-major stores: written element-wise to a row-major LDS tile.
// Diagonal SYRK tiles store only their upper triangle, mirrored in place, so the
// output is exactly symmetric.
//
// Packed tiles (PK). When the valid extent m leaves the last 128 rows of the padded
// extent M empty (m <= M - 128), the last tile column holds one 128-wide unit of real
// output, columns c0 = M - 256 .. M - 129. A launch of 256 x 256 tiles would spend half
// of every tile of that column on padding, so the PK kernel's full tiles stop one tile
// column short and packed tiles cover the unit: 512 rows x 128 columns per workgroup
// (two 256-row sub-tiles of the a panel against one 128-row b panel), 8 wavefronts of
// 64 x 128 each, the same inner loop. A matrix's packed tiles follow its full tiles in
// one launch: in a launch of their own they re-read every row panel from HBM (the
// m = 1408 X X^T packed tiles ran 1.7x as long as a full tile each, memory-bound). The unit's own 128 x 128 diagonal block lies in
// one packed tile and is stored symmetric as a diagonal tile is; rows and columns from
// M - 128 on are neither computed into the output nor stored. Readers of the result
// never reach them: the products contract over K <= M - 128 and mask rows beyond m.
// Per matrix the packed layout takes T(T-1)/2 + ceil((2T - 1)/4) workgroups instead
// of T(T+1)/2 (T = M / 256): 18 instead of 21 at m = 1408.
constexpr int V2_BK = 64, V2_ROWB = V2_BK * 2, V2_TILEB = 256 * V2_ROWB;
constexpr int V2_STAGEB = 2 * V2_TILEB;
constexpr int V2_EP_PITCH = 256 + 8;  // staging row pitch (elements)
constexpr int V2_SMEM = (2 * V2_STAGEB > 256 * V2_EP_PITCH * 2) ? 2 * V2_STAGEB
                                                                   : 256 * V2_EP_PITCH * 2;
constexpr int V2P_TP = 512 + 8;  // packed: transposed staging, 128 rows of 512
constexpr int V2P_RP = 128 + 8;  // packed: row-major staging, 512 rows of 128
constexpr int v2_smem(bool pk) {
  return !pk ? V2_SMEM
             : std::max(2 * (512 + 128) * V2_ROWB, std::max(128 * V2P_TP * 2, 512 * V2P_RP * 2));
}
static_assert(v2_smem(true) <= 160 * 1024, "packed SYRK tile fits the LDS");

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Chunk swizzle of a K-contiguous operand panel row (rows of 128 B in LDS); a row offset
// by a multiple of 16 keeps its swizzle.
MUON_DEVICE int kswz(int row) { return (row >> 1) & 7; }

MUON_DEVICE void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

MUON_DEVICE void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }

#define MUON_MFMA(C, A, B) "v_mfma_f32_32x32x16_bf16 %[" #C "], %[" #A "], %[" #B "], %[" #C "]\n\t"
// One k-substep of a 64 x 128 wave tile (2 x 4 accumulators of 32 x 32): 8 MFMAs on
// the current fragments (ca, cb), interleaved with the LDS reads of the next
// fragments (na from aa, aa + 4 KB; nb from ba + 0/4/8/12 KB), which are complete
// when the block ends.
MUON_DEVICE void mfma_substep(f32x16 (&acc)[2][4], const bf16x8_mfma (&ca)[2],
                              const bf16x8_mfma (&cb)[4], bf16x8_mfma (&na)[2],
                              bf16x8_mfma (&nb)[4], uint32_t aa, uint32_t ba) {
  asm volatile(
      "ds_read_b128 %[na0], %[aa]\n\t"
      MUON_MFMA(c00, ca0, cb0)
      "ds_read_b128 %[nb0], %[ba]\n\t"
      MUON_MFMA(c01, ca0, cb1)
      "ds_read_b128 %[na1], %[aa] offset:4096\n\t"
      MUON_MFMA(c02, ca0, cb2)
      "ds_read_b128 %[nb1], %[ba] offset:4096\n\t"
      MUON_MFMA(c03, ca0, cb3)
      "ds_read_b128 %[nb2], %[ba] offset:8192\n\t"
      MUON_MFMA(c10, ca1, cb0)
      "ds_read_b128 %[nb3], %[ba] offset:12288\n\t"
      MUON_MFMA(c11, ca1, cb1)
      MUON_MFMA(c12, ca1, cb2)
      MUON_MFMA(c13, ca1, cb3)
      "s_waitcnt lgkmcnt(0)"
      : [c00] "+v"(acc[0][0]), [c01] "+v"(acc[0][1]), [c02] "+v"(acc[0][2]),
        [c03] "+v"(acc[0][3]), [c10] "+v"(acc[1][0]), [c11] "+v"(acc[1][1]),
        [c12] "+v"(acc[1][2]), [c13] "+v"(acc[1][3]), [na0] "=&v"(na[0]), [na1] "=&v"(na[1]),
        [nb0] "=&v"(nb[0]), [nb1] "=&v"(nb[1]), [nb2] "=&v"(nb[2]), [nb3] "=&v"(nb[3])
      : [ca0] "v"(ca[0]), [ca1] "v"(ca[1]), [cb0] "v"(cb[0]), [cb1] "v"(cb[1]),
        [cb2] "v"(cb[2]), [cb3] "v"(cb[3]), [aa] "v"(aa), [ba] "v"(ba));
}
// The right half of mfma_substep (accumulator columns fn 2-3, a diagonal tile's wave
// block whose left half lies below the diagonal): 4 MFMAs, reading the next a fragments
// and b fragments 2-3.
MUON_DEVICE void mfma_substep_r(f32x16 (&acc)[2][4], const bf16x8_mfma (&ca)[2],
                                const bf16x8_mfma (&cb)[4], bf16x8_mfma (&na)[2],
                                bf16x8_mfma (&nb)[4], uint32_t aa, uint32_t ba) {
  asm volatile(
      "ds_read_b128 %[na0], %[aa]\n\t"
      MUON_MFMA(c02, ca0, cb2)
      "ds_read_b128 %[na1], %[aa] offset:4096\n\t"
      MUON_MFMA(c03, ca0, cb3)
      "ds_read_b128 %[nb2], %[ba] offset:8192\n\t"
      MUON_MFMA(c12, ca1, cb2)
      "ds_read_b128 %[nb3], %[ba] offset:12288\n\t"
      MUON_MFMA(c13, ca1, cb3)
      "s_waitcnt lgkmcnt(0)"
      : [c02] "+v"(acc[0][2]), [c03] "+v"(acc[0][3]), [c12] "+v"(acc[1][2]),
        [c13] "+v"(acc[1][3]), [na0] "=&v"(na[0]), [na1] "=&v"(na[1]), [nb2] "=&v"(nb[2]),
        [nb3] "=&v"(nb[3])
      : [ca0] "v"(ca[0]), [ca1] "v"(ca[1]), [cb2] "v"(cb[2]), [cb3] "v"(cb[3]), [aa] "v"(aa),
        [ba] "v"(ba));
}

MUON_DEVICE void frag_load_r(bf16x8_mfma (&na)[2], bf16x8_mfma (&nb)[4], uint32_t aa, uint32_t ba) {
  asm volatile(
      "ds_read_b128 %[na0], %[aa]\n\t"
      "ds_read_b128 %[na1], %[aa] offset:4096\n\t"
      "ds_read_b128 %[nb2], %[ba] offset:8192\n\t"
      "ds_read_b128 %[nb3], %[ba] offset:12288\n\t"
      "s_waitcnt lgkmcnt(0)"
      : [na0] "=&v"(na[0]), [na1] "=&v"(na[1]), [nb2] "=&v"(nb[2]), [nb3] "=&v"(nb[3])
      : [aa] "v"(aa), [ba] "v"(ba));
}

#undef MUON_MFMA

MUON_DEVICE void frag_load(bf16x8_mfma (&na)[2], bf16x8_mfma (&nb)[4], uint32_t aa, uint32_t ba) {
  asm volatile(
      "ds_read_b128 %[na0], %[aa]\n\t"
      "ds_read_b128 %[na1], %[aa] offset:4096\n\t"
      "ds_read_b128 %[nb0], %[ba]\n\t"
      "ds_read_b128 %[nb1], %[ba] offset:4096\n\t"
      "ds_read_b128 %[nb2], %[ba] offset:8192\n\t"
      "ds_read_b128 %[nb3], %[ba] offset:12288\n\t"
      "s_waitcnt lgkmcnt(0)"
      : [na0] "=&v"(na[0]), [na1] "=&v"(na[1]), [nb0] "=&v"(nb[0]), [nb1] "=&v"(nb[1]),
        [nb2] "=&v"(nb[2]), [nb3] "=&v"(nb[3])
      : [aa] "v"(aa), [ba] "v"(ba));
}

// The MFMAs run inside inline asm, which the compiler's hazard recognizer does not
// see: VALU access to their accumulators needs the XDL result latency (at most 19
// wait states on gfx950 for a 32x32 MFMA) in between, and an MFMA reading srcC
// written by VALU needs 2.
MUON_DEVICE void mfma_to_valu_wait() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }
MUON_DEVICE void valu_to_mfma_wait() { asm volatile("s_nop 4" ::: "memory"); }

typedef __attribute__((ext_vector_type(2))) float f2x;
typedef __attribute__((ext_vector_type(2))) __bf16 bf2x;  // v_cvt_pk_bf16_f32 (RNE)

// A finished 64 x 128 wave tile as bf16 pairs, converted once with the hardware RNE pair
// conversion: hv[fm][fn][2 rg + h] holds rows fm*32 + rg*8 + fh*4 + 2h and + 1 of the
// lane's column fn*32 + lane%32. Unless `full`, elements outside the valid extent are
// cleared to +0 (whatever they held): rem_i counts the valid rows from this lane's first
// row (fh*4 included), rem_j the valid columns from its column.
MUON_DEVICE void v2_pack(const f32x16 (&acc)[2][4], float alpha, bool full, int rem_i,
                         int rem_j, uint32_t (&hv)[2][4][8]) {
#pragma unroll
  for (int fm = 0; fm < 2; ++fm)
#pragma unroll
    for (int fn = 0; fn < 4; ++fn)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const f2x v = {alpha * acc[fm][fn][r], alpha * acc[fm][fn][r + 1]};
        hv[fm][fn][r >> 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2x));
      }
  if (full) return;
#pragma unroll
  for (int fm = 0; fm < 2; ++fm)
#pragma unroll
    for (int fn = 0; fn < 4; ++fn)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const int il0 = fm * 32 + (r >> 2) * 8 + (r & 3);
        const bool vj = fn * 32 < rem_j;
        const uint32_t keep = (vj && il0 < rem_i ? 0x0000ffffu : 0u) |
                              (vj && il0 + 1 < rem_i ? 0xffff0000u : 0u);
        hv[fm][fn][r >> 1] &= keep;
      }
}

MUON_DEVICE int clamp_rem(int64_t v) { return (int)std::max<int64_t>(-1, std::min<int64_t>(v, 1 << 20)); }

template <int MODE, bool PK>
__global__ __launch_bounds__(512, 1) void gemm_bf16_v2_kernel(GemmArgs g) {
  // PK: the launch mixes the full tiles of the first T-1 tile columns' triangle with the
  // packed tiles of the last column; each matrix's packed tiles follow its full tiles in
  // the tile order, so the workgroups of one XCD share the matrix's row panels in L2
  constexpr int NW = 8, WM = 64, WN = 128, FM = 2, FN = 4;
  extern __shared__ __align__(16) uint8_t smem[];

  int bidx, tm = 0, tn = 0;
  bool pk = false;  // this workgroup's tile is a packed one
  // arow0: first output row; packed: rows arow0 .. arow0 + 511 (logical), the second
  // sub-tile's operand rows read from arow1, which differs from arow0 + 256 only when
  // that sub-tile lies wholly in the padding (it then re-reads valid rows, unstored)
  int64_t arow0, arow1, brow0;
  if constexpr (PK) {
    const int64_t L = xcd_tile(blockIdx.x, (int64_t)gridDim.x, g.tiles_per_batch);
    bidx = (int)(L / g.tiles_per_batch);
    int t = (int)(L % g.tiles_per_batch);
    const int T1 = g.tiles_m - 1;
    const int ntri = T1 * (T1 + 1) / 2;
    const int64_t mpad = (int64_t)g.tiles_m * 256;
    if (t < ntri) {
      int r = 0;
      while (t >= T1 - r) {
        t -= T1 - r;
        ++r;
      }
      tm = r;
      tn = r + t;
      arow0 = (int64_t)tm * 256;
      arow1 = arow0 + 256;
      brow0 = (int64_t)tn * 256;
    } else {
      pk = true;
      arow0 = (int64_t)(t - ntri) * 512;
      arow1 = std::min(arow0 + 256, mpad - 256);
      brow0 = mpad - 256;
    }
  } else {
    map_tile(g, MODE, bidx, tm, tn);
    arow0 = (int64_t)tm * 256;
    arow1 = arow0 + 256;
    brow0 = (int64_t)tn * 256;
  }
  // operand panels: full tiles 256 a rows and 256 b rows (waves 4 x 2), packed tiles
  // 512 a rows and 128 b rows (waves 8 x 1); each wave computes 64 x 128 either way
  const int arows = pk ? 512 : 256;
  const int stageb = (pk ? 640 : 512) * V2_ROWB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // A full diagonal tile (tm == tn) stores only its upper triangle, 10 of its 16 64 x 64
  // units. For B = b A + c A A, and for X X^T with K <= 4096, its waves take the 64 x 128
  // blocks in another order so that each SIMD's two waves (w and w + 4) carry 3, 3, 2 and 2
  // of those units: waves 0-3 compute blocks (0, 0), (0, 1), (1, 1), (2, 1) whole (mode 0),
  // waves 4 and 5 blocks (1, 0) and (3, 1) only in their right half, accumulator columns
  // fn 2-3 (mode 1), waves 6 and 7 blocks (2, 0) and (3, 0), wholly below the diagonal, not
  // at all (mode 2). Its a and b panels are the same rows: only the a panel is loaded.
  const bool dg = MODE == MODE_SYRK && !pk && tm == tn && (g.beta != 0.0f || g.K <= 4096);
  const int wm = pk ? wave : (dg ? (0x32312100 >> (4 * wave)) & 15 : wave >> 1);
  const int wn = pk ? 0 : (dg ? (0x00101110 >> (4 * wave)) & 15 : wave & 1);
  const int wmode = dg ? (0x22110000 >> (4 * wave)) & 15 : 0;
  const bf16_t* A = (const bf16_t*)g.a + (int64_t)bidx * g.sa;
  const bf16_t* B = (const bf16_t*)g.b + (int64_t)bidx * g.sb;
  const int lda_b = (int)(g.lda * 2), ldb_b = (int)(g.ldb * 2);
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(A + arow0 * g.lda), 0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(B + brow0 * g.ldb), 0, 0x7fffffff, 0x00020000);
  // load slab q*NW + wave = rows (q*NW + wave)*8 .. +7; lane -> row lane/8, chunk
  // position lane%8, which holds logical chunk (lane%8) ^ kswz(row)
  const int r_in = wave * 8 + (lane >> 3);
  const int lch = (lane & 7) ^ kswz(r_in);
  const int voa = r_in * lda_b + lch * 16;
  const int vob = r_in * ldb_b + lch * 16;
  // PK: per-lane byte offsets of the a-panel slabs (slabs 4-7, packed tiles only, from
  // the second sub-tile's rows arow1)
  int voq[8];
#pragma unroll
  for (int q = 0; q < 8; ++q)
    voq[q] = voa + (int)((q >= 4 ? arow1 - arow0 + (q - 4) * NW * 8 : q * NW * 8) * lda_b);
  // A K-tile's DMA in two halves, issued in different substeps: the a panel of K-tile
  // k + 2 after the barrier of K-tile k, the b panel of K-tile k + 2 before the first
  // substep of K-tile k + 1 (all of a CU's loads of one K-tile issued together queue in
  // the load path and hold up the MFMAs behind them; in halves the products run 3-5%
  // faster)
  auto issue_a = [&](int kt, int st) {
    uint8_t* sa = smem + st * stageb;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int slab = q * NW + wave;
      if (q < 4 || pk) {
        const int vo = PK ? voq[q] : voa;
        const int so = PK ? kt * V2_ROWB : q * NW * 8 * lda_b + kt * V2_ROWB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_ptr_t)(sa + slab * 1024), 16, vo, so,
                                                 0, 0);
      }
    }
  };
  auto issue_b = [&](int kt, int st) {
    if (dg) return;
    uint8_t* sb = smem + st * stageb + arows * V2_ROWB;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int slab = q * NW + wave;
      if (q < 2 || !pk)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, (lds_ptr_t)(sb + slab * 1024), 16, vob,
                                                 q * NW * 8 * ldb_b + kt * V2_ROWB, 0, 0);
    }
  };

  // MFMA fragment read offsets: lane -> row lane%32 of the fragment, logical chunk
  // 2*ks + lane/32 for k-substep ks
  const int fr = lane & 31, fh = lane >> 5;
  int foff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) foff[ks] = fr * V2_ROWB + (((ks * 2 + fh) ^ kswz(fr)) << 4);
  const int abase = wm * WM * V2_ROWB, bbase = (dg ? 0 : arows * V2_ROWB) + wn * WN * V2_ROWB;

  float alpha = g.alpha, beta = g.beta;
  if (g.scale_mode != 0) {
    const float s = g.scale[bidx];
    if (g.scale_mode == 1) {
      alpha *= s;
      beta *= s;
    } else {
      alpha *= s * s;
    }
  }
  const float ratio = beta != 0.0f ? beta / alpha : 0.0f;
  // K-tile whose k range equals this wave's output rows (WM == BK), as read
  const int64_t wrow = pk && wm >= 4 ? arow1 + (wm - 4) * WM : arow0 + wm * WM;
  const int kdiag = ratio != 0.0f ? (int)(wrow / V2_BK) : -1;

  const int KT = (int)(g.K / V2_BK);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  auto aaddr = [&](int st, int ks) -> uint32_t { return lds0 + st * stageb + abase + foff[ks]; };
  auto baddr = [&](int st, int ks) -> uint32_t { return lds0 + st * stageb + bbase + foff[ks]; };
  // one K loop and epilogue per MFMA mode, so no path merges into another's registers
  auto kloop = [&](auto mode_c) {
  constexpr int MC = decltype(mode_c)::value;
  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  auto substep = [&](const bf16x8_mfma (&ca)[FM], const bf16x8_mfma (&cb)[FN],
                     bf16x8_mfma (&na)[FM], bf16x8_mfma (&nb)[FN], uint32_t aa, uint32_t ba) {
    if constexpr (MC == 0)
      mfma_substep(acc, ca, cb, na, nb, aa, ba);
    else if constexpr (MC == 1)
      mfma_substep_r(acc, ca, cb, na, nb, aa, ba);
  };
  bf16x8_mfma a0[FM], b0[FN], a1[FM], b1[FN];
  issue_a(0, 0);
  issue_b(0, 0);
  wait_vmcnt0();
  lds_barrier();
  if (KT > 1) issue_a(1, 1);
  if constexpr (MC == 0)
    frag_load(a0, b0, aaddr(0, 0), baddr(0, 0));
  else if constexpr (MC == 1)
    frag_load_r(a0, b0, aaddr(0, 0), baddr(0, 0));
  for (int kt = 0; kt < KT; ++kt) {
    const int cs = kt & 1;
    if (kt + 1 < KT) issue_b(kt + 1, cs ^ 1);
    substep(a0, b0, a1, b1, aaddr(cs, 1), baddr(cs, 1));
    substep(a1, b1, a0, b0, aaddr(cs, 2), baddr(cs, 2));
    substep(a0, b0, a1, b1, aaddr(cs, 3), baddr(cs, 3));
    if (MC != 2 && kt == kdiag) {
      // cin(i, j) = b(j, i): row j of the b panel, k offset i - kt*BK (4 consecutive
      // rows i of one accumulator group are 8 contiguous bytes of that row)
      mfma_to_valu_wait();
      const uint8_t* sb = smem + cs * stageb + bbase;
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            const int jl = fn * 32 + fr;  // row within this wave's b rows
            const int kl = fm * 32 + rg * 8 + fh * 4;
            const uint2 w = *(const uint2*)(sb + jl * V2_ROWB +
                                            (((kl >> 3) ^ kswz(jl)) << 4) + (kl & 7) * 2);
            acc[fm][fn][rg * 4 + 0] += ratio * bf16_to_f32((bf16_t)(w.x & 0xffffu));
            acc[fm][fn][rg * 4 + 1] += ratio * bf16_to_f32((bf16_t)(w.x >> 16));
            acc[fm][fn][rg * 4 + 2] += ratio * bf16_to_f32((bf16_t)(w.y & 0xffffu));
            acc[fm][fn][rg * 4 + 3] += ratio * bf16_to_f32((bf16_t)(w.y >> 16));
          }
      valu_to_mfma_wait();
    }
    wait_vmcnt0();
    lds_barrier();
    if (kt + 2 < KT) issue_a(kt + 2, cs);
    substep(a1, b1, a0, b0, aaddr(cs ^ 1, 0), baddr(cs ^ 1, 0));
  }
  mfma_to_valu_wait();

  // ---- epilogue: stage through LDS, store 16-byte row chunks ----
  bf16_t* T = (bf16_t*)smem;
  if (PK && pk) {
    // Packed tile: logical rows arow0 + il (il < 512) against columns c0 + jl (jl <
    // 128), c0 = brow0. Rows below c0 are off-diagonal (stored, and mirrored into rows
    // c0 + jl); rows c0 .. c0 + 127 are the unit's diagonal block (upper triangle
    // stored, mirrored in place); later rows are padding, not stored.
    const int64_t c0 = brow0;
    bf16_t* out = (bf16_t*)g.out + (int64_t)bidx * g.so;
    uint32_t hv[FM][FN][8];
    v2_pack(acc, alpha, arow0 + 512 <= g.Mv && c0 + 128 <= g.Nv,
            clamp_rem(g.Mv - (arow0 + wm * WM + fh * 4)), clamp_rem(g.Nv - (c0 + fr)), hv);
    // mirror: T[jl][il], 4 consecutive il per lane -> one 8-byte write
    lds_barrier();
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const int jl = fn * 32 + fr;
          const int il = wm * WM + fm * 32 + rg * 8 + fh * 4;
          *(uint2*)(T + jl * V2P_TP + il) = make_uint2(hv[fm][fn][2 * rg], hv[fm][fn][2 * rg + 1]);
        }
    lds_barrier();
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
      const int id = it * 512 + tid;
      const int jl = id >> 6, c = (id & 63) * 8;
      if (arow0 + c < c0) {  // 8 rows of one off-diagonal unit
        const uint4 w = *(const uint4*)(T + jl * V2P_TP + c);
        *(uint4*)(out + (c0 + jl) * g.ldo + arow0 + c) = w;
      }
    }
    // row-major: T[il][jl]
    lds_barrier();
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int il = wm * WM + fm * 32 + (r >> 2) * 8 + fh * 4 + (r & 3);
          const int jl = fn * 32 + fr;
          T[il * V2P_RP + jl] = (bf16_t)(hv[fm][fn][r >> 1] >> (16 * (r & 1)));
        }
    lds_barrier();
    const int dl0 = (int)(c0 - arow0);  // staging row of the diagonal block's first row
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
      const int id = it * 512 + tid;
      const int il = id >> 4, c = (id & 15) * 8;
      const int dr = il - dl0;  // row within the diagonal block (< 0: off-diagonal)
      if (dr >= 128) continue;  // padding rows
      uint4 w;
      if (dr < 0 || c >= dr) {
        w = *(const uint4*)(T + il * V2P_RP + c);
      } else {
        // diagonal block, chunk reaching below the diagonal: those columns come from
        // the computed (upper) element of the mirror position
        uint16_t e[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
          e[q] = (c + q < dr) ? T[(dl0 + c + q) * V2P_RP + dr] : T[il * V2P_RP + c + q];
        __builtin_memcpy(&w, e, 16);
      }
      *(uint4*)(out + (arow0 + il) * g.ldo + c0 + c) = w;
    }
    return;
  }
  const bool diag = MODE == MODE_SYRK && tm == tn;
  const int row0w = wm * WM, col0w = wn * WN;  // wave origin within the tile
  uint32_t hv[FM][FN][8];
  v2_pack(acc, alpha, arow0 + 256 <= g.Mv && brow0 + 256 <= g.Nv,
          clamp_rem(g.Mv - (arow0 + row0w + fh * 4)), clamp_rem(g.Nv - (brow0 + col0w + fr)), hv);
  bf16_t* out = g.out ? (bf16_t*)g.out + (int64_t)bidx * g.so : nullptr;
  bf16_t* out_t = g.out_t ? (bf16_t*)g.out_t + (int64_t)bidx * g.st : nullptr;
  const int64_t ldt = MODE == MODE_SYRK ? g.ldo : g.ldt;
  if (MODE == MODE_SYRK && !diag) out_t = out;  // mirror half of the symmetric output
  const bool do_t = out_t != nullptr && !diag;
  const bool do_o = out != nullptr;

  if (do_t) {
    // transposed stage: T[j][i], 4 consecutive i per lane -> one 8-byte write
    lds_barrier();
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const int jl = col0w + fn * 32 + fr;
          const int il = row0w + fm * 32 + rg * 8 + fh * 4;
          *(uint2*)(T + jl * V2_EP_PITCH + il) = make_uint2(hv[fm][fn][2 * rg], hv[fm][fn][2 * rg + 1]);
        }
    lds_barrier();
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
      const int id = it * 512 + tid;
      const int jl = id >> 5, c = (id & 31) * 8;
      const uint4 w = *(const uint4*)(T + jl * V2_EP_PITCH + c);
      *(uint4*)(out_t + (brow0 + jl) * ldt + arow0 + c) = w;
    }
  }
  if (do_o) {
    // row-major stage: T[i][j]
    lds_barrier();
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int il = row0w + fm * 32 + (r >> 2) * 8 + fh * 4 + (r & 3);
          const int jl = col0w + fn * 32 + fr;
          T[il * V2_EP_PITCH + jl] = (bf16_t)(hv[fm][fn][r >> 1] >> (16 * (r & 1)));
        }
    lds_barrier();
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
      const int id = it * 512 + tid;
      const int il = id >> 5, c = (id & 31) * 8;
      uint4 w;
      if (!diag || c >= il) {
        w = *(const uint4*)(T + il * V2_EP_PITCH + c);
      } else {
        // diagonal tile, chunk reaching below the diagonal: those columns come from
        // the computed (upper) element of the mirror position
        uint16_t e[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
          e[q] = (c + q < il) ? T[(c + q) * V2_EP_PITCH + il] : T[il * V2_EP_PITCH + c + q];
        __builtin_memcpy(&w, e, 16);
      }
      *(uint4*)(out + (arow0 + il) * g.ldo + brow0 + c) = w;
    }
  }
  };
  if (wmode == 0)
    kloop(std::integral_constant<int, 0>{});
  else if (wmode == 1)
    kloop(std::integral_constant<int, 1>{});
  else
    kloop(std::integral_constant<int, 2>{});
}

// ----------------------------------------------------------------------------------
// bf16 X' = alpha * (B X + ratio * X) with X read in its own row-major layout.
//
// The a operand (B, rows i, k contiguous) is staged as in gemm_bf16_v2_kernel. The
// b operand is X itself, whose rows are k: each K-tile stages a 64 x 256 panel
// X[k][j] (rows of 512 B, 16-byte chunk c of row k stored at chunk c ^ ((k & 3) << 2))
// and the MFMA fragments, which need 8 consecutive k of one column j per lane, come
// from ds_read_b64_tr_b16: within a group of 16 lanes, lane r points at 4 consecutive
// elements of row kb + r/4, columns jb + 4 (r % 4) .. +3, and lane i receives column
// jb + i of rows kb .. kb+3. Two such reads (kb, kb + 4) fill one fragment. The
// swizzle puts the four rows of one read in four different 64-byte bank groups.
//
// The MFMA takes the X fragment as its first operand, so an accumulator holds X'
// transposed: lane l has row i = l % 32 and 4 consecutive columns j of a 32 x 32
// block. Stores of X' are then 8-byte row pieces straight from registers, and the
// beta term X(i, j .. j+3) is 8 contiguous bytes of row k = i of the X panel.
// No X^T is kept in memory; X ping-pongs between two buffers because every tile
// reads whole columns of X.
constexpr int NN_XROWB = 512;                        // X panel row: 256 bf16
constexpr int NN_ATILEB = 256 * V2_ROWB;             // B panel: 256 rows x 64 k
constexpr int NN_XTILEB = V2_BK * NN_XROWB;          // X panel: 64 k x 256 j
constexpr int NN_STAGEB = NN_ATILEB + NN_XTILEB;

typedef __attribute__((ext_vector_type(4))) short i16x4;

MUON_DEVICE void nn_join(bf16x8_mfma (&cx)[4], const i16x4 (&lo)[4], const i16x4 (&hi)[4]) {
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const i16x4 l = lo[f], h = hi[f];
    const __attribute__((ext_vector_type(8))) short v =
        __builtin_shufflevector(l, h, 0, 1, 2, 3, 4, 5, 6, 7);
    cx[f] = __builtin_bit_cast(bf16x8_mfma, v);
  }
}

// ----------------------------------------------------------------------------------
// Persistent bf16 X' = alpha * (B X + ratio * X): 4 wavefronts (2 x 2), each owning a
// 128 x 128 block of the 256 x 256 tile, accumulators in AGPRs (256 per lane).
//
// Against 8 waves of 64 x 128 (measured 2-8% slower on the same box) a wave reads 8 KB of
// fragments from LDS per 16 MFMAs instead of 6 KB per 8, and with one wave per SIMD the DMA of
// K-tile k + 2 is issued from inside the MFMA stream of K-tile k (B panel) and k + 1 (X panel),
// one buffer_load ... lds after each of a substep's first 8 MFMAs, M0 stepping through the
// destination slabs. The grid is one workgroup per CU; each walks a list of tiles with
// the operand pipeline running across tile boundaries: the last two K-tiles of a tile
// prefetch the first two of the next, so a tile's epilogue overlaps the next tile's loads.
//
// All CUs finish their tiles together, so each epilogue is a chip-wide burst of 32 MB
// (4 MB per XCD, the size of its L2). The epilogue therefore stages each wave's 32-row
// blocks through 8 KB of LDS and writes whole 256-byte rows with non-temporal stores:
// measured against stores straight from the accumulators (16-byte row pieces through
// L2), the burst no longer evicts the operand panels the XCD's CUs share, and the
// product runs 5-8% faster.
//
// Tiles are dealt to the 8 XCDs (workgroup b runs on XCD b % 8) in stripes of 64
// consecutive tiles: the workgroups of one XCD share its L2 across neighbouring tiles
// (GM = 8 tile rows per column group, as map_tile), and all XCDs work on the same
// matrices at a time. The beta term reads the staged X panel during the
// two K-tiles whose k range covers the wave's output rows, holds the values in 128
// VGPRs (bf16 pairs) and adds them in the epilogue.
constexpr int N4_EPB = 32 * 256;                 // epilogue staging per wave: 32 rows
constexpr int N4_STRIPE = 64;                    // tiles per XCD stripe
constexpr int N4_SMEM = 2 * NN_STAGEB + 4 * N4_EPB;  // 160 KiB
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

// buffer descriptor words (raw, stride 0, 2^31 - 1 bytes; num_records 0 for `none`)
MUON_DEVICE u32x4 n4_rsrc(const void* base, bool none) {
  const uint64_t a = (uint64_t)base;
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, none ? 0u : 0x7fffffffu, 0x00020000u};
}

#define MF(C, X, B) "v_mfma_f32_32x32x16_bf16 %[" #C "], %[" #X "], %[" #B "], %[" #C "]\n\t"
#define TRL(D, XA, O) "ds_read_b64_tr_b16 %[" #D "], %[" #XA "] offset:%[" #O "]\n\t"
#define N4_ACC_OUT                                                                          \
  [c00] "+a"(acc[0][0]), [c01] "+a"(acc[0][1]), [c02] "+a"(acc[0][2]), [c03] "+a"(acc[0][3]), \
  [c10] "+a"(acc[1][0]), [c11] "+a"(acc[1][1]), [c12] "+a"(acc[1][2]), [c13] "+a"(acc[1][3]), \
  [c20] "+a"(acc[2][0]), [c21] "+a"(acc[2][1]), [c22] "+a"(acc[2][2]), [c23] "+a"(acc[2][3]), \
  [c30] "+a"(acc[3][0]), [c31] "+a"(acc[3][1]), [c32] "+a"(acc[3][2]), [c33] "+a"(acc[3][3]), \
  [nb0] "=&v"(nb[0]), [nb1] "=&v"(nb[1]), [nb2] "=&v"(nb[2]), [nb3] "=&v"(nb[3]),              \
  [l0] "=&v"(nxl[0]), [h0] "=&v"(nxh[0]), [l1] "=&v"(nxl[1]), [h1] "=&v"(nxh[1]),              \
  [l2] "=&v"(nxl[2]), [h2] "=&v"(nxh[2]), [l3] "=&v"(nxl[3]), [h3] "=&v"(nxh[3])
#define N4_FRAG_IN                                                                          \
  [cb0] "v"(cb[0]), [cb1] "v"(cb[1]), [cb2] "v"(cb[2]), [cb3] "v"(cb[3]), [cx0] "v"(cx[0]),    \
  [cx1] "v"(cx[1]), [cx2] "v"(cx[2]), [cx3] "v"(cx[3]), [ba] "v"(ba), [x0] "v"(xa[0]),         \
  [x1] "v"(xa[1]), [x2] "v"(xa[2]), [x3] "v"(xa[3]), [o0] "i"(XO), [o1] "i"(XO + 4 * NN_XROWB)

// One k-substep of the 128 x 128 wave tile: 16 MFMAs (accumulator (fm, fn) takes X
// fragment fn as srcA and B fragment fm as srcB) interleaved with the 12 LDS reads of
// the next substep's fragments (X: two tr reads per fragment at xa[f] + XO and + 2 KB;
// B: b128 at ba + 4 KB * fm), complete when the block ends.
template <int XO>
MUON_DEVICE void nn4_substep(f32x16 (&acc)[4][4], const bf16x8_mfma (&cb)[4],
                             const bf16x8_mfma (&cx)[4], bf16x8_mfma (&nb)[4], i16x4 (&nxl)[4],
                             i16x4 (&nxh)[4], uint32_t ba, const uint32_t (&xa)[4]) {
  asm volatile(
      TRL(l0, x0, o0) MF(c00, cx0, cb0)
      TRL(h0, x0, o1) MF(c01, cx1, cb0)
      TRL(l1, x1, o0) MF(c02, cx2, cb0)
      TRL(h1, x1, o1) MF(c03, cx3, cb0)
      TRL(l2, x2, o0) MF(c10, cx0, cb1)
      TRL(h2, x2, o1) MF(c11, cx1, cb1)
      TRL(l3, x3, o0) MF(c12, cx2, cb1)
      TRL(h3, x3, o1) MF(c13, cx3, cb1)
      "ds_read_b128 %[nb0], %[ba]\n\t" MF(c20, cx0, cb2)
      "ds_read_b128 %[nb1], %[ba] offset:4096\n\t" MF(c21, cx1, cb2)
      "ds_read_b128 %[nb2], %[ba] offset:8192\n\t" MF(c22, cx2, cb2)
      "ds_read_b128 %[nb3], %[ba] offset:12288\n\t" MF(c23, cx3, cb2)
      MF(c30, cx0, cb3) MF(c31, cx1, cb3) MF(c32, cx2, cb3) MF(c33, cx3, cb3)
      "s_waitcnt lgkmcnt(0)"
      : N4_ACC_OUT
      : N4_FRAG_IN);
}

// nn4_substep plus the DMA of half a K-tile into one stage: this wave's 8 slabs of one
// operand panel (B panel: rows 32 q + 8 wave .. +7; X panel: rows 8 q + 2 wave, +1; LDS
// slab 4 q + wave of that panel), one buffer_load ... lds after each of the first 8
// MFMAs. M0 holds the LDS destination; each M0 write is separated from its load by an
// MFMA (the one wait state the hardware needs). t steps the scalar byte offset by one
// slab group (st).
//
// A K-tile's two halves go out in two different substeps (the B panel of K-tile k + 2
// right after the barrier, the X panel of K-tile k + 2 in the next substep): the 64
// loads of one K-tile per CU, issued in one substep, queued in the load path and held
// up the MFMAs behind them (about 37 issue cycles per load); in halves the main loop
// takes 7-8% fewer cycles.
#define DL "buffer_load_dwordx4 %[vo], %[rs], %[t] offen lds\n\t"
#define DN "s_add_u32 m0, m0, 0x1000\n\ts_add_u32 %[t], %[t], %[st]\n\t"
template <int XO>
MUON_DEVICE void nn4_substep_dma(f32x16 (&acc)[4][4], const bf16x8_mfma (&cb)[4],
                                 const bf16x8_mfma (&cx)[4], bf16x8_mfma (&nb)[4],
                                 i16x4 (&nxl)[4], i16x4 (&nxh)[4], uint32_t ba,
                                 const uint32_t (&xa)[4], int vo, u32x4 rs, int so, int st,
                                 uint32_t m0) {
  int t;
  asm volatile(
      "s_mov_b32 m0, %[m0]\n\ts_mov_b32 %[t], %[so]\n\t"
      TRL(l0, x0, o0) MF(c00, cx0, cb0) DL
      DN TRL(h0, x0, o1) MF(c01, cx1, cb0) DL
      DN TRL(l1, x1, o0) MF(c02, cx2, cb0) DL
      DN TRL(h1, x1, o1) MF(c03, cx3, cb0) DL
      DN TRL(l2, x2, o0) MF(c10, cx0, cb1) DL
      DN TRL(h2, x2, o1) MF(c11, cx1, cb1) DL
      DN TRL(l3, x3, o0) MF(c12, cx2, cb1) DL
      DN TRL(h3, x3, o1) MF(c13, cx3, cb1) DL
      "ds_read_b128 %[nb0], %[ba]\n\t" MF(c20, cx0, cb2)
      "ds_read_b128 %[nb1], %[ba] offset:4096\n\t" MF(c21, cx1, cb2)
      "ds_read_b128 %[nb2], %[ba] offset:8192\n\t" MF(c22, cx2, cb2)
      "ds_read_b128 %[nb3], %[ba] offset:12288\n\t" MF(c23, cx3, cb2)
      MF(c30, cx0, cb3) MF(c31, cx1, cb3) MF(c32, cx2, cb3) MF(c33, cx3, cb3)
      "s_waitcnt lgkmcnt(0)"
      : N4_ACC_OUT, [t] "=&s"(t)
      : N4_FRAG_IN, [vo] "v"(vo), [rs] "s"(rs), [so] "s"(so), [st] "s"(st), [m0] "s"(m0)
      : "m0", "scc", "memory");
}
#undef DL
#undef DN

// The B panel half of a K-tile without MFMAs (pipeline start).
MUON_DEVICE void nn4_dma_half(int vo, u32x4 rs, int so, int st, uint32_t m0) {
  int t;
  asm volatile(
      "s_mov_b32 m0, %[m0]\n\ts_mov_b32 %[t], %[so]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[vo], %[rs], %[t] offen lds\n\t"
      "s_add_u32 m0, m0, 0x1000\n\ts_add_u32 %[t], %[t], %[st]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[vo], %[rs], %[t] offen lds\n\t"
      "s_add_u32 m0, m0, 0x1000\n\ts_add_u32 %[t], %[t], %[st]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[vo], %[rs], %[t] offen lds\n\t"
      "s_add_u32 m0, m0, 0x1000\n\ts_add_u32 %[t], %[t], %[st]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[vo], %[rs], %[t] offen lds\n\t"
      "s_add_u32 m0, m0, 0x1000\n\ts_add_u32 %[t], %[t], %[st]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[vo], %[rs], %[t] offen lds\n\t"
      "s_add_u32 m0, m0, 0x1000\n\ts_add_u32 %[t], %[t], %[st]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[vo], %[rs], %[t] offen lds\n\t"
      "s_add_u32 m0, m0, 0x1000\n\ts_add_u32 %[t], %[t], %[st]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[vo], %[rs], %[t] offen lds\n\t"
      "s_add_u32 m0, m0, 0x1000\n\ts_add_u32 %[t], %[t], %[st]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[vo], %[rs], %[t] offen lds\n\t"
      : [t] "=&s"(t)
      : [vo] "v"(vo), [rs] "s"(rs), [so] "s"(so), [st] "s"(st), [m0] "s"(m0)
      : "m0", "scc", "memory");
}

#define DA "buffer_load_dwordx4 %[voa], %[rsa], %[ta] offen lds\n\t"
#define DX "buffer_load_dwordx4 %[vox], %[rsx], %[tx] offen lds\n\t"
#define NA "s_add_u32 m0, m0, 0x1000\n\ts_add_u32 %[ta], %[ta], %[sta]\n\t"
#define NX "s_add_u32 m0, m0, 0x1000\n\ts_add_u32 %[tx], %[tx], %[stx]\n\t"
// The DMA of one K-tile without MFMAs (pipeline start).
MUON_DEVICE void nn4_dma(int voa, int vox, u32x4 rsa, u32x4 rsx, int soa, int sox, int sta,
                         int stx, uint32_t m0a, uint32_t m0x) {
  int ta, tx;
  asm volatile(
      "s_mov_b32 m0, %[m0a]\n\ts_mov_b32 %[ta], %[soa]\n\ts_nop 0\n\t"
      DA NA "s_nop 0\n\t" DA NA "s_nop 0\n\t" DA NA "s_nop 0\n\t" DA
      NA "s_nop 0\n\t" DA NA "s_nop 0\n\t" DA NA "s_nop 0\n\t" DA NA "s_nop 0\n\t" DA
      "s_mov_b32 m0, %[m0x]\n\ts_mov_b32 %[tx], %[sox]\n\ts_nop 0\n\t"
      DX NX "s_nop 0\n\t" DX NX "s_nop 0\n\t" DX NX "s_nop 0\n\t" DX
      NX "s_nop 0\n\t" DX NX "s_nop 0\n\t" DX NX "s_nop 0\n\t" DX NX "s_nop 0\n\t" DX
      : [ta] "=&s"(ta), [tx] "=&s"(tx)
      : [voa] "v"(voa), [vox] "v"(vox), [rsa] "s"(rsa), [rsx] "s"(rsx), [soa] "s"(soa),
        [sox] "s"(sox), [sta] "s"(sta), [stx] "s"(stx), [m0a] "s"(m0a), [m0x] "s"(m0x)
      : "m0", "scc", "memory");
}
#undef DA
#undef DX
#undef NA
#undef NX

template <int XO>
MUON_DEVICE void nn4_frag_load(bf16x8_mfma (&nb)[4], i16x4 (&nxl)[4], i16x4 (&nxh)[4], uint32_t ba,
                               const uint32_t (&xa)[4]) {
  asm volatile(
      TRL(l0, x0, o0) TRL(h0, x0, o1) TRL(l1, x1, o0) TRL(h1, x1, o1)
      TRL(l2, x2, o0) TRL(h2, x2, o1) TRL(l3, x3, o0) TRL(h3, x3, o1)
      "ds_read_b128 %[nb0], %[ba]\n\t"
      "ds_read_b128 %[nb1], %[ba] offset:4096\n\t"
      "ds_read_b128 %[nb2], %[ba] offset:8192\n\t"
      "ds_read_b128 %[nb3], %[ba] offset:12288\n\t"
      "s_waitcnt lgkmcnt(0)"
      : [nb0] "=&v"(nb[0]), [nb1] "=&v"(nb[1]), [nb2] "=&v"(nb[2]), [nb3] "=&v"(nb[3]),
        [l0] "=&v"(nxl[0]), [h0] "=&v"(nxh[0]), [l1] "=&v"(nxl[1]), [h1] "=&v"(nxh[1]),
        [l2] "=&v"(nxl[2]), [h2] "=&v"(nxh[2]), [l3] "=&v"(nxl[3]), [h3] "=&v"(nxh[3])
      : [ba] "v"(ba), [x0] "v"(xa[0]), [x1] "v"(xa[1]), [x2] "v"(xa[2]), [x3] "v"(xa[3]),
        [o0] "i"(XO), [o1] "i"(XO + 4 * NN_XROWB));
}
#undef MF
#undef TRL
#undef N4_ACC_OUT
#undef N4_FRAG_IN

// X(i, j .. j+3) for the accumulators of rows H0, H0 + 1 (panel row k = h*32 + lane%32,
// columns 128 wn + 32 fn + 8 rg + 4 (lane/32)) from the staged X panel at sx, as bf16
// pairs. The LDS base is laundered so the lane addresses are formed here and not kept
// live across the main loop.
template <int H0>
MUON_DEVICE void nn4_beta_rows(u32x2 (&xb)[4][4][4], uint32_t sx, int wn, int fr, int fh) {
  asm volatile("" : "+v"(sx));
  const uint32_t base = sx + fr * NN_XROWB + wn * 256 + fh * 8;
#pragma unroll
  for (int fn = 0; fn < 4; ++fn) {
    // logical 16-byte chunk 16 wn + 4 fn + rg sits at position ^ ((k & 3) << 2)
    const uint32_t b2 = base + (((fn ^ (fr & 3)) << 2) << 4);
    asm volatile(
        "ds_read_b64 %0, %8 offset:0\n\t"
        "ds_read_b64 %1, %8 offset:16\n\t"
        "ds_read_b64 %2, %8 offset:32\n\t"
        "ds_read_b64 %3, %8 offset:48\n\t"
        "ds_read_b64 %4, %8 offset:%9\n\t"
        "ds_read_b64 %5, %8 offset:%10\n\t"
        "ds_read_b64 %6, %8 offset:%11\n\t"
        "ds_read_b64 %7, %8 offset:%12\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(xb[H0][fn][0]), "=&v"(xb[H0][fn][1]), "=&v"(xb[H0][fn][2]),
          "=&v"(xb[H0][fn][3]), "=&v"(xb[H0 + 1][fn][0]), "=&v"(xb[H0 + 1][fn][1]),
          "=&v"(xb[H0 + 1][fn][2]), "=&v"(xb[H0 + 1][fn][3])
        : "v"(b2), "i"(32 * NN_XROWB), "i"(32 * NN_XROWB + 16), "i"(32 * NN_XROWB + 32),
          "i"(32 * NN_XROWB + 48));
  }
}

// Tile t of the launch -> (matrix, row origin, column origin); GM tile rows per column
// group, as map_tile.
MUON_DEVICE void nn4_tile(const GemmArgs& g, int t, int& bidx, int64_t& arow0, int64_t& bcol0) {
  bidx = t / g.tiles_per_batch;
  const int r = t - bidx * g.tiles_per_batch;
  const int GM = 8, TN = g.tiles_n, TM = g.tiles_m;
  const int group = r / (GM * TN);
  const int first = group * GM;
  const int gsz = min(TM - first, GM);
  const int local = r - group * (GM * TN);
  arow0 = (int64_t)(first + local % gsz) * 256;
  bcol0 = (int64_t)(local / gsz) * 256;
}

__global__ __launch_bounds__(256, 1) void gemm_bf16_nn4_kernel(GemmArgs g) {
  constexpr int FM = 4, FN = 4, WM = 128, WN = 128;
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // this workgroup's tiles: XCD x's list holds tcount tiles and its gx workgroups take
  // every gx-th one starting at their index l within the XCD. The list: stripes x, x + 8,
  // x + 16, ... of N4_STRIPE consecutive tiles while whole rounds of 8 stripes remain,
  // then an equal share of the rest. All XCDs thus work on the same matrices at a time,
  // so the operand panels their L2s miss on come from one matrix's worth of data (which
  // the Infinity Cache holds) rather than from 8 matrices (contiguous ranges per XCD:
  // 4% slower on the 4096 x 14336 bucket).
  const int G = gridDim.x, T = g.tiles_total;
  const int x = blockIdx.x & 7, l = blockIdx.x >> 3;
  const int gx = (G >> 3) + (x < (G & 7) ? 1 : 0);
  const int nfull = T / (8 * N4_STRIPE) * N4_STRIPE;  // tiles per XCD in whole rounds
  const int rq = (T - 8 * nfull) >> 3, rr = (T - 8 * nfull) & 7;
  const int tcount = nfull + rq + (x < rr ? 1 : 0);
  auto tile_of = [&](int i) {
    return i < nfull ? ((i / N4_STRIPE) * 8 + x) * N4_STRIPE + i % N4_STRIPE
                     : 8 * nfull + x * rq + min(x, rr) + (i - nfull);
  };
  int li = l;
  if (li >= tcount) return;

  const int lda_b = (int)(g.lda * 2), ldx_b = (int)(g.ldb * 2);
  // DMA lanes: B panel row 8 wave + lane/8 (+ 32 q), logical chunk (lane%8) ^ kswz(row);
  // X panel row 2 wave + lane/32 (+ 8 q), chunk (lane%32) ^ ((row & 3) << 2)
  const int ra_in = wave * 8 + (lane >> 3);
  const int voa = ra_in * lda_b + (((lane & 7) ^ kswz(ra_in)) << 4);
  const int rx_in = wave * 2 + (lane >> 5);
  const int vox = rx_in * ldx_b + (((lane & 31) ^ ((rx_in & 3) << 2)) << 4);
  const int sta = 32 * lda_b, stx = 8 * ldx_b;
  const bf16_t* const A0 = (const bf16_t*)g.a;
  const bf16_t* const X0 = (const bf16_t*)g.b;

  // B fragment rows (k contiguous, as gemm_bf16_v2_kernel) and X fragment tr-read offsets:
  // group g = lane/16, r = lane%16 points at panel row 8 (g/2) + r/4 (+ 16 ks, + 4 for
  // the high half), column 128 wn + 32 f + 16 (g%2) + 4 (r%4)
  const int fr = lane & 31, fh = lane >> 5;
  int foff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) foff[ks] = fr * V2_ROWB + (((ks * 2 + fh) ^ kswz(fr)) << 4);
  const int abase = wm * WM * V2_ROWB;
  const int tg = lane >> 4, trr = lane & 15, ts = trr >> 2;
  uint32_t xoff[4];
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int chunk = wn * 16 + ((f ^ ts) << 2) + (tg & 1) * 2 + ((trr & 3) >> 1);
    xoff[f] = NN_ATILEB + (8 * (tg >> 1) + ts) * NN_XROWB + chunk * 16 + (trr & 1) * 8;
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  auto baddr = [&](int st, int ks) -> uint32_t { return lds0 + st * NN_STAGEB + abase + foff[ks]; };
  uint32_t xa[4];
  auto set_xa = [&](int st) {
#pragma unroll
    for (int f = 0; f < 4; ++f) xa[f] = lds0 + st * NN_STAGEB + xoff[f];
  };
  const uint32_t m0w = lds0 + wave * 1024;
  // even: the last two K-tiles of a tile prefetch the next tile's first two into stages
  // (KT - 2) & 1 and (KT - 1) & 1, and every tile starts reading stage 0
  const int KT = (int)(g.K / V2_BK);

  // current tile and its descriptors; the next tile's (num_records 0 if none)
  int bidx;
  int64_t arow0, bcol0;
  nn4_tile(g, tile_of(li), bidx, arow0, bcol0);
  u32x4 rsa = n4_rsrc(A0 + (int64_t)bidx * g.sa + arow0 * g.lda, false);
  u32x4 rsx = n4_rsrc(X0 + (int64_t)bidx * g.sb + bcol0, false);

  bf16x8_mfma b0[FM], b1[FM], x0[FN], x1[FN];
  i16x4 xl[FN], xh[FN];
  nn4_dma(voa, vox, rsa, rsx, 0, 0, sta, stx, m0w, m0w + NN_ATILEB);
  wait_vmcnt0();
  lds_barrier();
  // K-tile 1: the B panel now, the X panel with the first substep of K-tile 0
  nn4_dma_half(voa, rsa, V2_ROWB, sta, m0w + NN_STAGEB);
  set_xa(0);
  nn4_frag_load<0>(b0, xl, xh, baddr(0, 0), xa);
  nn_join(x0, xl, xh);

  f32x16 acc[FM][FN];
  for (;;) {
    const int lnext = li + gx;
    const bool has_next = lnext < tcount;
    int nbidx = 0;
    int64_t narow0 = 0, nbcol0 = 0;
    if (has_next) nn4_tile(g, tile_of(lnext), nbidx, narow0, nbcol0);
    const u32x4 rsa_n = n4_rsrc(A0 + (int64_t)nbidx * g.sa + narow0 * g.lda, !has_next);
    const u32x4 rsx_n = n4_rsrc(X0 + (int64_t)nbidx * g.sb + nbcol0, !has_next);

    float alpha = g.alpha, beta = g.beta;
    if (g.scale_mode == 1) {
      const float sc = g.scale[bidx];
      alpha *= sc;
      beta *= sc;
    }
    const float ratio = beta != 0.0f ? beta / alpha : 0.0f;
    // the wave's 128 output rows are the k rows of K-tiles kd0 and kd0 + 1
    const int kd0 = ratio != 0.0f ? (int)((arow0 + wm * WM) / V2_BK) : -8;

#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    u32x2 xb[FM][FN][4];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) xb[i][j][r] = u32x2{0u, 0u};

    int kt = 0;
    do {
      const int cs = kt & 1;
      set_xa(cs);
      // the X panel of K-tile kt + 1 of this tile (or K-tile 0 of the next) into stage
      // cs ^ 1; its B panel went out with the previous DMA substep
      const bool c1 = kt + 1 < KT;
      const int k1 = c1 ? kt + 1 : kt + 1 - KT;
      nn4_substep_dma<1 * 16 * NN_XROWB>(acc, b0, x0, b1, xl, xh, baddr(cs, 1), xa, vox,
                                         c1 ? rsx : rsx_n, k1 * V2_BK * ldx_b, stx,
                                         m0w + (cs ^ 1) * NN_STAGEB + NN_ATILEB);
      nn_join(x1, xl, xh);
      nn4_substep<2 * 16 * NN_XROWB>(acc, b1, x1, b0, xl, xh, baddr(cs, 2), xa);
      nn_join(x0, xl, xh);
      nn4_substep<3 * 16 * NN_XROWB>(acc, b0, x0, b1, xl, xh, baddr(cs, 3), xa);
      nn_join(x1, xl, xh);
      if (kt == kd0) nn4_beta_rows<0>(xb, lds0 + cs * NN_STAGEB + NN_ATILEB, wn, fr, fh);
      if (kt == kd0 + 1) nn4_beta_rows<2>(xb, lds0 + cs * NN_STAGEB + NN_ATILEB, wn, fr, fh);
      wait_vmcnt0();
      lds_barrier();
      // the B panel of K-tile kt + 2 of this tile, or K-tile kt + 2 - KT of the next,
      // into stage cs
      const bool c2 = kt + 2 < KT;
      const int k2 = c2 ? kt + 2 : kt + 2 - KT;
      set_xa(cs ^ 1);
      nn4_substep_dma<0>(acc, b1, x1, b0, xl, xh, baddr(cs ^ 1, 0), xa, voa, c2 ? rsa : rsa_n,
                         k2 * V2_ROWB, sta, m0w + cs * NN_STAGEB);
      nn_join(x0, xl, xh);
    } while (++kt < KT);
    mfma_to_valu_wait();

    // epilogue: accumulator (fm, fn) element 4 rg + q is X'(i, j + q) with
    // i = 128 wm + 32 fm + lane%32, j = 128 wn + 32 fn + 8 rg + 4 (lane/32). Each 32-row
    // block fm goes through the wave's LDS staging rows (16-byte chunk k of row r kept at
    // chunk k ^ (r & 15), so both the 8-byte writes and the 16-byte reads are free of
    // bank conflicts), then out as 4 whole rows of 256 bytes per non-temporal store.
    // The staging rows are the wave's own and LDS serves one wave's accesses in order.
    bf16_t* outw = (bf16_t*)g.out + (int64_t)bidx * g.so + (arow0 + wm * WM) * g.ldo + bcol0 + wn * WN;
    const __amdgpu_buffer_rsrc_t rso =
        __builtin_amdgcn_make_buffer_rsrc((void*)outw, 0, 0x7fffffff, 0x00020000);
    const int ldo_b = (int)(g.ldo * 2);
    const uint32_t ep = lds0 + 2 * NN_STAGEB + wave * N4_EPB;
    const uint32_t epw = ep + fr * 256 + fh * 8;   // row fr, this lane's 8-byte half
    const uint32_t epr = ep + (lane >> 4) * 256;  // rows lane/16 + 4 i
    const int vor = (lane >> 4) * ldo_b + (lane & 15) * 16;
    // valid extents from this lane's first row / column (zeros are stored beyond);
    // most tiles lie inside both and take the unmasked path
    const bool full = arow0 + 256 <= g.Mv && bcol0 + 256 <= g.Nv;
    const int rem_i = (int)g.Mv - (int)(arow0 + wm * WM + fr);
    const int rem_j = (int)g.Nv - (int)(bcol0 + wn * WN + fh * 4);
    auto emit = [&](auto masked) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          // one accumulator at a time out of the AGPRs
          f32x16 av;
          asm volatile("" : "=v"(av) : "0"(acc[fm][fn]));
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            const u32x2 xw = xb[fm][fn][rg];
            f2x v01 = {alpha * (av[rg * 4 + 0] + ratio * __uint_as_float(xw.x << 16)),
                       alpha * (av[rg * 4 + 1] + ratio * __uint_as_float(xw.x & 0xffff0000u))};
            f2x v23 = {alpha * (av[rg * 4 + 2] + ratio * __uint_as_float(xw.y << 16)),
                       alpha * (av[rg * 4 + 3] + ratio * __uint_as_float(xw.y & 0xffff0000u))};
            if (decltype(masked)::value) {
              const int jq = fn * 32 + rg * 8;
              const bool vi = fm * 32 < rem_i;
              v01.x = vi && jq + 0 < rem_j ? v01.x : 0.0f;
              v01.y = vi && jq + 1 < rem_j ? v01.y : 0.0f;
              v23.x = vi && jq + 2 < rem_j ? v23.x : 0.0f;
              v23.y = vi && jq + 3 < rem_j ? v23.y : 0.0f;
            }
            const u32x2 w = {__builtin_bit_cast(uint32_t, __builtin_convertvector(v01, bf2x)),
                             __builtin_bit_cast(uint32_t, __builtin_convertvector(v23, bf2x))};
            // addresses are formed here rather than hoisted into registers for the loop
            uint32_t ea = epw, fx = fr & 15;
            asm volatile("" : "+v"(ea), "+v"(fx));
            *(u32x2 __attribute__((address_space(3)))*)(ea + (((4 * fn + rg) ^ fx) << 4)) = w;
          }
        }
        uint32_t ra = epr, lc = lane & 15, lr = lane >> 4;
        int vs = vor;
        asm volatile("" : "+v"(ra), "+v"(vs), "+v"(lc), "+v"(lr));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t c = lc ^ ((4 * i + lr) & 15);
          const u32x4 q4 = *(const u32x4 __attribute__((address_space(3)))*)(ra + i * 1024 + (c << 4));
          // aux 2: non-temporal
          __builtin_amdgcn_raw_buffer_store_b128(q4, rso, vs + i * 4 * ldo_b, fm * 32 * ldo_b, 2);
        }
      }
    };
    if (full)
      emit(std::false_type{});
    else
      emit(std::true_type{});
    if (!has_next) break;
    li = lnext;
    bidx = nbidx;
    arow0 = narow0;
    bcol0 = nbcol0;
    rsa = rsa_n;
    rsx = rsx_n;
  }
}

// ----------------------------------------------------------------------------------
// The persistent B X kernel on 16 x 16 x 32 MFMAs, for K of at least 768.
//
// Same tiling, waves, LDS layout, tile order and epilogue staging as gemm_bf16_nn4_kernel;
// the wave's 128 x 128 block is 8 x 8 accumulators of 16 x 16 (AGPRs) and a K-tile is two
// 32-k substeps of 64 MFMAs. A single wave issues v_mfma_f32_32x32x16_bf16 at most every 32
// cycles and each 16-byte fragment read between them costs it issue time; with
// v_mfma_f32_16x16x32_bf16 the same LDS bytes per FLOP ride along at almost no cost: a
// probe loop with this kernel's reads, DMA and barrier took 35.7 cycles per
// 32 x 32 x 16-equivalent against about 48 for the 32 x 32 x 16 loop.
//
// Fragments (lane l, r = l % 16, g = l / 16): srcA is X^T, 8 consecutive k (two tr reads)
// of column 16 fj + r; srcB is B, 8 consecutive k (one b128) of row 16 fi + r; the
// accumulator register q of block (fi, fj) is X'(16 fi + r, 16 fj + 4 g + q).
//
// The X panel's chunk swizzle adds row bit 3 to gemm_bf16_nn4_kernel's: chunk c of row k sits
// at c ^ ((k & 3) << 2) ^ (((k >> 3) & 1) << 1). A transposing read serves 32 lanes at a time,
// lanes 0-15 from rows 8 g' .. +3 and lanes 16-31 from rows 8 g' + 8 .. +11 (g' even); with
// the low-bit swizzle alone both groups hit the same 32 banks (35% of LDS-active cycles were
// bank conflicts), with bit 3 they use the other 32. The DMA takes the row parity of each X
// slab from one of two per-lane offsets (slab q holds rows 8 q .. 8 q + 7).
//
// The beta term is added during the two K-tiles whose k range is the wave's rows (no
// registers hold X values through the loop, which the double-buffered fragments need), by
// 32 more MFMAs per substep (n16_beta), so the accumulators never leave their AGPRs; those
// two K-tiles are peeled off the loop. It takes its own K-loop structure and per-tile work,
// so below K = 768 (where that work weighs more) gemm_bf16_nn4_kernel is used instead.
#define M16(C, X, B) "v_mfma_f32_16x16x32_bf16 %[" #C "], %[" #X "], %[" #B "], %[" #C "]\n\t"
#define N16_OUT(ACC)                                                                      \
  [c0] "+a"(ACC[0]), [c1] "+a"(ACC[1]), [c2] "+a"(ACC[2]), [c3] "+a"(ACC[3]),               \
  [c4] "+a"(ACC[4]), [c5] "+a"(ACC[5]), [c6] "+a"(ACC[6]), [c7] "+a"(ACC[7]),               \
  [nb] "=&v"(nb), [nl] "=&v"(nl), [nh] "=&v"(nh)
#define N16_IN                                                                            \
  [b] "v"(cb), [x0] "v"(cx[0]), [x1] "v"(cx[1]), [x2] "v"(cx[2]), [x3] "v"(cx[3]),          \
  [x4] "v"(cx[4]), [x5] "v"(cx[5]), [x6] "v"(cx[6]), [x7] "v"(cx[7]), [ba] "v"(ba),         \
  [xa] "v"(xa), [o0] "i"(XO), [o1] "i"(XO + 4 * NN_XROWB), [ob] "i"(FI * 16 * V2_ROWB)
// One block of a 32-k substep: the 8 MFMAs of row block FI (accumulators acc[0..7] hold
// X' rows 16 FI + lane%16, columns 16 fj + 4 (lane/16) .. +3) on the current fragments,
// with 3 reads of the next substep's fragments: both halves of X fragment FI (tr reads at
// xa + XO, + 2 KB) and B fragment FI (b128 at ba + 2 KB FI).
// SW (the last iteration of a tall matrix, whose update is applied in the parameter's
// layout): the operands swapped, srcA the B fragment and srcB the X fragments, so the
// accumulators hold X' columns 16 fj + lane%16, rows 16 FI + 4 (lane/16) .. +3, i.e. the
// transpose of the block within each 16 x 16 accumulator (the same products and sums).
#define M16S(C, X, B) "v_mfma_f32_16x16x32_bf16 %[" #C "], %[" #B "], %[" #X "], %[" #C "]\n\t"
#define N16_BLOCK(M)                                                                      \
  "ds_read_b64_tr_b16 %[nl], %[xa] offset:%[o0]\n\t" M(c0, x0, b)                          \
  M(c1, x1, b) M(c2, x2, b)                                                               \
  "ds_read_b64_tr_b16 %[nh], %[xa] offset:%[o1]\n\t" M(c3, x3, b)                          \
  M(c4, x4, b) M(c5, x5, b)                                                               \
  "ds_read_b128 %[nb], %[ba] offset:%[ob]\n\t" M(c6, x6, b)                                \
  M(c7, x7, b)
template <int FI, int XO, bool SW = false>
MUON_DEVICE void n16_block(f32x4 (&acc)[8], const bf16x8_mfma& cb, const bf16x8_mfma (&cx)[8],
                           bf16x8_mfma& nb, i16x4& nl, i16x4& nh, uint32_t ba, uint32_t xa) {
  if constexpr (SW)
    asm volatile(N16_BLOCK(M16S) : N16_OUT(acc) : N16_IN);
  else
    asm volatile(N16_BLOCK(M16) : N16_OUT(acc) : N16_IN);
}
// The same as the first block of a tile: the MFMAs start from zero (C = 0) and define the
// accumulators, so no instruction zeroes them between tiles.
#define M16Z(C, X, B) "v_mfma_f32_16x16x32_bf16 %[" #C "], %[" #X "], %[" #B "], 0\n\t"
#define M16SZ(C, X, B) "v_mfma_f32_16x16x32_bf16 %[" #C "], %[" #B "], %[" #X "], 0\n\t"
#define N16_OUTZ(ACC)                                                                     \
  [c0] "=a"(ACC[0]), [c1] "=a"(ACC[1]), [c2] "=a"(ACC[2]), [c3] "=a"(ACC[3]),               \
  [c4] "=a"(ACC[4]), [c5] "=a"(ACC[5]), [c6] "=a"(ACC[6]), [c7] "=a"(ACC[7]),               \
  [nb] "=&v"(nb), [nl] "=&v"(nl), [nh] "=&v"(nh)
template <int FI, int XO, bool SW = false>
MUON_DEVICE void n16_block_z(f32x4 (&acc)[8], const bf16x8_mfma& cb, const bf16x8_mfma (&cx)[8],
                             bf16x8_mfma& nb, i16x4& nl, i16x4& nh, uint32_t ba, uint32_t xa) {
  if constexpr (SW)
    asm volatile(N16_BLOCK(M16SZ) : N16_OUTZ(acc) : N16_IN);
  else
    asm volatile(N16_BLOCK(M16Z) : N16_OUTZ(acc) : N16_IN);
}
#undef M16Z
#undef M16SZ
#undef N16_OUTZ
// The same with two loads of the DMA of a K-tile (slabs 2 FI and 2 FI + 1 of the 16 this
// wave issues per K-tile: B panel slabs for FI < 4, X panel slabs for FI >= 4), each after an
// MFMA, with per-lane offsets vo0 and vo1. m0 and the scalar offsets of both loads come in
// precomputed.
#define N16_BLOCK_DMA(M)                                                                  \
  "s_mov_b32 m0, %[m00]\n\t"                                                              \
  "ds_read_b64_tr_b16 %[nl], %[xa] offset:%[o0]\n\t" M(c0, x0, b)                          \
  "buffer_load_dwordx4 %[vo0], %[rs], %[so0] offen lds\n\t"                               \
  M(c1, x1, b) "s_mov_b32 m0, %[m01]\n\t" M(c2, x2, b)                                    \
  "ds_read_b64_tr_b16 %[nh], %[xa] offset:%[o1]\n\t" M(c3, x3, b)                          \
  "buffer_load_dwordx4 %[vo1], %[rs], %[so1] offen lds\n\t"                               \
  M(c4, x4, b) M(c5, x5, b)                                                               \
  "ds_read_b128 %[nb], %[ba] offset:%[ob]\n\t" M(c6, x6, b)                                \
  M(c7, x7, b)
#define N16_DMA_IN                                                                        \
  N16_IN, [vo0] "v"(vo0), [vo1] "v"(vo1), [rs] "s"(rs), [so0] "s"(so0), [so1] "s"(so1),    \
      [m00] "s"(m00), [m01] "s"(m01)
template <int FI, int XO, bool SW = false>
MUON_DEVICE void n16_block_dma(f32x4 (&acc)[8], const bf16x8_mfma& cb, const bf16x8_mfma (&cx)[8],
                               bf16x8_mfma& nb, i16x4& nl, i16x4& nh, uint32_t ba, uint32_t xa,
                               int vo0, int vo1, u32x4 rs, int so0, int so1, uint32_t m00,
                               uint32_t m01) {
  if constexpr (SW)
    asm volatile(N16_BLOCK_DMA(M16S) : N16_OUT(acc) : N16_DMA_IN : "m0", "memory");
  else
    asm volatile(N16_BLOCK_DMA(M16) : N16_OUT(acc) : N16_DMA_IN : "m0", "memory");
}
#undef N16_BLOCK
#undef N16_BLOCK_DMA
#undef N16_DMA_IN
#undef N16_OUT
#undef N16_IN
#undef M16
#undef M16S

#define DA "buffer_load_dwordx4 %[voa], %[rsa], %[ta] offen lds\n\t"
#define DXE "buffer_load_dwordx4 %[voxe], %[rsx], %[tx] offen lds\n\t"
#define DXO "buffer_load_dwordx4 %[voxo], %[rsx], %[tx] offen lds\n\t"
#define NA "s_add_u32 m0, m0, 0x1000\n\ts_add_u32 %[ta], %[ta], %[sta]\n\ts_nop 0\n\t"
#define NX "s_add_u32 m0, m0, 0x1000\n\ts_add_u32 %[tx], %[tx], %[stx]\n\ts_nop 0\n\t"
// The DMA of one K-tile without MFMAs (pipeline start); X slab q takes the per-lane offsets
// of its row parity (voxe for even q, voxo for odd).
MUON_DEVICE void n16_dma(int voa, int voxe, int voxo, u32x4 rsa, u32x4 rsx, int soa, int sox,
                         int sta, int stx, uint32_t m0a, uint32_t m0x) {
  int ta, tx;
  asm volatile(
      "s_mov_b32 m0, %[m0a]\n\ts_mov_b32 %[ta], %[soa]\n\ts_nop 0\n\t"
      DA NA DA NA DA NA DA NA DA NA DA NA DA NA DA
      "s_mov_b32 m0, %[m0x]\n\ts_mov_b32 %[tx], %[sox]\n\ts_nop 0\n\t"
      DXE NX DXO NX DXE NX DXO NX DXE NX DXO NX DXE NX DXO
      : [ta] "=&s"(ta), [tx] "=&s"(tx)
      : [voa] "v"(voa), [voxe] "v"(voxe), [voxo] "v"(voxo), [rsa] "s"(rsa), [rsx] "s"(rsx),
        [soa] "s"(soa), [sox] "s"(sox), [sta] "s"(sta), [stx] "s"(stx), [m0a] "s"(m0a),
        [m0x] "s"(m0x)
      : "m0", "scc", "memory");
}
#undef DA
#undef DXE
#undef DXO
#undef NA
#undef NX

// All 24 fragment reads of one substep without MFMAs (pipeline start).
template <int XO>
MUON_DEVICE void n16_frag_load(bf16x8_mfma (&nb)[8], i16x4 (&nl)[8], i16x4 (&nh)[8], uint32_t ba,
                               const uint32_t (&xa)[8]) {
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    asm volatile("ds_read_b64_tr_b16 %0, %3 offset:%4\n\t"
                 "ds_read_b64_tr_b16 %1, %3 offset:%5\n\t"
                 "ds_read_b128 %2, %6 offset:%7"
                 : "=&v"(nl[f]), "=&v"(nh[f]), "=&v"(nb[f])
                 : "v"(xa[f]), "i"(XO), "i"(XO + 4 * NN_XROWB), "v"(ba), "i"(0));
    ba += 16 * V2_ROWB;
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

MUON_DEVICE void n16_join(bf16x8_mfma (&cx)[8], const i16x4 (&lo)[8], const i16x4 (&hi)[8]) {
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    const __attribute__((ext_vector_type(8))) short v = __builtin_shufflevector(lo[f], hi[f], 0, 1, 2, 3, 4, 5, 6, 7);
    cx[f] = __builtin_bit_cast(bf16x8_mfma, v);
  }
}

// One 32-k substep: 8 blocks, then the wait for its 24 reads. The first of a tile (Z)
// starts the accumulators from zero.
template <int XO, bool SW = false, bool Z = false>
MUON_DEVICE void n16_substep(f32x4 (&acc)[8][8], const bf16x8_mfma (&cb)[8], const bf16x8_mfma (&cx)[8],
                             bf16x8_mfma (&nb)[8], i16x4 (&nl)[8], i16x4 (&nh)[8], uint32_t ba,
                             const uint32_t (&xa)[8]) {
  if constexpr (Z) {
    n16_block_z<0, XO, SW>(acc[0], cb[0], cx, nb[0], nl[0], nh[0], ba, xa[0]);
    n16_block_z<1, XO, SW>(acc[1], cb[1], cx, nb[1], nl[1], nh[1], ba, xa[1]);
    n16_block_z<2, XO, SW>(acc[2], cb[2], cx, nb[2], nl[2], nh[2], ba, xa[2]);
    n16_block_z<3, XO, SW>(acc[3], cb[3], cx, nb[3], nl[3], nh[3], ba, xa[3]);
    n16_block_z<4, XO, SW>(acc[4], cb[4], cx, nb[4], nl[4], nh[4], ba, xa[4]);
    n16_block_z<5, XO, SW>(acc[5], cb[5], cx, nb[5], nl[5], nh[5], ba, xa[5]);
    n16_block_z<6, XO, SW>(acc[6], cb[6], cx, nb[6], nl[6], nh[6], ba, xa[6]);
    n16_block_z<7, XO, SW>(acc[7], cb[7], cx, nb[7], nl[7], nh[7], ba, xa[7]);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    return;
  }
  n16_block<0, XO, SW>(acc[0], cb[0], cx, nb[0], nl[0], nh[0], ba, xa[0]);
  n16_block<1, XO, SW>(acc[1], cb[1], cx, nb[1], nl[1], nh[1], ba, xa[1]);
  n16_block<2, XO, SW>(acc[2], cb[2], cx, nb[2], nl[2], nh[2], ba, xa[2]);
  n16_block<3, XO, SW>(acc[3], cb[3], cx, nb[3], nl[3], nh[3], ba, xa[3]);
  n16_block<4, XO, SW>(acc[4], cb[4], cx, nb[4], nl[4], nh[4], ba, xa[4]);
  n16_block<5, XO, SW>(acc[5], cb[5], cx, nb[5], nl[5], nh[5], ba, xa[5]);
  n16_block<6, XO, SW>(acc[6], cb[6], cx, nb[6], nl[6], nh[6], ba, xa[6]);
  n16_block<7, XO, SW>(acc[7], cb[7], cx, nb[7], nl[7], nh[7], ba, xa[7]);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// The substep after the barrier, carrying the DMA of one whole K-tile into one stage: blocks
// 0-3 load the B panel slabs (rows 32 q + 8 wave .. +7, q = 0..7), blocks 4-7 the X panel
// slabs (rows 8 q + 2 wave, +1).
template <int XO, bool SW = false>
MUON_DEVICE void n16_substep_dma(f32x4 (&acc)[8][8], const bf16x8_mfma (&cb)[8],
                                 const bf16x8_mfma (&cx)[8], bf16x8_mfma (&nb)[8], i16x4 (&nl)[8],
                                 i16x4 (&nh)[8], uint32_t ba, const uint32_t (&xa)[8], int voa,
                                 int voxe, int voxo, u32x4 rsa, u32x4 rsx, int soa, int sox, int sta, int stx,
                                 uint32_t m0a, uint32_t m0x) {
  n16_block_dma<0, XO, SW>(acc[0], cb[0], cx, nb[0], nl[0], nh[0], ba, xa[0], voa, voa, rsa, soa, soa + sta, m0a, m0a + 0x1000);
  n16_block_dma<1, XO, SW>(acc[1], cb[1], cx, nb[1], nl[1], nh[1], ba, xa[1], voa, voa, rsa, soa + 2 * sta, soa + 3 * sta, m0a + 0x2000, m0a + 0x3000);
  n16_block_dma<2, XO, SW>(acc[2], cb[2], cx, nb[2], nl[2], nh[2], ba, xa[2], voa, voa, rsa, soa + 4 * sta, soa + 5 * sta, m0a + 0x4000, m0a + 0x5000);
  n16_block_dma<3, XO, SW>(acc[3], cb[3], cx, nb[3], nl[3], nh[3], ba, xa[3], voa, voa, rsa, soa + 6 * sta, soa + 7 * sta, m0a + 0x6000, m0a + 0x7000);
  n16_block_dma<4, XO, SW>(acc[4], cb[4], cx, nb[4], nl[4], nh[4], ba, xa[4], voxe, voxo, rsx, sox, sox + stx, m0x, m0x + 0x1000);
  n16_block_dma<5, XO, SW>(acc[5], cb[5], cx, nb[5], nl[5], nh[5], ba, xa[5], voxe, voxo, rsx, sox + 2 * stx, sox + 3 * stx, m0x + 0x2000, m0x + 0x3000);
  n16_block_dma<6, XO, SW>(acc[6], cb[6], cx, nb[6], nl[6], nh[6], ba, xa[6], voxe, voxo, rsx, sox + 4 * stx, sox + 5 * stx, m0x + 0x4000, m0x + 0x5000);
  n16_block_dma<7, XO, SW>(acc[7], cb[7], cx, nb[7], nl[7], nh[7], ba, xa[7], voxe, voxo, rsx, sox + 6 * stx, sox + 7 * stx, m0x + 0x6000, m0x + 0x7000);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// The beta term on the matrix cores: ratio * X(i, j) = sum_k X(k, j) (ratio delta(k, i)), so
// an MFMA with the substep's X fragment as srcA (k = the substep's 32 rows) and a diagonal
// fragment as srcB adds it to the accumulators of the two row blocks those rows are. ratio is
// split into two bf16 parts, hi = RNE(ratio) and lo = RNE(ratio - hi): hi + lo carries 16
// significant bits of the fp32 ratio, so the coefficient applied is a (1 + d) with
// |d| <= about 2^-17 (plus the fp32 rounding of beta / alpha), far below the bf16 output's
// resolution; each bf16 x bf16 product is exact in the fp32 accumulator. The accumulators
// never leave their AGPRs. (A read-modify-write
// through VGPRs made the compiler move accumulators between AGPRs next to the inline-asm
// MFMAs, whose latency it does not see, and the moves raced their results: B X then differed
// by an ulp from run to run.) db[par][part]: lane l (r = l%16, g = l/16) holds B(k, n) for
// k = 8 g .. 8 g + 7, n = r: part at k = 16 par + r, else zero.
MUON_DEVICE void n16_beta_frags(float ratio, int lane, bf16x8_mfma (&db)[2][2]) {
  const float hi = bf16_to_f32(f32_to_bf16(ratio));
  const float lo = ratio - hi;
  const uint32_t parts[2] = {(uint32_t)f32_to_bf16(hi), (uint32_t)f32_to_bf16(lo)};
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int par = 0; par < 2; ++par)
#pragma unroll
    for (int pt = 0; pt < 2; ++pt) {
      const int e = 16 * par + r - 8 * g;  // element of this lane's 8 holding the diagonal
      uint32_t w[4];
#pragma unroll
      for (int d = 0; d < 4; ++d)
        w[d] = (e == 2 * d ? parts[pt] : 0u) | (e == 2 * d + 1 ? parts[pt] << 16 : 0u);
      db[par][pt] = __builtin_bit_cast(bf16x8_mfma, u32x4{w[0], w[1], w[2], w[3]});
    }
}

#define M16(C, X, B) "v_mfma_f32_16x16x32_bf16 %[" #C "], %[" #X "], %[" #B "], %[" #C "]\n\t"
#define M16S(C, X, B) "v_mfma_f32_16x16x32_bf16 %[" #C "], %[" #B "], %[" #X "], %[" #C "]\n\t"
#define NB_ROW(M, P, F, B)                                                                   \
  M(P##0, x0, B) M(P##1, x1, B) M(P##2, x2, B) M(P##3, x3, B)                                 \
  M(P##4, x4, B) M(P##5, x5, B) M(P##6, x6, B) M(P##7, x7, B)
#define NB_ALL(M) NB_ROW(M, a, FI, d0h) NB_ROW(M, b, FI + 1, d1h) NB_ROW(M, a, FI, d0l) NB_ROW(M, b, FI + 1, d1l)
#define NB_OUT                                                                               \
  [a0] "+a"(acc[FI][0]), [a1] "+a"(acc[FI][1]), [a2] "+a"(acc[FI][2]), [a3] "+a"(acc[FI][3]),   \
  [a4] "+a"(acc[FI][4]), [a5] "+a"(acc[FI][5]), [a6] "+a"(acc[FI][6]), [a7] "+a"(acc[FI][7]),   \
  [b0] "+a"(acc[FI + 1][0]), [b1] "+a"(acc[FI + 1][1]), [b2] "+a"(acc[FI + 1][2]),             \
  [b3] "+a"(acc[FI + 1][3]), [b4] "+a"(acc[FI + 1][4]), [b5] "+a"(acc[FI + 1][5]),             \
  [b6] "+a"(acc[FI + 1][6]), [b7] "+a"(acc[FI + 1][7])
#define NB_IN                                                                                \
  [x0] "v"(cx[0]), [x1] "v"(cx[1]), [x2] "v"(cx[2]), [x3] "v"(cx[3]), [x4] "v"(cx[4]),        \
  [x5] "v"(cx[5]), [x6] "v"(cx[6]), [x7] "v"(cx[7]), [d0h] "v"(db[0][0]), [d0l] "v"(db[0][1]), \
  [d1h] "v"(db[1][0]), [d1l] "v"(db[1][1])
// ratio * X added to row blocks FI and FI + 1 (rows 32 ks .. 32 ks + 31 of the K-tile whose
// X fragments cx are the substep's): 32 MFMAs, the hi parts of both row blocks first. The
// diagonal fragment serves as srcA as well (SW): its per-lane layout is the same.
template <int FI, bool SW = false>
MUON_DEVICE void n16_beta(f32x4 (&acc)[8][8], const bf16x8_mfma (&cx)[8],
                          const bf16x8_mfma (&db)[2][2]) {
  if constexpr (SW)
    asm volatile(NB_ALL(M16S) : NB_OUT : NB_IN);
  else
    asm volatile(NB_ALL(M16) : NB_OUT : NB_IN);
}
#undef NB_ALL
#undef NB_OUT
#undef NB_IN
#undef M16S
#undef NB_ROW
#undef M16

// APPLY 0: X' stored into the workspace. APPLY 1 / 2 (the last iteration, bf16 parameters):
// X' is not stored; each bf16 element of it is the update u of one parameter element, applied
// as the post-pass does (apply_elem: cautious weight decay and the shape-scaled step) and the
// parameter written back. 1: a wide matrix (parameter row i = X' row i); 2: a tall matrix
// (parameter row j = X' column j), computed with swapped MFMA operands so the accumulators
// hold parameter rows.
// MODE (APPLY 1, 2): the form of the apply, from the uniform wd and cautious (below).
template <int APPLY, int MODE = 0>
__global__ __launch_bounds__(256, 1) void gemm_bf16_nn16_kernel(GemmArgs g, MuonApply ap) {
  constexpr int WM = 128, WN = 128;
  constexpr bool SW = APPLY == 2;
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  const int G = gridDim.x, T = g.tiles_total;
  const int x = blockIdx.x & 7, l = blockIdx.x >> 3;
  const int gx = (G >> 3) + (x < (G & 7) ? 1 : 0);
  const int nfull = T / (8 * N4_STRIPE) * N4_STRIPE;
  const int rq = (T - 8 * nfull) >> 3, rr = (T - 8 * nfull) & 7;
  const int tcount = nfull + rq + (x < rr ? 1 : 0);
  auto tile_of = [&](int i) {
    return i < nfull ? ((i / N4_STRIPE) * 8 + x) * N4_STRIPE + i % N4_STRIPE
                     : 8 * nfull + x * rq + min(x, rr) + (i - nfull);
  };
  int li = l;
  if (li >= tcount) return;

  const int lda_b = (int)(g.lda * 2), ldx_b = (int)(g.ldb * 2);
  const int ra_in = wave * 8 + (lane >> 3);
  const int voa = ra_in * lda_b + (((lane & 7) ^ kswz(ra_in)) << 4);
  const int rx_in = wave * 2 + (lane >> 5);
  const int vox = rx_in * ldx_b + (((lane & 31) ^ ((rx_in & 3) << 2)) << 4);
  const int voxo = rx_in * ldx_b + (((lane & 31) ^ ((rx_in & 3) << 2) ^ 2) << 4);
  const int sta = 32 * lda_b, stx = 8 * ldx_b;
  const bf16_t* const A0 = (const bf16_t*)g.a;
  const bf16_t* const X0 = (const bf16_t*)g.b;

  // fragment addresses. B (srcB): lane l -> panel row 128 wm + 16 fi + l%16, logical chunk
  // 4 ks + l/16 (8 consecutive k). X (srcA): tr reads, lane l -> panel row 32 ks + 8 (l/16) +
  // (l%16)/4 (+4 for the high half), columns 128 wn + 16 fj + 4 (l%4) .. +3.
  const int fr = lane & 15, fg = lane >> 4;
  int foff[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) foff[ks] = fr * V2_ROWB + (((ks * 4 + fg) ^ kswz(fr)) << 4);
  const int abase = wm * WM * V2_ROWB;
  uint32_t xoff[8];
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    const int chunk = (wn * 16 + f * 2 + ((fr & 3) >> 1)) ^ (((fr >> 2) & 3) << 2) ^ ((fg & 1) << 1);
    xoff[f] = NN_ATILEB + (8 * fg + (fr >> 2)) * NN_XROWB + chunk * 16 + (fr & 1) * 8;
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  auto baddr = [&](int st, int ks) -> uint32_t { return lds0 + st * NN_STAGEB + abase + foff[ks]; };
  uint32_t xa[8];
  auto set_xa = [&](int st) {
#pragma unroll
    for (int f = 0; f < 8; ++f) xa[f] = lds0 + st * NN_STAGEB + xoff[f];
  };
  const uint32_t m0w = lds0 + wave * 1024;
  const int KT = (int)(g.K / V2_BK);

  int bidx;
  int64_t arow0, bcol0;
  nn4_tile(g, tile_of(li), bidx, arow0, bcol0);
  u32x4 rsa = n4_rsrc(A0 + (int64_t)bidx * g.sa + arow0 * g.lda, false);
  u32x4 rsx = n4_rsrc(X0 + (int64_t)bidx * g.sb + bcol0, false);

  bf16x8_mfma b0[8], b1[8], x0[8], x1[8];
  i16x4 xl[8], xh[8];
  // K-tiles 0 and 1 of the first tile
  n16_dma(voa, vox, voxo, rsa, rsx, 0, 0, sta, stx, m0w, m0w + NN_ATILEB);
  wait_vmcnt0();
  lds_barrier();
  n16_dma(voa, vox, voxo, rsa, rsx, V2_ROWB, V2_BK * ldx_b, sta, stx, m0w + NN_STAGEB,
          m0w + NN_STAGEB + NN_ATILEB);
  set_xa(0);
  n16_frag_load<0>(b0, xl, xh, baddr(0, 0), xa);
  n16_join(x0, xl, xh);

  f32x4 acc[8][8];
  for (;;) {
    const int lnext = li + gx;
    const bool has_next = lnext < tcount;
    int nbidx = 0;
    int64_t narow0 = 0, nbcol0 = 0;
    if (has_next) nn4_tile(g, tile_of(lnext), nbidx, narow0, nbcol0);
    const u32x4 rsa_n = n4_rsrc(A0 + (int64_t)nbidx * g.sa + narow0 * g.lda, !has_next);
    const u32x4 rsx_n = n4_rsrc(X0 + (int64_t)nbidx * g.sb + nbcol0, !has_next);

    float alpha = g.alpha, beta = g.beta;
    if (g.scale_mode == 1) {
      const float sc = g.scale[bidx];
      alpha *= sc;
      beta *= sc;
    }
    const float ratio = beta != 0.0f ? beta / alpha : 0.0f;
    // the wave's 128 output rows are the k rows of K-tiles kd0 and kd0 + 1; rows at or beyond
    // K are padding, whose X rows are zero
    const int kd = (int)((arow0 + wm * WM) / V2_BK);
    const int kd0 = ratio != 0.0f && kd < KT ? kd : -1;

    // one K-tile: substep 0 (reading substep 1's fragments), wait for K-tile kt + 1's DMA,
    // barrier, substep 1 (reading K-tile kt + 1's first fragments) with the DMA of K-tile
    // kt + 2 (this tile's or the next's) into this K-tile's stage. In the two K-tiles whose k
    // range is the wave's rows (peeled off the loops), each substep also adds ratio * X to
    // the two row blocks its 32 k rows are.
    // first: the tile's K-tile 0, whose first MFMAs start from zero (a compile-time true or
    // false, or a run-time test)
    auto kstep = [&](int kt, auto beta_fi0, auto first) {
      constexpr int FB = decltype(beta_fi0)::value;
      const int cs = kt & 1;
      set_xa(cs);
      if constexpr (std::is_same_v<decltype(first), bool>) {
        if (first)
          n16_substep<16 * NN_XROWB * 2, SW, true>(acc, b0, x0, b1, xl, xh, baddr(cs, 1), xa);
        else
          n16_substep<16 * NN_XROWB * 2, SW>(acc, b0, x0, b1, xl, xh, baddr(cs, 1), xa);
      } else {
        n16_substep<16 * NN_XROWB * 2, SW, decltype(first)::value>(acc, b0, x0, b1, xl, xh,
                                                                     baddr(cs, 1), xa);
      }
      if constexpr (FB >= 0) {
        bf16x8_mfma db[2][2];
        n16_beta_frags(ratio, lane, db);
        n16_beta<FB, SW>(acc, x0, db);
      }
      n16_join(x1, xl, xh);
      wait_vmcnt0();
      lds_barrier();
      const bool c2 = kt + 2 < KT;
      const int k2 = c2 ? kt + 2 : kt + 2 - KT;
      set_xa(cs ^ 1);
      const uint32_t m0a = m0w + cs * NN_STAGEB;
      n16_substep_dma<0, SW>(acc, b1, x1, b0, xl, xh, baddr(cs ^ 1, 0), xa, voa, vox, voxo, c2 ? rsa : rsa_n,
                         c2 ? rsx : rsx_n, k2 * V2_ROWB, k2 * V2_BK * ldx_b, sta, stx, m0a,
                         m0a + NN_ATILEB);
      if constexpr (FB >= 0) {
        bf16x8_mfma db[2][2];
        n16_beta_frags(ratio, lane, db);
        n16_beta<FB + 2, SW>(acc, x1, db);
      }
      n16_join(x0, xl, xh);
    };
    using no_beta = std::integral_constant<int, -1>;
    using beta_lo = std::integral_constant<int, 0>;
    using beta_hi = std::integral_constant<int, 4>;
    const std::true_type first{};
    const std::false_type later{};
    // Leaving a loop that the peeled beta K-tiles follow, the compiler may copy accumulators
    // between registers before any asm that follows the loop; it does not see the MFMAs in
    // the asm, so the last K-tile of such a loop ends with their latency.
    if constexpr (APPLY == 0) {
      // K-tile 0 peeled off every loop, so the loops carry no test for it (B X 1.6% faster on
      // the Llama set than with the test in the loops)
      int kt;
      if (kd0 == 0) {
        kstep(0, beta_lo{}, first);
        kstep(1, beta_hi{}, later);
        kt = 2;
      } else {
        kstep(0, no_beta{}, first);
        kt = 1;
        if (kd0 > 0) {
          for (; kt < kd0; ++kt) {
            kstep(kt, no_beta{}, later);
            if (kt + 1 == kd0) mfma_to_valu_wait();
          }
          kstep(kt++, beta_lo{}, later);
          kstep(kt++, beta_hi{}, later);
        }
      }
      for (; kt < KT; ++kt) kstep(kt, no_beta{}, later);
    } else {
      // the apply kernels test for K-tile 0 in the loops: peeled, their larger epilogue spilled
      // (their launches took 7% longer on the MoE experts)
      int kt = 0;
      if (kd0 >= 0) {
        for (; kt < kd0; ++kt) {
          kstep(kt, no_beta{}, kt == 0);
          if (kt + 1 == kd0) mfma_to_valu_wait();
        }
        kstep(kt, beta_lo{}, kt == 0);
        ++kt;
        kstep(kt++, beta_hi{}, later);
      }
      for (; kt < KT; ++kt) kstep(kt, no_beta{}, kt == 0);
    }
    mfma_to_valu_wait();

    // epilogue: accumulator (fi, fj) element q is X'(i, j + q) with i = 128 wm + 16 fi +
    // lane%16, j = 128 wn + 16 fj + 4 (lane/16) (SW: X'(i + q, j) with i = 128 wm + 16 fi +
    // 4 (lane/16), j = 128 wn + 16 fj + lane%16). Two row blocks (32 rows) at a time go through
    // the wave's LDS staging rows (16-byte chunk k of row r at chunk k ^ (r & 15)), then out as
    // 4 whole rows of 256 bytes per non-temporal store.
    const uint32_t ep = lds0 + 2 * NN_STAGEB + wave * N4_EPB;
    const uint32_t epr = ep + (lane >> 4) * 256;
    // staging rows 32 p .. 32 p + 31: X' rows (APPLY 0, 1) or X' columns (APPLY 2), packed bf16
    auto stage = [&](int p, auto masked, int rem_i, int rem_j) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          f32x4 av;
          if constexpr (SW)
            asm volatile("" : "=v"(av) : "0"(acc[k][2 * p + h]));
          else
            asm volatile("" : "=v"(av) : "0"(acc[2 * p + h][k]));
          f2x v01 = {alpha * av[0], alpha * av[1]};
          f2x v23 = {alpha * av[2], alpha * av[3]};
          if (decltype(masked)::value) {
            const int fi = 2 * p + h, jq = k * 16;
            const bool vi = fi * 16 < rem_i;
            v01.x = vi && jq + 0 < rem_j ? v01.x : 0.0f;
            v01.y = vi && jq + 1 < rem_j ? v01.y : 0.0f;
            v23.x = vi && jq + 2 < rem_j ? v23.x : 0.0f;
            v23.y = vi && jq + 3 < rem_j ? v23.y : 0.0f;
          }
          const u32x2 w = {__builtin_bit_cast(uint32_t, __builtin_convertvector(v01, bf2x)),
                           __builtin_bit_cast(uint32_t, __builtin_convertvector(v23, bf2x))};
          uint32_t ea = ep + (h * 16 + fr) * 256 + (fg & 1) * 8, fx = fr;
          asm volatile("" : "+v"(ea), "+v"(fx));
          *(u32x2 __attribute__((address_space(3)))*)(ea + (((2 * k + (fg >> 1)) ^ fx) << 4)) = w;
        }
      }
    };
    if constexpr (APPLY == 0) {
      bf16_t* outw = (bf16_t*)g.out + (int64_t)bidx * g.so + (arow0 + wm * WM) * g.ldo + bcol0 + wn * WN;
      const __amdgpu_buffer_rsrc_t rso =
          __builtin_amdgcn_make_buffer_rsrc((void*)outw, 0, 0x7fffffff, 0x00020000);
      const int ldo_b = (int)(g.ldo * 2);
      const int vor = (lane >> 4) * ldo_b + (lane & 15) * 16;
      const bool full = arow0 + 256 <= g.Mv && bcol0 + 256 <= g.Nv;
      const int rem_i = (int)g.Mv - (int)(arow0 + wm * WM + fr);
      const int rem_j = (int)g.Nv - (int)(bcol0 + wn * WN + 4 * fg);
      auto emit = [&](auto masked) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          stage(p, masked, rem_i, rem_j);
          uint32_t ra = epr, lc = lane & 15, lr = lane >> 4;
          int vs = vor;
          asm volatile("" : "+v"(ra), "+v"(vs), "+v"(lc), "+v"(lr));
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const uint32_t c = lc ^ ((4 * i + lr) & 15);
            const u32x4 q4 = *(const u32x4 __attribute__((address_space(3)))*)(ra + i * 1024 + (c << 4));
            __builtin_amdgcn_raw_buffer_store_b128(q4, rso, vs + i * 4 * ldo_b, p * 32 * ldo_b, 2);
          }
        }
      };
      if (full)
        emit(std::false_type{});
      else
        emit(std::true_type{});
    } else {
      // the parameter block of this wave: rows orow0 .., columns ocol0 .. of matrix mb of
      // tensor t; staging row r of round p is parameter row orow0 + 32 p + r, chunk c its
      // columns ocol0 + 8 c .. + 7
      const int t = (int)(bidx / ap.nb);
      const int64_t mb = bidx - (int64_t)t * ap.nb;
      const float adj = ap.adj[t];
      const int64_t orow0 = SW ? bcol0 + wn * WN : arow0 + wm * WM;
      const int64_t ocol0 = SW ? arow0 + wm * WM : bcol0 + wn * WN;
      bf16_t* pw = (bf16_t*)ap.params[t] + mb * ap.prows * ap.pcols + orow0 * ap.pcols + ocol0;
      const __amdgpu_buffer_rsrc_t rsp =
          __builtin_amdgcn_make_buffer_rsrc((void*)pw, 0, 0x7fffffff, 0x00020000);
      const int ldp_b = (int)(ap.pcols * 2);
      const int lr = lane >> 4, lc = lane & 15;
      const int vop = lr * ldp_b + lc * 16;
      const int vrows = (int)std::min<int64_t>(ap.prows - orow0, 1 << 20);  // valid rows from orow0
      const bool vcol = ocol0 + lc * 8 < ap.pcols;                          // whole 8-column chunks
      // Chunk i of round p is parameter row 32 p + 4 i + lane/16 of the block; its row offset is
      // the scalar offset of the access. A lane outside the parameter (padding rows or columns)
      // takes a per-lane offset past the descriptor's range instead of a branch: its loads
      // read zeros and its stores are dropped, so the code stays straight and the loads of
      // round p + 1 go out before round p is applied.
      const float adjr = bf16_to_f32(f32_to_bf16(adj));
      auto voff = [&](int p, int i) -> int {
        return vcol && lr < vrows - (p * 32 + 4 * i) ? vop : (int)0x80000000;
      };
      // apply_elem<bf16, bf16> in three straight forms (apply_bf16x8, one kernel each: MODE 1
      // cautious weight decay, 2 plain weight decay, 0 no weight decay)
      auto rounds = [&](auto mode_c) {
        constexpr int AM = decltype(mode_c)::value;
        u32x4 pv[2][8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          pv[0][i] = __builtin_amdgcn_raw_buffer_load_b128(rsp, voff(0, i), 4 * i * ldp_b, 2);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          if (p < 3) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
              pv[(p + 1) & 1][i] = __builtin_amdgcn_raw_buffer_load_b128(
                  rsp, voff(p + 1, i), ((p + 1) * 32 + 4 * i) * ldp_b, 2);
          }
          stage(p, std::false_type{}, 0, 0);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const uint32_t c = lc ^ ((4 * i + lr) & 15);
            const u32x4 q4 = *(const u32x4 __attribute__((address_space(3)))*)(epr + i * 1024 + (c << 4));
            const u32x4 o4 = apply_bf16x8<AM>(q4, pv[p & 1][i], adj, adjr, ap.wd);
            __builtin_amdgcn_raw_buffer_store_b128(o4, rsp, voff(p, i), (p * 32 + 4 * i) * ldp_b, 2);
          }
        }
      };
      rounds(std::integral_constant<int, MODE>{});
    }
    if (!has_next) break;
    li = lnext;
    bidx = nbidx;
    arow0 = narow0;
    bcol0 = nbcol0;
    rsa = rsa_n;
    rsx = rsx_n;
  }
}

// ----------------------------------------------------------------------------------
// The SYRK kernel (X X^T, A A) on 16 x 16 x 32 MFMAs.
//
// Tiles, tile order, waves (8, two per SIMD, 64 x 128 each), LDS stages and epilogue
// staging as gemm_bf16_v2_kernel; the wave's block is 4 x 8 accumulators of 16 x 16 and a
// K-tile is two 32-k substeps of 32 MFMAs, each substep reading the next one's 12 fragments
// (4 a, 8 b) between its MFMAs. The DMA of K-tile k + 2 is spread over the second substep
// of K-tile k (two loads per block of 8 MFMAs), right after the barrier that ends the reads
// of its stage. On the Llama shapes X X^T and A A run 6-7% faster than on 32 x 32 x 16
// MFMAs; launches with packed tiles measured 2-5% slower on X X^T (also with a K loop per
// tile kind) and stay on gemm_bf16_v2_kernel.
//
// Fragments (lane l, r = l % 16, g = l / 16): srcA is a-panel row 16 fi + r, srcB is
// b-panel row 16 fj + r, both 8 consecutive k (logical chunk 4 ks + g of the row); the
// accumulator register q of block (fi, fj) is C(16 fi + 4 g + q, 16 fj + r).
#define S16(C, B) "v_mfma_f32_16x16x32_bf16 %[" #C "], %[a], %[" #B "], %[" #C "]\n\t"
#define S16_OUT                                                                             \
  [c0] "+v"(acc[0]), [c1] "+v"(acc[1]), [c2] "+v"(acc[2]), [c3] "+v"(acc[3]),                \
  [c4] "+v"(acc[4]), [c5] "+v"(acc[5]), [c6] "+v"(acc[6]), [c7] "+v"(acc[7]),                \
  [na] "=&v"(na), [nb0] "=&v"(nb0), [nb1] "=&v"(nb1)
#define S16_IN                                                                              \
  [a] "v"(ca), [b0] "v"(cb[0]), [b1] "v"(cb[1]), [b2] "v"(cb[2]), [b3] "v"(cb[3]),           \
  [b4] "v"(cb[4]), [b5] "v"(cb[5]), [b6] "v"(cb[6]), [b7] "v"(cb[7]), [aa] "v"(aa),          \
  [ba] "v"(ba), [oa] "i"(FI * 16 * V2_ROWB), [ob0] "i"(2 * FI * 16 * V2_ROWB),                \
  [ob1] "i"((2 * FI + 1) * 16 * V2_ROWB)
#define S16_RA "ds_read_b128 %[na], %[aa] offset:%[oa]\n\t"
#define S16_RB0 "ds_read_b128 %[nb0], %[ba] offset:%[ob0]\n\t"
#define S16_RB1 "ds_read_b128 %[nb1], %[ba] offset:%[ob1]\n\t"
#define S16_M0(N) "s_mov_b32 m0, %[mz" #N "]\n\t"
#define S16_DL(N) "buffer_load_dwordx4 %[vo" #N "], %[rs" #N "], %[so" #N "] offen lds\n\t"
#define S16_LD(N)                                                                           \
  [vo##N] "v"(vo##N), [rs##N] "s"(rs##N), [so##N] "s"(so##N), [mz##N] "s"(mz##N)
// One block of a 32-k substep: the 8 MFMAs of a fragment FI (accumulators acc[0..7]) with
// the reads of the next substep's a fragment FI (aa + 2 KB FI) and b fragments 2 FI and
// 2 FI + 1 (ba + 2 KB (2 FI), + 2 KB (2 FI + 1)). MODE (diagonal tiles, below): 0 all 8
// column blocks; 1 column blocks 4-7 only (the same reads); 2 no MFMAs and no reads.
template <int FI, int MODE = 0>
MUON_DEVICE void s16_block(f32x4 (&acc)[8], const bf16x8_mfma& ca, const bf16x8_mfma (&cb)[8],
                           bf16x8_mfma& na, bf16x8_mfma& nb0, bf16x8_mfma& nb1, uint32_t aa,
                           uint32_t ba) {
  if constexpr (MODE == 0)
    asm volatile(S16_RA S16(c0, b0) S16(c1, b1) S16(c2, b2)
                 S16_RB0 S16(c3, b3) S16(c4, b4) S16(c5, b5)
                 S16_RB1 S16(c6, b6) S16(c7, b7)
                 : S16_OUT
                 : S16_IN);
  else if constexpr (MODE == 1)
    asm volatile(S16_RA S16(c4, b4) S16_RB0 S16(c5, b5) S16_RB1 S16(c6, b6) S16(c7, b7)
                 : S16_OUT
                 : S16_IN);
}
// The same with two loads of a K-tile's DMA, each after an MFMA that follows its M0 write
// (MODE 2: the loads alone, each one wait state after its M0 write).
template <int FI, int MODE = 0>
MUON_DEVICE void s16_block_dma(f32x4 (&acc)[8], const bf16x8_mfma& ca, const bf16x8_mfma (&cb)[8],
                               bf16x8_mfma& na, bf16x8_mfma& nb0, bf16x8_mfma& nb1, uint32_t aa,
                               uint32_t ba, int vo0, u32x4 rs0, int so0, uint32_t mz0, int vo1,
                               u32x4 rs1, int so1, uint32_t mz1) {
  if constexpr (MODE == 0)
    asm volatile(S16_M0(0) S16_RA S16(c0, b0) S16_DL(0) S16(c1, b1) S16_M0(1) S16(c2, b2)
                 S16_RB0 S16(c3, b3) S16_DL(1) S16(c4, b4) S16(c5, b5)
                 S16_RB1 S16(c6, b6) S16(c7, b7)
                 : S16_OUT
                 : S16_IN, S16_LD(0), S16_LD(1)
                 : "m0", "memory");
  else if constexpr (MODE == 1)
    asm volatile(S16_M0(0) S16_RA S16(c4, b4) S16_DL(0) S16_M0(1) S16_RB0 S16(c5, b5)
                 S16_DL(1) S16_RB1 S16(c6, b6) S16(c7, b7)
                 : S16_OUT
                 : S16_IN, S16_LD(0), S16_LD(1)
                 : "m0", "memory");
  else
    asm volatile(S16_M0(0) "s_nop 0\n\t" S16_DL(0) S16_M0(1) "s_nop 0\n\t" S16_DL(1)
                 :
                 : S16_LD(0), S16_LD(1)
                 : "m0", "memory");
}
#undef S16
#undef S16_OUT
#undef S16_IN
#undef S16_RA
#undef S16_RB0
#undef S16_RB1
#undef S16_M0
#undef S16_DL
#undef S16_LD

typedef bf16x8_mfma s16_frags[12];  // a fragments 0-3, b fragments 0-7

// One substep without DMA, then the wait for its 12 reads.
template <int MODE = 0>
MUON_DEVICE void s16_substep(f32x4 (&acc)[4][8], const s16_frags& c, s16_frags& n, uint32_t aa,
                             uint32_t ba) {
  const bf16x8_mfma(&cb)[8] = *(const bf16x8_mfma(*)[8]) & c[4];
  s16_block<0, MODE>(acc[0], c[0], cb, n[0], n[4], n[5], aa, ba);
  s16_block<1, MODE>(acc[1], c[1], cb, n[1], n[6], n[7], aa, ba);
  s16_block<2, MODE>(acc[2], c[2], cb, n[2], n[8], n[9], aa, ba);
  s16_block<3, MODE>(acc[3], c[3], cb, n[3], n[10], n[11], aa, ba);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// One substep with the DMA of one K-tile into one stage: this wave's slabs q = 0..3 of the a
// panel (scalar offsets soa + q sta, M0 ma + 8 KB q) and of the b panel (sob + q stb, mb +
// 8 KB q), two after each block. A slab is the wave's 1 KB of 8 panel rows. DIAG (a diagonal
// tile, whose b panel is its a panel): the a panel only.
template <int MODE = 0, bool DIAG = false>
MUON_DEVICE void s16_substep_dma(f32x4 (&acc)[4][8], const s16_frags& c, s16_frags& n, uint32_t aa,
                                 uint32_t ba, int voa, int vob, u32x4 rsa, u32x4 rsb, int soa,
                                 int sta, int sob, int stb, uint32_t ma, uint32_t mb) {
  const bf16x8_mfma(&cb)[8] = *(const bf16x8_mfma(*)[8]) & c[4];
  s16_block_dma<0, MODE>(acc[0], c[0], cb, n[0], n[4], n[5], aa, ba, voa, rsa, soa, ma, voa, rsa,
                         soa + sta, ma + 0x2000);
  s16_block_dma<1, MODE>(acc[1], c[1], cb, n[1], n[6], n[7], aa, ba, voa, rsa, soa + 2 * sta,
                         ma + 0x4000, voa, rsa, soa + 3 * sta, ma + 0x6000);
  if constexpr (DIAG) {
    s16_block<2, MODE>(acc[2], c[2], cb, n[2], n[8], n[9], aa, ba);
    s16_block<3, MODE>(acc[3], c[3], cb, n[3], n[10], n[11], aa, ba);
  } else {
    s16_block_dma<2, MODE>(acc[2], c[2], cb, n[2], n[8], n[9], aa, ba, vob, rsb, sob, mb, vob,
                           rsb, sob + stb, mb + 0x2000);
    s16_block_dma<3, MODE>(acc[3], c[3], cb, n[3], n[10], n[11], aa, ba, vob, rsb,
                           sob + 2 * stb, mb + 0x4000, vob, rsb, sob + 3 * stb, mb + 0x6000);
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// All 12 fragment reads of one substep without MFMAs (pipeline start).
MUON_DEVICE void s16_frag_load(s16_frags& n, uint32_t aa, uint32_t ba) {
#pragma unroll
  for (int f = 0; f < 4; ++f)
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(n[f]) : "v"(aa), "i"(f * 16 * V2_ROWB));
#pragma unroll
  for (int f = 0; f < 8; ++f)
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(n[4 + f]) : "v"(ba), "i"(f * 16 * V2_ROWB));
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// A finished 64 x 128 wave tile as bf16 pairs (hardware RNE pair conversion): hv[fi][fj][h]
// holds rows 16 fi + 4 g + 2 h and + 1 of the lane's column 16 fj + r. Unless `full`,
// elements outside the valid extent are cleared to +0: rem_i counts the valid rows from the
// lane's first row (4 g included), rem_j the valid columns from its column.
template <int FJ>
MUON_DEVICE void s16_pack(const f32x4 (&acc)[4][FJ], float alpha, bool full, int rem_i, int rem_j,
                          uint32_t (&hv)[4][FJ][2]) {
#pragma unroll
  for (int fi = 0; fi < 4; ++fi)
#pragma unroll
    for (int fj = 0; fj < FJ; ++fj)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f2x v = {alpha * acc[fi][fj][2 * h], alpha * acc[fi][fj][2 * h + 1]};
        hv[fi][fj][h] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2x));
      }
  if (full) return;
#pragma unroll
  for (int fi = 0; fi < 4; ++fi)
#pragma unroll
    for (int fj = 0; fj < FJ; ++fj)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int il0 = fi * 16 + 2 * h;
        const bool vj = fj * 16 < rem_j;
        const uint32_t keep = (vj && il0 < rem_i ? 0x0000ffffu : 0u) |
                              (vj && il0 + 1 < rem_i ? 0xffff0000u : 0u);
        hv[fi][fj][h] &= keep;
      }
}

__global__ __launch_bounds__(512, 1) void gemm_bf16_s16_kernel(GemmArgs g) {
  constexpr int NW = 8, WM = 64, WN = 128;
  extern __shared__ __align__(16) uint8_t smem[];

  int bidx, tm, tn;
  map_tile(g, MODE_SYRK, bidx, tm, tn);
  const int64_t arow0 = (int64_t)tm * 256, brow0 = (int64_t)tn * 256;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // A diagonal tile (tm == tn) stores only its upper triangle, 10 of its 16 64 x 64 units.
  // Its waves take the 64 x 128 blocks in another order, so that each SIMD's two waves
  // (waves w and w + 4 share a SIMD) carry 3, 3, 2 and 2 of those units instead of 2, 4, 1
  // and 3: waves 0-3 compute blocks (0, 0), (0, 1), (1, 1), (2, 1) whole (MFMA mode 0),
  // waves 4 and 5 blocks (1, 0) and (3, 1), of which only column blocks 4-7 reach the upper
  // triangle (mode 1), waves 6 and 7 blocks (2, 0) and (3, 0), wholly below it (mode 2: no
  // MFMAs). The a and b panels of a diagonal tile are the same rows: only the a panel is
  // loaded, and the b fragments are read from it. This applies to A A and to X X^T with
  // K <= 4096; X X^T over longer rows (K = 14336) ran 1 ms per Llama step slower in this form
  // and keeps whole 64 x 128 blocks and both panels (the epilogue treats its diagonal tiles
  // as diagonal either way).
  const bool dtile = tm == tn;
  const bool diag = dtile && (g.beta != 0.0f || g.K <= 4096);
  const int wm = diag ? (0x32312100 >> (4 * wave)) & 15 : wave >> 1;
  const int wn = diag ? (0x00101110 >> (4 * wave)) & 15 : wave & 1;
  const int wmode = diag ? (0x22110000 >> (4 * wave)) & 15 : 0;
  const bf16_t* A = (const bf16_t*)g.a + (int64_t)bidx * g.sa;
  const bf16_t* B = (const bf16_t*)g.b + (int64_t)bidx * g.sb;
  const int lda_b = (int)(g.lda * 2), ldb_b = (int)(g.ldb * 2);
  const u32x4 rsa = n4_rsrc(A + arow0 * g.lda, false);
  const u32x4 rsb = n4_rsrc(B + brow0 * g.ldb, false);
  const u32x4 rs_none = n4_rsrc(A, true);
  const __amdgpu_buffer_rsrc_t rsa_p =
      __builtin_amdgcn_make_buffer_rsrc((void*)(A + arow0 * g.lda), 0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb_p =
      __builtin_amdgcn_make_buffer_rsrc((void*)(B + brow0 * g.ldb), 0, 0x7fffffff, 0x00020000);
  // load slab q*NW + wave = panel rows (q*NW + wave)*8 .. +7; lane -> row lane/8, chunk
  // position lane%8, which holds logical chunk (lane%8) ^ kswz(row)
  const int r_in = wave * 8 + (lane >> 3);
  const int lch = (lane & 7) ^ kswz(r_in);
  const int voa = r_in * lda_b + lch * 16;
  const int vob = r_in * ldb_b + lch * 16;
  const int sta = NW * 8 * lda_b, stb = NW * 8 * ldb_b;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  const uint32_t m0w = lds0 + wave * 1024;

  // fragment read offsets: lane -> row r of the fragment, logical chunk 4 ks + g
  const int fr = lane & 15, fg = lane >> 4;
  int foff[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) foff[ks] = fr * V2_ROWB + (((ks * 4 + fg) ^ kswz(fr)) << 4);
  const int abase = wm * WM * V2_ROWB, bbase = (diag ? 0 : V2_TILEB) + wn * WN * V2_ROWB;

  float alpha = g.alpha, beta = g.beta;
  if (g.scale_mode != 0) {
    const float s = g.scale[bidx];
    if (g.scale_mode == 1) {
      alpha *= s;
      beta *= s;
    } else {
      alpha *= s * s;
    }
  }
  const float ratio = beta != 0.0f ? beta / alpha : 0.0f;
  // K-tile whose k range equals this wave's output rows (WM == BK)
  const int kdiag = ratio != 0.0f ? (int)((arow0 + wm * WM) / V2_BK) : -1;

  const int KT = (int)(g.K / V2_BK);
  auto aaddr = [&](int st, int ks) -> uint32_t { return lds0 + st * V2_STAGEB + abase + foff[ks]; };
  auto baddr = [&](int st, int ks) -> uint32_t { return lds0 + st * V2_STAGEB + bbase + foff[ks]; };
  // the DMA of K-tile kt into stage st (pipeline start; later K-tiles ride in the substeps)
  auto issue = [&](int kt, int st) {
    uint8_t* sa = smem + st * V2_STAGEB;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa_p, (lds_ptr_t)(sa + (q * NW + wave) * 1024), 16,
                                               voa, q * sta + kt * V2_ROWB, 0, 0);
      if (!diag)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsb_p, (lds_ptr_t)(sa + V2_TILEB + (q * NW + wave) * 1024), 16, vob,
            q * stb + kt * V2_ROWB, 0, 0);
    }
  };
  issue(0, 0);
  wait_vmcnt0();
  lds_barrier();
  if (KT > 1) issue(1, 1);
  // accumulators and fragments are declared per path: nothing of the K loop is live across
  // the branch on the mode
  auto kloop = [&](auto mode_c, auto diag_c) {
    constexpr int MODE = decltype(mode_c)::value;
    constexpr bool DIAG = decltype(diag_c)::value;
    f32x4 acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    s16_frags f0, f1;
    if (MODE != 2) s16_frag_load(f0, aaddr(0, 0), baddr(0, 0));
    for (int kt = 0; kt < KT; ++kt) {
      const int cs = kt & 1;
      s16_substep<MODE>(acc, f0, f1, aaddr(cs, 1), baddr(cs, 1));
      if (MODE != 2 && kt == kdiag) {
        // cin(i, j) = b(j, i): row j of the b panel, k offset i - kt*BK (the 4 rows of one
        // accumulator are 8 contiguous bytes of that row)
        mfma_to_valu_wait();
        const uint32_t sb = lds0 + cs * V2_STAGEB + bbase + fr * V2_ROWB + (fg & 1) * 8;
#pragma unroll
        for (int fi = 0; fi < 4; ++fi)
#pragma unroll
          for (int fj = 0; fj < 8; ++fj) {
            const u32x2 w = *(const u32x2 __attribute__((address_space(3)))*)(
                sb + fj * 16 * V2_ROWB + (((2 * fi + (fg >> 1)) ^ kswz(fr)) << 4));
            acc[fi][fj][0] += ratio * __uint_as_float(w.x << 16);
            acc[fi][fj][1] += ratio * __uint_as_float(w.x & 0xffff0000u);
            acc[fi][fj][2] += ratio * __uint_as_float(w.y << 16);
            acc[fi][fj][3] += ratio * __uint_as_float(w.y & 0xffff0000u);
          }
        valu_to_mfma_wait();
      }
      wait_vmcnt0();
      lds_barrier();
      // K-tile kt + 2 into this K-tile's stage; past the last K-tile the null descriptor
      // reads no memory
      const bool more = kt + 2 < KT;
      const int kb = (kt + 2) * V2_ROWB;
      const uint32_t ma = m0w + cs * V2_STAGEB;
      s16_substep_dma<MODE, DIAG>(acc, f1, f0, aaddr(cs ^ 1, 0), baddr(cs ^ 1, 0), voa, vob,
                                  more ? rsa : rs_none, more ? rsb : rs_none, kb, sta, kb, stb,
                                  ma, ma + V2_TILEB);
    }
    mfma_to_valu_wait();
    wait_vmcnt0();

    // ---- epilogue: stage through LDS, store 16-byte row chunks ----
    if (g.out == nullptr) return;
    bf16_t* T = (bf16_t*)smem;
    const int row0w = wm * WM, col0w = wn * WN;  // wave origin within the tile
    uint32_t hv[4][8][2];
    s16_pack(acc, alpha, arow0 + 256 <= g.Mv && brow0 + 256 <= g.Nv,
             clamp_rem(g.Mv - (arow0 + row0w + fg * 4)), clamp_rem(g.Nv - (brow0 + col0w + fr)), hv);
    bf16_t* out = (bf16_t*)g.out + (int64_t)bidx * g.so;
    if (!dtile) {
      // mirror half of the symmetric output: T[j][i], 4 consecutive i per lane -> one 8-byte
      // write
      lds_barrier();
#pragma unroll
      for (int fi = 0; fi < 4; ++fi)
#pragma unroll
        for (int fj = 0; fj < 8; ++fj) {
          const int jl = col0w + fj * 16 + fr;
          const int il = row0w + fi * 16 + fg * 4;
          *(uint2*)(T + jl * V2_EP_PITCH + il) = make_uint2(hv[fi][fj][0], hv[fi][fj][1]);
        }
      lds_barrier();
#pragma unroll 4
      for (int it = 0; it < 16; ++it) {
        const int id = it * 512 + tid;
        const int jl = id >> 5, c = (id & 31) * 8;
        const uint4 w = *(const uint4*)(T + jl * V2_EP_PITCH + c);
        *(uint4*)(out + (brow0 + jl) * g.ldo + arow0 + c) = w;
      }
    }
    // row-major stage: T[i][j]
    lds_barrier();
#pragma unroll
    for (int fi = 0; fi < 4; ++fi)
#pragma unroll
      for (int fj = 0; fj < 8; ++fj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int il = row0w + fi * 16 + fg * 4 + q;
          const int jl = col0w + fj * 16 + fr;
          T[il * V2_EP_PITCH + jl] = (bf16_t)(hv[fi][fj][q >> 1] >> (16 * (q & 1)));
        }
    lds_barrier();
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
      const int id = it * 512 + tid;
      const int il = id >> 5, c = (id & 31) * 8;
      uint4 w;
      if (!dtile || c >= il) {
        w = *(const uint4*)(T + il * V2_EP_PITCH + c);
      } else {
        // diagonal tile, chunk reaching below the diagonal: those columns come from the
        // computed (upper) element of the mirror position
        uint16_t e[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
          e[q] = (c + q < il) ? T[(c + q) * V2_EP_PITCH + il] : T[il * V2_EP_PITCH + c + q];
        __builtin_memcpy(&w, e, 16);
      }
      *(uint4*)(out + (arow0 + il) * g.ldo + brow0 + c) = w;
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  // one K loop and epilogue per mode, so no path merges into another's registers
  if (!diag)
    kloop(I0{}, std::false_type{});
  else if (wmode == 0)
    kloop(I0{}, std::true_type{});
  else if (wmode == 1)
    kloop(I1{}, std::true_type{});
  else
    kloop(I2{}, std::true_type{});
}

// ----------------------------------------------------------------------------------
// The SYRK on 128 x 128 tiles, for launches of at most two rounds of 256-row tiles, which
// leave CUs idle (12 matrices of 768 rows: 72 workgroups of 256-row tiles, 252 of 128-row
// ones; 32 of 1024 rows: 320 = 256 + 64, against 1152 in two workgroups per CU). Four
// waves (2 x 2, 64 x 64 each: 4 x 4 accumulators of 16 x 16) and 64 KB of LDS per
// workgroup, so that two workgroups share a CU (two waves per SIMD, as in
// gemm_bf16_s16_kernel). The same K-tile pipeline: two 32-k substeps of 16 MFMAs, each
// reading the next substep's 8 fragments (4 a, 4 b) between its MFMAs, and the DMA of
// K-tile k + 2 spread over the second substep of K-tile k (two loads per block). Fragments
// and accumulator layout as gemm_bf16_s16_kernel's.
constexpr int H_TILEB = 128 * V2_ROWB;  // one 128-row K-panel
constexpr int H_STAGEB = 2 * H_TILEB;   // a and b panels
constexpr int H_EP_PITCH = 128 + 8;     // staging row pitch (elements)
constexpr int H_SMEM = 2 * H_STAGEB;
static_assert(128 * H_EP_PITCH * 2 <= H_SMEM, "the 128-row staging fits the stages");

#define H16(C, B) "v_mfma_f32_16x16x32_bf16 %[" #C "], %[a], %[" #B "], %[" #C "]\n\t"
#define H16_OUT                                                                              \
  [c0] "+v"(acc[0]), [c1] "+v"(acc[1]), [c2] "+v"(acc[2]), [c3] "+v"(acc[3]), [na] "=&v"(na), \
  [nb] "=&v"(nb)
#define H16_IN                                                                               \
  [a] "v"(ca), [b0] "v"(cb[0]), [b1] "v"(cb[1]), [b2] "v"(cb[2]), [b3] "v"(cb[3]), [aa] "v"(aa), \
  [ba] "v"(ba), [oa] "i"(FI * 16 * V2_ROWB)
#define H16_RA "ds_read_b128 %[na], %[aa] offset:%[oa]\n\t"
#define H16_RB "ds_read_b128 %[nb], %[ba] offset:%[oa]\n\t"
#define H16_M0(N) "s_mov_b32 m0, %[mz" #N "]\n\t"
#define H16_DL(N) "buffer_load_dwordx4 %[vo" #N "], %[rs" #N "], %[so" #N "] offen lds\n\t"
#define H16_LD(N) [vo##N] "v"(vo##N), [rs##N] "s"(rs##N), [so##N] "s"(so##N), [mz##N] "s"(mz##N)
// One block of a 32-k substep: the 4 MFMAs of row block FI with the reads of the next
// substep's a fragment FI (aa + 2 KB FI) and b fragment FI (ba + 2 KB FI). MODE 0: all of
// it; 2 (a wave wholly below a diagonal tile's diagonal): nothing.
template <int FI, int MODE = 0>
MUON_DEVICE void h16_block(f32x4 (&acc)[4], const bf16x8_mfma& ca, const bf16x8_mfma (&cb)[4],
                           bf16x8_mfma& na, bf16x8_mfma& nb, uint32_t aa, uint32_t ba) {
  if constexpr (MODE == 0)
    asm volatile(H16_RA H16(c0, b0) H16(c1, b1) H16_RB H16(c2, b2) H16(c3, b3)
                 : H16_OUT
                 : H16_IN);
}
// The same with two loads of a K-tile's DMA, each after an MFMA that follows its M0 write
// (MODE 2: the loads alone, each one wait state after its M0 write).
template <int FI, int MODE = 0>
MUON_DEVICE void h16_block_dma(f32x4 (&acc)[4], const bf16x8_mfma& ca, const bf16x8_mfma (&cb)[4],
                               bf16x8_mfma& na, bf16x8_mfma& nb, uint32_t aa, uint32_t ba,
                               int vo0, u32x4 rs0, int so0, uint32_t mz0, int vo1, u32x4 rs1,
                               int so1, uint32_t mz1) {
  if constexpr (MODE == 0)
    asm volatile(H16_M0(0) H16_RA H16(c0, b0) H16_DL(0) H16(c1, b1) H16_M0(1) H16_RB
                 H16(c2, b2) H16_DL(1) H16(c3, b3)
                 : H16_OUT
                 : H16_IN, H16_LD(0), H16_LD(1)
                 : "m0", "memory");
  else
    asm volatile(H16_M0(0) "s_nop 0\n\t" H16_DL(0) H16_M0(1) "s_nop 0\n\t" H16_DL(1)
                 :
                 : H16_LD(0), H16_LD(1)
                 : "m0", "memory");
}
#undef H16
#undef H16_OUT
#undef H16_IN
#undef H16_RA
#undef H16_RB
#undef H16_M0
#undef H16_DL
#undef H16_LD

typedef bf16x8_mfma h16_frags[8];  // a fragments 0-3, b fragments 0-3

template <int MODE = 0>
MUON_DEVICE void h16_substep(f32x4 (&acc)[4][4], const h16_frags& c, h16_frags& n, uint32_t aa,
                             uint32_t ba) {
  const bf16x8_mfma(&cb)[4] = *(const bf16x8_mfma(*)[4]) & c[4];
  h16_block<0, MODE>(acc[0], c[0], cb, n[0], n[4], aa, ba);
  h16_block<1, MODE>(acc[1], c[1], cb, n[1], n[5], aa, ba);
  h16_block<2, MODE>(acc[2], c[2], cb, n[2], n[6], aa, ba);
  h16_block<3, MODE>(acc[3], c[3], cb, n[3], n[7], aa, ba);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// One substep with the DMA of one K-tile into one stage: this wave's slabs q = 0..3 of the
// a panel (scalar offsets soa + q sta, M0 ma + 4 KB q) and of the b panel (sob + q stb,
// mb + 4 KB q), two after each block. DIAG (a diagonal tile): the a panel only.
template <int MODE = 0, bool DIAG = false>
MUON_DEVICE void h16_substep_dma(f32x4 (&acc)[4][4], const h16_frags& c, h16_frags& n, uint32_t aa,
                                 uint32_t ba, int voa, int vob, u32x4 rsa, u32x4 rsb, int soa,
                                 int sta, int sob, int stb, uint32_t ma, uint32_t mb) {
  const bf16x8_mfma(&cb)[4] = *(const bf16x8_mfma(*)[4]) & c[4];
  h16_block_dma<0, MODE>(acc[0], c[0], cb, n[0], n[4], aa, ba, voa, rsa, soa, ma, voa, rsa,
                         soa + sta, ma + 0x1000);
  h16_block_dma<1, MODE>(acc[1], c[1], cb, n[1], n[5], aa, ba, voa, rsa, soa + 2 * sta,
                         ma + 0x2000, voa, rsa, soa + 3 * sta, ma + 0x3000);
  if constexpr (DIAG) {
    h16_block<2, MODE>(acc[2], c[2], cb, n[2], n[6], aa, ba);
    h16_block<3, MODE>(acc[3], c[3], cb, n[3], n[7], aa, ba);
  } else {
    h16_block_dma<2, MODE>(acc[2], c[2], cb, n[2], n[6], aa, ba, vob, rsb, sob, mb, vob, rsb,
                           sob + stb, mb + 0x1000);
    h16_block_dma<3, MODE>(acc[3], c[3], cb, n[3], n[7], aa, ba, vob, rsb, sob + 2 * stb,
                           mb + 0x2000, vob, rsb, sob + 3 * stb, mb + 0x3000);
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

MUON_DEVICE void h16_frag_load(h16_frags& n, uint32_t aa, uint32_t ba) {
#pragma unroll
  for (int f = 0; f < 4; ++f)
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(n[f]) : "v"(aa), "i"(f * 16 * V2_ROWB));
#pragma unroll
  for (int f = 0; f < 4; ++f)
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(n[4 + f]) : "v"(ba), "i"(f * 16 * V2_ROWB));
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

__global__ __launch_bounds__(256, 2) void gemm_bf16_s16h_kernel(GemmArgs g) {
  constexpr int NW = 4, WM = 64, WN = 64;
  extern __shared__ __align__(16) uint8_t smem[];

  int bidx, tm, tn;
  map_tile(g, MODE_SYRK, bidx, tm, tn);
  const int64_t arow0 = (int64_t)tm * 128, brow0 = (int64_t)tn * 128;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  // A diagonal tile (tm == tn) stores its upper triangle: wave (1, 0) lies wholly below the
  // diagonal and runs no MFMAs, and since the a and b panels are the same rows only the a
  // panel is loaded, the b fragments read from it.
  const bool diag = tm == tn;
  const bool idle = diag && wm == 1 && wn == 0;
  const bf16_t* A = (const bf16_t*)g.a + (int64_t)bidx * g.sa;
  const bf16_t* B = (const bf16_t*)g.b + (int64_t)bidx * g.sb;
  const int lda_b = (int)(g.lda * 2), ldb_b = (int)(g.ldb * 2);
  const u32x4 rsa = n4_rsrc(A + arow0 * g.lda, false);
  const u32x4 rsb = n4_rsrc(B + brow0 * g.ldb, false);
  const u32x4 rs_none = n4_rsrc(A, true);
  const __amdgpu_buffer_rsrc_t rsa_p =
      __builtin_amdgcn_make_buffer_rsrc((void*)(A + arow0 * g.lda), 0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb_p =
      __builtin_amdgcn_make_buffer_rsrc((void*)(B + brow0 * g.ldb), 0, 0x7fffffff, 0x00020000);
  // load slab q*NW + wave = panel rows (q*NW + wave)*8 .. +7; lane -> row lane/8, chunk
  // position lane%8, which holds logical chunk (lane%8) ^ kswz(row)
  const int r_in = wave * 8 + (lane >> 3);
  const int lch = (lane & 7) ^ kswz(r_in);
  const int voa = r_in * lda_b + lch * 16;
  const int vob = r_in * ldb_b + lch * 16;
  const int sta = NW * 8 * lda_b, stb = NW * 8 * ldb_b;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  const uint32_t m0w = lds0 + wave * 1024;

  const int fr = lane & 15, fg = lane >> 4;
  int foff[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) foff[ks] = fr * V2_ROWB + (((ks * 4 + fg) ^ kswz(fr)) << 4);
  const int abase = wm * WM * V2_ROWB, bbase = (diag ? 0 : H_TILEB) + wn * WN * V2_ROWB;

  float alpha = g.alpha, beta = g.beta;
  if (g.scale_mode != 0) {
    const float s = g.scale[bidx];
    if (g.scale_mode == 1) {
      alpha *= s;
      beta *= s;
    } else {
      alpha *= s * s;
    }
  }
  const float ratio = beta != 0.0f ? beta / alpha : 0.0f;
  // K-tile whose k range equals this wave's output rows (WM == BK)
  const int kdiag = ratio != 0.0f ? (int)((arow0 + wm * WM) / V2_BK) : -1;

  const int KT = (int)(g.K / V2_BK);
  auto aaddr = [&](int st, int ks) -> uint32_t { return lds0 + st * H_STAGEB + abase + foff[ks]; };
  auto baddr = [&](int st, int ks) -> uint32_t { return lds0 + st * H_STAGEB + bbase + foff[ks]; };
  auto issue = [&](int kt, int st) {
    uint8_t* sa = smem + st * H_STAGEB;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa_p, (lds_ptr_t)(sa + (q * NW + wave) * 1024), 16,
                                               voa, q * sta + kt * V2_ROWB, 0, 0);
      if (!diag)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsb_p, (lds_ptr_t)(sa + H_TILEB + (q * NW + wave) * 1024), 16, vob,
            q * stb + kt * V2_ROWB, 0, 0);
    }
  };
  issue(0, 0);
  wait_vmcnt0();
  lds_barrier();
  if (KT > 1) issue(1, 1);
  auto kloop = [&](auto mode_c, auto diag_c) {
    constexpr int MODE = decltype(mode_c)::value;
    constexpr bool DIAG = decltype(diag_c)::value;
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    h16_frags f0, f1;
    if (MODE != 2) h16_frag_load(f0, aaddr(0, 0), baddr(0, 0));
    for (int kt = 0; kt < KT; ++kt) {
      const int cs = kt & 1;
      h16_substep<MODE>(acc, f0, f1, aaddr(cs, 1), baddr(cs, 1));
      if (MODE != 2 && kt == kdiag) {
        // cin(i, j) = b(j, i): row j of the b panel, k offset i - kt*BK
        mfma_to_valu_wait();
        const uint32_t sb = lds0 + cs * H_STAGEB + bbase + fr * V2_ROWB + (fg & 1) * 8;
#pragma unroll
        for (int fi = 0; fi < 4; ++fi)
#pragma unroll
          for (int fj = 0; fj < 4; ++fj) {
            const u32x2 w = *(const u32x2 __attribute__((address_space(3)))*)(
                sb + fj * 16 * V2_ROWB + (((2 * fi + (fg >> 1)) ^ kswz(fr)) << 4));
            acc[fi][fj][0] += ratio * __uint_as_float(w.x << 16);
            acc[fi][fj][1] += ratio * __uint_as_float(w.x & 0xffff0000u);
            acc[fi][fj][2] += ratio * __uint_as_float(w.y << 16);
            acc[fi][fj][3] += ratio * __uint_as_float(w.y & 0xffff0000u);
          }
        valu_to_mfma_wait();
      }
      wait_vmcnt0();
      lds_barrier();
      // K-tile kt + 2 into this K-tile's stage; past the last K-tile the null descriptor
      // reads no memory
      const bool more = kt + 2 < KT;
      const int kb = (kt + 2) * V2_ROWB;
      const uint32_t ma = m0w + cs * H_STAGEB;
      h16_substep_dma<MODE, DIAG>(acc, f1, f0, aaddr(cs ^ 1, 0), baddr(cs ^ 1, 0), voa, vob,
                                  more ? rsa : rs_none, more ? rsb : rs_none, kb, sta, kb, stb,
                                  ma, ma + H_TILEB);
    }
    mfma_to_valu_wait();
    wait_vmcnt0();

    // ---- epilogue: stage through LDS, store 16-byte row chunks ----
    if (g.out == nullptr) return;
    bf16_t* T = (bf16_t*)smem;
    const int row0w = wm * WM, col0w = wn * WN;  // wave origin within the tile
    uint32_t hv[4][4][2];
    s16_pack<4>(acc, alpha, arow0 + 128 <= g.Mv && brow0 + 128 <= g.Nv,
                clamp_rem(g.Mv - (arow0 + row0w + fg * 4)),
                clamp_rem(g.Nv - (brow0 + col0w + fr)), hv);
    bf16_t* out = (bf16_t*)g.out + (int64_t)bidx * g.so;
    if (!diag) {
      // mirror half of the symmetric output: T[j][i], 4 consecutive i per lane
      lds_barrier();
#pragma unroll
      for (int fi = 0; fi < 4; ++fi)
#pragma unroll
        for (int fj = 0; fj < 4; ++fj) {
          const int jl = col0w + fj * 16 + fr;
          const int il = row0w + fi * 16 + fg * 4;
          *(uint2*)(T + jl * H_EP_PITCH + il) = make_uint2(hv[fi][fj][0], hv[fi][fj][1]);
        }
      lds_barrier();
#pragma unroll 4
      for (int it = 0; it < 8; ++it) {
        const int id = it * 256 + tid;
        const int jl = id >> 4, c = (id & 15) * 8;
        const uint4 w = *(const uint4*)(T + jl * H_EP_PITCH + c);
        *(uint4*)(out + (brow0 + jl) * g.ldo + arow0 + c) = w;
      }
    }
    // row-major stage: T[i][j]
    lds_barrier();
#pragma unroll
    for (int fi = 0; fi < 4; ++fi)
#pragma unroll
      for (int fj = 0; fj < 4; ++fj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int il = row0w + fi * 16 + fg * 4 + q;
          const int jl = col0w + fj * 16 + fr;
          T[il * H_EP_PITCH + jl] = (bf16_t)(hv[fi][fj][q >> 1] >> (16 * (q & 1)));
        }
    lds_barrier();
#pragma unroll 4
    for (int it = 0; it < 8; ++it) {
      const int id = it * 256 + tid;
      const int il = id >> 4, c = (id & 15) * 8;
      uint4 w;
      if (!diag || c >= il) {
        w = *(const uint4*)(T + il * H_EP_PITCH + c);
      } else {
        // diagonal tile, chunk reaching below the diagonal: those columns come from the
        // computed (upper) element of the mirror position
        uint16_t e[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
          e[q] = (c + q < il) ? T[(c + q) * H_EP_PITCH + il] : T[il * H_EP_PITCH + c + q];
        __builtin_memcpy(&w, e, 16);
      }
      *(uint4*)(out + (arow0 + il) * g.ldo + brow0 + c) = w;
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I2 = std::integral_constant<int, 2>;
  if (!diag)
    kloop(I0{}, std::false_type{});
  else if (!idle)
    kloop(I0{}, std::true_type{});
  else
    kloop(I2{}, std::true_type{});
}

// Wave grid of the register-staged bf16 kernel (gemm_bf16_kernel), which serves the
// masked gram_ path and SYRKs whose beta term has no alpha to fold into: 4 x 2
// wavefronts, each 64 x 128, two waves per SIMD.
#ifndef MUON_BF16_WGM
#define MUON_BF16_WGM 4
#endif
#ifndef MUON_BF16_WGN
#define MUON_BF16_WGN 2
#endif
constexpr int BF_WGM = MUON_BF16_WGM, BF_WGN = MUON_BF16_WGN;
constexpr int BF_NT = 64 * BF_WGM * BF_WGN;

// The bf16 kernels need more than the default 64 KiB of dynamic LDS; raise the
// per-kernel limit once per process for every instantiation.
int reserve_bf16_lds() {
  static int status = -1;
  static std::once_flag once;
  std::call_once(once, [] {
    const void* ks[2] = {(const void*)gemm_bf16_kernel<MODE_SYRK, false, BF_WGM, BF_WGN>,
                         (const void*)gemm_bf16_kernel<MODE_SYRK, true, BF_WGM, BF_WGN>};
    status = 0;
    for (const void* k : ks)
      if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, BF_SMEM) !=
          hipSuccess)
        status = -1;
    if (hipFuncSetAttribute((const void*)gemm_bf16_v2_kernel<MODE_SYRK, true>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, v2_smem(true)) !=
        hipSuccess)
      status = -1;
    if (hipFuncSetAttribute((const void*)gemm_bf16_s16_kernel,
                            hipFuncAttributeMaxDynamicSharedMemorySize, V2_SMEM) != hipSuccess)
      status = -1;
    if (hipFuncSetAttribute((const void*)gemm_bf16_s16h_kernel,
                            hipFuncAttributeMaxDynamicSharedMemorySize, H_SMEM) != hipSuccess)
      status = -1;
    if (hipFuncSetAttribute((const void*)gemm_bf16_nn4_kernel,
                            hipFuncAttributeMaxDynamicSharedMemorySize, N4_SMEM) != hipSuccess)
      status = -1;
    const void* n16[7] = {
        (const void*)gemm_bf16_nn16_kernel<0>,    (const void*)gemm_bf16_nn16_kernel<1, 0>,
        (const void*)gemm_bf16_nn16_kernel<1, 1>, (const void*)gemm_bf16_nn16_kernel<1, 2>,
        (const void*)gemm_bf16_nn16_kernel<2, 0>, (const void*)gemm_bf16_nn16_kernel<2, 1>,
        (const void*)gemm_bf16_nn16_kernel<2, 2>};
    for (const void* k : n16)
      if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, N4_SMEM) !=
          hipSuccess)
        status = -1;
  });
  return status;
}

// Compute units of the current device (the persistent kernel's grid), cached per device.
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Workgroups of a persistent launch over `blocks` tiles: as many rounds as one workgroup per
// CU needs, with the tiles spread evenly over them (a launch of a few hundred tiles leaves
// the CUs it does not need to kernels on other streams instead of idling them in its last
// round). Unchanged when the tile count is a multiple of the CU count.
// Whether a full-tile SYRK launch of `blocks` 256-row tiles (tiles_m per side, `batch`
// matrices) takes gemm_bf16_s16h_kernel's 128-row tiles instead: when it has at most two
// rounds of 256-row tiles (one workgroup per CU) and the 128-row tiles, two workgroups per
// CU with a quarter of the work each, need fewer rounds, counting a 128-row round as half
// a 256-row one at 85% of its efficiency (72 workgroups of 12 matrices of 768 rows: one
// round against one half-round; 320 of 32 matrices of 1024 rows: two rounds against three
// half-rounds; 200 would be one round against two half-rounds, and stays).
static bool use_h128(int tiles_m, int64_t batch, int64_t blocks) {
  const int64_t cus = device_cus();
  const int64_t th = 2 * (int64_t)tiles_m;
  const int64_t bh = th * (th + 1) / 2 * batch;
  const int64_t rounds = (blocks + cus - 1) / cus, rounds_h = (bh + 2 * cus - 1) / (2 * cus);
  return blocks <= 2 * cus && 20 * rounds_h <= 34 * rounds;
}

static int persistent_wgs(int64_t blocks) {
  const int64_t cus = device_cus();
  if (blocks <= cus) return (int)blocks;
  const int64_t rounds = (blocks + cus - 1) / cus;
  return (int)((blocks + rounds - 1) / rounds);
}

}  // namespace

// Launch one batched product. `dtype` selects bf16 (256-tiles) or fp32 (128-tiles).
// M/N are the (padded) output extents; they must be multiples of the tile unless
// `masked`. SYRK: a and b are the same K-contiguous rows. GEMM (NN): b is the
// K x N row-major operand (row pitch ldb) and the beta term reads cin = b's first
// M rows (cin(i, j) = b(i, j), true of X' = a X + B X); the bf16 kernels take it from
// the staged operand panels. Masked (arbitrary-extent) launches exist for SYRK only.
int muon_launch_gemm(int dtype, int mode, bool masked, int64_t batch, int64_t M, int64_t N,
                     int64_t K, const void* a, int64_t lda, int64_t sa, const void* b,
                     int64_t ldb, int64_t sb, const void* cin, int64_t ldc, int64_t sc,
                     void* out, int64_t ldo, int64_t so, void* out_t, int64_t ldt, int64_t st,
                     int64_t Mv, int64_t Nv, float alpha, float beta, const float* scale,
                     int scale_mode, hipStream_t stream) {
  GemmArgs g;
  g.a = a;
  g.b = b;
  g.cin = cin;
  g.out = out;
  g.out_t = out_t;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.ldo = ldo;
  g.ldt = ldt;
  g.sa = sa;
  g.sb = sb;
  g.sc = sc;
  g.so = so;
  g.st = st;
  g.Mv = Mv;
  g.Nv = Nv;
  g.Mt = M;
  g.Nt = N;
  g.Kt = K;
  g.alpha = alpha;
  g.beta = beta;
  g.scale = scale;
  g.scale_mode = scale_mode;
  g.store_out = out != nullptr;
  g.store_out_t = out_t != nullptr;
  const int bm = dtype == MUON_DT_BF16 ? BF_BM : F_BM;
  const int bk = dtype == MUON_DT_BF16 ? BF_BK : F_BK;
  g.tiles_m = (int)((M + bm - 1) / bm);
  g.tiles_n = (int)((N + bm - 1) / bm);
  g.K = masked ? round_up(K, bk) : K;
  if (!masked && (M % bm || N % bm || K % bk)) {
    muon_set_error("gemm: unmasked extents (%lld, %lld, %lld) not tile multiples", (long long)M,
                   (long long)N, (long long)K);
    return MUON_ERR_SHAPE;
  }
  if (masked && mode != MODE_SYRK) {
    muon_set_error("gemm: masked launches are SYRK only");
    return MUON_ERR_ARG;
  }
  // the bf16 kernels address one matrix's operands with 32-bit byte offsets
  const int64_t es = dtype == MUON_DT_BF16 ? 2 : 4;
  if (std::max(M * lda, (mode == MODE_SYRK ? M : K) * ldb) * es >= (int64_t)0x7fffffff) {
    muon_set_error("gemm: operand of %lld x %lld elements exceeds the 2 GiB per-matrix limit",
                   (long long)std::max(M, K), (long long)std::max(lda, ldb));
    return MUON_ERR_SHAPE;
  }
  if (mode == MODE_SYRK)
    g.tiles_per_batch = g.tiles_m * (g.tiles_m + 1) / 2;
  else
    g.tiles_per_batch = g.tiles_m * g.tiles_n;
  const int64_t blocks = (int64_t)g.tiles_per_batch * batch;
  if (blocks == 0) return MUON_OK;
  g.tiles_total = (int)std::min<int64_t>(blocks, 0x7fffffffLL);
  if (blocks > 0x7fffffffLL) {
    muon_set_error("gemm: grid too large (%lld workgroups)", (long long)blocks);
    return MUON_ERR_SHAPE;
  }
  dim3 grid((unsigned)blocks), block(256);
  if (dtype == MUON_DT_BF16) {
    if (reserve_bf16_lds() != 0) {
      muon_set_error("gemm: cannot reserve %d B of LDS", BF_SMEM);
      return MUON_ERR_LAUNCH;
    }
#define LAUNCH_BF(MODE_, MASK_)                                                        \
  do {                                                                                 \
    hipLaunchKernelGGL((gemm_bf16_kernel<MODE_, MASK_, BF_WGM, BF_WGN>), grid, dim3(BF_NT), \
                       BF_SMEM, stream, g);                                                \
  } while (0)
    if (mode == MODE_GEMM) {
      if (alpha == 0.0f) {
        muon_set_error("gemm: alpha must be nonzero");
        return MUON_ERR_ARG;
      }
      if (out_t != nullptr || K % 128 != 0) {
        muon_set_error("gemm: bf16 NN products take K a multiple of 128 and no transposed output");
        return MUON_ERR_ARG;
      }
      // persistent: at most one workgroup per CU walks the tile list
      const int wgs = persistent_wgs(blocks);
      if (K >= 768) {
        MuonApply none;
        none.nb = 1;
        hipLaunchKernelGGL(gemm_bf16_nn16_kernel<0>, dim3((unsigned)wgs), dim3(256), N4_SMEM,
                           stream, g, none);
      }
      else
        hipLaunchKernelGGL(gemm_bf16_nn4_kernel, dim3((unsigned)wgs), dim3(256), N4_SMEM, stream, g);
    } else if (!masked && (alpha != 0.0f || beta == 0.0f)) {
      // the last 128 rows padding only: the last tile column's real unit in packed tiles,
      // in the same launch as the full tiles
      const int T = g.tiles_m;
      if (T >= 2 && Mv <= M - 128 && Nv == Mv) {
        GemmArgs gp = g;
        gp.tiles_per_batch = (T - 1) * T / 2 + (2 * T - 1 + 3) / 4;
        gp.tiles_total = gp.tiles_per_batch * (int)batch;
        hipLaunchKernelGGL((gemm_bf16_v2_kernel<MODE_SYRK, true>),
                           dim3((unsigned)(gp.tiles_per_batch * batch)), dim3(512),
                           v2_smem(true), stream, gp);
      } else if (use_h128(g.tiles_m, batch, blocks)) {
        // at most two rounds of 256-row tiles, the CUs idle for much of them (72 workgroups,
        // or 320 in two rounds of 256 and 64): 128-row tiles, two workgroups per CU
        GemmArgs gh = g;
        gh.tiles_m = 2 * g.tiles_m;
        gh.tiles_per_batch = gh.tiles_m * (gh.tiles_m + 1) / 2;
        gh.tiles_total = gh.tiles_per_batch * (int)batch;
        hipLaunchKernelGGL(gemm_bf16_s16h_kernel, dim3((unsigned)gh.tiles_total), dim3(256),
                           H_SMEM, stream, gh);
      } else {
        // full tiles only: the 16 x 16 x 32 MFMA kernel
        hipLaunchKernelGGL(gemm_bf16_s16_kernel, grid, dim3(512), V2_SMEM, stream, g);
      }
    } else {
      if (masked) LAUNCH_BF(MODE_SYRK, true); else LAUNCH_BF(MODE_SYRK, false);
    }
#undef LAUNCH_BF
  } else if (dtype == MUON_DT_F32) {
    if (mode == MODE_SYRK) {
      if (masked)
        hipLaunchKernelGGL((gemm_f32_kernel<MODE_SYRK, true>), grid, block, 0, stream, g);
      else
        hipLaunchKernelGGL((gemm_f32_kernel<MODE_SYRK, false>), grid, block, 0, stream, g);
    } else {
      hipLaunchKernelGGL((gemm_f32_kernel<MODE_GEMM, false>), grid, block, 0, stream, g);
    }
  } else {
    muon_set_error("gemm: unsupported dtype %d", dtype);
    return MUON_ERR_DTYPE;
  }
  MUON_CHECK_LAUNCH("gemm");
  return MUON_OK;
}

// The last iteration's X' = a X + B X with the post-pass applied in its epilogue (bf16
// parameters, K >= 768: the 16 x 16 x 32 GEMM); extents and operands as muon_launch_gemm's
// GEMM mode, X' is not stored. tall: the parameter is the transpose of the iterate (its
// rows are the columns of X'). Parameter rows of whole 8-element chunks (pcols % 8 == 0) and
// 16-byte aligned tensors are the caller's to check.
int muon_launch_gemm_apply(int64_t batch, int64_t M, int64_t N, int64_t K, const void* a,
                           int64_t lda, int64_t sa, const void* b, int64_t ldb, int64_t sb,
                           int64_t Mv, int64_t Nv, float alpha, float beta, const float* scale,
                           int scale_mode, const MuonApply& ap, int tall, hipStream_t stream) {
  if (K < 768 || K % 128 || M % BF_BM || N % BF_BM || alpha == 0.0f || ap.nb <= 0 ||
      (batch + ap.nb - 1) / ap.nb > MUON_APPLY_MAX || ap.pcols % 8) {
    muon_set_error("gemm_apply: unsupported launch (K %lld, batch %lld)", (long long)K,
                   (long long)batch);
    return MUON_ERR_ARG;
  }
  if (std::max(M * lda, K * ldb) * 2 >= (int64_t)0x7fffffff ||
      ap.prows * ap.pcols * 2 >= (int64_t)0x7fffffff) {
    muon_set_error("gemm_apply: operand exceeds the 2 GiB per-matrix limit");
    return MUON_ERR_SHAPE;
  }
  GemmArgs g;
  memset(&g, 0, sizeof(g));
  g.a = a;
  g.b = b;
  g.cin = b;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldb;
  g.sa = sa;
  g.sb = sb;
  g.sc = sb;
  g.Mv = Mv;
  g.Nv = Nv;
  g.alpha = alpha;
  g.beta = beta;
  g.scale = scale;
  g.scale_mode = scale_mode;
  g.tiles_m = (int)(M / BF_BM);
  g.tiles_n = (int)(N / BF_BM);
  g.K = K;
  g.tiles_per_batch = g.tiles_m * g.tiles_n;
  const int64_t blocks = (int64_t)g.tiles_per_batch * batch;
  if (blocks == 0) return MUON_OK;
  if (blocks > 0x7fffffffLL) {
    muon_set_error("gemm_apply: grid too large (%lld tiles)", (long long)blocks);
    return MUON_ERR_SHAPE;
  }
  g.tiles_total = (int)blocks;
  if (reserve_bf16_lds() != 0) {
    muon_set_error("gemm_apply: cannot reserve LDS");
    return MUON_ERR_LAUNCH;
  }
  const int wgs = persistent_wgs(blocks);
  const int mode = ap.wd == 0.0f ? 0 : (ap.cautious ? 1 : 2);
#define LAUNCH_APPLY(A, M) \
  hipLaunchKernelGGL((gemm_bf16_nn16_kernel<A, M>), dim3((unsigned)wgs), dim3(256), N4_SMEM, stream, g, ap)
  if (tall) {
    if (mode == 0) LAUNCH_APPLY(2, 0); else if (mode == 1) LAUNCH_APPLY(2, 1); else LAUNCH_APPLY(2, 2);
  } else {
    if (mode == 0) LAUNCH_APPLY(1, 0); else if (mode == 1) LAUNCH_APPLY(1, 1); else LAUNCH_APPLY(1, 2);
  }
#undef LAUNCH_APPLY
  MUON_CHECK_LAUNCH("gemm_apply");
  return MUON_OK;
}
