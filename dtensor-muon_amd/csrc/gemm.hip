// Batched "NT" matrix products on CDNA4 MFMA for the Newton-Schulz / Polar Express
// iteration:  C[b](i, j) = alpha * sum_k A[b](i, k) * B[b](j, k) + beta * Cin[b](i, j)
// Both operands are K-contiguous rows, which is the native MFMA operand layout.
//
//  * SYRK mode  (A == B, upper-triangle tiles only, mirrored store): the Gram
//    products X X^T and A A (A symmetric) of pe_loop_triton / ns_loop_triton
//    (polar_express.py:98-104, newton_schulz.py:105-112; Triton gram_nd,
//    gram.py:21-106). The polynomial combination B = b*A + c*A^2 rides in the
//    epilogue (beta*Cin with Cin = A).
//  * GEMM mode: X' = a*X + B X (polar_express.py:109-110) with B symmetric, computed
//    as sum_k B(i, k) X^T(j, k); the epilogue writes X' row-major and, optionally,
//    its transpose, which the next iteration's GEMM consumes as its K-contiguous
//    operand.
//
// Operands live in workspaces whose extents are padded to the tile size and whose
// padding is rewritten as zeros by every producer, so the K loop and the stores
// need no masking (only the standalone gram_ path uses the masked variant).
#include <mutex>

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
  int store_out, store_out_t;
};

MUON_DEVICE void map_tile(const GemmArgs& g, int mode, int& bidx, int& tm, int& tn) {
  int64_t total = (int64_t)gridDim.x;
  int64_t L = blockIdx.x;
  // Dispatch hands consecutive workgroups to the 8 XCDs round-robin; remap so each
  // XCD (own L2) works through a contiguous range of (matrix, tile) indices.
  if ((total & 7) == 0) {
    int64_t per = total >> 3;
    L = (L & 7) * per + (L >> 3);
  }
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
    const int GM = 4;
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
// bf16: 256 x 256 x 64 tile, 4 wavefronts in 2 x 2, each 128 x 128 (4 x 4 MFMA
// 32x32x16 blocks, 256 fp32 accumulators per lane). LDS: double-buffered operand
// panels with an 8-element row pad (row pitch 144 B) so the 16-byte fragment reads
// of 32 consecutive rows hit distinct banks. Global loads for tile k+1 are issued
// before the MFMAs of tile k and parked in registers until the LDS slot frees up.
constexpr int BF_BM = 256, BF_BN = 256, BF_BK = 64, BF_LDSP = BF_BK + 8;
constexpr int BF_SMEM = 2 * (BF_BM + BF_BN) * BF_LDSP * 2;

template <int MODE, bool MASKED>
__global__ __launch_bounds__(256, 1) void gemm_bf16_kernel(GemmArgs g) {
  extern __shared__ __align__(16) uint8_t smem[];
  bf16_t* As = (bf16_t*)smem;
  bf16_t* Bs = As + 2 * BF_BM * BF_LDSP;

  int bidx, tm, tn;
  map_tile(g, MODE, bidx, tm, tn);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

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
  uint4 ra[8], rb[8];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int c = q * 256 + tid;
      const int r = c >> 3, cc = (c & 7) * 8;
      if (!MASKED) {
        typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
        u32x4 va = __builtin_amdgcn_raw_buffer_load_b128(rsa, voa, (int)(q * 32 * lda_b + k0 * 2), 0);
        u32x4 vb = __builtin_amdgcn_raw_buffer_load_b128(rsb, vob, (int)(q * 32 * ldb_b + k0 * 2), 0);
        ra[q] = make_uint4(va.x, va.y, va.z, va.w);
        rb[q] = make_uint4(vb.x, vb.y, vb.z, vb.w);
        (void)r;
        (void)cc;
      } else {
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
    for (int q = 0; q < 8; ++q) {
      const int c = q * 256 + tid;
      const int r = c >> 3, cc = (c & 7) * 8;
      *(uint4*)(as + r * BF_LDSP + cc) = ra[q];
      *(uint4*)(bs + r * BF_LDSP + cc) = rb[q];
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
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
    const bf16_t* as = As + cur * BF_BM * BF_LDSP + (wm * 128 + frow) * BF_LDSP + fk;
    const bf16_t* bs = Bs + cur * BF_BN * BF_LDSP + (wn * 128 + frow) * BF_LDSP + fk;
#pragma unroll
    for (int ks = 0; ks < BF_BK / 16; ++ks) {
      bf16x8_mfma af[4], bfr[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        uint4 va = *(const uint4*)(as + f * 32 * BF_LDSP + ks * 16);
        uint4 vb = *(const uint4*)(bs + f * 32 * BF_LDSP + ks * 16);
        af[f] = __builtin_bit_cast(bf16x8_mfma, va);
        bfr[f] = __builtin_bit_cast(bf16x8_mfma, vb);
      }
#pragma unroll
      for (int fm = 0; fm < 4; ++fm)
#pragma unroll
        for (int fn = 0; fn < 4; ++fn)
          acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[fm], bfr[fn], acc[fm][fn], 0, 0, 0);
    }
    if (kt + 1 < KT) sstore(cur ^ 1);
    __syncthreads();
  }

  epilogue<bf16_t, 4, 4, MASKED>(g, MODE, bidx, arow0 + wm * 128, brow0 + wn * 128, acc, lane,
                         MODE == MODE_SYRK && tm == tn);
}

// ----------------------------------------------------------------------------------
// fp32: 128 x 128 x 16 tile, 4 wavefronts in 2 x 2, each 64 x 64 (2 x 2 MFMA
// 32x32x2 f32 blocks). Used for the fp32 iteration mode and fp32 gram_.
constexpr int F_BM = 128, F_BN = 128, F_BK = 16, F_LDSP = F_BK + 4;

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
        bfr[f] = Bs[cur][(wn * 64 + f * 32 + frow) * F_LDSP + ks * 2 + fk];
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

// The bf16 kernels need more than the default 64 KiB of dynamic LDS; raise the
// per-kernel limit once per process for every instantiation.
int reserve_bf16_lds() {
  static int status = -1;
  static std::once_flag once;
  std::call_once(once, [] {
    const void* ks[4] = {(const void*)gemm_bf16_kernel<MODE_GEMM, false>,
                         (const void*)gemm_bf16_kernel<MODE_GEMM, true>,
                         (const void*)gemm_bf16_kernel<MODE_SYRK, false>,
                         (const void*)gemm_bf16_kernel<MODE_SYRK, true>};
    status = 0;
    for (const void* k : ks)
      if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, BF_SMEM) !=
          hipSuccess)
        status = -1;
  });
  return status;
}

}  // namespace

// Launch one batched product. `dtype` selects bf16 (256-tiles) or fp32 (128-tiles).
// M/N are the (padded) row extents of the a/b operands; they must be multiples of
// the tile unless `masked`.
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
  if (mode == MODE_SYRK)
    g.tiles_per_batch = g.tiles_m * (g.tiles_m + 1) / 2;
  else
    g.tiles_per_batch = g.tiles_m * g.tiles_n;
  const int64_t blocks = (int64_t)g.tiles_per_batch * batch;
  if (blocks == 0) return MUON_OK;
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
    hipLaunchKernelGGL((gemm_bf16_kernel<MODE_, MASK_>), grid, block, BF_SMEM, stream, g); \
  } while (0)
    if (mode == MODE_SYRK) {
      if (masked) LAUNCH_BF(MODE_SYRK, true); else LAUNCH_BF(MODE_SYRK, false);
    } else {
      if (masked) LAUNCH_BF(MODE_GEMM, true); else LAUNCH_BF(MODE_GEMM, false);
    }
#undef LAUNCH_BF
  } else if (dtype == MUON_DT_F32) {
    if (mode == MODE_SYRK) {
      if (masked)
        hipLaunchKernelGGL((gemm_f32_kernel<MODE_SYRK, true>), grid, block, 0, stream, g);
      else
        hipLaunchKernelGGL((gemm_f32_kernel<MODE_SYRK, false>), grid, block, 0, stream, g);
    } else {
      if (masked)
        hipLaunchKernelGGL((gemm_f32_kernel<MODE_GEMM, true>), grid, block, 0, stream, g);
      else
        hipLaunchKernelGGL((gemm_f32_kernel<MODE_GEMM, false>), grid, block, 0, stream, g);
    }
  } else {
    muon_set_error("gemm: unsupported dtype %d", dtype);
    return MUON_ERR_DTYPE;
  }
  MUON_CHECK_LAUNCH("gemm");
  return MUON_OK;
}
