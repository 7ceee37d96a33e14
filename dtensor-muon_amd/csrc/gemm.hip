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
// bf16, software-pipelined: 256 x 256 x 64 tile, 4 wavefronts (2 x 2), each 128 x 128
// (one wave per SIMD, 256 accumulators in AGPRs). The largest per-wave tile keeps
// LDS traffic per MFMA at its minimum (8 fragment reads per 16 MFMAs); a single wave
// per SIMD then hides latency by explicit pipelining instead of by wave switching:
//   * fragments are double-buffered: the 8 LDS reads of k-substep s+1 are issued
//     between the 16 MFMAs of substep s;
//   * global loads run two K-tiles ahead (issued in substep 3 of tile k for tile k+2,
//     parked in registers) and are written to LDS in substep 2 of tile k+1, spread
//     between that substep's MFMAs;
//   * one barrier per K-tile, placed before substep 3 so that substep's MFMAs (whose
//     fragments are already in registers) overlap the barrier and the first reads of
//     the next tile.
// sched_group_barrier pins the interleaving so the compiler cannot hoist all loads
// ahead of the MFMAs.
#define SG_MFMA 0x008
#define SG_VMEM_READ 0x020
#define SG_DS_READ 0x100
#define SG_DS_WRITE 0x200

template <int MODE>
__global__ __launch_bounds__(256, 1) void gemm_bf16_pipe_kernel(GemmArgs g) {
  constexpr int NT = 256, FM = 4, FN = 4, CPT = 8, RPQ = 32;
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
  const int64_t lda_b = g.lda * 2, ldb_b = g.ldb * 2;
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(A + arow0 * g.lda), 0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(B + brow0 * g.ldb), 0, 0x7fffffff, 0x00020000);
  const int voa = (int)((tid >> 3) * lda_b + (tid & 7) * 16);
  const int vob = (int)((tid >> 3) * ldb_b + (tid & 7) * 16);
  typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
  u32x4 ra[CPT], rb[CPT];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      ra[q] = __builtin_amdgcn_raw_buffer_load_b128(rsa, voa, (int)(q * RPQ * lda_b + k0 * 2), 0);
      rb[q] = __builtin_amdgcn_raw_buffer_load_b128(rsb, vob, (int)(q * RPQ * ldb_b + k0 * 2), 0);
    }
  };
  // LDS write address of this thread's chunk q: row q*32 + tid/8, column (tid%8)*8
  const int swr = (tid >> 3) * BF_LDSP + (tid & 7) * 8;
  auto sstore = [&](int buf) {
    bf16_t* as = As + buf * BF_BM * BF_LDSP + swr;
    bf16_t* bs = Bs + buf * BF_BN * BF_LDSP + swr;
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      *(u32x4*)(as + q * RPQ * BF_LDSP) = ra[q];
      *(u32x4*)(bs + q * RPQ * BF_LDSP) = rb[q];
    }
  };

  const int frow = lane & 31, fk = (lane >> 5) * 8;
  const int afo = (wm * 128 + frow) * BF_LDSP + fk;
  const int bfo = (wn * 128 + frow) * BF_LDSP + fk;
  bf16x8_mfma af[2][FM], bfr[2][FN];
  auto fload = [&](int buf, int ks, int set) {
    const bf16_t* as = As + buf * BF_BM * BF_LDSP + afo + ks * 16;
    const bf16_t* bs = Bs + buf * BF_BN * BF_LDSP + bfo + ks * 16;
#pragma unroll
    for (int f = 0; f < FM; ++f) af[set][f] = *(const bf16x8_mfma*)(as + f * 32 * BF_LDSP);
#pragma unroll
    for (int f = 0; f < FN; ++f) bfr[set][f] = *(const bf16x8_mfma*)(bs + f * 32 * BF_LDSP);
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  auto mfmas = [&](int set) {
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
        acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[set][fm], bfr[set][fn],
                                                               acc[fm][fn], 0, 0, 0);
  };

  const int KT = (int)(g.K / BF_BK);
  // prologue: tile 0 into LDS, tile 1 into registers, substep-0 fragments of tile 0
  gload(0);
  sstore(0);
  __syncthreads();
  gload(KT > 1 ? BF_BK : 0);
  fload(0, 0, 0);

  // The loop body is branch-free so each substep is one scheduling region: in the
  // last two iterations the loads fetch a clamped (valid) K-tile and the stores fill
  // a buffer that is never read again.
  const int64_t klast = (int64_t)(KT - 1) * BF_BK;
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    // substep 0: read fragments of substep 1
    fload(buf, 1, 1);
    mfmas(0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
    }
    // substep 1: read fragments of substep 2
    fload(buf, 2, 0);
    mfmas(1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
    }
    // substep 2: read fragments of substep 3, write tile kt+1 into the other buffer
    fload(buf, 3, 1);
    sstore(buf ^ 1);
    mfmas(0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
      __builtin_amdgcn_sched_group_barrier(SG_DS_WRITE, 2, 0);
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
    }
    // substep 3: barrier (tile kt+1 is in LDS, nobody reads tile kt's buffer any more),
    // then substep-0 fragments of tile kt+1 and global loads of tile kt+2 between the
    // MFMAs that finish tile kt
    __syncthreads();
    fload(buf ^ 1, 0, 0);
    gload(min((int64_t)(kt + 2) * BF_BK, klast));
    mfmas(1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
      __builtin_amdgcn_sched_group_barrier(SG_VMEM_READ, 2, 0);
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
    }
  }

  epilogue<bf16_t, FM, FN, false>(g, MODE, bidx, arow0 + wm * 128, brow0 + wn * 128, acc, lane,
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

// Wave grid of the bf16 tile used by the library: 4 x 2 wavefronts (each 64 x 128,
// two waves per SIMD). Measured on MI355X at the Llama step shapes, it runs the B X
// GEMM at 760-770 TFLOP/s and the SYRKs at 810-850, against 560-770 for 2 x 2 and
// 620-830 for the software-pipelined single-wave variant.
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
    const void* ks[4] = {(const void*)gemm_bf16_kernel<MODE_GEMM, false, BF_WGM, BF_WGN>,
                         (const void*)gemm_bf16_kernel<MODE_GEMM, true, BF_WGM, BF_WGN>,
                         (const void*)gemm_bf16_kernel<MODE_SYRK, false, BF_WGM, BF_WGN>,
                         (const void*)gemm_bf16_kernel<MODE_SYRK, true, BF_WGM, BF_WGN>};
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
    hipLaunchKernelGGL((gemm_bf16_kernel<MODE_, MASK_, BF_WGM, BF_WGN>), grid, dim3(BF_NT), \
                       BF_SMEM, stream, g);                                                \
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
