// HBM-bound elementwise passes around the orthogonalization.
//
// All passes walk the stored (param-layout) matrices in 64 x 64 tiles so the
// pre-pass can emit both the stored layout and its transpose (through LDS) in one
// read of the gradient and momentum, and reduce the Frobenius-norm partials of each
// tile in a fixed order (deterministic, no atomics).
#include "common.h"

namespace {

constexpr int TILE = 64;

struct PrepassArgs {
  void* grads[MUON_MAX_TENSORS];
  void* bufs[MUON_MAX_TENSORS];
  int64_t nb, rows, cols;
  int64_t s_pitch, s_mstride;  // source (grad) row pitch and matrix stride, elements
  void* direct;        // stored-layout output (workspace), matrix 0 of this launch
  int64_t d_pitch, d_mstride;
  void* trans;         // transposed output (workspace)
  int64_t t_pitch, t_mstride;
  float* partials;     // [matrix][tile]
  int64_t parts;       // partials per matrix
  int tiles_c;         // tiles along cols of the padded stored layout
  float momentum;
  int nesterov, maximize, has_buf, write_grad;
  int write_direct;    // 0: no, 1: every element, 2: padding only (source is the direct buffer)
};

// g -> (momentum) -> x for one element; mirrors muon.py:39-56 op for op:
// buf' = buf * mu + g ; g' = g + buf' * mu (Nesterov) or buf'.
template <int GDT, int BDT>
MUON_DEVICE float momentum_elem(const PrepassArgs& a, void* gp, void* bp, int64_t idx) {
#pragma clang fp contract(off)
  float g = Elem<GDT>::load(gp, idx);
  if (a.maximize) g = -g;
  if (!a.has_buf) return g;
  float buf = Elem<BDT>::load(bp, idx);
  float nb = buf * a.momentum;
  nb = nb + g;
  Elem<BDT>::store(bp, idx, nb);
  // The per-tensor reference keeps using the fp32 value it just stored (rounded
  // into a low-precision buffer only by the copy), muon.py:49-56.
  if (!a.nesterov) return nb;
  float t = nb * a.momentum;
  return g + t;
}

// grid: x = tile index within the padded stored matrix, y = matrix of this launch.
template <int GDT, int BDT, int WDT, int VEC>
__global__ __launch_bounds__(256) void prepass_kernel(PrepassArgs a) {
#pragma clang fp contract(off)
  __shared__ float tile[TILE][TILE + 1];
  __shared__ float wsum[4];
  const int mat = blockIdx.y;
  const int tr = blockIdx.x / a.tiles_c, tc = blockIdx.x % a.tiles_c;
  const int t = (int)(mat / a.nb);
  const int64_t mb = mat % a.nb;
  void* gp = a.grads[t];
  void* bp = a.bufs[t];
  const int64_t base = mb * a.s_mstride;
  const int tid = threadIdx.x;
  const int64_t r0 = (int64_t)tr * TILE, c0 = (int64_t)tc * TILE;

  float ss = 0.0f;
  // Stored layout: 64 rows x 64 cols; each thread VEC consecutive columns.
  constexpr int TPR = TILE / VEC;          // threads per row
  constexpr int RPP = 256 / TPR;           // rows per pass
  const int cl = (tid % TPR) * VEC;
  if constexpr (VEC == 8) {
    // 16-byte accesses: the host guarantees cols % 8 == 0, a pitch multiple of 8 and
    // 16-byte aligned tensors, so each 8-column chunk is wholly valid or wholly padding
#pragma unroll
    for (int rp = 0; rp < TILE / RPP; ++rp) {
      const int rl = rp * RPP + tid / TPR;
      const int64_t r = r0 + rl;
      const int64_t c = c0 + cl;
      const bool valid = r < a.rows && c < a.cols;
      float xv[8];
      if (valid) {
        const int64_t idx = base + r * a.s_pitch + c;
        float g[8];
        Vec8<GDT>::load(gp, idx, g);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (a.maximize) g[e] = -g[e];
        float gq[8];
        if (a.has_buf) {
          float b[8], nb[8];
          Vec8<BDT>::load(bp, idx, b);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float m = b[e] * a.momentum;
            nb[e] = m + g[e];
          }
          Vec8<BDT>::store(bp, idx, nb);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            if (a.nesterov) {
              float tt = nb[e] * a.momentum;
              gq[e] = g[e] + tt;
            } else {
              gq[e] = nb[e];
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) gq[e] = g[e];
        }
        if (a.write_grad) Vec8<GDT>::store(gp, idx, gq);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xv[e] = Elem<WDT>::round(gq[e]);
          ss += xv[e] * xv[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[e] = 0.0f;
      }
      if (a.trans) {
#pragma unroll
        for (int e = 0; e < 8; ++e) tile[rl][cl + e] = xv[e];
      }
      if (a.write_direct == 1 || (a.write_direct == 2 && !valid))
        Vec8<WDT>::store(a.direct, (int64_t)mat * a.d_mstride + r * a.d_pitch + c, xv);
    }
    if (a.trans) {
    __syncthreads();
#pragma unroll
    for (int rp = 0; rp < TILE / RPP; ++rp) {
      const int cc = rp * RPP + tid / TPR;
      float tv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) tv[e] = tile[cl + e][cc];
      Vec8<WDT>::store(a.trans, (int64_t)mat * a.t_mstride + (c0 + cc) * a.t_pitch + r0 + cl, tv);
    }
    }
  } else {
#pragma unroll
  for (int rp = 0; rp < TILE / RPP; ++rp) {
    const int rl = rp * RPP + tid / TPR;
    const int64_t r = r0 + rl;
    float xv[VEC];
    bool valid[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const int64_t c = c0 + cl + e;
      float x = 0.0f;
      valid[e] = r < a.rows && c < a.cols;
      if (valid[e]) {
        const int64_t idx = base + r * a.s_pitch + c;
        float gq = momentum_elem<GDT, BDT>(a, gp, bp, idx);
        if (a.write_grad) Elem<GDT>::store(gp, idx, gq);
        x = Elem<WDT>::round(gq);
        ss += x * x;
      }
      xv[e] = x;
      if (a.trans) tile[rl][cl + e] = x;
    }
    if (a.write_direct) {
      const int64_t o = (int64_t)mat * a.d_mstride + r * a.d_pitch + c0 + cl;
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        if (a.write_direct == 1 || !valid[e]) Elem<WDT>::store(a.direct, o + e, xv[e]);
    }
  }
  if (a.trans) {
  __syncthreads();
  // Transposed layout: row (c0 + cc) of the transpose holds column cc of the tile.
#pragma unroll
  for (int rp = 0; rp < TILE / RPP; ++rp) {
    const int cc = rp * RPP + tid / TPR;
    const int64_t o = (int64_t)mat * a.t_mstride + (c0 + cc) * a.t_pitch + r0 + cl;
#pragma unroll
    for (int e = 0; e < VEC; ++e) Elem<WDT>::store(a.trans, o + e, tile[cl + e][cc]);
  }
  }
  }
  ss = warp_sum(ss);
  if ((tid & 63) == 0) wsum[tid >> 6] = ss;
  __syncthreads();
  if (tid == 0) {
    float s = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
    a.partials[(int64_t)mat * a.parts + blockIdx.x] = s;
  }
}

// The same pass over a 64-row x 256-column slab (four 64 x 64 tiles side by side) per
// workgroup, for a bf16 workspace with 16-byte aligned rows: every global load of the slab
// is issued before any arithmetic and all streamed traffic is non-temporal (measured:
// 4 tiles per workgroup with loads first and non-temporal access move 22% more bytes per
// second than one tile per workgroup on MI355X). Lane -> row tid/32 of each 8-row pass,
// 8 columns at chunk tid%32, so each lane stays in one tile (chunk/8) and the tile's
// norm partial is a fixed-order sum of its 16 lanes per wave and the 4 waves. Tall
// matrices: X0 gets the slab transposed through LDS (256 rows of 64 values).
template <int GDT, int BDT>
__global__ __launch_bounds__(256) void prepass_slab_kernel(PrepassArgs a) {
#pragma clang fp contract(off)
  constexpr int SLAB_C = 4 * TILE, NP = TILE / 8;
  __shared__ bf16_t tileT[TILE][SLAB_C + 8];
  __shared__ float wsum[4][4];
  const int mat = blockIdx.y;
  const int slabs_c = a.tiles_c / 4;
  const int tr = blockIdx.x / slabs_c, sc = blockIdx.x % slabs_c;
  const int t = (int)(mat / a.nb);
  const int64_t mb = mat % a.nb;
  void* gp = a.grads[t];
  void* bp = a.bufs[t];
  const int64_t base = mb * a.s_mstride;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int chunk = tid & 31, rsub = tid >> 5;
  const int64_t r0 = (int64_t)tr * TILE, c0 = (int64_t)sc * SLAB_C;
  const int64_t c = c0 + chunk * 8;
  const bool cvalid = c < a.cols;

  Raw8<GDT> gr[NP];
  Raw8<BDT> br[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int64_t r = r0 + p * 8 + rsub;
    if (r < a.rows && cvalid) {
      const int64_t idx = base + r * a.s_pitch + c;
      gr[p].load(gp, idx);
      if (a.has_buf) br[p].load(bp, idx);
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int rl = p * 8 + rsub;
    const int64_t r = r0 + rl;
    const bool valid = r < a.rows && cvalid;
    float xv[8];
    if (valid) {
      const int64_t idx = base + r * a.s_pitch + c;
      float g[8];
      gr[p].unpack(g);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (a.maximize) g[e] = -g[e];
      float gq[8];
      if (a.has_buf) {
        float b[8], nb[8];
        br[p].unpack(b);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float m = b[e] * a.momentum;
          nb[e] = m + g[e];
        }
        br[p].pack(nb);
        br[p].store(bp, idx);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (a.nesterov) {
            float tt = nb[e] * a.momentum;
            gq[e] = g[e] + tt;
          } else {
            gq[e] = nb[e];
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) gq[e] = g[e];
      }
      if (a.write_grad) {
        gr[p].pack(gq);
        gr[p].store(gp, idx);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xv[e] = Elem<MUON_DT_BF16>::round(gq[e]);
        ss += xv[e] * xv[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[e] = 0.0f;
    }
    Raw8<MUON_DT_BF16> xr;
    xr.pack(xv);
    if (a.trans) {
      const uint4 w = xr.w[0];
      uint32_t* d = (uint32_t*)&tileT[rl][chunk * 8];
      d[0] = w.x;
      d[1] = w.y;
      d[2] = w.z;
      d[3] = w.w;
    } else if (a.write_direct == 1) {
      xr.store(a.direct, (int64_t)mat * a.d_mstride + r * a.d_pitch + c);
    }
  }
  if (a.trans) {
    __syncthreads();
    // X0 row (c0 + cc) holds stored column cc of the slab's 64 rows
#pragma unroll 2
    for (int it = 0; it < (SLAB_C * TILE / 8) / 256; ++it) {
      const int id = it * 256 + tid;
      const int cc = id >> 3, rr = (id & 7) * 8;
      uint16_t ev[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) ev[k] = tileT[rr + k][cc];
      uint4 w;
      __builtin_memcpy(&w, ev, 16);
      st_nt((bf16_t*)a.trans + (int64_t)mat * a.t_mstride + (c0 + cc) * a.t_pitch + r0 + rr, w);
    }
  }
  // tile partials: lanes of one tile are chunk bits 0-2 and lane bit 5 within each wave
  float v = ss;
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 4, 64);
  v += __shfl_xor(v, 32, 64);
  if (lane < 32 && (lane & 7) == 0) wsum[lane >> 3][wave] = v;
  __syncthreads();
  if (tid < 4)
    a.partials[(int64_t)mat * a.parts + (int64_t)tr * a.tiles_c + sc * 4 + tid] =
        ((wsum[tid][0] + wsum[tid][1]) + wsum[tid][2]) + wsum[tid][3];
}

// Momentum only (no workspace): buf' and g' as in momentum_elem, g' stored into the
// grad tensor when write_grad. Used when the orthogonalization is supplied by the
// caller (the module-level zeropower seam) and needs g' as a tensor.
template <int GDT, int BDT>
__global__ __launch_bounds__(256) void momentum_kernel(PrepassArgs a, int64_t numel) {
#pragma clang fp contract(off)
  const int t = blockIdx.y;
  void* gp = a.grads[t];
  void* bp = a.bufs[t];
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < numel;
       i += (int64_t)gridDim.x * 256) {
    float gq = momentum_elem<GDT, BDT>(a, gp, bp, i);
    if (a.write_grad) Elem<GDT>::store(gp, i, gq);
  }
}

// scale[b] = 1 / (sqrt(sum of partials) * prescale + eps); one workgroup per matrix,
// fixed-order reduction in double.
__global__ __launch_bounds__(256) void finalize_scale_kernel(const float* partials,
                                                             int64_t parts, float* scale,
                                                             float prescale, float eps) {
#pragma clang fp contract(off)
  __shared__ double red[256];
  const int64_t b = blockIdx.x;
  const float* p = partials + b * parts;
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < parts; i += 256) s += (double)p[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float norm = (float)sqrt(red[0]);
    float denom = norm * prescale;
    denom = denom + eps;
    scale[b] = 1.0f / denom;
  }
}

// x *= scale[b] over the padded stored-layout matrices (steps == 0 path).
template <int WDT>
__global__ __launch_bounds__(256) void scale_kernel(void* x, int64_t mstride,
                                                    const float* scale) {
  const int64_t b = blockIdx.y;
  const float s = scale[b];
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < mstride;
       i += (int64_t)gridDim.x * 256) {
    const int64_t idx = b * mstride + i;
    Elem<WDT>::store(x, idx, Elem<WDT>::load(x, idx) * s);
  }
}

struct PostArgs {
  void* params[MUON_MAX_TENSORS];
  float adj[MUON_MAX_TENSORS];
  const void* u;        // matrix 0 of this launch; (TRANS) U(r, c) at u[c * u_pitch + r]
  int64_t u_pitch, u_mstride;
  const float* rscale;  // (ROWSCALE) per stored row multiplier, matrix 0 of this launch
  int64_t rs_mstride;
  float uscale[MUON_MAX_TENSORS];  // per tensor: u <- round_UDT(u * uscale) when has_uscale
  int has_uscale;
  int64_t nb, rows, cols;
  int tiles_c;
  float wd;
  int cautious;
};

// TRANS: U is the wide-orientation iterate of a tall matrix, U(r, c) = u[c][r] (the
// workspace after the iteration); the 64 x 64 block u[c0 .. c0+63][r0 .. r0+63] is read
// with coalesced 16-byte loads and transposed through LDS. Its extents are padded to a
// multiple of 64, so the block is in bounds.
// With uscale, u is first replaced by round(u * uscale[t]) in U's dtype (a split_sizes row
// block's `u * scales[i]`, base.py:98). ROWSCALE (NorMuon): u is then multiplied by its
// row's scale and the result is an fp32 tensor, so the apply runs in fp32 whatever U's
// storage dtype (normuon.py:44-55, 125-134).
template <int PDT, int UDT, int VEC, bool TRANS, bool ROWSCALE>
__global__ __launch_bounds__(256) void postpass_kernel(PostArgs a) {
#pragma clang fp contract(off)
  const int mat = blockIdx.y;
  const int tr = blockIdx.x / a.tiles_c, tc = blockIdx.x % a.tiles_c;
  const int t = (int)(mat / a.nb);
  const int64_t mb = mat % a.nb;
  void* pp = a.params[t];
  const float adj = a.adj[t];
  const int tid = threadIdx.x;
  const int64_t r0 = (int64_t)tr * TILE, c0 = (int64_t)tc * TILE;
  constexpr int TPR = TILE / VEC;
  constexpr int RPP = 256 / TPR;
  const int cl = (tid % TPR) * VEC;
  __shared__ float ut[TRANS ? TILE : 1][TILE + 1];  // ut[r - r0][c - c0]
  if constexpr (TRANS) {
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int id = it * 256 + tid;
      const int cc = id >> 3, rr = (id & 7) * 8;
      float v[8];
      Vec8<UDT>::load(a.u, (int64_t)mat * a.u_mstride + (c0 + cc) * a.u_pitch + r0 + rr, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) ut[rr + e][cc] = v[e];
    }
    __syncthreads();
  }
#pragma unroll
  for (int rp = 0; rp < TILE / RPP; ++rp) {
    const int64_t r = r0 + rp * RPP + tid / TPR;
    if (r >= a.rows) continue;
    if constexpr (VEC == 8) {
      const int64_t c = c0 + cl;
      if (c >= a.cols) continue;
      const int64_t pi = mb * a.rows * a.cols + r * a.cols + c;
      const int64_t ui = (int64_t)mat * a.u_mstride + r * a.u_pitch + c;
      float p[8], u[8], o[8];
      Vec8<PDT>::load(pp, pi, p);
      if constexpr (TRANS) {
#pragma unroll
        for (int e = 0; e < 8; ++e) u[e] = ut[r - r0][cl + e];
      } else {
        Vec8<UDT>::load(a.u, ui, u);
      }
      if (a.has_uscale) {
#pragma unroll
        for (int e = 0; e < 8; ++e) u[e] = Elem<UDT>::round(u[e] * a.uscale[t]);
      }
      if constexpr (ROWSCALE) {
        const float rs = a.rscale[(int64_t)mat * a.rs_mstride + r];
#pragma unroll
        for (int e = 0; e < 8; ++e) u[e] = u[e] * rs;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o[e] = apply_elem<PDT, ROWSCALE ? MUON_DT_F32 : UDT>(p[e], u[e], a.wd, a.cautious, adj);
      Vec8<PDT>::store(pp, pi, o);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const int64_t c = c0 + cl + e;
        if (c >= a.cols) continue;
        const int64_t pi = mb * a.rows * a.cols + r * a.cols + c;
        const int64_t ui = (int64_t)mat * a.u_mstride + r * a.u_pitch + c;
        const float p = Elem<PDT>::load(pp, pi);
        float u = TRANS ? ut[r - r0][cl + e] : Elem<UDT>::load(a.u, ui);
        if (a.has_uscale) u = Elem<UDT>::round(u * a.uscale[t]);
        if (ROWSCALE) u = u * a.rscale[(int64_t)mat * a.rs_mstride + r];
        Elem<PDT>::store(pp, pi,
                         apply_elem<PDT, ROWSCALE ? MUON_DT_F32 : UDT>(p, u, a.wd, a.cautious, adj));
      }
    }
  }
}

// The post-pass over a 64-row x 256-column slab of stored elements per workgroup (four
// tiles side by side), loads first and non-temporal access, as prepass_slab_kernel.
// TRANS (a tall result in the workspace, bf16): the rows of the wide iterate that hold the
// slab's valid columns (at most 256 x 64) are read with coalesced 128-byte rows into LDS
// first. Only rows below `cols` are read: the iterate may have as few as 64 rows.
template <int PDT, int UDT, bool TRANS, bool ROWSCALE>
__global__ __launch_bounds__(256) void postpass_slab_kernel(PostArgs a) {
#pragma clang fp contract(off)
  constexpr int SLAB_C = 4 * TILE, NP = TILE / 8;
  __shared__ uint16_t ut[TRANS ? SLAB_C : 1][TILE + 1];  // ut[c - c0][r - r0], raw bits
  const int mat = blockIdx.y;
  const int slabs_c = (a.tiles_c + 3) / 4;
  const int tr = blockIdx.x / slabs_c, sc = blockIdx.x % slabs_c;
  const int t = (int)(mat / a.nb);
  const int64_t mb = mat % a.nb;
  void* pp = a.params[t];
  const float adj = a.adj[t];
  const int tid = threadIdx.x, chunk = tid & 31, rsub = tid >> 5;
  const int64_t r0 = (int64_t)tr * TILE, c0 = (int64_t)sc * SLAB_C;
  const int64_t c = c0 + chunk * 8;
  const bool cvalid = c < a.cols;
  Raw8<PDT> pr[NP];
  Raw8<UDT> ur[NP];
  if constexpr (TRANS) {
#pragma unroll
    for (int it = 0; it < (SLAB_C * TILE / 8) / 256; ++it) {
      const int id = it * 256 + tid;
      const int cc = id >> 3, rr = (id & 7) * 8;
      if (c0 + cc >= a.cols) continue;
      const uint4 w = ld_nt((const uint16_t*)a.u + (int64_t)mat * a.u_mstride +
                            (c0 + cc) * a.u_pitch + r0 + rr);
      const uint32_t q[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        ut[cc][rr + 2 * k] = (uint16_t)(q[k] & 0xffffu);
        ut[cc][rr + 2 * k + 1] = (uint16_t)(q[k] >> 16);
      }
    }
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int64_t r = r0 + p * 8 + rsub;
    if (r < a.rows && cvalid) {
      pr[p].load(pp, mb * a.rows * a.cols + r * a.cols + c);
      if (!TRANS) ur[p].load(a.u, (int64_t)mat * a.u_mstride + r * a.u_pitch + c);
    }
  }
  if (TRANS) __syncthreads();
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int rl = p * 8 + rsub;
    const int64_t r = r0 + rl;
    if (r >= a.rows || !cvalid) continue;
    float pv[8], u[8], o[8];
    pr[p].unpack(pv);
    if constexpr (TRANS) {
#pragma unroll
      for (int e = 0; e < 8; ++e) u[e] = bf16_to_f32(ut[chunk * 8 + e][rl]);
    } else {
      ur[p].unpack(u);
    }
    if (a.has_uscale) {
#pragma unroll
      for (int e = 0; e < 8; ++e) u[e] = Elem<UDT>::round(u[e] * a.uscale[t]);
    }
    if constexpr (ROWSCALE) {
      const float rs = a.rscale[(int64_t)mat * a.rs_mstride + r];
#pragma unroll
      for (int e = 0; e < 8; ++e) u[e] = u[e] * rs;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o[e] = apply_elem<PDT, ROWSCALE ? MUON_DT_F32 : UDT>(pv[e], u[e], a.wd, a.cautious, adj);
    pr[p].pack(o);
    pr[p].store(pp, mb * a.rows * a.cols + r * a.cols + c);
  }
}

// ---- NorMuon ---------------------------------------------------------------------------
// ss[r] = sum over the columns of stored row r of U^2 (fp32, fixed order), for the 64
// stored rows r0 .. r0+63 of one matrix per workgroup. TRANS: U is the wide iterate of a
// tall matrix, stored row r = its column r (lanes over r, coalesced; the 4 waves split the
// columns and are combined in order). Otherwise lanes stride over the columns of a row
// (VEC consecutive values each) and a butterfly sums them.
struct RowSsArgs {
  const void* u;  // matrix 0 of this launch
  int64_t u_pitch, u_mstride, rows, cols;
  float* ss;      // matrix 0 of this launch, pitch ss_mstride
  int64_t ss_mstride;
  int64_t nb;     // matrices per tensor
  float uscale[MUON_MAX_TENSORS];  // per tensor: U <- round_UDT(U * uscale) when has_uscale
  int has_uscale;
};

template <int UDT, int VEC, bool TRANS>
__global__ __launch_bounds__(256) void row_sumsq_kernel(RowSsArgs a) {
#pragma clang fp contract(off)
  __shared__ float part[4][64];
  const int mat = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * 64;
  const int64_t base = (int64_t)mat * a.u_mstride;
  float* ss = a.ss + (int64_t)mat * a.ss_mstride;
  const float us = a.uscale[mat / a.nb];
  if constexpr (TRANS) {
    const int64_t r = r0 + lane;
    float s = 0.0f;
    if (r < a.rows)
      for (int64_t c = wave; c < a.cols; c += 4) {
        float v = Elem<UDT>::load(a.u, base + c * a.u_pitch + r);
        if (a.has_uscale) v = Elem<UDT>::round(v * us);
        s += v * v;
      }
    part[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && r < a.rows) ss[r] = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
  } else {
    for (int i = 0; i < 16; ++i) {
      const int64_t r = r0 + wave * 16 + i;
      if (r >= a.rows) break;
      float s = 0.0f;
      if constexpr (VEC == 8) {
        for (int64_t c = (int64_t)lane * 8; c < a.cols; c += 512) {
          float v[8];
          Vec8<UDT>::load(a.u, base + r * a.u_pitch + c, v);
          if (a.has_uscale) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = Elem<UDT>::round(v[e] * us);
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) s += v[e] * v[e];
        }
      } else {
        for (int64_t c = lane; c < a.cols; c += 64) {
          float v = Elem<UDT>::load(a.u, base + r * a.u_pitch + c);
          if (a.has_uscale) v = Elem<UDT>::round(v * us);
          s += v * v;
        }
      }
      s = warp_sum(s);
      if (lane == 0) ss[r] = s;
    }
  }
}

// The transposed case with 16-byte loads: row r of the update is column r of the stored
// result (tall matrices), so a lane takes 8 consecutive rows (8 consecutive elements of a
// stored row) and a workgroup 512 rows; wave w sums stored rows w, w + 4, ... with four
// loads in flight. The same sums in the same order as row_sumsq_kernel<UDT, 1, true>.
// Needs rows % 8 == 0 and 16-byte aligned stored rows.
template <int UDT>
__global__ __launch_bounds__(256) void row_sumsq_t8_kernel(RowSsArgs a) {
#pragma clang fp contract(off)
  __shared__ float part[4][512];
  const int mat = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t rb = (int64_t)blockIdx.x * 512;
  const int64_t r = rb + lane * 8;
  const int64_t base = (int64_t)mat * a.u_mstride;
  float* ss = a.ss + (int64_t)mat * a.ss_mstride;
  const float us = a.uscale[mat / a.nb];
  float s[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  if (r < a.rows) {
    int64_t c = wave;
    for (; c + 12 < a.cols; c += 16) {
      float v[4][8];
#pragma unroll
      for (int q = 0; q < 4; ++q) Vec8<UDT>::load(a.u, base + (c + 4 * q) * a.u_pitch + r, v[q]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = a.has_uscale ? Elem<UDT>::round(v[q][e] * us) : v[q][e];
          s[e] += x * x;
        }
      }
    }
    for (; c < a.cols; c += 4) {
      float v[8];
      Vec8<UDT>::load(a.u, base + c * a.u_pitch + r, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = a.has_uscale ? Elem<UDT>::round(v[e] * us) : v[e];
        s[e] += x * x;
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) part[wave][lane * 8 + e] = s[e];
  __syncthreads();
  for (int k = tid; k < 512; k += 256) {
    if (rb + k < a.rows) ss[rb + k] = ((part[0][k] + part[1][k]) + part[2][k]) + part[3][k];
  }
}

// Per (row block, matrix): v' = lerp(v, ss / cols, w) into the variance state, row
// multipliers d = 1 / (sqrt(v') + 1e-8), and the Frobenius rescale
// f = ||U|| / max(||U d||, 1e-8) with ||U||^2 = sum ss and ||U d||^2 = sum ss d^2 (double,
// fixed order); ss[r] is replaced by d_r * f.
struct NormuonArgs {
  float* ss;  // matrix 0 of this launch
  int64_t ss_mstride;
  void* vars[MUON_MAX_TENSORS];
  int64_t nb, rows, cols;
  int64_t split_start[MUON_MAX_SPLITS + 1];
  float w;    // lerp weight 1 - beta2
};

MUON_DEVICE float torch_lerp(float a, float b, float w) {
#pragma clang fp contract(off)
  // at::lerp for floating types: a + w (b - a) for |w| < 0.5, else b - (b - a)(1 - w)
  if (fabsf(w) < 0.5f) {
    const float d = b - a;
    return a + w * d;
  }
  const float d = b - a;
  const float om = 1.0f - w;
  return b - d * om;
}

template <int VDT>
__global__ __launch_bounds__(256) void normuon_finalize_kernel(NormuonArgs a) {
#pragma clang fp contract(off)
  __shared__ double r1[256], r2[256];
  __shared__ float fac;
  const int mat = blockIdx.y, blk = blockIdx.x, tid = threadIdx.x;
  const int t = (int)(mat / a.nb);
  const int64_t mb = mat % a.nb;
  float* ss = a.ss + (int64_t)mat * a.ss_mstride;
  void* vp = a.vars[t];
  const int64_t rs = a.split_start[blk], re = a.split_start[blk + 1];
  const float colsf = (float)a.cols;
  double s1 = 0.0, s2 = 0.0;
  for (int64_t r = rs + tid; r < re; r += 256) {
    const float q = ss[r];
    const float mean = q / colsf;
    const int64_t vi = mb * a.rows + r;
    const float vn = torch_lerp(Elem<VDT>::load(vp, vi), mean, a.w);
    Elem<VDT>::store(vp, vi, vn);
    const float den = sqrtf(vn) + 1e-8f;
    const float d = 1.0f / den;
    s1 += (double)q;
    s2 += (double)q * (double)d * (double)d;
    ss[r] = d;
  }
  r1[tid] = s1;
  r2[tid] = s2;
  __syncthreads();
  for (int h = 128; h > 0; h >>= 1) {
    if (tid < h) {
      r1[tid] += r1[tid + h];
      r2[tid] += r2[tid + h];
    }
    __syncthreads();
  }
  if (tid == 0) {
    const float norm_u = sqrtf((float)r1[0]);
    const float norm_new = fmaxf(sqrtf((float)r2[0]), 1e-8f);
    fac = norm_u / norm_new;
  }
  __syncthreads();
  const float f = fac;
  for (int64_t r = rs + tid; r < re; r += 256) ss[r] = ss[r] * f;
}

// Copy the stored-layout result out of the workspace (with dtype conversion).
template <int WDT, int ODT>
__global__ __launch_bounds__(256) void extract_kernel(const void* src, int64_t pitch,
                                                      int64_t mstride, void* dst, int64_t rows,
                                                      int64_t cols) {
  const int64_t b = blockIdx.y;
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / cols, c = i % cols;
    Elem<ODT>::store(dst, b * n + i, Elem<WDT>::load(src, b * mstride + r * pitch + c));
  }
}

// As extract_kernel for a tall matrix whose result is held transposed (element (r, c) at
// src[c * pitch + r], extents padded to 64): one 64 x 64 block per workgroup through LDS.
template <int WDT, int ODT>
__global__ __launch_bounds__(256) void extract_t_kernel(const void* src, int64_t pitch,
                                                        int64_t mstride, void* dst, int64_t rows,
                                                        int64_t cols, int tiles_c) {
  __shared__ float tile[TILE][TILE + 1];  // tile[c - c0][r - r0]
  const int64_t b = blockIdx.y;
  const int64_t r0 = (int64_t)(blockIdx.x / tiles_c) * TILE, c0 = (int64_t)(blockIdx.x % tiles_c) * TILE;
  for (int i = threadIdx.x; i < TILE * TILE; i += 256) {
    const int cc = i / TILE, rr = i % TILE;
    tile[cc][rr] = Elem<WDT>::load(src, b * mstride + (c0 + cc) * pitch + r0 + rr);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < TILE * TILE; i += 256) {
    const int rr = i / TILE, cc = i % TILE;
    const int64_t r = r0 + rr, c = c0 + cc;
    if (r < rows && c < cols) Elem<ODT>::store(dst, (b * rows + r) * cols + c, tile[cc][rr]);
  }
}

template <int GDT, int BDT, int WDT>
void launch_prepass_t(const PrepassArgs& a, dim3 grid, bool vec8, hipStream_t s) {
  if (vec8 && WDT == MUON_DT_BF16 && a.write_direct != 2 && (a.tiles_c % 4) == 0) {
    dim3 sgrid(grid.x / 4, grid.y);
    hipLaunchKernelGGL((prepass_slab_kernel<GDT, BDT>), sgrid, dim3(256), 0, s, a);
  } else if (vec8) {
    hipLaunchKernelGGL((prepass_kernel<GDT, BDT, WDT, 8>), grid, dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((prepass_kernel<GDT, BDT, WDT, 1>), grid, dim3(256), 0, s, a);
  }
}

template <int GDT, int BDT>
int launch_prepass_w(int wdt, const PrepassArgs& a, dim3 grid, bool vec8, hipStream_t s) {
  if (wdt == MUON_DT_BF16)
    launch_prepass_t<GDT, BDT, MUON_DT_BF16>(a, grid, vec8, s);
  else if (wdt == MUON_DT_F32)
    launch_prepass_t<GDT, BDT, MUON_DT_F32>(a, grid, vec8, s);
  else
    return MUON_ERR_DTYPE;
  return MUON_OK;
}

template <int GDT>
int launch_prepass_b(int bdt, int wdt, const PrepassArgs& a, dim3 grid, bool vec8,
                     hipStream_t s) {
  switch (bdt) {
    case MUON_DT_F32: return launch_prepass_w<GDT, MUON_DT_F32>(wdt, a, grid, vec8, s);
    case MUON_DT_BF16: return launch_prepass_w<GDT, MUON_DT_BF16>(wdt, a, grid, vec8, s);
    case MUON_DT_F16: return launch_prepass_w<GDT, MUON_DT_F16>(wdt, a, grid, vec8, s);
  }
  return MUON_ERR_DTYPE;
}

template <int PDT, int UDT, bool TRANS>
void launch_post_t(const PostArgs& a, dim3 grid, bool vec8, hipStream_t s) {
  if (vec8 && (!TRANS || UDT == MUON_DT_BF16)) {
    // slabs of 4 tiles side by side (a partial last slab stops at the valid columns)
    const int tiles_r = (int)(grid.x / a.tiles_c);
    dim3 sgrid((unsigned)(tiles_r * ((a.tiles_c + 3) / 4)), grid.y);
    if (a.rscale)
      hipLaunchKernelGGL((postpass_slab_kernel<PDT, UDT, TRANS, true>), sgrid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((postpass_slab_kernel<PDT, UDT, TRANS, false>), sgrid, dim3(256), 0, s, a);
    return;
  }
  if (a.rscale) {
    if (vec8)
      hipLaunchKernelGGL((postpass_kernel<PDT, UDT, 8, TRANS, true>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((postpass_kernel<PDT, UDT, 1, TRANS, true>), grid, dim3(256), 0, s, a);
  } else {
    if (vec8)
      hipLaunchKernelGGL((postpass_kernel<PDT, UDT, 8, TRANS, false>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((postpass_kernel<PDT, UDT, 1, TRANS, false>), grid, dim3(256), 0, s, a);
  }
}

// A transposed U comes from the workspace only (bf16 or fp32).
template <int PDT>
int launch_post_u(int udt, bool trans, const PostArgs& a, dim3 grid, bool vec8, hipStream_t s) {
  switch (udt) {
    case MUON_DT_F32:
      if (trans)
        launch_post_t<PDT, MUON_DT_F32, true>(a, grid, vec8, s);
      else
        launch_post_t<PDT, MUON_DT_F32, false>(a, grid, vec8, s);
      return MUON_OK;
    case MUON_DT_BF16:
      if (trans)
        launch_post_t<PDT, MUON_DT_BF16, true>(a, grid, vec8, s);
      else
        launch_post_t<PDT, MUON_DT_BF16, false>(a, grid, vec8, s);
      return MUON_OK;
    case MUON_DT_F16:
      if (trans) return MUON_ERR_DTYPE;
      launch_post_t<PDT, MUON_DT_F16, false>(a, grid, vec8, s);
      return MUON_OK;
  }
  return MUON_ERR_DTYPE;
}

template <int WDT, int ODT>
void launch_extract_t(const void* src, int64_t pitch, int64_t mstride, void* dst, int64_t rows,
                      int64_t cols, int64_t batch, hipStream_t s) {
  const int64_t tr = (rows + TILE - 1) / TILE, tc = (cols + TILE - 1) / TILE;
  hipLaunchKernelGGL((extract_t_kernel<WDT, ODT>), dim3((unsigned)(tr * tc), (unsigned)batch),
                     dim3(256), 0, s, src, pitch, mstride, dst, rows, cols, (int)tc);
}

template <int WDT>
int launch_extract_o(int odt, const void* src, int64_t pitch, int64_t mstride, int trans,
                     void* dst, int64_t rows, int64_t cols, int64_t batch, hipStream_t s) {
  if (trans) {
    switch (odt) {
      case MUON_DT_F32: launch_extract_t<WDT, MUON_DT_F32>(src, pitch, mstride, dst, rows, cols, batch, s); return MUON_OK;
      case MUON_DT_BF16: launch_extract_t<WDT, MUON_DT_BF16>(src, pitch, mstride, dst, rows, cols, batch, s); return MUON_OK;
      case MUON_DT_F16: launch_extract_t<WDT, MUON_DT_F16>(src, pitch, mstride, dst, rows, cols, batch, s); return MUON_OK;
    }
    return MUON_ERR_DTYPE;
  }
  const int64_t n = rows * cols;
  dim3 grid((unsigned)std::min<int64_t>((n + 255) / 256, 4096), (unsigned)batch);
  switch (odt) {
    case MUON_DT_F32:
      hipLaunchKernelGGL((extract_kernel<WDT, MUON_DT_F32>), grid, dim3(256), 0, s, src, pitch,
                         mstride, dst, rows, cols);
      return MUON_OK;
    case MUON_DT_BF16:
      hipLaunchKernelGGL((extract_kernel<WDT, MUON_DT_BF16>), grid, dim3(256), 0, s, src, pitch,
                         mstride, dst, rows, cols);
      return MUON_OK;
    case MUON_DT_F16:
      hipLaunchKernelGGL((extract_kernel<WDT, MUON_DT_F16>), grid, dim3(256), 0, s, src, pitch,
                         mstride, dst, rows, cols);
      return MUON_OK;
  }
  return MUON_ERR_DTYPE;
}

}  // namespace

// ---- launchers used by api.hip ------------------------------------------------------

// One prepass launch over ntensors (<= MUON_MAX_TENSORS) tensors whose matrices
// start at workspace matrix `mat0`.
int muon_launch_prepass(int ntensors, void* const* grads, void* const* bufs, int gdt, int bdt,
                        int64_t nb, int64_t rows, int64_t cols, int64_t s_pitch,
                        int64_t s_mstride, float momentum, int nesterov, int maximize,
                        int write_grad, int write_direct, void* direct, int64_t d_pitch,
                        void* trans, const OrthLayout& L, void* ws, int wdt, int64_t mat0,
                        hipStream_t s) {
  PrepassArgs a;
  for (int i = 0; i < ntensors; ++i) {
    a.grads[i] = grads[i];
    a.bufs[i] = bufs ? bufs[i] : nullptr;
  }
  a.nb = nb;
  a.rows = rows;
  a.cols = cols;
  a.s_pitch = s_pitch;
  a.s_mstride = s_mstride;
  char* w = (char*)ws;
  const int64_t rows_pad = L.tall ? L.n_pad : L.m_pad;
  const int64_t cols_pad = L.tall ? L.m_pad : L.n_pad;
  const int64_t mst = L.m_pad * L.x_pitch;  // X0's matrix stride
  a.direct = direct ? (char*)direct + mat0 * mst * L.es : nullptr;
  a.trans = trans ? (char*)trans + mat0 * mst * L.es : nullptr;
  if (write_direct && !direct) write_direct = 0;
  a.d_pitch = d_pitch;
  a.t_pitch = L.x_pitch;  // a transposed (tall) matrix's rows in X0
  a.d_mstride = mst;
  a.t_mstride = mst;
  a.partials = (float*)(w + L.off_part) + mat0 * L.parts;
  a.parts = L.parts;
  a.tiles_c = (int)(cols_pad / TILE);
  a.momentum = momentum;
  a.nesterov = nesterov;
  a.maximize = maximize;
  a.has_buf = bufs != nullptr;
  a.write_grad = write_grad;
  a.write_direct = write_direct;
  bool vec8 = (cols % 8) == 0 && (s_pitch % 8) == 0 && (nb == 1 || (s_mstride % 8) == 0);
  for (int i = 0; i < ntensors; ++i)
    if (((uintptr_t)grads[i] & 15) || (bufs && ((uintptr_t)bufs[i] & 15))) vec8 = false;
  dim3 grid((unsigned)((rows_pad / TILE) * (cols_pad / TILE)), (unsigned)(ntensors * nb));
  int rc;
  switch (gdt) {
    case MUON_DT_F32: rc = launch_prepass_b<MUON_DT_F32>(bdt, wdt, a, grid, vec8, s); break;
    case MUON_DT_BF16: rc = launch_prepass_b<MUON_DT_BF16>(bdt, wdt, a, grid, vec8, s); break;
    case MUON_DT_F16: rc = launch_prepass_b<MUON_DT_F16>(bdt, wdt, a, grid, vec8, s); break;
    default: rc = MUON_ERR_DTYPE;
  }
  if (rc != MUON_OK) {
    muon_set_error("prepass: unsupported dtypes (grad %d, buf %d, ws %d)", gdt, bdt, wdt);
    return rc;
  }
  MUON_CHECK_LAUNCH("prepass");
  return MUON_OK;
}

template <int GDT>
int launch_momentum_b(int bdt, const PrepassArgs& a, int64_t numel, dim3 grid, hipStream_t s) {
  switch (bdt) {
    case MUON_DT_F32:
      hipLaunchKernelGGL((momentum_kernel<GDT, MUON_DT_F32>), grid, dim3(256), 0, s, a, numel);
      return MUON_OK;
    case MUON_DT_BF16:
      hipLaunchKernelGGL((momentum_kernel<GDT, MUON_DT_BF16>), grid, dim3(256), 0, s, a, numel);
      return MUON_OK;
    case MUON_DT_F16:
      hipLaunchKernelGGL((momentum_kernel<GDT, MUON_DT_F16>), grid, dim3(256), 0, s, a, numel);
      return MUON_OK;
  }
  return MUON_ERR_DTYPE;
}

int muon_launch_momentum(int ntensors, void* const* grads, void* const* bufs, int gdt, int bdt,
                         int64_t numel, float momentum, int nesterov, int maximize,
                         int write_grad, hipStream_t s) {
  PrepassArgs a;
  for (int i = 0; i < ntensors; ++i) {
    a.grads[i] = grads[i];
    a.bufs[i] = bufs[i];
  }
  a.momentum = momentum;
  a.nesterov = nesterov;
  a.maximize = maximize;
  a.has_buf = 1;
  a.write_grad = write_grad;
  dim3 grid((unsigned)std::min<int64_t>((numel + 255) / 256, 8192), (unsigned)ntensors);
  int rc;
  switch (gdt) {
    case MUON_DT_F32: rc = launch_momentum_b<MUON_DT_F32>(bdt, a, numel, grid, s); break;
    case MUON_DT_BF16: rc = launch_momentum_b<MUON_DT_BF16>(bdt, a, numel, grid, s); break;
    case MUON_DT_F16: rc = launch_momentum_b<MUON_DT_F16>(bdt, a, numel, grid, s); break;
    default: rc = MUON_ERR_DTYPE;
  }
  if (rc != MUON_OK) {
    muon_set_error("momentum: unsupported dtypes (grad %d, buf %d)", gdt, bdt);
    return rc;
  }
  MUON_CHECK_LAUNCH("momentum");
  return MUON_OK;
}

int muon_launch_finalize(const OrthLayout& L, void* ws, int64_t batch, float prescale,
                         float eps, hipStream_t s) {
  char* w = (char*)ws;
  hipLaunchKernelGGL(finalize_scale_kernel, dim3((unsigned)batch), dim3(256), 0, s,
                     (const float*)(w + L.off_part), L.parts, (float*)(w + L.off_scale),
                     prescale, eps);
  MUON_CHECK_LAUNCH("finalize_scale");
  return MUON_OK;
}

int muon_launch_scale(const OrthLayout& L, void* x, int wdt, int64_t batch, const float* scale,
                      hipStream_t s) {
  const int64_t mst = L.m_pad * L.x_pitch;
  dim3 grid((unsigned)std::min<int64_t>((mst + 255) / 256, 4096), (unsigned)batch);
  if (wdt == MUON_DT_BF16)
    hipLaunchKernelGGL((scale_kernel<MUON_DT_BF16>), grid, dim3(256), 0, s, x, mst, scale);
  else
    hipLaunchKernelGGL((scale_kernel<MUON_DT_F32>), grid, dim3(256), 0, s, x, mst, scale);
  MUON_CHECK_LAUNCH("scale");
  return MUON_OK;
}

int muon_launch_postpass(int ntensors, void* const* params, const float* adj, int pdt,
                         const void* u, int udt, int64_t u_pitch, int64_t u_mstride, int u_trans,
                         const float* rscale, int64_t rs_mstride, const float* uscale,
                         int64_t nb, int64_t rows, int64_t cols, float wd, int cautious,
                         hipStream_t s) {
  PostArgs a;
  a.rscale = rscale;
  a.rs_mstride = rs_mstride;
  a.has_uscale = uscale != nullptr;
  for (int i = 0; i < ntensors; ++i) a.uscale[i] = uscale ? uscale[i] : 1.0f;
  for (int i = 0; i < ntensors; ++i) {
    a.params[i] = params[i];
    a.adj[i] = adj[i];
  }
  a.u = u;
  a.u_pitch = u_pitch;
  a.u_mstride = u_mstride;
  a.nb = nb;
  a.rows = rows;
  a.cols = cols;
  a.wd = wd;
  a.cautious = cautious;
  const int64_t tiles_r = (rows + TILE - 1) / TILE, tiles_c = (cols + TILE - 1) / TILE;
  a.tiles_c = (int)tiles_c;
  // the transposed read needs 64-padded extents and 16-byte rows (the workspace layout)
  if (u_trans && ((u_pitch % TILE) || (u_mstride % 8) || ((uintptr_t)u & 15))) {
    muon_set_error("postpass: transposed update must come from the workspace");
    return MUON_ERR_ALIGN;
  }
  bool vec8 = (cols % 8) == 0 && (u_pitch % 8) == 0 && (u_mstride % 8) == 0 &&
              !((uintptr_t)u & 15);
  for (int i = 0; i < ntensors; ++i)
    if ((uintptr_t)params[i] & 15) vec8 = false;
  dim3 grid((unsigned)(tiles_r * tiles_c), (unsigned)(ntensors * nb));
  int rc;
  switch (pdt) {
    case MUON_DT_F32: rc = launch_post_u<MUON_DT_F32>(udt, u_trans, a, grid, vec8, s); break;
    case MUON_DT_BF16: rc = launch_post_u<MUON_DT_BF16>(udt, u_trans, a, grid, vec8, s); break;
    case MUON_DT_F16: rc = launch_post_u<MUON_DT_F16>(udt, u_trans, a, grid, vec8, s); break;
    default: rc = MUON_ERR_DTYPE;
  }
  if (rc != MUON_OK) {
    muon_set_error("postpass: unsupported dtypes (param %d, u %d)", pdt, udt);
    return rc;
  }
  MUON_CHECK_LAUNCH("postpass");
  return MUON_OK;
}

int muon_launch_extract(const void* src, int wdt, int64_t pitch, int64_t mstride, int trans,
                        void* dst, int odt, int64_t rows, int64_t cols, int64_t batch,
                        hipStream_t s) {
  int rc;
  if (wdt == MUON_DT_BF16)
    rc = launch_extract_o<MUON_DT_BF16>(odt, src, pitch, mstride, trans, dst, rows, cols, batch, s);
  else
    rc = launch_extract_o<MUON_DT_F32>(odt, src, pitch, mstride, trans, dst, rows, cols, batch, s);
  if (rc != MUON_OK) {
    muon_set_error("extract: unsupported dtype %d", odt);
    return rc;
  }
  MUON_CHECK_LAUNCH("extract");
  return MUON_OK;
}

// NorMuon row statistics and finalize for nmat matrices of rows x cols starting at u
// (pitch / matrix stride in elements, transposed as the post-pass reads it), scratch ss
// (pitch ss_mstride per matrix); splits: nsplits + 1 row offsets; uscale (per tensor,
// nullable): the statistics are those of round(U * uscale[t]), as the post-pass applies.
int muon_launch_normuon_stats(int ntensors, void* const* vars, int vdt, const void* u, int udt,
                              int64_t u_pitch, int64_t u_mstride, int u_trans, int64_t nb,
                              int64_t rows, int64_t cols, float* ss, int64_t ss_mstride,
                              const int64_t* split_start, int nsplits, const float* uscale,
                              float w, hipStream_t s) {
  const int64_t nmat = (int64_t)ntensors * nb;
  RowSsArgs ra;
  ra.nb = nb;
  ra.has_uscale = uscale != nullptr;
  for (int i = 0; i < ntensors; ++i) ra.uscale[i] = uscale ? uscale[i] : 1.0f;
  ra.u = u;
  ra.u_pitch = u_pitch;
  ra.u_mstride = u_mstride;
  ra.rows = rows;
  ra.cols = cols;
  ra.ss = ss;
  ra.ss_mstride = ss_mstride;
  dim3 grid((unsigned)((rows + 63) / 64), (unsigned)nmat);
  const bool vec8 = !u_trans && (cols % 8) == 0 && (u_pitch % 8) == 0 && (u_mstride % 8) == 0 &&
                    !((uintptr_t)u & 15);
  const bool t8 = u_trans && (rows % 8) == 0 && (u_pitch % 8) == 0 && (u_mstride % 8) == 0 &&
                  !((uintptr_t)u & 15);
  const dim3 grid8((unsigned)((rows + 511) / 512), (unsigned)nmat);
#define ROWSS(UDT_)                                                                        \
  do {                                                                                     \
    if (t8)                                                                                \
      hipLaunchKernelGGL((row_sumsq_t8_kernel<UDT_>), grid8, dim3(256), 0, s, ra);          \
    else if (u_trans)                                                                      \
      hipLaunchKernelGGL((row_sumsq_kernel<UDT_, 1, true>), grid, dim3(256), 0, s, ra);     \
    else if (vec8)                                                                         \
      hipLaunchKernelGGL((row_sumsq_kernel<UDT_, 8, false>), grid, dim3(256), 0, s, ra);    \
    else                                                                                   \
      hipLaunchKernelGGL((row_sumsq_kernel<UDT_, 1, false>), grid, dim3(256), 0, s, ra);    \
  } while (0)
  switch (udt) {
    case MUON_DT_F32: ROWSS(MUON_DT_F32); break;
    case MUON_DT_BF16: ROWSS(MUON_DT_BF16); break;
    case MUON_DT_F16: ROWSS(MUON_DT_F16); break;
    default:
      muon_set_error("normuon: unsupported update dtype %d", udt);
      return MUON_ERR_DTYPE;
  }
#undef ROWSS
  NormuonArgs na;
  na.ss = ss;
  na.ss_mstride = ss_mstride;
  for (int i = 0; i < ntensors; ++i) na.vars[i] = vars[i];
  na.nb = nb;
  na.rows = rows;
  na.cols = cols;
  for (int i = 0; i <= nsplits; ++i) na.split_start[i] = split_start[i];
  na.w = w;
  dim3 fgrid((unsigned)nsplits, (unsigned)nmat);
  switch (vdt) {
    case MUON_DT_F32:
      hipLaunchKernelGGL((normuon_finalize_kernel<MUON_DT_F32>), fgrid, dim3(256), 0, s, na);
      break;
    case MUON_DT_BF16:
      hipLaunchKernelGGL((normuon_finalize_kernel<MUON_DT_BF16>), fgrid, dim3(256), 0, s, na);
      break;
    case MUON_DT_F16:
      hipLaunchKernelGGL((normuon_finalize_kernel<MUON_DT_F16>), fgrid, dim3(256), 0, s, na);
      break;
    default:
      muon_set_error("normuon: unsupported variance dtype %d", vdt);
      return MUON_ERR_DTYPE;
  }
  MUON_CHECK_LAUNCH("normuon_stats");
  return MUON_OK;
}

// ---- zero fill ---------------------------------------------------------------------
// A kernel rather than hipMemsetAsync, so that a caller may capture it in a HIP graph.
// 2-byte stores: every dtype of the library is 2 or 4 bytes wide and aligned to its size.
namespace {
__global__ __launch_bounds__(256) void zero_fill_kernel(uint16_t* dst, int64_t halves) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < halves; i += stride)
    dst[i] = 0;
}
}  // namespace

int muon_launch_zero(void* dst, int64_t bytes, hipStream_t s) {
  if (bytes <= 0) return MUON_OK;
  if (bytes % 2 || ((uintptr_t)dst & 1)) {
    muon_set_error("zero_fill: %lld bytes at %p are not whole 2-byte elements", (long long)bytes,
                   dst);
    return MUON_ERR_ALIGN;
  }
  const int64_t halves = bytes / 2;
  dim3 grid((unsigned)std::min<int64_t>((halves + 255) / 256, 4096));
  hipLaunchKernelGGL(zero_fill_kernel, grid, dim3(256), 0, s, (uint16_t*)dst, halves);
  MUON_CHECK_LAUNCH("zero_fill");
  return MUON_OK;
}
