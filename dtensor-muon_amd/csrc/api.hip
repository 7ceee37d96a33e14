// C ABI entry points (include/muon_amd.h): argument checks, workspace layout and the
// launch sequence of one Muon step. Kernels live in gemm.hip, elementwise.hip, lp.hip.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "common.h"

// ---- launchers defined in the kernel files ------------------------------------------
int muon_launch_gemm(int dtype, int mode, bool masked, int64_t batch, int64_t M, int64_t N,
                     int64_t K, const void* a, int64_t lda, int64_t sa, const void* b,
                     int64_t ldb, int64_t sb, const void* cin, int64_t ldc, int64_t sc,
                     void* out, int64_t ldo, int64_t so, void* out_t, int64_t ldt, int64_t st,
                     int64_t Mv, int64_t Nv, float alpha, float beta, const float* scale,
                     int scale_mode, hipStream_t stream);
int muon_launch_gemm_apply(int64_t batch, int64_t M, int64_t N, int64_t K, const void* a,
                           int64_t lda, int64_t sa, const void* b, int64_t ldb, int64_t sb,
                           int64_t Mv, int64_t Nv, float alpha, float beta, const float* scale,
                           int scale_mode, const MuonApply& ap, int tall, hipStream_t stream);
int muon_launch_prepass(int ntensors, void* const* grads, void* const* bufs, int gdt, int bdt,
                        int64_t nb, int64_t rows, int64_t cols, int64_t s_pitch,
                        int64_t s_mstride, float momentum, int nesterov, int maximize,
                        int write_grad, int write_direct, void* direct, int64_t d_pitch,
                        void* trans, const OrthLayout& L, void* ws, int wdt, int64_t mat0,
                        hipStream_t s);
int muon_launch_finalize(const OrthLayout& L, void* ws, int64_t batch, float prescale,
                         float eps, hipStream_t s);
int muon_launch_momentum(int ntensors, void* const* grads, void* const* bufs, int gdt, int bdt,
                         int64_t numel, float momentum, int nesterov, int maximize,
                         int write_grad, hipStream_t s);
int muon_launch_scale(const OrthLayout& L, void* x, int wdt, int64_t batch, const float* scale,
                      hipStream_t s);
int muon_launch_postpass(int ntensors, void* const* params, const float* adj, int pdt,
                         const void* u, int udt, int64_t u_pitch, int64_t u_mstride, int u_trans,
                         const float* rscale, int64_t rs_mstride, const float* uscale,
                         int64_t nb, int64_t rows, int64_t cols, float wd, int cautious,
                         hipStream_t s);
int muon_launch_normuon_stats(int ntensors, void* const* vars, int vdt, const void* u, int udt,
                              int64_t u_pitch, int64_t u_mstride, int u_trans, int64_t nb,
                              int64_t rows, int64_t cols, float* ss, int64_t ss_mstride,
                              const int64_t* split_start, int nsplits, const float* uscale,
                              float w, hipStream_t s);
int muon_launch_extract(const void* src, int wdt, int64_t pitch, int64_t mstride, int trans,
                        void* dst, int odt, int64_t rows, int64_t cols, int64_t batch,
                        hipStream_t s);
int muon_check_lp_format(int qformat, int64_t numel, int64_t block);
int muon_launch_lp_prepass_tiled(int ntensors, void* const* grads, int gdt, void* const* codes,
                                 void* const* scales, const float* qmap, int qf, int64_t block,
                                 int64_t nb, int64_t rows, int64_t cols, float momentum,
                                 int nesterov, int maximize, const OrthLayout& L, void* ws,
                                 int64_t mat0, hipStream_t s);
int muon_launch_lp_prepass(int ntensors, void* const* grads, int gdt, void* const* codes,
                           void* const* scales, const float* qmap, int qf, int64_t block,
                           int64_t nb, int64_t rows, int64_t cols, float momentum,
                           int nesterov, int maximize, void* direct, int64_t d_pitch,
                           int64_t d_mstride, hipStream_t s);
int64_t muon_short_parts(int64_t n_pad);
int muon_launch_zero(void* dst, int64_t bytes, hipStream_t s);
int muon_launch_short_gram(const OrthLayout& L, const void* x, float* part, int64_t batch,
                           hipStream_t s);
int muon_launch_short_poly(const OrthLayout& L, float* part, void* bm, int64_t batch, float pa,
                           float pb, const float* scale, int first, hipStream_t s);
int muon_launch_short_bx(const OrthLayout& L, const void* x, void* xo, const void* bm,
                         float* part, int64_t batch, float alpha, float beta, const float* scale,
                         int first, int gram, hipStream_t s);
int muon_launch_short_bx_apply(const OrthLayout& L, const void* x, const void* bm,
                               int64_t batch, float alpha, float beta, const float* scale,
                               int first, const MuonApply& ap, hipStream_t s);

enum { MODE_GEMM = 0, MODE_SYRK = 1 };

static thread_local char g_err[512];

void muon_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

// ---- kernel timing (muon_timing_*) -------------------------------------------------
namespace {
struct TimingRec {
  int kind;
  double work;
  hipEvent_t ev0, ev1;
};
struct TimingState {
  std::mutex mu;
  bool on = false;
  std::vector<hipEvent_t> free_events;
  std::vector<TimingRec> recs;
};
TimingState g_timing;
const size_t kMaxTimedLaunches = 65536;

hipEvent_t take_event() {
  if (!g_timing.free_events.empty()) {
    hipEvent_t e = g_timing.free_events.back();
    g_timing.free_events.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Brackets the launches made during its lifetime with events on `s` when timing is on.
class Timed {
 public:
  Timed(int kind, double work, hipStream_t s) : kind_(kind), work_(work), s_(s) {
    if (!g_timing.on) return;
    std::lock_guard<std::mutex> lock(g_timing.mu);
    if (g_timing.recs.size() >= kMaxTimedLaunches) return;
    ev0_ = take_event();
    ev1_ = take_event();
    if (ev0_ && ev1_ && hipEventRecord(ev0_, s_) != hipSuccess) ev0_ = nullptr;
  }
  ~Timed() {
    if (!ev0_ || !ev1_) return;
    if (hipEventRecord(ev1_, s_) != hipSuccess) return;
    std::lock_guard<std::mutex> lock(g_timing.mu);
    g_timing.recs.push_back({kind_, work_, ev0_, ev1_});
  }

 private:
  int kind_;
  double work_;
  hipStream_t s_;
  hipEvent_t ev0_ = nullptr, ev1_ = nullptr;
};
}  // namespace

// Padding granule of the workspace extents: the bf16 tile (256); fp32 tiles (128)
// divide it. A short bf16 iterate (m <= 64) pads its rows to SHORT_ROWS only.
static const int64_t PAD = 256;
static const int64_t SHORT_ROWS = 64;
static const int64_t SHORT_PART_BYTES = 3 * 1024 * 4;
// Extra row pitch of the 256-row iterates wider than 4096 columns, in elements (128 bytes
// in bf16): with rows of a 4096 x 14336 iterate 28 KB apart B X ran 2.3-2.7% and X X^T
// 1.5-1.9% slower than with 128 more bytes per row (the Llama step 397.3 against 389.5 ms),
// measured in alternation on one box; at 4096 columns the padding changed nothing, at
// 2048 (the MoE experts) X X^T lost 2%, at 8192 and 11008 it measured within 1% either way.
static const int64_t X_PITCH_PAD = 64;
static const int64_t X_PITCH_PAD_FROM = 4096;

OrthLayout muon_orth_layout(int dtype, int64_t batch, int64_t rows, int64_t cols) {
  OrthLayout L;
  memset(&L, 0, sizeof(L));
  L.rows = rows;
  L.cols = cols;
  L.tall = rows > cols;
  L.m = std::min(rows, cols);
  L.n = std::max(rows, cols);
  L.short_m = dtype == MUON_DT_BF16 && L.m <= SHORT_ROWS;
  L.m_pad = L.short_m ? SHORT_ROWS : round_up(std::max<int64_t>(L.m, 1), PAD);
  L.n_pad = round_up(std::max<int64_t>(L.n, 1), PAD);
  L.x_pitch = !L.short_m && L.n_pad > X_PITCH_PAD_FROM ? L.n_pad + X_PITCH_PAD : L.n_pad;
  L.es = dtype == MUON_DT_F32 ? 4 : 2;
  L.batch = batch;
  L.parts = (L.m_pad / 64) * (L.n_pad / 64);
  L.gparts = L.short_m ? muon_short_parts(L.n_pad) : 0;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off = (size_t)round_up((int64_t)(off + bytes), 256);
    return o;
  };
  const size_t xs = (size_t)(batch * L.m_pad * L.x_pitch * L.es);
  const size_t as = (size_t)(batch * L.m_pad * L.m_pad * L.es);
  L.off_x0 = take(xs);
  L.off_x1 = take(xs);
  L.off_a = take(as);
  L.off_b = take(as);
  L.off_part = take((size_t)(batch * L.parts * 4));
  L.off_scale = take((size_t)(batch * 4));
  L.off_qtab = take((size_t)MUON_QTAB_BYTES);
  L.off_rows = take((size_t)(batch * L.n_pad * 4));  // per stored row (NorMuon)
  L.off_gpart = take((size_t)(batch * L.gparts * SHORT_PART_BYTES));
  L.total = off;
  return L;
}

// ---- static scratch of the allocation-free entry point -------------------------------
// One array per GPU (each device holds its own copy of a __device__ variable), held until
// the process ends. Host code must not use the array's name as a device address: its
// address on each device comes from hipGetSymbolAddress, looked up once per device with
// that device current (muon_amd_init, else the entry point's first call on the device).
static __device__ __align__(256) unsigned char scratch[MUON_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Address of the current device's scratch array (looked up on first use per device).
int current_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    muon_set_error("scratch: no usable current HIP device (%d)", dev);
    return MUON_ERR_DEVICE;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      muon_set_error("scratch: hipGetSymbolAddress failed on device %d: %s", dev,
                     hipGetErrorString(e));
      return MUON_ERR_DEVICE;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MUON_OK;
}
}  // namespace

static bool iter_dtype_ok(int dt) { return dt == MUON_DT_BF16 || dt == MUON_DT_F32; }
static bool io_dtype_ok(int dt) {
  return dt == MUON_DT_BF16 || dt == MUON_DT_F32 || dt == MUON_DT_F16;
}

extern "C" {

int muon_amd_abi_version(void) { return 5; }

const char* muon_amd_last_error(void) { return g_err; }

int muon_amd_init(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    muon_set_error("init: no HIP device");
    return MUON_ERR_DEVICE;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
    muon_set_error("init: hipGetDeviceProperties failed");
    return MUON_ERR_DEVICE;
  }
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    muon_set_error("init: device %d is %s; this library is built for gfx950 only", dev,
                   prop.gcnArchName);
    return MUON_ERR_DEVICE;
  }
  void* sp = nullptr;
  return current_scratch(&sp);  // this device's static scratch address, once
}

int muon_gram(const void* x, void* y, int dtype, int64_t batch, int64_t M, int64_t K,
              void* stream) {
  if (!iter_dtype_ok(dtype)) {
    muon_set_error("gram: dtype %d not supported (bf16 or fp32)", dtype);
    return MUON_ERR_DTYPE;
  }
  if (batch < 0 || M < 0 || K < 0) {
    muon_set_error("gram: negative extent");
    return MUON_ERR_SHAPE;
  }
  if (batch == 0 || M == 0) return MUON_OK;
  if (K == 0)  // an empty contraction: y = 0 (x is never read)
    return muon_launch_zero(y, batch * M * M * (dtype == MUON_DT_F32 ? 4 : 2),
                            (hipStream_t)stream);
  if (dtype == MUON_DT_BF16 && M % PAD == 0 && K % 64 == 0 && !((uintptr_t)x & 15) &&
      !((uintptr_t)y & 15))
    // whole 256-row tiles and 64-wide K-tiles: the iteration's SYRK reads the caller's
    // operands in place
    return muon_launch_gemm(dtype, MODE_SYRK, false, batch, M, M, K, x, K, M * K, x, K, M * K,
                            nullptr, 0, 0, y, M, M * M, nullptr, 0, 0, M, M, 1.0f, 0.0f,
                            nullptr, 0, (hipStream_t)stream);
  return muon_launch_gemm(dtype, MODE_SYRK, true, batch, M, M, K, x, K,
                          M * K, x, K, M * K, nullptr, 0, 0, y, M, M * M, nullptr, 0, 0, M, M,
                          1.0f, 0.0f, nullptr, 0, (hipStream_t)stream);
}

int64_t muon_orth_workspace_bytes(int dtype, int64_t batch, int64_t rows, int64_t cols) {
  if (!iter_dtype_ok(dtype) || batch < 0 || rows <= 0 || cols <= 0) return -1;
  return (int64_t)muon_orth_layout(dtype, batch, rows, cols).total;
}

int muon_orth_result(int dtype, int64_t batch, int64_t rows, int64_t cols, int steps,
                     int64_t* offset_bytes, int64_t* row_pitch, int64_t* matrix_stride,
                     int* transposed) {
  if (!iter_dtype_ok(dtype) || rows <= 0 || cols <= 0 || steps < 0) {
    muon_set_error("orth_result: bad arguments");
    return MUON_ERR_ARG;
  }
  OrthLayout L = muon_orth_layout(dtype, batch, rows, cols);
  // The iterate after `steps` GEMMs (or the scaled input for steps == 0) is in
  // X[steps % 2], in the wide orientation; a tall matrix's result is its transpose.
  *offset_bytes = (int64_t)((steps % 2) ? L.off_x1 : L.off_x0);
  *row_pitch = L.x_pitch;
  *matrix_stride = L.m_pad * L.x_pitch;
  *transposed = L.tall;
  return MUON_OK;
}

int muon_prepass(int ntensors, void* const* grads, void* const* bufs, int g_dtype,
                 int buf_dtype, int64_t nb, int64_t rows, int64_t cols, float momentum,
                 int nesterov, int maximize, int write_back_grad, void* ws, int ws_dtype,
                 int64_t ws_batch, void* stream) {
  if (!iter_dtype_ok(ws_dtype) || !io_dtype_ok(g_dtype) || (bufs && !io_dtype_ok(buf_dtype))) {
    muon_set_error("prepass: unsupported dtype (grad %d, buf %d, ws %d)", g_dtype, buf_dtype,
                   ws_dtype);
    return MUON_ERR_DTYPE;
  }
  if (ntensors < 0 || nb <= 0 || rows <= 0 || cols <= 0) {
    muon_set_error("prepass: bad extents (ntensors %d, nb %lld)", ntensors, (long long)nb);
    return MUON_ERR_SHAPE;
  }
  hipStream_t s = (hipStream_t)stream;
  if (!ws) {
    // momentum only: g' goes back into the grad tensors (write_back_grad) or stays
    // in the buffers (no Nesterov)
    if (!bufs) {
      muon_set_error("prepass: nothing to do without buffers or a workspace");
      return MUON_ERR_ARG;
    }
    for (int t0 = 0; t0 < ntensors; t0 += MUON_MAX_TENSORS) {
      const int cnt = std::min(MUON_MAX_TENSORS, ntensors - t0);
      int rc = muon_launch_momentum(cnt, grads + t0, bufs + t0, g_dtype, buf_dtype,
                                    nb * rows * cols, momentum, nesterov, maximize,
                                    write_back_grad, s);
      if (rc != MUON_OK) return rc;
    }
    return MUON_OK;
  }
  if ((int64_t)ntensors * nb > ws_batch) {
    muon_set_error("prepass: %lld matrices exceed the workspace capacity %lld",
                   (long long)ntensors * nb, (long long)ws_batch);
    return MUON_ERR_SHAPE;
  }
  OrthLayout L = muon_orth_layout(ws_dtype, ws_batch, rows, cols);
  const int ges = g_dtype == MUON_DT_F32 ? 4 : 2, bes = buf_dtype == MUON_DT_F32 ? 4 : 2;
  const double per_elem = ges + (bufs ? 2.0 * bes : 0.0) + L.es + (write_back_grad ? ges : 0);
  Timed timed(MUON_K_PREPASS, per_elem * (double)ntensors * nb * rows * cols, s);
  // X0 holds the wide iterate: the stored layout itself, or its transpose (tall)
  char* x0 = (char*)ws + L.off_x0;
  for (int t0 = 0; t0 < ntensors; t0 += MUON_MAX_TENSORS) {
    const int cnt = std::min(MUON_MAX_TENSORS, ntensors - t0);
    int rc = muon_launch_prepass(cnt, grads + t0, bufs ? bufs + t0 : nullptr, g_dtype,
                                 buf_dtype, nb, rows, cols, cols, rows * cols, momentum,
                                 nesterov, maximize, write_back_grad, L.tall ? 0 : 1,
                                 L.tall ? nullptr : x0, L.x_pitch, L.tall ? x0 : nullptr, L, ws,
                                 ws_dtype, (int64_t)t0 * nb, s);
    if (rc != MUON_OK) return rc;
  }
  return MUON_OK;
}

// The iteration; with `ap` (eligible shapes only, checked by the caller) the last X' is
// not stored but applied to the parameters in the GEMM's epilogue.
// The parameters of a fused apply: per tensor a bf16 pointer and lr * lr_ratio, nb matrices
// of prows x pcols each, wd and cautious. The last product's launches take them in chunks of
// at most MUON_APPLY_MAX tensors (the table a launch carries).
struct ApplyReq {
  void* const* params;
  const float* adj;
  int ntensors;
  int64_t nb, prows, pcols;
  float wd;
  int cautious;
};

// Run `launch(m0, cnt, table)` for consecutive chunks of the apply's tensors: matrices
// m0 .. m0 + cnt - 1 of the launch, the chunk's table.
extern "C++" template <typename F>
static int apply_chunks(const ApplyReq& r, F&& launch) {
  MuonApply ap;
  memset(&ap, 0, sizeof(ap));
  ap.nb = r.nb;
  ap.prows = r.prows;
  ap.pcols = r.pcols;
  ap.wd = r.wd;
  ap.cautious = r.cautious;
  for (int t0 = 0; t0 < r.ntensors; t0 += MUON_APPLY_MAX) {
    const int cnt = std::min(MUON_APPLY_MAX, r.ntensors - t0);
    for (int t = 0; t < cnt; ++t) {
      ap.params[t] = r.params[t0 + t];
      ap.adj[t] = r.adj[t0 + t];
    }
    const int rc = launch((int64_t)t0 * r.nb, (int64_t)cnt * r.nb, ap);
    if (rc != MUON_OK) return rc;
  }
  return MUON_OK;
}

static int orth_run_impl(void* ws, int ws_dtype, int64_t ws_batch, int64_t batch, int64_t rows,
                         int64_t cols, const double* coeffs, int steps, float prescale,
                         float eps, const ApplyReq* ap, void* stream) {
  if (!iter_dtype_ok(ws_dtype)) {
    muon_set_error("orth_run: unsupported dtype %d", ws_dtype);
    return MUON_ERR_DTYPE;
  }
  if (batch < 0 || batch > ws_batch || rows <= 0 || cols <= 0 || steps < 0 ||
      (steps > 0 && !coeffs)) {
    muon_set_error("orth_run: bad arguments (batch %lld of %lld, steps %d)", (long long)batch,
                   (long long)ws_batch, steps);
    return MUON_ERR_ARG;
  }
  if (batch == 0) return MUON_OK;
  OrthLayout L = muon_orth_layout(ws_dtype, ws_batch, rows, cols);
  hipStream_t s = (hipStream_t)stream;
  char* w = (char*)ws;
  int rc;
  {
    Timed t(MUON_K_OTHER, 0.0, s);
    rc = muon_launch_finalize(L, ws, batch, prescale, eps, s);
  }
  if (rc != MUON_OK) return rc;
  const float* scale = (const float*)(w + L.off_scale);
  char* X[2] = {w + L.off_x0, w + L.off_x1};
  char* A = w + L.off_a;
  char* B = w + L.off_b;
  const int64_t mp = L.m_pad, np = L.n_pad, xp = L.x_pitch;
  if (steps == 0) {
    Timed t(MUON_K_OTHER, 0.0, s);
    return muon_launch_scale(L, X[0], ws_dtype, batch, scale, s);
  }
  const double bm = (double)batch, md = (double)L.m, nd = (double)L.n;
  if (L.short_m) {
    // 64-row iterate: B X streams X once per iteration and leaves the next iteration's
    // Gram partials behind, so its launch also carries the next X X^T's work
    float* part = (float*)(w + L.off_gpart);
    {
      Timed t(MUON_K_SYRK_XX, bm * md * (md + 1) * nd, s);
      rc = muon_launch_short_gram(L, X[0], part, batch, s);
    }
    if (rc != MUON_OK) return rc;
    for (int it = 0; it < steps; ++it) {
      const float a = (float)coeffs[3 * it], b = (float)coeffs[3 * it + 1],
                  c = (float)coeffs[3 * it + 2];
      const int first = it == 0;
      const int more = it + 1 < steps;
      {
        Timed t(MUON_K_SYRK_AA, bm * md * (md + 1) * md, s);
        rc = muon_launch_short_poly(L, part, B, batch, c, b, scale, first, s);
      }
      if (rc != MUON_OK) return rc;
      if (ap && !more) {
        Timed t(MUON_K_GEMM_BX_APPLY, bm * 2.0 * md * md * nd, s);
        const int64_t xs = 64 * L.n_pad * 2, bs = 64 * 64 * 2;  // bytes per matrix
        rc = apply_chunks(*ap, [&](int64_t m0, int64_t cnt, const MuonApply& tab) {
          return muon_launch_short_bx_apply(L, X[it & 1] + m0 * xs, B + m0 * bs, cnt, 1.0f, a,
                                            scale + m0, first, tab, s);
        });
      } else {
        Timed t(MUON_K_GEMM_BX, bm * 2.0 * md * md * nd + (more ? bm * md * (md + 1) * nd : 0.0), s);
        rc = muon_launch_short_bx(L, X[it & 1], X[(it + 1) & 1], B, part, batch, 1.0f, a, scale,
                                  first, more, s);
      }
      if (rc != MUON_OK) return rc;
    }
    return MUON_OK;
  }
  // A A and B X contract over the m valid rows of X (the rest of the padding is zero):
  // the bf16 kernels take K in whole pairs of 64-wide K-tiles
  const int64_t kq = ws_dtype == MUON_DT_BF16 ? std::min(mp, round_up(L.m, 128)) : mp;
  for (int it = 0; it < steps; ++it) {
    const float a = (float)coeffs[3 * it], b = (float)coeffs[3 * it + 1],
                c = (float)coeffs[3 * it + 2];
    const bool first = it == 0;
    char* Xc = X[it & 1];
    char* Xn = X[(it + 1) & 1];
    // A = X X^T (the first iteration folds the Frobenius prescale s in as s^2)
    {
    Timed t(MUON_K_SYRK_XX, bm * md * (md + 1) * nd, s);
    rc = muon_launch_gemm(ws_dtype, MODE_SYRK, false, batch, mp, mp, np, Xc, xp, mp * xp, Xc, xp,
                          mp * xp, nullptr, 0, 0, A, mp, mp * mp, nullptr, 0, 0, L.m, L.m, 1.0f,
                          0.0f, scale, first ? 2 : 0, s);
    }
    if (rc != MUON_OK) return rc;
    // B = b*A + c*(A A)
    {
    Timed t(MUON_K_SYRK_AA, bm * md * (md + 1) * md, s);
    rc = muon_launch_gemm(ws_dtype, MODE_SYRK, false, batch, mp, mp, kq, A, mp, mp * mp, A, mp,
                          mp * mp, A, mp, mp * mp, B, mp, mp * mp, nullptr, 0, 0, L.m, L.m, c, b,
                          nullptr, 0, s);
    }
    if (rc != MUON_OK) return rc;
    // X' = a*X + B X into the other buffer (every tile reads whole columns of X); the
    // result stays in the wide orientation (readers of a tall result transpose on load)
    if (ap && it + 1 == steps) {
      Timed t(MUON_K_GEMM_BX_APPLY, bm * 2.0 * md * md * nd, s);
      rc = apply_chunks(*ap, [&](int64_t m0, int64_t cnt, const MuonApply& tab) {
        return muon_launch_gemm_apply(cnt, mp, np, kq, B + m0 * mp * mp * 2, mp, mp * mp,
                                      Xc + m0 * mp * xp * 2, xp, mp * xp, L.m, L.n, 1.0f, a,
                                      scale + m0, first ? 1 : 0, tab, L.tall, s);
      });
    } else {
    Timed t(MUON_K_GEMM_BX, bm * 2.0 * md * md * nd, s);
    rc = muon_launch_gemm(ws_dtype, MODE_GEMM, false, batch, mp, np, kq, B, mp, mp * mp, Xc, xp,
                          mp * xp, Xc, xp, mp * xp, Xn, xp, mp * xp, nullptr, 0, 0, L.m, L.n,
                          1.0f, a, scale, first ? 1 : 0, s);
    }
    if (rc != MUON_OK) return rc;
  }
  return MUON_OK;
}

int muon_orth_run(void* ws, int ws_dtype, int64_t ws_batch, int64_t batch, int64_t rows,
                  int64_t cols, const double* coeffs, int steps, float prescale, float eps,
                  void* stream) {
  return orth_run_impl(ws, ws_dtype, ws_batch, batch, rows, cols, coeffs, steps, prescale, eps,
                       nullptr, stream);
}

int muon_orth_run_apply(void* ws, int ws_dtype, int64_t ws_batch, int64_t batch, int64_t rows,
                        int64_t cols, const double* coeffs, int steps, float prescale,
                        float eps, int ntensors, void* const* params, int p_dtype, int64_t nb,
                        const float* adjusted_lrs, float wd, int cautious, void* stream) {
  bool fuse = ws_dtype == MUON_DT_BF16 && p_dtype == MUON_DT_BF16 && steps > 0 && rows > 0 &&
              cols > 0 && nb > 0 && ntensors > 0 && (int64_t)ntensors * nb == batch && batch <= ws_batch && params && adjusted_lrs &&
              cols % 8 == 0;
  if (fuse) {
    const OrthLayout L = muon_orth_layout(ws_dtype, ws_batch, rows, cols);
    const int64_t kq = std::min(L.m_pad, round_up(L.m, 128));
    // the tiled path from K = 768; iterates of at most 64 rows when the parameter is wide
    // (its rows are the iterate's)
    fuse = L.short_m ? !L.tall : kq >= 768;
    for (int t = 0; fuse && t < ntensors; ++t) fuse = params[t] && !((uintptr_t)params[t] & 15);
  }
  if (!fuse) {
    int rc = muon_orth_run(ws, ws_dtype, ws_batch, batch, rows, cols, coeffs, steps, prescale,
                           eps, stream);
    if (rc != MUON_OK) return rc;
    return muon_postpass(ntensors, params, p_dtype, nullptr, 0, ws, ws_dtype, ws_batch, steps,
                         nb, rows, cols, adjusted_lrs, nullptr, wd, cautious, stream);
  }
  const ApplyReq ap = {params, adjusted_lrs, ntensors, nb, rows, cols, wd, cautious};
  return orth_run_impl(ws, ws_dtype, ws_batch, batch, rows, cols, coeffs, steps, prescale, eps,
                       &ap, stream);
}

int muon_orth_extract(const void* ws, int ws_dtype, int64_t ws_batch, int64_t batch,
                      int64_t rows, int64_t cols, int steps, void* out, int out_dtype,
                      void* stream) {
  if (!iter_dtype_ok(ws_dtype) || !io_dtype_ok(out_dtype)) {
    muon_set_error("orth_extract: unsupported dtype");
    return MUON_ERR_DTYPE;
  }
  if (batch < 0 || batch > ws_batch) {
    muon_set_error("orth_extract: bad batch");
    return MUON_ERR_ARG;
  }
  if (batch == 0) return MUON_OK;
  int64_t off, pitch, mst;
  int trans;
  int rc = muon_orth_result(ws_dtype, ws_batch, rows, cols, steps, &off, &pitch, &mst, &trans);
  if (rc != MUON_OK) return rc;
  return muon_launch_extract((const char*)ws + off, ws_dtype, pitch, mst, trans, out, out_dtype,
                             rows, cols, batch, (hipStream_t)stream);
}

int muon_postpass(int ntensors, void* const* params, int p_dtype, const void* u, int u_dtype,
                  const void* ws, int ws_dtype, int64_t ws_batch, int steps, int64_t nb,
                  int64_t rows, int64_t cols, const float* adjusted_lrs, const float* u_scales,
                  float wd, int cautious, void* stream) {
  if (!io_dtype_ok(p_dtype)) {
    muon_set_error("postpass: unsupported param dtype %d", p_dtype);
    return MUON_ERR_DTYPE;
  }
  if (ntensors < 0 || nb <= 0 || rows <= 0 || cols <= 0) {
    muon_set_error("postpass: bad extents");
    return MUON_ERR_SHAPE;
  }
  const char* ubase;
  int udt, trans = 0;
  int64_t pitch, mst;
  if (u) {
    if (!io_dtype_ok(u_dtype)) {
      muon_set_error("postpass: unsupported update dtype %d", u_dtype);
      return MUON_ERR_DTYPE;
    }
    ubase = (const char*)u;
    udt = u_dtype;
    pitch = cols;
    mst = rows * cols;
  } else {
    if (!iter_dtype_ok(ws_dtype) || (int64_t)ntensors * nb > ws_batch) {
      muon_set_error("postpass: bad workspace arguments");
      return MUON_ERR_ARG;
    }
    int64_t off;
    int rc = muon_orth_result(ws_dtype, ws_batch, rows, cols, steps, &off, &pitch, &mst, &trans);
    if (rc != MUON_OK) return rc;
    ubase = (const char*)ws + off;
    udt = ws_dtype;
  }
  const int es = udt == MUON_DT_F32 ? 4 : 2;
  const int pes = p_dtype == MUON_DT_F32 ? 4 : 2;
  hipStream_t s = (hipStream_t)stream;
  Timed timed(MUON_K_POSTPASS, (es + 2.0 * pes) * (double)ntensors * nb * rows * cols, s);
  for (int t0 = 0; t0 < ntensors; t0 += MUON_MAX_TENSORS) {
    const int cnt = std::min(MUON_MAX_TENSORS, ntensors - t0);
    int rc = muon_launch_postpass(cnt, params + t0, adjusted_lrs + t0, p_dtype,
                                  ubase + (int64_t)t0 * nb * mst * es, udt, pitch, mst, trans,
                                  nullptr, 0, u_scales ? u_scales + t0 : nullptr, nb, rows, cols,
                                  wd, cautious, s);
    if (rc != MUON_OK) return rc;
  }
  return MUON_OK;
}

// NorMuon post-pass on an update U at ubase (pitch / matrix stride in elements; trans: a
// tall result in the workspace's wide layout), with the per-row statistics in ss (one
// float per stored row, ss_mst floats per matrix, at least chunk x nb matrices, reused by
// each chunk of MUON_MAX_TENSORS tensors in stream order). Every ss value the kernels
// read is written first, so ss needs no clearing.
static int normuon_postpass_on(int ntensors, void* const* params, int p_dtype,
                               void* const* variances, int v_dtype, const char* ubase, int udt,
                               int64_t pitch, int64_t mst, int trans, float* ss, int64_t ss_mst,
                               int64_t nb, int64_t rows, int64_t cols, const int64_t* starts,
                               int nb_split, const float* adjusted_lrs, const float* u_scales,
                               float wd, int cautious, double beta2, hipStream_t s) {
  const int es = udt == MUON_DT_F32 ? 4 : 2;
  const int pes = p_dtype == MUON_DT_F32 ? 4 : 2;
  const float w = (float)(1.0 - beta2);
  Timed timed(MUON_K_POSTPASS, (2.0 * es + 2.0 * pes) * (double)ntensors * nb * rows * cols, s);
  for (int t0 = 0; t0 < ntensors; t0 += MUON_MAX_TENSORS) {
    const int cnt = std::min(MUON_MAX_TENSORS, ntensors - t0);
    const char* uc = ubase + (int64_t)t0 * nb * mst * es;
    const float* usc = u_scales ? u_scales + t0 : nullptr;
    int rc = muon_launch_normuon_stats(cnt, variances + t0, v_dtype, uc, udt, pitch, mst, trans,
                                       nb, rows, cols, ss, ss_mst, starts, nb_split, usc, w, s);
    if (rc != MUON_OK) return rc;
    rc = muon_launch_postpass(cnt, params + t0, adjusted_lrs + t0, p_dtype, uc, udt, pitch, mst,
                              trans, ss, ss_mst, usc, nb, rows, cols, wd, cautious, s);
    if (rc != MUON_OK) return rc;
  }
  return MUON_OK;
}

// Row-block offsets of a NorMuon call: the whole matrix, or split_sizes summing to rows.
static int normuon_row_blocks(const char* who, const int64_t* split_sizes, int nsplits,
                              int64_t rows, int64_t* starts, int* nb_split) {
  *nb_split = 1;
  starts[0] = 0;
  starts[1] = rows;
  if (!split_sizes || nsplits <= 0) return MUON_OK;
  if (nsplits > MUON_MAX_SPLITS) {
    muon_set_error("%s: %d row blocks exceed the maximum %d", who, nsplits, MUON_MAX_SPLITS);
    return MUON_ERR_ARG;
  }
  int64_t acc = 0;
  for (int i = 0; i < nsplits; ++i) {
    if (split_sizes[i] <= 0) {
      muon_set_error("%s: row block %d has size %lld", who, i, (long long)split_sizes[i]);
      return MUON_ERR_SHAPE;
    }
    starts[i] = acc;
    acc += split_sizes[i];
  }
  if (acc != rows) {
    muon_set_error("%s: row blocks sum to %lld, not %lld rows", who, (long long)acc,
                   (long long)rows);
    return MUON_ERR_SHAPE;
  }
  starts[nsplits] = rows;
  *nb_split = nsplits;
  return MUON_OK;
}

int muon_normuon_postpass(int ntensors, void* const* params, int p_dtype,
                          void* const* variances, int v_dtype, const void* u, int u_dtype,
                          void* ws, int ws_dtype, int64_t ws_batch, int steps, int64_t nb,
                          int64_t rows, int64_t cols, const int64_t* split_sizes, int nsplits,
                          const float* adjusted_lrs, const float* u_scales, float wd,
                          int cautious, double beta2, void* stream) {
  if (!io_dtype_ok(p_dtype) || !io_dtype_ok(v_dtype)) {
    muon_set_error("normuon_postpass: unsupported param/variance dtype (%d, %d)", p_dtype,
                   v_dtype);
    return MUON_ERR_DTYPE;
  }
  if (ntensors < 0 || nb <= 0 || rows <= 0 || cols <= 0) {
    muon_set_error("normuon_postpass: bad extents");
    return MUON_ERR_SHAPE;
  }
  if (!ws || !iter_dtype_ok(ws_dtype) || (int64_t)ntensors * nb > ws_batch) {
    muon_set_error("normuon_postpass: a workspace for the %lld matrices is required",
                   (long long)ntensors * nb);
    return MUON_ERR_ARG;
  }
  int64_t starts[MUON_MAX_SPLITS + 1];
  int nb_split;
  int rc = normuon_row_blocks("normuon_postpass", split_sizes, nsplits, rows, starts, &nb_split);
  if (rc != MUON_OK) return rc;
  OrthLayout L = muon_orth_layout(ws_dtype, ws_batch, rows, cols);
  const char* ubase;
  int udt, trans = 0;
  int64_t pitch, mst;
  if (u) {
    if (!io_dtype_ok(u_dtype)) {
      muon_set_error("normuon_postpass: unsupported update dtype %d", u_dtype);
      return MUON_ERR_DTYPE;
    }
    ubase = (const char*)u;
    udt = u_dtype;
    pitch = cols;
    mst = rows * cols;
  } else {
    int64_t off;
    rc = muon_orth_result(ws_dtype, ws_batch, rows, cols, steps, &off, &pitch, &mst, &trans);
    if (rc != MUON_OK) return rc;
    ubase = (const char*)ws + off;
    udt = ws_dtype;
  }
  float* ss = (float*)((char*)ws + L.off_rows);  // stored rows <= n <= n_pad per matrix
  return normuon_postpass_on(ntensors, params, p_dtype, variances, v_dtype, ubase, udt, pitch,
                             mst, trans, ss, L.n_pad, nb, rows, cols, starts, nb_split,
                             adjusted_lrs, u_scales, wd, cautious, beta2, (hipStream_t)stream);
}

int muon_normuon_postpass_noalloc(int ntensors, void* const* params, int p_dtype,
                                  void* const* variances, int v_dtype, const void* u,
                                  int u_dtype, int64_t nb, int64_t rows, int64_t cols,
                                  const int64_t* split_sizes, int nsplits,
                                  const float* adjusted_lrs, const float* u_scales, float wd,
                                  int cautious, double beta2, void* stream) {
  if (!io_dtype_ok(p_dtype) || !io_dtype_ok(v_dtype) || !io_dtype_ok(u_dtype)) {
    muon_set_error("normuon_postpass_noalloc: unsupported dtype (param %d, variance %d, u %d)",
                   p_dtype, v_dtype, u_dtype);
    return MUON_ERR_DTYPE;
  }
  if (ntensors < 0 || nb <= 0 || rows <= 0 || cols <= 0) {
    muon_set_error("normuon_postpass_noalloc: bad extents");
    return MUON_ERR_SHAPE;
  }
  if (!u) {
    muon_set_error("normuon_postpass_noalloc: the update u is required");
    return MUON_ERR_ARG;
  }
  // one float per stored row of each matrix of a chunk of MUON_MAX_TENSORS tensors
  const int64_t need = (int64_t)std::min(ntensors, MUON_MAX_TENSORS) * nb * rows * 4;
  if (need > MUON_NOALLOC_SCRATCH_BYTES) {
    muon_set_error("normuon_postpass_noalloc: %lld bytes of row statistics exceed the %d-byte "
                   "scratch (at most %d tensors per chunk x nb x rows x 4 B)",
                   (long long)need, MUON_NOALLOC_SCRATCH_BYTES, MUON_MAX_TENSORS);
    return MUON_ERR_SHAPE;
  }
  int64_t starts[MUON_MAX_SPLITS + 1];
  int nb_split;
  int rc = normuon_row_blocks("normuon_postpass_noalloc", split_sizes, nsplits, rows, starts,
                              &nb_split);
  if (rc != MUON_OK) return rc;
  if (ntensors == 0) return MUON_OK;
  void* sp = nullptr;
  rc = current_scratch(&sp);
  if (rc != MUON_OK) return rc;
  return normuon_postpass_on(ntensors, params, p_dtype, variances, v_dtype, (const char*)u,
                             u_dtype, cols, rows * cols, 0, (float*)sp, rows, nb, rows, cols,
                             starts, nb_split, adjusted_lrs, u_scales, wd, cautious, beta2,
                             (hipStream_t)stream);
}

int muon_lp_prepass(int ntensors, void* const* grads, int g_dtype, void* const* codes,
                    void* const* scales, const float* qmap, int qformat, int64_t block,
                    int64_t nb, int64_t rows, int64_t cols, float momentum, int nesterov,
                    int maximize, void* ws, int ws_dtype, int64_t ws_batch, void* stream) {
  if (ws_dtype != MUON_DT_BF16 || !io_dtype_ok(g_dtype)) {
    muon_set_error("lp_prepass: workspace must be bf16 and grads bf16/fp16/fp32");
    return MUON_ERR_DTYPE;
  }
  if (ntensors < 0 || nb <= 0 || rows <= 0 || cols <= 0 || (int64_t)ntensors * nb > ws_batch) {
    muon_set_error("lp_prepass: bad extents");
    return MUON_ERR_SHAPE;
  }
  int rc = muon_check_lp_format(qformat, nb * rows * cols, block);
  if (rc != MUON_OK) return rc;
  if (qformat != MUON_Q_FP8 && !qmap) {
    muon_set_error("lp_prepass: missing qmap");
    return MUON_ERR_ARG;
  }
  OrthLayout L = muon_orth_layout(ws_dtype, ws_batch, rows, cols);
  hipStream_t s = (hipStream_t)stream;
  char* w = (char*)ws;
  {
    // one pass writing X0 and the norm partials directly, when the shape allows it
    const double ges = g_dtype == MUON_DT_F32 ? 4.0 : 2.0;
    const double code_b = qformat == MUON_Q_4BIT ? 0.5 : 1.0;
    const double per_elem = ges + 2.0 * code_b + 8.0 / (double)block + 2.0;
    Timed timed(MUON_K_LP_PREPASS, per_elem * (double)ntensors * nb * rows * cols, s);
    rc = MUON_OK;
    for (int t0 = 0; t0 < ntensors && rc == MUON_OK; t0 += MUON_MAX_TENSORS) {
      const int cnt = std::min(MUON_MAX_TENSORS, ntensors - t0);
      rc = muon_launch_lp_prepass_tiled(cnt, grads + t0, g_dtype, codes + t0, scales + t0, qmap,
                                        qformat, block, nb, rows, cols, momentum, nesterov,
                                        maximize, L, ws, (int64_t)t0 * nb, s);
      if (rc != MUON_OK && t0 > 0) return rc;  // shape checks are the same for every chunk
    }
    if (rc == MUON_OK) return MUON_OK;
    if (rc != MUON_ERR_SHAPE) return rc;
  }
  // general path: the stored-layout X goes to X0 (wide) or, for a tall matrix, to X1
  // (n_pad x m_pad) from where the second pass below transposes it into X0
  char* direct = w + (L.tall ? L.off_x1 : L.off_x0);
  const int64_t d_pitch = L.tall ? L.m_pad : L.x_pitch;
  const int64_t mst = L.m_pad * (L.tall ? L.n_pad : L.x_pitch);
  {
  const double ges = g_dtype == MUON_DT_F32 ? 4.0 : 2.0;
  const double code_b = qformat == MUON_Q_4BIT ? 0.5 : 1.0;
  const double per_elem = ges + 2.0 * code_b + 8.0 / (double)block + 2.0;
  Timed timed(MUON_K_LP_PREPASS, per_elem * (double)ntensors * nb * rows * cols, s);
  for (int t0 = 0; t0 < ntensors; t0 += MUON_MAX_TENSORS) {
    const int cnt = std::min(MUON_MAX_TENSORS, ntensors - t0);
    rc = muon_launch_lp_prepass(cnt, grads + t0, g_dtype, codes + t0, scales + t0, qmap,
                                qformat, block, nb, rows, cols, momentum, nesterov, maximize,
                                direct + (int64_t)t0 * nb * mst * L.es, d_pitch, mst, s);
    if (rc != MUON_OK) return rc;
  }
  }
  Timed timed_t(MUON_K_OTHER, 0.0, s);
  // Norm partials (and, tall, the transpose into X0) from the stored-layout X just
  // written: a plain (no momentum) prepass reading the valid region of the workspace;
  // for a wide matrix it rewrites only the padding of X0 in place.
  const int64_t nmat = (int64_t)ntensors * nb;
  char* x0 = w + L.off_x0;
  for (int64_t m0 = 0; m0 < nmat; m0 += MUON_MAX_TENSORS) {
    const int cnt = (int)std::min<int64_t>(MUON_MAX_TENSORS, nmat - m0);
    void* srcs[MUON_MAX_TENSORS];
    for (int i = 0; i < cnt; ++i) srcs[i] = direct + (m0 + i) * mst * L.es;
    rc = muon_launch_prepass(cnt, srcs, nullptr, MUON_DT_BF16, MUON_DT_BF16, 1, rows, cols,
                             d_pitch, mst, 0.0f, 0, 0, 0, L.tall ? 0 : 2, L.tall ? nullptr : x0,
                             L.x_pitch, L.tall ? x0 : nullptr, L, ws, ws_dtype, m0, s);
    if (rc != MUON_OK) return rc;
  }
  return MUON_OK;
}

int muon_timing_enable(int on) {
  std::lock_guard<std::mutex> lock(g_timing.mu);
  for (auto& r : g_timing.recs) {
    g_timing.free_events.push_back(r.ev0);
    g_timing.free_events.push_back(r.ev1);
  }
  g_timing.recs.clear();
  g_timing.on = on != 0;
  return MUON_OK;
}

int muon_timing_read(double* ms, int64_t* launches, double* work) {
  std::lock_guard<std::mutex> lock(g_timing.mu);
  for (int k = 0; k < MUON_K_COUNT; ++k) {
    ms[k] = 0.0;
    launches[k] = 0;
    work[k] = 0.0;
  }
  for (auto& r : g_timing.recs) {
    if (hipEventSynchronize(r.ev1) != hipSuccess) {
      muon_set_error("timing: hipEventSynchronize failed");
      return MUON_ERR_DEVICE;
    }
    float t = 0.0f;
    if (hipEventElapsedTime(&t, r.ev0, r.ev1) != hipSuccess) {
      muon_set_error("timing: hipEventElapsedTime failed");
      return MUON_ERR_DEVICE;
    }
    ms[r.kind] += t;
    launches[r.kind] += 1;
    work[r.kind] += r.work;
  }
  return MUON_OK;
}

}  // extern "C"
