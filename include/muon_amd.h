/*
 * muon_amd.h — C ABI of the MI355X-native Muon optimizer step (libmuon_amd.so).
 *
 * The library replaces the device-side work of muonium's `Muon.step()` hot path
 * (tonyf/dtensor-muon, package `muonium`). Every entry point takes plain device
 * pointers, sizes and a hipStream_t passed as `void*`; nothing allocates, frees or
 * synchronizes: the caller (the Python host package, or any FFI user) owns every
 * buffer. All launches are asynchronous on the given stream.
 *
 * Return value: MUON_OK (0) or one of the MUON_ERR_* codes; the text of the last
 * error on the calling thread is available from muon_amd_last_error().
 *
 * Shapes. A "tensor" handed to the step entry points is `nb` stored matrices of
 * `rows x cols`, contiguous (row-major, matrix after matrix): the transformed
 * gradient shape of muonium's `_init_muon_group` (optim.py:395-401). The
 * orthogonalization runs on the wide orientation X (m x n, m = min(rows, cols)),
 * transposing tall matrices as pe_loop/ns_loop do (polar_express.py:52-54,
 * newton_schulz.py:41-43).
 *
 * Workspace. The iteration works in a caller-allocated workspace whose size comes
 * from muon_orth_workspace_bytes(); the same (dtype, batch, rows, cols) quadruple
 * must be passed to every call that touches it. Its contents need no
 * initialization: every call rewrites what it reads later.
 */
#ifndef MUON_AMD_H
#define MUON_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
#define MUON_DT_F32 0
#define MUON_DT_BF16 1
#define MUON_DT_F16 2

/* status codes */
#define MUON_OK 0
#define MUON_ERR_SHAPE 1
#define MUON_ERR_DTYPE 2
#define MUON_ERR_ALIGN 3
#define MUON_ERR_LAUNCH 4
#define MUON_ERR_ARG 5
#define MUON_ERR_DEVICE 6

/* quantized-state formats (muon_lp_*) */
#define MUON_Q_8BIT 8
#define MUON_Q_4BIT 4
#define MUON_Q_FP8 0

/* Maximum tensors per multi-tensor launch; larger lists are chunked internally. */
#define MUON_MAX_TENSORS 32

/* ABI version of this header (bumped on any signature change): 5. */
int muon_amd_abi_version(void);

/* Text of the last error reported on the calling thread ("" if none). */
const char* muon_amd_last_error(void);

/* Checks that the current HIP device is a gfx950 (MI355X) and that the code
 * objects load. No counterpart in the reference (Triton JIT-compiles on first use). */
int muon_amd_init(void);

/* ---- Gram kernel -------------------------------------------------------------
 * y[b] = x[b] @ x[b]^T for b < batch; x is (batch, M, K) contiguous, y is
 * (batch, M, M) contiguous, both `dtype` (bf16 or fp32), fp32 accumulation, output
 * exactly symmetric (upper-triangle tiles computed, lower mirrored).
 * Replaces: muonium/kernels/gram.py:109-152 `gram_(d_in, d_out)` (the Triton
 * `gram_nd`, gram.py:21-106). The contract checks of gram.py:114-130 live in the
 * Python wrapper, which raises the reference's AssertionError. */
int muon_gram(const void* x, void* y, int dtype, int64_t batch, int64_t M, int64_t K,
              void* stream);

/* ---- Orthogonalization workspace ---------------------------------------------- */
int64_t muon_orth_workspace_bytes(int dtype, int64_t batch, int64_t rows, int64_t cols);

/* Location of the orthogonalized result U (rows x cols) inside the workspace after
 * muon_orth_run(..., steps, ...): byte offset of matrix 0, row pitch and matrix stride
 * in elements of the wide iterate (m x n). *transposed is 1 for a tall matrix
 * (rows > cols), whose U(r, c) is then at row c, column r of that iterate. */
int muon_orth_result(int dtype, int64_t batch, int64_t rows, int64_t cols, int steps,
                     int64_t* offset_bytes, int64_t* row_pitch, int64_t* matrix_stride,
                     int* transposed);

/* ---- Pre-pass: momentum / Nesterov -> bf16 X (both layouts) + norm partials ------
 * For tensor t < ntensors (each nb matrices of rows x cols, elementwise):
 *   g  = maximize ? -grad : grad                                  (muon.py:41-42)
 *   buf' = buf * momentum + g        (fp32 math, stored in buf's dtype) (muon.py:49-50)
 *   g' = nesterov ? g + buf' * momentum : buf'                     (muon.py:53-56)
 *   X[t*nb + i] = cast(g', iteration dtype)                        (orthogonalize.py:101-102)
 * With bufs == NULL the momentum step is skipped (g' = g): the zeropower cast path.
 * write_back_grad stores g' into grad (the foreach driver's in-place Nesterov
 * update of the gradient list, muon.py:117-118). The sum of squares of the cast
 * values is accumulated per matrix for the Frobenius prescale (polar_express.py:89).
 * With ws == NULL only the momentum step runs (buf' in place, g' into grad when
 * write_back_grad): for a caller-supplied orthogonalizer that needs g' as a tensor.
 * Replaces: muonium/optim/algorithms/muon.py:39-56 and :108-119, plus the
 * `torch.stack(...).bfloat16()` of orthogonalize.py:159-161. */
int muon_prepass(int ntensors, void* const* grads, void* const* bufs, int g_dtype,
                 int buf_dtype, int64_t nb, int64_t rows, int64_t cols, float momentum,
                 int nesterov, int maximize, int write_back_grad, void* ws, int ws_dtype,
                 int64_t ws_batch, void* stream);

/* ---- Iteration: Newton-Schulz / Polar Express on the workspace -----------------
 * For the first `batch` matrices of the workspace: X /= (||X||_F * prescale + eps),
 * then for each of `steps` coefficient triples (a, b, c) (coeffs is steps*3 doubles):
 *   A = X X^T;  B = b*A + c*A A;  X = a*X + B X
 * in bf16 (fp32 accumulation) or fp32 according to ws_dtype.
 * Replaces: muonium/orthogonalize/polar_express.py:71-115 `pe_loop_triton`
 * (prescale 1.02) and newton_schulz.py:60-107 `ns_loop_triton` (prescale 1.0). */
int muon_orth_run(void* ws, int ws_dtype, int64_t ws_batch, int64_t batch, int64_t rows,
                  int64_t cols, const double* coeffs, int steps, float prescale, float eps,
                  void* stream);

/* muon_orth_run followed by muon_postpass of its result (u = NULL, the same arguments),
 * with the post-pass fused into the last iteration's X = a*X + B X where the shapes allow
 * (bf16 workspace and parameters; on the iterate's short side either at least 768 valid
 * rows after padding to 128, or at most 64 rows with the parameter stored wide;
 * ntensors * nb == batch, parameter rows a multiple of 8 elements in the stored
 * orientation, 16-byte aligned parameters; the last product launches once per 128 tensors):
 * each bf16 element of the last X' is applied to its parameter element
 * (cautious weight decay and the shape-scaled step, exactly as muon_postpass) and X' is
 * not stored, so the workspace does not hold U afterwards. Otherwise the two calls run
 * one after the other. Replaces the orthogonalize-then-apply sequence of
 * muonium/optim/algorithms/muon.py:101-140 (foreach_update) and :58-77 (update). */
int muon_orth_run_apply(void* ws, int ws_dtype, int64_t ws_batch, int64_t batch, int64_t rows,
                        int64_t cols, const double* coeffs, int steps, float prescale,
                        float eps, int ntensors, void* const* params, int p_dtype, int64_t nb,
                        const float* adjusted_lrs, float wd, int cautious, void* stream);

/* Copy U (first `batch` matrices, stored layout) out of the workspace into a
 * contiguous (batch, rows, cols) tensor of out_dtype. Replaces the return/unbind of
 * orthogonalize.py:101-102, :159-162. */
int muon_orth_extract(const void* ws, int ws_dtype, int64_t ws_batch, int64_t batch,
                      int64_t rows, int64_t cols, int steps, void* out, int out_dtype,
                      void* stream);

/* ---- Post-pass: cautious weight decay + shape-scaled apply ----------------------
 * For tensor t, element e (u from the workspace when u == NULL, else from the
 * contiguous tensor u of u_dtype holding ntensors*nb*rows*cols elements):
 *   v = wd != 0 ? (cautious ? u + (wd*p)*(u*p > 0) : u + wd*p) : u    (muon.py:62-69)
 *   p = round(p - adjusted_lrs[t] * v)                                 (muon.py:71-77)
 * in fp32 with no contraction; when wd == 0 the product adjusted_lr*u keeps u's dtype
 * (eager type promotion of a 0-dim fp32 tensor times a bf16 tensor: adjusted_lr is cast
 * to u's dtype, the product rounded to it). With u_scales (one per tensor, NULL for none)
 * u is first replaced by u * u_scales[t] rounded to u's dtype: the split_sizes row-block
 * rescale `u * scales[i]` of base.py:98 applied to a block handed over as its own tensor.
 * Replaces: muonium/optim/algorithms/muon.py:59-77 and :121-140. */
int muon_postpass(int ntensors, void* const* params, int p_dtype, const void* u, int u_dtype,
                  const void* ws, int ws_dtype, int64_t ws_batch, int steps, int64_t nb,
                  int64_t rows, int64_t cols, const float* adjusted_lrs, const float* u_scales,
                  float wd, int cautious, void* stream);

/* ---- NorMuon post-pass ------------------------------------------------------------
 * muon_postpass for the "normuon" algorithm: the update U (from the workspace when
 * u == NULL, else the contiguous tensor u of u_dtype, as in muon_postpass) is first
 * normalized per stored row (normuon.py:16-55), per row block when split_sizes is given
 * (nsplits blocks of stored rows summing to `rows`, at most MUON_MAX_SPLITS):
 *   r_i   = mean_j U(i, j)^2                          (fp32)
 *   v_i'  = lerp(v_i, r_i, 1 - beta2)                 (torch.lerp; v = variances[t], one
 *                                                      value per stored row, v_dtype)
 *   U'    = U(i, :) / (sqrt(v_i') + 1e-8)
 *   U''   = U' * ||U||_F / max(||U'||_F, 1e-8)        (norms per matrix and row block)
 * and v_i' is stored into the variance state; then cautious weight decay and the apply
 * run on U'' in fp32 exactly as muon_postpass. With u_scales (one per tensor, NULL for
 * none) U is first replaced by U * u_scales[t] rounded to U's dtype, before the statistics:
 * the split_sizes row-block rescale `u * scales[i]` of base.py:98, for a row block handed
 * over as its own tensor. The workspace (same quadruple as the other calls; required also
 * with an explicit u) holds the per-row scratch.
 * Replaces: muonium/optim/algorithms/normuon.py:16-55 (_normuon_normalize), :118-134
 * (NorMuon.update after the orthogonalization) and :182-203 (foreach_update). */
#define MUON_MAX_SPLITS 16
int muon_normuon_postpass(int ntensors, void* const* params, int p_dtype,
                          void* const* variances, int v_dtype, const void* u, int u_dtype,
                          void* ws, int ws_dtype, int64_t ws_batch, int steps, int64_t nb,
                          int64_t rows, int64_t cols, const int64_t* split_sizes, int nsplits,
                          const float* adjusted_lrs, const float* u_scales, float wd,
                          int cautious, double beta2, void* stream);

/* ---- Allocation-free NorMuon post-pass ------------------------------------------------
 * No counterpart in the reference: for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving or training loops, harnesses that forbid
 * hipMalloc). Same arithmetic and results as muon_normuon_postpass with an explicit update
 * u (required here) and no workspace: the per-row statistics live in a static device array
 * of MUON_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends. A call needs
 * min(ntensors, MUON_MAX_TENSORS) * nb * rows * 4 bytes of it and is refused with
 * MUON_ERR_SHAPE beyond (rows up to 131072 for 32 single-matrix tensors). Nothing is
 * allocated and nothing needs clearing between calls (every value read is written first
 * by the same call). All calls on one GPU share its array: calls that overlap in time on
 * one GPU (on different streams) race and must be serialized by the caller. */
#define MUON_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
int muon_normuon_postpass_noalloc(int ntensors, void* const* params, int p_dtype,
                                  void* const* variances, int v_dtype, const void* u,
                                  int u_dtype, int64_t nb, int64_t rows, int64_t cols,
                                  const int64_t* split_sizes, int nsplits,
                                  const float* adjusted_lrs, const float* u_scales, float wd,
                                  int cautious, double beta2, void* stream);

/* ---- Quantized momentum (MuonLP) -------------------------------------------------
 * State of one tensor of `numel` values: codes (uint8; numel bytes for 8-bit and
 * fp8, numel/2 for 4-bit with element 2i in the high nibble) and one fp32 scale per
 * block of `block` consecutive values. 8/4-bit codes index the 256/16-entry fp32
 * `qmap`; value = qmap[code] * scale. fp8 codes are float8_e4m3fn; value =
 * float(code) * scale. Quantizing a block: absmax = max(|x|) clipped at 1e-12;
 * scale = absmax (fp8: absmax / 448); y = x / scale (IEEE division); 8/4-bit code =
 * largest i with qmap[i] <= y, then i+1 if y - qmap[i] >= (qmap[i+1]-qmap[i])*0.5.
 * Replaces the torchao 0.17.0 OptimState8bit / OptimState4bit / OptimStateFp8
 * arithmetic reached from muonium/optim/optim_lp.py:118-133 via muon.py:45,50. */
int muon_lp_quantize(const float* src, void* codes, float* scales, const float* qmap,
                     int qformat, int64_t numel, int64_t block, void* stream);
int muon_lp_dequantize(const void* codes, const float* scales, const float* qmap,
                       int qformat, int64_t numel, int64_t block, float* dst, void* stream);

/* Fused dequant -> momentum -> requant pre-pass for quantized momentum buffers:
 * as muon_prepass, with buf = dequant(codes, scales) and buf' requantized in
 * place; Nesterov uses the unquantized buf' (muon.py:49-56). */
int muon_lp_prepass(int ntensors, void* const* grads, int g_dtype, void* const* codes,
                    void* const* scales, const float* qmap, int qformat, int64_t block,
                    int64_t nb, int64_t rows, int64_t cols, float momentum, int nesterov,
                    int maximize, void* ws, int ws_dtype, int64_t ws_batch, void* stream);

/* ---- Kernel timing (measurement support) ------------------------------------------
 * No counterpart in the reference. While enabled, every kernel the step entry points
 * launch is bracketed by hipEvents on its own stream; muon_timing_read() waits for
 * the last event and returns, per kernel kind (MUON_K_*), the summed duration in ms,
 * the launch count and the summed algorithmic work (FLOP for the products, bytes for
 * the elementwise passes, as documented per kind). Capacity: 65536 launches. */
#define MUON_K_SYRK_XX 0   /* A = X X^T: m(m+1) n FLOP per matrix (upper triangle) */
#define MUON_K_SYRK_AA 1   /* B = b A + c A A: m(m+1) m FLOP per matrix */
#define MUON_K_GEMM_BX 2   /* X = a X + B X: 2 m^2 n FLOP per matrix */
#define MUON_K_PREPASS 3   /* bytes: grad + 2 * buffer + one bf16 X per element */
#define MUON_K_POSTPASS 4  /* bytes: u + 2 * param per element */
#define MUON_K_LP_PREPASS 5 /* bytes: grad + 2 * codes + 2 * scales + one bf16 X */
#define MUON_K_OTHER 6     /* finalize / transpose / scale / extract (no work counted) */
#define MUON_K_GEMM_BX_APPLY 7 /* the last X = a X + B X with the post-pass fused
                                  (muon_orth_run_apply): 2 m^2 n FLOP per matrix; the apply
                                  moves 2 * param bytes per element besides */
#define MUON_K_COUNT 8
int muon_timing_enable(int on);
int muon_timing_read(double* ms, int64_t* launches, double* work);

#ifdef __cplusplus
}
#endif

#endif /* MUON_AMD_H */
