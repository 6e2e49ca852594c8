/*
 * fused_layernorm.h -- C ABI of the MI355X (gfx950) fused normalization library (libfln.so).
 *
 * Plain pointers and sizes only: no torch types cross this boundary.  Every tensor is a dense
 * row-major [rows, cols] array (row stride == cols); per-column parameters are [cols]; per-row
 * statistics are fp32 [rows].  `stream` is a hipStream_t (NULL = the null stream).  All calls
 * are asynchronous with respect to the host and return 0 on success, FLN_ERR_INVALID for bad
 * arguments (detected before anything is launched), or a nonzero hipError_t value from the
 * launch.  fln_error_string() turns a code into text.
 *
 * Each entry point names the reference interface it replaces (paths relative to the
 * JonSnow1807/Fused-LayerNorm-CUDA-Operator tree).
 */
#ifndef FUSED_LAYERNORM_H
#define FUSED_LAYERNORM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type codes. */
#define FLN_F32 0
#define FLN_BF16 1
#define FLN_F16 2
#define FLN_F64 3 /* forward only (the reference dispatches fp32/fp64 in its built kernels) */
#define FLN_F8E4M3FN 4 /* OCP fp8 e4m3fn, output of fln_layernorm_fp8_forward only */

/* GELU flavours for fln_layernorm_gelu. */
#define FLN_GELU_NONE 0
#define FLN_GELU_ERF 1  /* 0.5 v (1 + erf(v / sqrt 2)) -- torch approximate='none' */
/* 0.5 v (1 + tanh(sqrt(2/pi)(v + 0.044715 v^3))) -- the reference's gelu() */
#define FLN_GELU_TANH 2

#define FLN_OK 0
#define FLN_ERR_INVALID 1 /* == hipErrorInvalidValue */
/* fln_layernorm_backward_noalloc only: the call needs more workspace than its fixed per-device
 * scratch holds (negative, so it never collides with a hipError_t value). */
#define FLN_ERR_TOO_LARGE (-2)

/* y = LN(x) [* gamma + beta].  gamma and beta may each be NULL (then that term is skipped).
 * Replaces `layernorm_cuda` (csrc/layernorm_cuda_kernel.cu:152-178) behind
 * `layernorm` (csrc/bindings.cpp:19-28). */
int fln_layernorm(const void* x, const void* gamma, const void* beta, void* y, int64_t rows,
                  int64_t cols, int dtype, float eps, void* stream);

/* y = GELU(LN(x) [* gamma + beta]), gelu_mode = FLN_GELU_ERF or FLN_GELU_TANH.
 * Replaces `layernorm_gelu_cuda` (csrc/layernorm_cuda_kernel.cu:180-206) behind
 * `layernorm_gelu` (csrc/bindings.cpp:30-39). */
int fln_layernorm_gelu(const void* x, const void* gamma, const void* beta, void* y, int64_t rows,
                       int64_t cols, int dtype, float eps, int gelu_mode, void* stream);

/* LayerNorm + GELU forward that also writes the row statistics the backward needs (mean and
 * rstd of x, fp32; either may be NULL).  The reference's layernorm_gelu_cuda
 * (csrc/layernorm_cuda_kernel.cu:180-206) returns only y; this is its training form. */
int fln_layernorm_gelu_forward(const void* x, const void* gamma, const void* beta, void* y,
                               float* mean, float* rstd, int64_t rows, int64_t cols, int dtype,
                               float eps, int gelu_mode, void* stream);

/* Training forward: y plus fp32 mean[rows] and rstd[rows] (either may be NULL).
 * Replaces `layernorm_forward_cuda` (csrc/layernorm.h:15-22, csrc/layernorm_cuda.cpp:14-21) and
 * `layernorm_forward_cuda_optimized` (csrc/layernorm_cuda_kernel_optimized.cu:171-212), called
 * from `layernorm_forward` (csrc/layernorm_cuda.cpp:49-94). */
int fln_layernorm_forward(const void* x, const void* gamma, const void* beta, void* y, float* mean,
                          float* rstd, int64_t rows, int64_t cols, int dtype, float eps,
                          void* stream);

/* Workspace (bytes) the backward entry points use: the two-stage column reduction's partial
 * rows and, for rows wider than the register and LDS kernels hold (16-bit or fp32 rows of more
 * than 16384 columns, long rows on the unaligned path), per-row statistics.  Required whenever
 * dgamma / dbeta is requested; passing it for dx alone lets such rows take the two-pass
 * kernels instead of the slower looped one. */
size_t fln_backward_workspace_bytes(int64_t rows, int64_t cols, int dtype);

/* LayerNorm backward.  dx = rstd (g - mean(g) - xhat mean(g xhat)), g = dy * gamma,
 * xhat = (x - mean) rstd; dgamma = sum_rows dy xhat; dbeta = sum_rows dy.
 * dx, dgamma, dbeta may each be NULL (the reference's output_mask).  dres, if not NULL, is an
 * incoming gradient [rows, cols] added into dx (backward of a fused residual add).
 * dparam_dtype is the element type of dgamma/dbeta (FLN_F32 or `dtype`).  workspace must hold
 * fln_backward_workspace_bytes(rows, cols, dtype) bytes whenever dgamma or dbeta is requested.
 * Replaces `layernorm_backward_cuda` (csrc/layernorm.h:24-32, csrc/layernorm_cuda.cpp:33-41),
 * declared but never defined in the reference; called from `layernorm_backward`
 * (csrc/layernorm_cuda.cpp:97-141). */
int fln_layernorm_backward(const void* dy, const void* x, const float* mean, const float* rstd,
                           const void* gamma, const void* dres, void* dx, void* dgamma,
                           void* dbeta, int64_t rows, int64_t cols, int dtype, int dparam_dtype,
                           void* workspace, size_t workspace_bytes, void* stream);

/* fln_layernorm_backward without a workspace argument, for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  The workspace is a fixed 32 MiB scratch array in device memory
 * (a __device__ array of the backward's code object: held on every device where libfln's
 * backward kernels are loaded, until the process ends, whether or not this entry point is
 * called); nothing is allocated per call.  Enough for the register and LDS kernels' one
 * partial row per CU up to 16384 columns (8 MiB at 8192 x 4096); a call that needs more
 * returns FLN_ERR_TOO_LARGE before
 * anything is launched.  Every call on a device shares that device's scratch: calls that
 * overlap on one device (other streams, other host threads) race, so serialize them.  The
 * stream must belong to the current device (FLN_ERR_INVALID otherwise).  Results equal
 * fln_layernorm_backward's bit for bit. */
int fln_layernorm_backward_noalloc(const void* dy, const void* x, const float* mean,
                                   const float* rstd, const void* gamma, const void* dres,
                                   void* dx, void* dgamma, void* dbeta, int64_t rows, int64_t cols,
                                   int dtype, int dparam_dtype, void* stream);

/* Backward of y = GELU(LayerNorm(x) * gamma + beta) (gelu_mode FLN_GELU_ERF or _TANH, as in
 * the forward): the GELU input is recomputed from mean / rstd / gamma / beta, then
 * dx, dgamma = sum dy GELU'(a) xhat, dbeta = sum dy GELU'(a) as fln_layernorm_backward (same
 * workspace, same NULL rules).  No counterpart in the reference (it has no backward for its
 * fused LayerNorm + GELU). */
int fln_layernorm_gelu_backward(const void* dy, const void* x, const float* mean,
                                const float* rstd, const void* gamma, const void* beta, void* dx,
                                void* dgamma, void* dbeta, int64_t rows, int64_t cols, int dtype,
                                int dparam_dtype, int gelu_mode, void* workspace,
                                size_t workspace_bytes, void* stream);

/* RMSNorm forward: y = x rstd [* weight], rstd = 1/sqrt(mean(x^2) + eps); rstd[rows] optional.
 * No counterpart in the reference (new capability on the same path). */
int fln_rmsnorm_forward(const void* x, const void* weight, void* y, float* rstd, int64_t rows,
                        int64_t cols, int dtype, float eps, void* stream);

/* RMSNorm backward: dx = rstd (g - xhat mean(g xhat)), g = dy * weight, xhat = x rstd;
 * dweight = sum_rows dy xhat.  Same optional-output and workspace rules as
 * fln_layernorm_backward.  No counterpart in the reference. */
int fln_rmsnorm_backward(const void* dy, const void* x, const float* rstd, const void* weight,
                         const void* dres, void* dx, void* dweight, int64_t rows, int64_t cols,
                         int dtype, int dweight_dtype, void* workspace, size_t workspace_bytes,
                         void* stream);

/* Residual add + LayerNorm: h = x + residual (rounded to dtype), y = LN(h) [* gamma + beta];
 * statistics are taken over the rounded h.  h, mean, rstd may be NULL.
 * No counterpart in the reference. */
int fln_add_layernorm_forward(const void* x, const void* residual, const void* gamma,
                              const void* beta, void* h, void* y, float* mean, float* rstd,
                              int64_t rows, int64_t cols, int dtype, float eps, void* stream);

/* Residual add + RMSNorm: h = x + residual (rounded), y = h rstd [* weight].
 * No counterpart in the reference. */
int fln_add_rmsnorm_forward(const void* x, const void* residual, const void* weight, void* h,
                            void* y, float* rstd, int64_t rows, int64_t cols, int dtype, float eps,
                            void* stream);

/* LayerNorm with OCP fp8 e4m3fn output: v = LN(x) [* gamma + beta] in fp32,
 * scale[r] = max_j |v_rj| / 448, q = sat_rne_e4m3fn(v / scale[r]) (one byte per element);
 * a row whose max is 0 gets scale 0 and all-zero codes.  A row whose statistics are not usable
 * (a NaN or an infinity in it, an fp32 sum over it that overflows, or a constant row with
 * eps = 0: mean not finite or rstd outside (0, inf)) gets scale NaN, so its codes read as NaN;
 * gamma and beta are taken to be finite.  The fp8 and MXFP8 entry points below share this rule
 * (MXFP8: every block scale of such a row is 0xFF, E8M0's NaN).  mean and rstd may be NULL.
 * No counterpart in the reference. */
int fln_layernorm_fp8_forward(const void* x, const void* gamma, const void* beta, uint8_t* q,
                              float* scale, float* mean, float* rstd, int64_t rows, int64_t cols,
                              int dtype, float eps, void* stream);

/* RMSNorm with fp8 e4m3fn output: v = x rstd [* weight], per-row scale and codes as in
 * fln_layernorm_fp8_forward.  rstd may be NULL.  No counterpart in the reference. */
int fln_rmsnorm_fp8_forward(const void* x, const void* weight, uint8_t* q, float* scale,
                            float* rstd, int64_t rows, int64_t cols, int dtype, float eps,
                            void* stream);

/* Residual add + LayerNorm with fp8 output: h = x + residual (rounded to dtype, stored when h
 * is not NULL), then fln_layernorm_fp8_forward of h.  No counterpart in the reference. */
int fln_add_layernorm_fp8_forward(const void* x, const void* residual, const void* gamma,
                                  const void* beta, void* h, uint8_t* q, float* scale,
                                  float* mean, float* rstd, int64_t rows, int64_t cols,
                                  int dtype, float eps, void* stream);

/* Residual add + RMSNorm with fp8 output (the pre-norm feeding an fp8 GEMM): h = x + residual
 * (rounded, stored when h is not NULL), then fln_rmsnorm_fp8_forward of h.
 * No counterpart in the reference. */
int fln_add_rmsnorm_fp8_forward(const void* x, const void* residual, const void* weight,
                                void* h, uint8_t* q, float* scale, float* rstd, int64_t rows,
                                int64_t cols, int dtype, float eps, void* stream);

/* LayerNorm with OCP MX fp8 output (MXFP8 E4M3, OCP Microscaling Formats v1.0): v = LN(x)
 * [* gamma + beta] in fp32; every block of 32 consecutive elements of a row shares the scale
 * 2^e, e = floor(log2 max|v_block|) - 8 clamped to [-127, 127], stored as the E8M0 byte e + 127
 * in block_scale[rows, cols / 32]; q = sat_rne_e4m3fn(v * 2^-e).  cols must be a multiple of
 * 32.  mean and rstd may be NULL.  No counterpart in the reference. */
int fln_layernorm_mxfp8_forward(const void* x, const void* gamma, const void* beta, uint8_t* q,
                                uint8_t* block_scale, float* mean, float* rstd, int64_t rows,
                                int64_t cols, int dtype, float eps, void* stream);

/* RMSNorm with MXFP8 E4M3 output (block rule of fln_layernorm_mxfp8_forward).
 * No counterpart in the reference. */
int fln_rmsnorm_mxfp8_forward(const void* x, const void* weight, uint8_t* q,
                              uint8_t* block_scale, float* rstd, int64_t rows, int64_t cols,
                              int dtype, float eps, void* stream);

/* Residual add + RMSNorm with MXFP8 E4M3 output: h = x + residual (rounded, stored when h is
 * not NULL), then fln_rmsnorm_mxfp8_forward of h.  No counterpart in the reference. */
int fln_add_rmsnorm_mxfp8_forward(const void* x, const void* residual, const void* weight,
                                  void* h, uint8_t* q, uint8_t* block_scale, float* rstd,
                                  int64_t rows, int64_t cols, int dtype, float eps,
                                  void* stream);

/* Elementwise fp32 -> OCP fp8 e4m3fn (saturating, round-to-nearest-even) with the same device
 * conversion the fp8 forward uses; n elements, any alignment.  A standalone quantizer for
 * callers that scale themselves (and a direct check of the conversion).
 * No counterpart in the reference. */
int fln_fp8_e4m3fn_encode(const float* x, uint8_t* q, int64_t n, void* stream);

/* Forward kernel routes (fln_forward_plan). */
#define FLN_ROUTE_NONE (-1)     /* empty call: nothing is launched */
#define FLN_ROUTE_REGISTERS 0   /* rows held in VGPRs of one or more wave64s (fwd_reg_kernel) */
#define FLN_ROUTE_LDS 1         /* row parked in LDS, the next row in flight (fwd_lds_kernel) */
#define FLN_ROUTE_LDS_REG 2     /* half of each row in LDS, half in registers (fwd_lds_kernel) */
#define FLN_ROUTE_WIDE 3        /* row streamed in passes over L2 / HBM (fwd_wide_kernel) */
#define FLN_ROUTE_SPLIT 4       /* few rows: each split over several blocks (fwd_split_*) */
#define FLN_ROUTE_LOOP 5        /* one block per row, scalar passes (fwd_loop_kernel) */

typedef struct fln_forward_plan {
  int route;            /* FLN_ROUTE_* */
  int vector_elems;     /* elements per lane load: 16 bytes' worth on the vector path, else 1 */
  int waves_per_row;    /* register route: wave64s per row (0 on the other routes) */
  int vectors_per_lane; /* register route: vectors of the row per lane (0 on the other routes) */
  int exact;            /* register route: 1 if no lane holds a masked slot */
  int threads;          /* threads per block */
} fln_forward_plan_t;

/* The launch plan the forward entry points take for a contiguous, 16-byte aligned
 * [rows, cols] input of `dtype` whose output overlaps no input: fp8 = 0 (output in dtype),
 * 1 (fp8 e4m3fn with a per-row scale) or 2 (MXFP8); residual = 0 / 1 (residual-add flavour);
 * gelu_mode FLN_GELU_*; num_cus the CU count to plan for (0: the current device).  It is the
 * dispatcher's own rule (the same function decides the launches, under the same FLN_* knobs),
 * computed on the host without touching a device when num_cus > 0.  Backs
 * `fused_layernorm.functional.get_optimal_config`, which the reference computes from CUDA
 * heuristics in Python (fused_layernorm/functional.py:47-74). */
int fln_forward_plan(int64_t rows, int64_t cols, int dtype, int fp8, int residual,
                     int gelu_mode, int num_cus, fln_forward_plan_t* plan);

/* Host utilities with the reference's meaning (csrc/layernorm_cuda.cpp:144-164 and :167-195).
 * fln_get_performance_hints writes a NUL-terminated string into buf (truncated to buflen) and
 * returns the full length; it reads the CU count of the current device. */
int64_t fln_get_memory_usage(int batch_size, int hidden_size, int use_mixed_precision);
int fln_get_performance_hints(int batch_size, int hidden_size, char* buf, size_t buflen);

/* Library version ("1.0.0", as the reference's __version__, csrc/layernorm_cuda.cpp:230). */
const char* fln_version(void);
/* HIP runtime version the library was built against (the reference's __cuda_version__). */
int fln_hip_version(void);
const char* fln_error_string(int code);
/* Re-reads the FLN_* tuning and debugging environment variables (FLN_FORCE_LOOP, FLN_FWD_EPL,
 * FLN_FWD_WPR, FLN_FWD_GRID_MULT, FLN_FWD_NO_LDS, FLN_FWD_NO_WIDE, FLN_DEBUG_GEOMETRY,
 * FLN_BWD_EPL, FLN_BWD_WPR, FLN_BWD_THREADS, FLN_BWD_NO_LDS, FLN_BWD_NO_TWO_PASS); they are
 * otherwise read once, at the first launch.  No counterpart in the reference: for tests and
 * tuning sweeps. */
void fln_reload_tuning(void);

#ifdef __cplusplus
}
#endif

#endif /* FUSED_LAYERNORM_H */
