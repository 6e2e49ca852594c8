// fln_forward.hip -- forward normalization kernels for gfx950 and their C-ABI entry points.
//
// Path replaced: the reference's `layernorm_kernel` / `layernorm_gelu_kernel`
// (csrc/layernorm_cuda_kernel.cu:39-148) and `layernorm_forward_kernel_optimized`
// (csrc/layernorm_cuda_kernel_optimized.cu:54-168).  Those launch one block per row and read the
// row from global memory three times.  Here a row is read from HBM once, with 16-byte vector
// loads, into VGPRs of one or more wave64s ("row group"); mean and variance are two passes over
// the registers (the reference's two-pass, biased-variance, rsqrt(var + eps) arithmetic,
// csrc/layernorm_cuda_kernel.cu:57-81), and the normalized row is written once.
//
// Kernel flavours (all share the register-resident structure):
//   * LayerNorm / RMSNorm (runtime flag), optional affine (gamma, beta each optional),
//   * optional GELU epilogue (erf or tanh),
//   * optional residual add (h = x + r rounded to the I/O type, statistics over h),
//   * output in the I/O type, or OCP fp8 e4m3fn codes plus a per-row fp32 scale.
// Rows too long for registers (or odd rows beyond 4096 elements) take a looped fallback that
// keeps the same arithmetic but re-reads the row (from L2) on each pass.
//
// The kernels live in fln_forward_impl.h and are instantiated per I/O type in
// fln_forward_{f32,bf16,f16,f64}.hip; this file validates arguments and holds the entry points.
#include "fln_device.h"
#include "fln_internal.h"

namespace fln {

__global__ __launch_bounds__(256) void fp8_encode_kernel(const float* __restrict__ x,
                                                         uint8_t* __restrict__ q, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    q[i] = fp8x1(x[i]);
}

int launch_forward_f32(const FwdParams& p, bool out_fp8, hipStream_t s);
int launch_forward_bf16(const FwdParams& p, bool out_fp8, hipStream_t s);
int launch_forward_f16(const FwdParams& p, bool out_fp8, hipStream_t s);
int launch_forward_f64(const FwdParams& p, hipStream_t s);
int plan_forward_f32(int64_t rows, int64_t cols, int fp8, bool res, int gelu, int64_t cus,
                     fln_forward_plan_t* out);
int plan_forward_bf16(int64_t rows, int64_t cols, int fp8, bool res, int gelu, int64_t cus,
                      fln_forward_plan_t* out);
int plan_forward_f16(int64_t rows, int64_t cols, int fp8, bool res, int gelu, int64_t cus,
                     fln_forward_plan_t* out);

int launch_forward(const FwdParams& p, int dtype, bool out_fp8, hipStream_t s) {
  if (p.rows < 0 || p.cols < 0 || p.rows > INT32_MAX || p.cols > INT32_MAX) return FLN_ERR_INVALID;
  if (!(p.eps >= 0.0f) || p.gelu < 0 || p.gelu > 2) return FLN_ERR_INVALID;
  if (p.rows == 0 || p.cols == 0) return FLN_OK;
  if (!p.x || !p.y) return FLN_ERR_INVALID;
  if (p.res == nullptr && p.h != nullptr) return FLN_ERR_INVALID;
  if (out_fp8 && !p.mx && !p.scale) return FLN_ERR_INVALID;
  if (out_fp8 && p.mx && (!p.bscale || p.cols % 32 != 0)) return FLN_ERR_INVALID;
  if (p.rms && p.beta) return FLN_ERR_INVALID;
  const CallDevice device_scope;
  switch (dtype) {
    case FLN_F32: return launch_forward_f32(p, out_fp8, s);
    case FLN_BF16: return launch_forward_bf16(p, out_fp8, s);
    case FLN_F16: return launch_forward_f16(p, out_fp8, s);
    case FLN_F64: return out_fp8 ? FLN_ERR_INVALID : launch_forward_f64(p, s);
    default:
      return FLN_ERR_INVALID;
  }
}

}  // namespace fln

using fln::FwdParams;

extern "C" int fln_forward_plan(int64_t rows, int64_t cols, int dtype, int fp8, int residual,
                                int gelu_mode, int num_cus, fln_forward_plan_t* plan) {
  if (!plan || rows < 0 || cols < 0 || rows > INT32_MAX || cols > INT32_MAX) return FLN_ERR_INVALID;
  if (fp8 < 0 || fp8 > 2 || gelu_mode < 0 || gelu_mode > 2 || num_cus < 0) return FLN_ERR_INVALID;
  if (fp8 && (gelu_mode != FLN_GELU_NONE || dtype == FLN_F64)) return FLN_ERR_INVALID;
  if (fp8 == 2 && cols % 32 != 0) return FLN_ERR_INVALID;
  if (dtype == FLN_F64 && residual) return FLN_ERR_INVALID;
  *plan = fln_forward_plan_t{FLN_ROUTE_NONE, 0, 0, 0, 0, 0};
  if (rows == 0 || cols == 0) return FLN_OK;  // nothing is launched
  const int64_t cus = num_cus > 0 ? num_cus : fln::device_cu_count();
  switch (dtype) {
    case FLN_F32: return fln::plan_forward_f32(rows, cols, fp8, residual != 0, gelu_mode, cus, plan);
    case FLN_BF16: return fln::plan_forward_bf16(rows, cols, fp8, residual != 0, gelu_mode, cus, plan);
    case FLN_F16: return fln::plan_forward_f16(rows, cols, fp8, residual != 0, gelu_mode, cus, plan);
    case FLN_F64:  // fp64 always takes the looped kernel with fp64 accumulation
      *plan = fln_forward_plan_t{FLN_ROUTE_LOOP, 1, 0, 0, 0, cols >= 4096 ? 1024 : 256};
      return FLN_OK;
    default: return FLN_ERR_INVALID;
  }
}

extern "C" int fln_layernorm(const void* x, const void* gamma, const void* beta, void* y,
                             int64_t rows, int64_t cols, int dtype, float eps, void* stream) {
  FwdParams p{};
  p.x = x; p.gamma = gamma; p.beta = beta; p.y = y;
  p.rows = rows; p.cols = cols; p.eps = eps;
  return fln::launch_forward(p, dtype, false, static_cast<hipStream_t>(stream));
}

extern "C" int fln_layernorm_gelu(const void* x, const void* gamma, const void* beta, void* y,
                                  int64_t rows, int64_t cols, int dtype, float eps, int gelu_mode,
                                  void* stream) {
  if (gelu_mode != FLN_GELU_ERF && gelu_mode != FLN_GELU_TANH) return FLN_ERR_INVALID;
  FwdParams p{};
  p.x = x; p.gamma = gamma; p.beta = beta; p.y = y;
  p.rows = rows; p.cols = cols; p.eps = eps; p.gelu = gelu_mode;
  return fln::launch_forward(p, dtype, false, static_cast<hipStream_t>(stream));
}

extern "C" int fln_layernorm_gelu_forward(const void* x, const void* gamma, const void* beta,
                                          void* y, float* mean, float* rstd, int64_t rows,
                                          int64_t cols, int dtype, float eps, int gelu_mode,
                                          void* stream) {
  if (gelu_mode != FLN_GELU_ERF && gelu_mode != FLN_GELU_TANH) return FLN_ERR_INVALID;
  FwdParams p{};
  p.x = x; p.gamma = gamma; p.beta = beta; p.y = y; p.mean = mean; p.rstd = rstd;
  p.rows = rows; p.cols = cols; p.eps = eps; p.gelu = gelu_mode;
  return fln::launch_forward(p, dtype, false, static_cast<hipStream_t>(stream));
}

extern "C" int fln_layernorm_forward(const void* x, const void* gamma, const void* beta, void* y,
                                     float* mean, float* rstd, int64_t rows, int64_t cols,
                                     int dtype, float eps, void* stream) {
  FwdParams p{};
  p.x = x; p.gamma = gamma; p.beta = beta; p.y = y; p.mean = mean; p.rstd = rstd;
  p.rows = rows; p.cols = cols; p.eps = eps;
  return fln::launch_forward(p, dtype, false, static_cast<hipStream_t>(stream));
}

extern "C" int fln_rmsnorm_forward(const void* x, const void* weight, void* y, float* rstd,
                                   int64_t rows, int64_t cols, int dtype, float eps,
                                   void* stream) {
  FwdParams p{};
  p.x = x; p.gamma = weight; p.y = y; p.rstd = rstd;
  p.rows = rows; p.cols = cols; p.eps = eps; p.rms = 1;
  return fln::launch_forward(p, dtype, false, static_cast<hipStream_t>(stream));
}

extern "C" int fln_add_layernorm_forward(const void* x, const void* residual, const void* gamma,
                                         const void* beta, void* h, void* y, float* mean,
                                         float* rstd, int64_t rows, int64_t cols, int dtype,
                                         float eps, void* stream) {
  if (!residual) return FLN_ERR_INVALID;
  FwdParams p{};
  p.x = x; p.res = residual; p.gamma = gamma; p.beta = beta; p.h = h; p.y = y;
  p.mean = mean; p.rstd = rstd; p.rows = rows; p.cols = cols; p.eps = eps;
  return fln::launch_forward(p, dtype, false, static_cast<hipStream_t>(stream));
}

extern "C" int fln_add_rmsnorm_forward(const void* x, const void* residual, const void* weight,
                                       void* h, void* y, float* rstd, int64_t rows, int64_t cols,
                                       int dtype, float eps, void* stream) {
  if (!residual) return FLN_ERR_INVALID;
  FwdParams p{};
  p.x = x; p.res = residual; p.gamma = weight; p.h = h; p.y = y; p.rstd = rstd;
  p.rows = rows; p.cols = cols; p.eps = eps; p.rms = 1;
  return fln::launch_forward(p, dtype, false, static_cast<hipStream_t>(stream));
}

extern "C" int fln_layernorm_fp8_forward(const void* x, const void* gamma, const void* beta,
                                         uint8_t* q, float* scale, float* mean, float* rstd,
                                         int64_t rows, int64_t cols, int dtype, float eps,
                                         void* stream) {
  if (dtype == FLN_F64) return FLN_ERR_INVALID;
  FwdParams p{};
  p.x = x; p.gamma = gamma; p.beta = beta; p.y = q; p.scale = scale; p.mean = mean; p.rstd = rstd;
  p.rows = rows; p.cols = cols; p.eps = eps;
  return fln::launch_forward(p, dtype, true, static_cast<hipStream_t>(stream));
}

extern "C" int fln_rmsnorm_fp8_forward(const void* x, const void* weight, uint8_t* q,
                                       float* scale, float* rstd, int64_t rows, int64_t cols,
                                       int dtype, float eps, void* stream) {
  if (dtype == FLN_F64) return FLN_ERR_INVALID;
  FwdParams p{};
  p.x = x; p.gamma = weight; p.y = q; p.scale = scale; p.rstd = rstd;
  p.rows = rows; p.cols = cols; p.eps = eps; p.rms = 1;
  return fln::launch_forward(p, dtype, true, static_cast<hipStream_t>(stream));
}

extern "C" int fln_add_layernorm_fp8_forward(const void* x, const void* residual,
                                             const void* gamma, const void* beta, void* h,
                                             uint8_t* q, float* scale, float* mean, float* rstd,
                                             int64_t rows, int64_t cols, int dtype, float eps,
                                             void* stream) {
  if (dtype == FLN_F64 || !residual) return FLN_ERR_INVALID;
  FwdParams p{};
  p.x = x; p.res = residual; p.gamma = gamma; p.beta = beta; p.h = h; p.y = q;
  p.scale = scale; p.mean = mean; p.rstd = rstd; p.rows = rows; p.cols = cols; p.eps = eps;
  return fln::launch_forward(p, dtype, true, static_cast<hipStream_t>(stream));
}

extern "C" int fln_add_rmsnorm_fp8_forward(const void* x, const void* residual,
                                           const void* weight, void* h, uint8_t* q, float* scale,
                                           float* rstd, int64_t rows, int64_t cols, int dtype,
                                           float eps, void* stream) {
  if (dtype == FLN_F64 || !residual) return FLN_ERR_INVALID;
  FwdParams p{};
  p.x = x; p.res = residual; p.gamma = weight; p.h = h; p.y = q; p.scale = scale;
  p.rstd = rstd; p.rows = rows; p.cols = cols; p.eps = eps; p.rms = 1;
  return fln::launch_forward(p, dtype, true, static_cast<hipStream_t>(stream));
}

extern "C" int fln_layernorm_mxfp8_forward(const void* x, const void* gamma, const void* beta,
                                           uint8_t* q, uint8_t* block_scale, float* mean,
                                           float* rstd, int64_t rows, int64_t cols, int dtype,
                                           float eps, void* stream) {
  if (dtype == FLN_F64) return FLN_ERR_INVALID;
  FwdParams p{};
  p.x = x; p.gamma = gamma; p.beta = beta; p.y = q; p.bscale = block_scale; p.mx = 1;
  p.mean = mean; p.rstd = rstd; p.rows = rows; p.cols = cols; p.eps = eps;
  return fln::launch_forward(p, dtype, true, static_cast<hipStream_t>(stream));
}

extern "C" int fln_rmsnorm_mxfp8_forward(const void* x, const void* weight, uint8_t* q,
                                         uint8_t* block_scale, float* rstd, int64_t rows,
                                         int64_t cols, int dtype, float eps, void* stream) {
  if (dtype == FLN_F64) return FLN_ERR_INVALID;
  FwdParams p{};
  p.x = x; p.gamma = weight; p.y = q; p.bscale = block_scale; p.mx = 1; p.rstd = rstd;
  p.rows = rows; p.cols = cols; p.eps = eps; p.rms = 1;
  return fln::launch_forward(p, dtype, true, static_cast<hipStream_t>(stream));
}

extern "C" int fln_add_rmsnorm_mxfp8_forward(const void* x, const void* residual,
                                             const void* weight, void* h, uint8_t* q,
                                             uint8_t* block_scale, float* rstd, int64_t rows,
                                             int64_t cols, int dtype, float eps, void* stream) {
  if (dtype == FLN_F64 || !residual) return FLN_ERR_INVALID;
  FwdParams p{};
  p.x = x; p.res = residual; p.gamma = weight; p.h = h; p.y = q; p.bscale = block_scale;
  p.mx = 1; p.rstd = rstd; p.rows = rows; p.cols = cols; p.eps = eps; p.rms = 1;
  return fln::launch_forward(p, dtype, true, static_cast<hipStream_t>(stream));
}

extern "C" int fln_fp8_e4m3fn_encode(const float* x, uint8_t* q, int64_t n, void* stream) {
  if (n < 0) return FLN_ERR_INVALID;
  if (n == 0) return FLN_OK;
  if (!x || !q) return FLN_ERR_INVALID;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fln::fp8_encode_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, q, n);
  return static_cast<int>(hipGetLastError());
}
