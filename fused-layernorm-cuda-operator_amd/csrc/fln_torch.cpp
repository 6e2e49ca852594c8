// fln_torch.cpp -- PyTorch binding of libfln: the extension module `fused_layernorm_cuda`
// (drop-in for the reference's module of that name: csrc/bindings.cpp:41-44 and
// csrc/layernorm_cuda.cpp:198-238) and the `fused_layernorm::*` operator schemas used by
// torch.compile.
//
// This file is host C++ only.  It validates arguments (before anything is launched), allocates
// outputs through the caching allocator, and calls the C ABI of libfln on the current HIP stream
// of the input's device.  The kernels live behind include/fused_layernorm.h.
#include <torch/extension.h>
#include <torch/library.h>

#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/autograd/function.h>
#include <torch/csrc/autograd/functions/utils.h>
#include <torch/csrc/autograd/saved_variable.h>

#include <array>
#include <mutex>
#include <optional>
#include <string>
#include <tuple>
#include <vector>

#include "fused_layernorm.h"

namespace {

using at::Tensor;
using OptT = std::optional<Tensor>;

int dtype_code(const Tensor& t) {
  switch (t.scalar_type()) {
    case at::kFloat: return FLN_F32;
    case at::kBFloat16: return FLN_BF16;
    case at::kHalf: return FLN_F16;
    case at::kDouble: return FLN_F64;
    default: return -1;
  }
}

void check(int rc, const char* what) {
  TORCH_CHECK(rc == FLN_OK, what, " failed: ", fln_error_string(rc), " (code ", rc, ")");
}

void* stream_of(const Tensor& t) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

// Shape of the normalized problem: rows x cols with cols = last dimension.
struct Shape {
  int64_t rows;
  int64_t cols;
};

Shape check_input(const Tensor& x, const char* name, bool allow_f64) {
  TORCH_CHECK(x.defined(), name, " must be defined");
  TORCH_CHECK(x.is_cuda(), name, " must be a GPU (HIP) tensor");
  TORCH_CHECK(x.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(x.dim() >= 1, name, " must have at least one dimension");
  const int code = dtype_code(x);
  TORCH_CHECK(code == FLN_F32 || code == FLN_BF16 || code == FLN_F16 ||
                  (allow_f64 && code == FLN_F64),
              name, " has unsupported dtype ", x.scalar_type(),
              allow_f64 ? " (float32, float64, bfloat16, float16 are supported)"
                        : " (float32, bfloat16, float16 are supported)");
  const int64_t cols = x.size(-1);
  return {cols == 0 ? 0 : x.numel() / cols, cols};
}

void check_param(const OptT& p, const Tensor& x, int64_t cols, const char* name) {
  if (!p.has_value() || !p->defined()) return;
  const Tensor& t = *p;
  TORCH_CHECK(t.is_cuda(), name, " must be a GPU (HIP) tensor");
  TORCH_CHECK(t.device() == x.device(), name, " must be on the same device as the input");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(t.dim() == 1, name, " must be 1D");
  TORCH_CHECK(t.size(0) == cols, name, " size must match hidden dimension (", t.size(0),
              " vs ", cols, ")");
  TORCH_CHECK(t.scalar_type() == x.scalar_type(), name, " must have the input's dtype (",
              t.scalar_type(), " vs ", x.scalar_type(), ")");
}

const void* ptr_or_null(const OptT& p) {
  return (p.has_value() && p->defined()) ? p->data_ptr() : nullptr;
}

bool has(const OptT& p) { return p.has_value() && p->defined(); }

void check_affine_pair(const OptT& w, const OptT& b) {
  TORCH_CHECK(has(w) == has(b),
              "gamma and beta must be given together (the affine step applies both or neither)");
}

void check_stats(const Tensor& s, int64_t rows, const Tensor& x, const char* name) {
  TORCH_CHECK(s.defined() && s.is_cuda() && s.device() == x.device(), name,
              " must be a GPU tensor on the input's device");
  TORCH_CHECK(s.scalar_type() == at::kFloat, name, " must be float32");
  TORCH_CHECK(s.is_contiguous() && s.numel() == rows, name, " must hold one value per row (",
              rows, "), got ", s.numel());
}

Tensor stats_like(const Tensor& x, int64_t rows) {
  std::vector<int64_t> shape(x.sizes().begin(), x.sizes().end() - 1);
  if (shape.empty()) shape.push_back(1);
  (void)rows;
  return at::empty(shape, x.options().dtype(at::kFloat));
}

// ------------------------------------------------------------------------------------------
// Forward family.
// ------------------------------------------------------------------------------------------

// Reference `layernorm(input, gamma, beta, epsilon)` (csrc/bindings.cpp:19-28).
Tensor layernorm(const Tensor& input, const OptT& gamma, const OptT& beta, double eps) {
  const Shape s = check_input(input, "input", true);
  check_param(gamma, input, s.cols, "gamma");
  check_param(beta, input, s.cols, "beta");
  check_affine_pair(gamma, beta);
  c10::hip::HIPGuard guard(input.device().index());
  Tensor y = at::empty_like(input);
  check(fln_layernorm(input.data_ptr(), ptr_or_null(gamma), ptr_or_null(beta), y.data_ptr(),
                      s.rows, s.cols, dtype_code(input), static_cast<float>(eps),
                      stream_of(input)),
        "layernorm");
  return y;
}

// Reference `layernorm_gelu(input, gamma, beta, epsilon)` (csrc/bindings.cpp:30-39), whose GELU
// is the tanh form (csrc/layernorm_cuda_kernel.cu:31-36): that is the default here;
// approximate="none" selects the exact erf form.
int gelu_code(const std::string& approximate) {
  TORCH_CHECK(approximate == "tanh" || approximate == "none",
              "approximate must be 'tanh' or 'none', got '", approximate, "'");
  return approximate == "tanh" ? FLN_GELU_TANH : FLN_GELU_ERF;
}

// GELU(LayerNorm(x)) -> (y, mean, rstd): the operator form, whose statistics feed the fused
// backward below.
std::tuple<Tensor, Tensor, Tensor> layer_norm_gelu_fwd(const Tensor& input, const OptT& gamma,
                                                       const OptT& beta, double eps,
                                                       const std::string& approximate) {
  const int mode = gelu_code(approximate);
  const Shape s = check_input(input, "input", true);
  check_param(gamma, input, s.cols, "gamma");
  check_param(beta, input, s.cols, "beta");
  c10::hip::HIPGuard guard(input.device().index());
  Tensor y = at::empty_like(input);
  Tensor mean = stats_like(input, s.rows);
  Tensor rstd = stats_like(input, s.rows);
  check(fln_layernorm_gelu_forward(input.data_ptr(), ptr_or_null(gamma), ptr_or_null(beta),
                                   y.data_ptr(), mean.data_ptr<float>(), rstd.data_ptr<float>(),
                                   s.rows, s.cols, dtype_code(input), static_cast<float>(eps),
                                   mode, stream_of(input)),
        "layer_norm_gelu forward");
  return {y, mean, rstd};
}

// Reference `layernorm_gelu` (csrc/bindings.cpp:30-39): output only.
Tensor layernorm_gelu(const Tensor& input, const OptT& gamma, const OptT& beta, double eps,
                      const std::string& approximate) {
  check_affine_pair(gamma, beta);
  const int mode = gelu_code(approximate);
  const Shape s = check_input(input, "input", true);
  check_param(gamma, input, s.cols, "gamma");
  check_param(beta, input, s.cols, "beta");
  c10::hip::HIPGuard guard(input.device().index());
  Tensor y = at::empty_like(input);
  check(fln_layernorm_gelu(input.data_ptr(), ptr_or_null(gamma), ptr_or_null(beta),
                           y.data_ptr(), s.rows, s.cols, dtype_code(input),
                           static_cast<float>(eps), mode, stream_of(input)),
        "layernorm_gelu");
  return y;
}

// Reference `forward(input, gamma, beta, epsilon) -> [out, mean, rstd]`
// (csrc/layernorm_cuda.cpp:49-94); mean/rstd are always float32 here.
std::tuple<Tensor, Tensor, Tensor> layer_norm_fwd(const Tensor& input, const OptT& gamma,
                                                  const OptT& beta, double eps) {
  const Shape s = check_input(input, "input", true);
  check_param(gamma, input, s.cols, "gamma");
  check_param(beta, input, s.cols, "beta");
  c10::hip::HIPGuard guard(input.device().index());
  Tensor y = at::empty_like(input);
  Tensor mean = stats_like(input, s.rows);
  Tensor rstd = stats_like(input, s.rows);
  check(fln_layernorm_forward(input.data_ptr(), ptr_or_null(gamma), ptr_or_null(beta),
                              y.data_ptr(), mean.data_ptr<float>(), rstd.data_ptr<float>(),
                              s.rows, s.cols, dtype_code(input), static_cast<float>(eps),
                              stream_of(input)),
        "layer_norm forward");
  return {y, mean, rstd};
}

std::vector<Tensor> forward(const Tensor& input, const OptT& gamma, const OptT& beta,
                            double eps) {
  TORCH_CHECK(input.dim() == 2, "Input must be 2D (batch_size, hidden_size)");
  check_affine_pair(gamma, beta);
  auto r = layer_norm_fwd(input, gamma, beta, eps);
  return {std::get<0>(r), std::get<1>(r), std::get<2>(r)};
}

std::tuple<Tensor, Tensor> rms_norm_fwd(const Tensor& input, const OptT& weight, double eps) {
  const Shape s = check_input(input, "input", false);
  check_param(weight, input, s.cols, "weight");
  c10::hip::HIPGuard guard(input.device().index());
  Tensor y = at::empty_like(input);
  Tensor rstd = stats_like(input, s.rows);
  check(fln_rmsnorm_forward(input.data_ptr(), ptr_or_null(weight), y.data_ptr(),
                            rstd.data_ptr<float>(), s.rows, s.cols, dtype_code(input),
                            static_cast<float>(eps), stream_of(input)),
        "rms_norm forward");
  return {y, rstd};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> add_layer_norm_fwd(const Tensor& input,
                                                              const Tensor& residual,
                                                              const OptT& gamma,
                                                              const OptT& beta, double eps) {
  const Shape s = check_input(input, "input", true);
  check_input(residual, "residual", true);
  TORCH_CHECK(residual.sizes() == input.sizes() && residual.scalar_type() == input.scalar_type() &&
                  residual.device() == input.device(),
              "residual must match the input's shape, dtype and device");
  check_param(gamma, input, s.cols, "gamma");
  check_param(beta, input, s.cols, "beta");
  c10::hip::HIPGuard guard(input.device().index());
  Tensor y = at::empty_like(input);
  Tensor h = at::empty_like(input);
  Tensor mean = stats_like(input, s.rows);
  Tensor rstd = stats_like(input, s.rows);
  check(fln_add_layernorm_forward(input.data_ptr(), residual.data_ptr(), ptr_or_null(gamma),
                                  ptr_or_null(beta), h.data_ptr(), y.data_ptr(),
                                  mean.data_ptr<float>(), rstd.data_ptr<float>(), s.rows, s.cols,
                                  dtype_code(input), static_cast<float>(eps), stream_of(input)),
        "add_layer_norm forward");
  return {y, h, mean, rstd};
}

std::tuple<Tensor, Tensor, Tensor> add_rms_norm_fwd(const Tensor& input, const Tensor& residual,
                                                    const OptT& weight, double eps) {
  const Shape s = check_input(input, "input", false);
  check_input(residual, "residual", false);
  TORCH_CHECK(residual.sizes() == input.sizes() && residual.scalar_type() == input.scalar_type() &&
                  residual.device() == input.device(),
              "residual must match the input's shape, dtype and device");
  check_param(weight, input, s.cols, "weight");
  c10::hip::HIPGuard guard(input.device().index());
  Tensor y = at::empty_like(input);
  Tensor h = at::empty_like(input);
  Tensor rstd = stats_like(input, s.rows);
  check(fln_add_rmsnorm_forward(input.data_ptr(), residual.data_ptr(), ptr_or_null(weight),
                                h.data_ptr(), y.data_ptr(), rstd.data_ptr<float>(), s.rows,
                                s.cols, dtype_code(input), static_cast<float>(eps),
                                stream_of(input)),
        "add_rms_norm forward");
  return {y, h, rstd};
}

std::tuple<Tensor, Tensor> layer_norm_fp8_fwd(const Tensor& input, const OptT& gamma,
                                              const OptT& beta, double eps) {
  const Shape s = check_input(input, "input", false);
  check_param(gamma, input, s.cols, "gamma");
  check_param(beta, input, s.cols, "beta");
  c10::hip::HIPGuard guard(input.device().index());
  Tensor q = at::empty(input.sizes(), input.options().dtype(at::kFloat8_e4m3fn));
  Tensor scale = stats_like(input, s.rows);
  check(fln_layernorm_fp8_forward(input.data_ptr(), ptr_or_null(gamma), ptr_or_null(beta),
                                  static_cast<uint8_t*>(q.data_ptr()), scale.data_ptr<float>(),
                                  nullptr, nullptr, s.rows, s.cols, dtype_code(input),
                                  static_cast<float>(eps), stream_of(input)),
        "layer_norm fp8 forward");
  return {q, scale};
}

std::tuple<Tensor, Tensor> rms_norm_fp8_fwd(const Tensor& input, const OptT& weight,
                                            double eps) {
  const Shape s = check_input(input, "input", false);
  check_param(weight, input, s.cols, "weight");
  c10::hip::HIPGuard guard(input.device().index());
  Tensor q = at::empty(input.sizes(), input.options().dtype(at::kFloat8_e4m3fn));
  Tensor scale = stats_like(input, s.rows);
  check(fln_rmsnorm_fp8_forward(input.data_ptr(), ptr_or_null(weight),
                                static_cast<uint8_t*>(q.data_ptr()), scale.data_ptr<float>(),
                                nullptr, s.rows, s.cols, dtype_code(input),
                                static_cast<float>(eps), stream_of(input)),
        "rms_norm fp8 forward");
  return {q, scale};
}

void check_residual(const Tensor& residual, const Tensor& input) {
  check_input(residual, "residual", false);
  TORCH_CHECK(residual.sizes() == input.sizes() && residual.scalar_type() == input.scalar_type() &&
                  residual.device() == input.device(),
              "residual must match the input's shape, dtype and device");
}

std::tuple<Tensor, Tensor, Tensor> add_layer_norm_fp8_fwd(const Tensor& input,
                                                          const Tensor& residual,
                                                          const OptT& gamma, const OptT& beta,
                                                          double eps) {
  const Shape s = check_input(input, "input", false);
  check_residual(residual, input);
  check_param(gamma, input, s.cols, "gamma");
  check_param(beta, input, s.cols, "beta");
  c10::hip::HIPGuard guard(input.device().index());
  Tensor q = at::empty(input.sizes(), input.options().dtype(at::kFloat8_e4m3fn));
  Tensor scale = stats_like(input, s.rows);
  Tensor h = at::empty_like(input);
  check(fln_add_layernorm_fp8_forward(input.data_ptr(), residual.data_ptr(), ptr_or_null(gamma),
                                      ptr_or_null(beta), h.data_ptr(),
                                      static_cast<uint8_t*>(q.data_ptr()),
                                      scale.data_ptr<float>(), nullptr, nullptr, s.rows, s.cols,
                                      dtype_code(input), static_cast<float>(eps),
                                      stream_of(input)),
        "add_layer_norm fp8 forward");
  return {q, scale, h};
}

std::tuple<Tensor, Tensor, Tensor> add_rms_norm_fp8_fwd(const Tensor& input,
                                                        const Tensor& residual,
                                                        const OptT& weight, double eps) {
  const Shape s = check_input(input, "input", false);
  check_residual(residual, input);
  check_param(weight, input, s.cols, "weight");
  c10::hip::HIPGuard guard(input.device().index());
  Tensor q = at::empty(input.sizes(), input.options().dtype(at::kFloat8_e4m3fn));
  Tensor scale = stats_like(input, s.rows);
  Tensor h = at::empty_like(input);
  check(fln_add_rmsnorm_fp8_forward(input.data_ptr(), residual.data_ptr(), ptr_or_null(weight),
                                    h.data_ptr(), static_cast<uint8_t*>(q.data_ptr()),
                                    scale.data_ptr<float>(), nullptr, s.rows, s.cols,
                                    dtype_code(input), static_cast<float>(eps),
                                    stream_of(input)),
        "add_rms_norm fp8 forward");
  return {q, scale, h};
}

// OCP MX fp8 outputs: codes as float8_e4m3fn [rows, cols], block scales as float8_e8m0fnu
// [rows, cols / 32] (torch's E8M0 type: the byte e + 127 for the scale 2^e).
Tensor mx_scales_like(const Tensor& input, const Shape& s) {
  TORCH_CHECK(s.cols % 32 == 0, "MX fp8 output needs the normalized size to be a multiple of 32, "
              "got ", s.cols);
  std::vector<int64_t> shape(input.sizes().begin(), input.sizes().end() - 1);
  shape.push_back(s.cols / 32);
  return at::empty(shape, input.options().dtype(at::kFloat8_e8m0fnu));
}

std::tuple<Tensor, Tensor> layer_norm_mxfp8_fwd(const Tensor& input, const OptT& gamma,
                                                const OptT& beta, double eps) {
  const Shape s = check_input(input, "input", false);
  check_param(gamma, input, s.cols, "gamma");
  check_param(beta, input, s.cols, "beta");
  c10::hip::HIPGuard guard(input.device().index());
  Tensor q = at::empty(input.sizes(), input.options().dtype(at::kFloat8_e4m3fn));
  Tensor sc = mx_scales_like(input, s);
  check(fln_layernorm_mxfp8_forward(input.data_ptr(), ptr_or_null(gamma), ptr_or_null(beta),
                                    static_cast<uint8_t*>(q.data_ptr()),
                                    static_cast<uint8_t*>(sc.data_ptr()), nullptr, nullptr,
                                    s.rows, s.cols, dtype_code(input), static_cast<float>(eps),
                                    stream_of(input)),
        "layer_norm mxfp8 forward");
  return {q, sc};
}

std::tuple<Tensor, Tensor> rms_norm_mxfp8_fwd(const Tensor& input, const OptT& weight,
                                              double eps) {
  const Shape s = check_input(input, "input", false);
  check_param(weight, input, s.cols, "weight");
  c10::hip::HIPGuard guard(input.device().index());
  Tensor q = at::empty(input.sizes(), input.options().dtype(at::kFloat8_e4m3fn));
  Tensor sc = mx_scales_like(input, s);
  check(fln_rmsnorm_mxfp8_forward(input.data_ptr(), ptr_or_null(weight),
                                  static_cast<uint8_t*>(q.data_ptr()),
                                  static_cast<uint8_t*>(sc.data_ptr()), nullptr, s.rows, s.cols,
                                  dtype_code(input), static_cast<float>(eps), stream_of(input)),
        "rms_norm mxfp8 forward");
  return {q, sc};
}

std::tuple<Tensor, Tensor, Tensor> add_rms_norm_mxfp8_fwd(const Tensor& input,
                                                          const Tensor& residual,
                                                          const OptT& weight, double eps) {
  const Shape s = check_input(input, "input", false);
  check_residual(residual, input);
  check_param(weight, input, s.cols, "weight");
  c10::hip::HIPGuard guard(input.device().index());
  Tensor q = at::empty(input.sizes(), input.options().dtype(at::kFloat8_e4m3fn));
  Tensor sc = mx_scales_like(input, s);
  Tensor h = at::empty_like(input);
  check(fln_add_rmsnorm_mxfp8_forward(input.data_ptr(), residual.data_ptr(), ptr_or_null(weight),
                                      h.data_ptr(), static_cast<uint8_t*>(q.data_ptr()),
                                      static_cast<uint8_t*>(sc.data_ptr()), nullptr, s.rows,
                                      s.cols, dtype_code(input), static_cast<float>(eps),
                                      stream_of(input)),
        "add_rms_norm mxfp8 forward");
  return {q, sc, h};
}

// ------------------------------------------------------------------------------------------
// Backward family.  Masked-off outputs come back as empty (0-element) tensors through the
// operator schema and as None through the pybind `backward`.
// ------------------------------------------------------------------------------------------
// Always passed (also for dx alone): rows past the register kernels use it for their row
// statistics, and torch's caching allocator makes it cheap.
Tensor workspace_for(const Tensor& x, int64_t rows, int64_t cols) {
  const size_t bytes = fln_backward_workspace_bytes(rows, cols, dtype_code(x));
  return at::empty({static_cast<int64_t>((bytes + 3) / 4)}, x.options().dtype(at::kFloat));
}

std::tuple<Tensor, Tensor, Tensor> layer_norm_bwd(const Tensor& grad_out, const Tensor& input,
                                                  const Tensor& mean, const Tensor& rstd,
                                                  const OptT& gamma, const OptT& beta,
                                                  std::array<bool, 3> output_mask,
                                                  const OptT& grad_extra) {
  const Shape s = check_input(input, "input", false);
  check_input(grad_out, "grad_output", false);
  TORCH_CHECK(grad_out.sizes() == input.sizes(), "grad_output shape must match input shape");
  TORCH_CHECK(grad_out.scalar_type() == input.scalar_type(),
              "grad_output dtype must match input dtype");
  check_stats(mean, s.rows, input, "mean");
  check_stats(rstd, s.rows, input, "rstd");
  check_param(gamma, input, s.cols, "gamma");
  check_param(beta, input, s.cols, "beta");
  if (has(grad_extra)) {
    check_input(*grad_extra, "grad_extra", false);
    TORCH_CHECK(grad_extra->sizes() == input.sizes() &&
                    grad_extra->scalar_type() == input.scalar_type(),
                "grad_extra must match the input's shape and dtype");
  }
  c10::hip::HIPGuard guard(input.device().index());
  const bool want_dx = output_mask[0];
  const bool want_dg = output_mask[1] && has(gamma);
  const bool want_db = output_mask[2] && has(beta);
  Tensor dx = want_dx ? at::empty_like(input) : at::empty({0}, input.options());
  Tensor dg = want_dg ? at::empty_like(*gamma) : at::empty({0}, input.options());
  Tensor db = want_db ? at::empty_like(*beta) : at::empty({0}, input.options());
  Tensor ws;
  ws = workspace_for(input, s.rows, s.cols);
  check(fln_layernorm_backward(grad_out.data_ptr(), input.data_ptr(), mean.data_ptr<float>(),
                               rstd.data_ptr<float>(), ptr_or_null(gamma),
                               ptr_or_null(grad_extra), want_dx ? dx.data_ptr() : nullptr,
                               want_dg ? dg.data_ptr() : nullptr,
                               want_db ? db.data_ptr() : nullptr, s.rows, s.cols,
                               dtype_code(input), dtype_code(input),
                               ws.defined() ? ws.data_ptr() : nullptr,
                               ws.defined() ? static_cast<size_t>(ws.numel()) * 4 : 0,
                               stream_of(input)),
        "layer_norm backward");
  return {dx, dg, db};
}

std::tuple<Tensor, Tensor, Tensor> layer_norm_gelu_bwd(const Tensor& grad_out,
                                                       const Tensor& input, const Tensor& mean,
                                                       const Tensor& rstd, const OptT& gamma,
                                                       const OptT& beta,
                                                       const std::string& approximate,
                                                       std::array<bool, 3> output_mask) {
  const int mode = gelu_code(approximate);
  const Shape s = check_input(input, "input", false);
  check_input(grad_out, "grad_output", false);
  TORCH_CHECK(grad_out.sizes() == input.sizes(), "grad_output shape must match input shape");
  TORCH_CHECK(grad_out.scalar_type() == input.scalar_type(),
              "grad_output dtype must match input dtype");
  check_stats(mean, s.rows, input, "mean");
  check_stats(rstd, s.rows, input, "rstd");
  check_param(gamma, input, s.cols, "gamma");
  check_param(beta, input, s.cols, "beta");
  c10::hip::HIPGuard guard(input.device().index());
  const bool want_dx = output_mask[0];
  const bool want_dg = output_mask[1] && has(gamma);
  const bool want_db = output_mask[2] && has(beta);
  Tensor dx = want_dx ? at::empty_like(input) : at::empty({0}, input.options());
  Tensor dg = want_dg ? at::empty_like(*gamma) : at::empty({0}, input.options());
  Tensor db = want_db ? at::empty_like(*beta) : at::empty({0}, input.options());
  Tensor ws;
  ws = workspace_for(input, s.rows, s.cols);
  check(fln_layernorm_gelu_backward(grad_out.data_ptr(), input.data_ptr(),
                                    mean.data_ptr<float>(), rstd.data_ptr<float>(),
                                    ptr_or_null(gamma), ptr_or_null(beta),
                                    want_dx ? dx.data_ptr() : nullptr,
                                    want_dg ? dg.data_ptr() : nullptr,
                                    want_db ? db.data_ptr() : nullptr, s.rows, s.cols,
                                    dtype_code(input), dtype_code(input), mode,
                                    ws.defined() ? ws.data_ptr() : nullptr,
                                    ws.defined() ? static_cast<size_t>(ws.numel()) * 4 : 0,
                                    stream_of(input)),
        "layer_norm_gelu backward");
  return {dx, dg, db};
}

// Reference `backward(grad_output, input, mean, rstd, gamma, beta, output_mask)`
// (csrc/layernorm_cuda.cpp:97-141, :208-216).
std::vector<std::optional<Tensor>> backward(const Tensor& grad_out, const Tensor& input,
                                            const Tensor& mean, const Tensor& rstd,
                                            const OptT& gamma, const OptT& beta,
                                            std::array<bool, 3> output_mask) {
  auto r = layer_norm_bwd(grad_out, input, mean, rstd, gamma, beta, output_mask, std::nullopt);
  const bool dg = output_mask[1] && has(gamma), db = output_mask[2] && has(beta);
  return {output_mask[0] ? OptT(std::get<0>(r)) : std::nullopt,
          dg ? OptT(std::get<1>(r)) : std::nullopt, db ? OptT(std::get<2>(r)) : std::nullopt};
}

std::tuple<Tensor, Tensor> rms_norm_bwd(const Tensor& grad_out, const Tensor& input,
                                        const Tensor& rstd, const OptT& weight,
                                        std::array<bool, 2> output_mask, const OptT& grad_extra) {
  const Shape s = check_input(input, "input", false);
  check_input(grad_out, "grad_output", false);
  TORCH_CHECK(grad_out.sizes() == input.sizes(), "grad_output shape must match input shape");
  TORCH_CHECK(grad_out.scalar_type() == input.scalar_type(),
              "grad_output dtype must match input dtype");
  check_stats(rstd, s.rows, input, "rstd");
  check_param(weight, input, s.cols, "weight");
  if (has(grad_extra)) {
    check_input(*grad_extra, "grad_extra", false);
    TORCH_CHECK(grad_extra->sizes() == input.sizes() &&
                    grad_extra->scalar_type() == input.scalar_type(),
                "grad_extra must match the input's shape and dtype");
  }
  c10::hip::HIPGuard guard(input.device().index());
  const bool want_dx = output_mask[0];
  const bool want_dw = output_mask[1] && has(weight);
  Tensor dx = want_dx ? at::empty_like(input) : at::empty({0}, input.options());
  Tensor dw = want_dw ? at::empty_like(*weight) : at::empty({0}, input.options());
  Tensor ws;
  ws = workspace_for(input, s.rows, s.cols);
  check(fln_rmsnorm_backward(grad_out.data_ptr(), input.data_ptr(), rstd.data_ptr<float>(),
                             ptr_or_null(weight), ptr_or_null(grad_extra),
                             want_dx ? dx.data_ptr() : nullptr, want_dw ? dw.data_ptr() : nullptr,
                             s.rows, s.cols, dtype_code(input), dtype_code(input),
                             ws.defined() ? ws.data_ptr() : nullptr,
                             ws.defined() ? static_cast<size_t>(ws.numel()) * 4 : 0,
                             stream_of(input)),
        "rms_norm backward");
  return {dx, dw};
}

// ------------------------------------------------------------------------------------------
// Host utilities (csrc/layernorm_cuda.cpp:144-195).
// ------------------------------------------------------------------------------------------
int64_t get_memory_usage(int batch_size, int hidden_size, bool use_mixed_precision) {
  return fln_get_memory_usage(batch_size, hidden_size, use_mixed_precision ? 1 : 0);
}

std::string get_performance_hints(int batch_size, int hidden_size) {
  const int n = fln_get_performance_hints(batch_size, hidden_size, nullptr, 0);
  std::string s(static_cast<size_t>(n) + 1, '\0');
  fln_get_performance_hints(batch_size, hidden_size, s.data(), s.size());
  s.resize(static_cast<size_t>(n));
  return s;
}

// ------------------------------------------------------------------------------------------
// LayerNorm with autograd in C++: the eager path of FusedLayerNorm / fused_layer_norm.  A
// Python torch.autograd.Function plus an operator call cost ~10 us per forward on the host (the
// GPU work at BERT shapes is ~3 us).  Here the output gets a graph node of its own, built the way
// PyTorch's generated autograd code builds one (edges to the inputs that require grad, saved
// variables, no type-erased context), and the kernels are called directly.  It saves what the
// reference's FusedLayerNormFunction saves (input, weight, bias, mean, rstd:
// fused_layernorm/layernorm.py:76; mean and rstd here as the two rows of one fp32 tensor).
// torch.compile keeps the fused_layernorm::layer_norm_fwd / layer_norm_bwd operators (the
// Python side chooses).
// ------------------------------------------------------------------------------------------
struct FusedLayerNormBackward : public torch::autograd::Node {
  torch::autograd::SavedVariable x_, w_, b_, stats_;
  bool has_w = false, has_b = false;

  torch::autograd::variable_list apply(torch::autograd::variable_list&& grads) override {
    std::lock_guard<std::mutex> lock(mutex_);
    const Tensor x = x_.unpack(), stats = stats_.unpack();
    const OptT w = has_w ? OptT(w_.unpack()) : std::nullopt;
    const OptT b = has_b ? OptT(b_.unpack()) : std::nullopt;
    const std::array<bool, 3> mask{task_should_compute_output(0),
                                   has_w && task_should_compute_output(1),
                                   has_b && task_should_compute_output(2)};
    if (!grads[0].defined() || !(mask[0] || mask[1] || mask[2])) return {Tensor(), Tensor(), Tensor()};
    const Tensor dy = grads[0].is_contiguous() ? grads[0] : grads[0].contiguous();
    auto r = layer_norm_bwd(dy, x, stats[0], stats[1], w, b, mask, std::nullopt);
    return {mask[0] ? std::get<0>(r) : Tensor(), mask[1] ? std::get<1>(r) : Tensor(),
            mask[2] ? std::get<2>(r) : Tensor()};
  }
  std::string name() const override { return "FusedLayerNormBackward"; }
  void release_variables() override {
    std::lock_guard<std::mutex> lock(mutex_);
    x_.reset_data();
    w_.reset_data();
    b_.reset_data();
    stats_.reset_data();
  }
};

// FusedLayerNorm.forward's eager call: LayerNorm over the last dimension, which must equal
// `normalized` (torch.nn.functional.layer_norm's error otherwise), with autograd.
Tensor layer_norm_autograd(const Tensor& input, int64_t normalized, const OptT& weight,
                           const OptT& bias, double eps) {
  TORCH_CHECK(input.dim() >= 1 && input.size(-1) == normalized,
              "Given normalized_shape=[", normalized, "], expected input with shape [*, ",
              normalized, "], but got input of size", input.sizes());
  const Tensor x = input.is_contiguous() ? input : input.contiguous();
  const Shape s = check_input(x, "input", true);
  check_param(weight, x, s.cols, "weight");
  check_param(bias, x, s.cols, "bias");
  c10::hip::HIPGuard guard(x.device().index());
  Tensor y = at::empty_like(x);
  Tensor stats = at::empty({2, s.rows}, x.options().dtype(at::kFloat));  // mean, rstd
  float* st = stats.data_ptr<float>();
  check(fln_layernorm_forward(x.data_ptr(), ptr_or_null(weight), ptr_or_null(bias),
                              y.data_ptr(), st, st + s.rows, s.rows, s.cols, dtype_code(x),
                              static_cast<float>(eps), stream_of(x)),
        "layer_norm forward");
  const bool wg = has(weight) && weight->requires_grad();
  const bool bg = has(bias) && bias->requires_grad();
  if (c10::GradMode::is_enabled() && (x.requires_grad() || wg || bg)) {
    std::shared_ptr<FusedLayerNormBackward> node(new FusedLayerNormBackward(),
                                                 torch::autograd::deleteNode);
    node->set_next_edges(torch::autograd::collect_next_edges(
        x, has(weight) ? *weight : Tensor(), has(bias) ? *bias : Tensor()));
    node->x_ = torch::autograd::SavedVariable(x, false);
    node->stats_ = torch::autograd::SavedVariable(stats, false);
    node->has_w = has(weight);
    node->has_b = has(bias);
    if (node->has_w) node->w_ = torch::autograd::SavedVariable(*weight, false);
    if (node->has_b) node->b_ = torch::autograd::SavedVariable(*bias, false);
    torch::autograd::set_history(y, node);
  }
  return y;
}

// RMSNorm with autograd in C++: the eager path of FusedRMSNorm / fused_rms_norm, built like
// layer_norm_autograd (saves input, weight, rstd).
struct FusedRMSNormBackward : public torch::autograd::Node {
  torch::autograd::SavedVariable x_, w_, rstd_;
  bool has_w = false;

  torch::autograd::variable_list apply(torch::autograd::variable_list&& grads) override {
    std::lock_guard<std::mutex> lock(mutex_);
    const Tensor x = x_.unpack(), rstd = rstd_.unpack();
    const OptT w = has_w ? OptT(w_.unpack()) : std::nullopt;
    const std::array<bool, 2> mask{task_should_compute_output(0),
                                   has_w && task_should_compute_output(1)};
    if (!grads[0].defined() || !(mask[0] || mask[1])) return {Tensor(), Tensor()};
    const Tensor dy = grads[0].is_contiguous() ? grads[0] : grads[0].contiguous();
    auto r = rms_norm_bwd(dy, x, rstd, w, mask, std::nullopt);
    return {mask[0] ? std::get<0>(r) : Tensor(), mask[1] ? std::get<1>(r) : Tensor()};
  }
  std::string name() const override { return "FusedRMSNormBackward"; }
  void release_variables() override {
    std::lock_guard<std::mutex> lock(mutex_);
    x_.reset_data();
    w_.reset_data();
    rstd_.reset_data();
  }
};

Tensor rms_norm_autograd(const Tensor& input, int64_t normalized, const OptT& weight,
                         double eps) {
  TORCH_CHECK(input.dim() >= 1 && input.size(-1) == normalized,
              "Given normalized_shape=[", normalized, "], expected input with shape [*, ",
              normalized, "], but got input of size", input.sizes());
  const Tensor x = input.is_contiguous() ? input : input.contiguous();
  auto r = rms_norm_fwd(x, weight, eps);
  Tensor y = std::get<0>(r);
  const bool wg = has(weight) && weight->requires_grad();
  if (c10::GradMode::is_enabled() && (x.requires_grad() || wg)) {
    std::shared_ptr<FusedRMSNormBackward> node(new FusedRMSNormBackward(),
                                               torch::autograd::deleteNode);
    node->set_next_edges(
        torch::autograd::collect_next_edges(x, has(weight) ? *weight : Tensor()));
    node->x_ = torch::autograd::SavedVariable(x, false);
    node->rstd_ = torch::autograd::SavedVariable(std::get<1>(r), false);
    node->has_w = has(weight);
    if (node->has_w) node->w_ = torch::autograd::SavedVariable(*weight, false);
    torch::autograd::set_history(y, node);
  }
  return y;
}

// The forward launch plan (fln_forward_plan): (route, vector_elems, waves_per_row,
// vectors_per_lane, exact, threads) for a contiguous, aligned input; backs
// fused_layernorm.functional.get_optimal_config (reference fused_layernorm/functional.py:47-74).
std::tuple<int, int, int, int, bool, int> forward_plan(int64_t rows, int64_t cols, int dtype,
                                                       int fp8, bool residual, int gelu,
                                                       int num_cus) {
  fln_forward_plan_t plan{};
  check(fln_forward_plan(rows, cols, dtype, fp8, residual ? 1 : 0, gelu, num_cus, &plan),
        "forward_plan");
  return {plan.route, plan.vector_elems, plan.waves_per_row, plan.vectors_per_lane,
          plan.exact != 0, plan.threads};
}

}  // namespace

// Operator schemas (namespace fused_layernorm): the torch.compile-visible surface.  Fake
// (meta) kernels and autograd formulas are registered from Python (fused_layernorm/ops.py).
TORCH_LIBRARY(fused_layernorm, m) {
  m.def("layer_norm_fwd(Tensor input, Tensor? weight, Tensor? bias, float eps) "
        "-> (Tensor, Tensor, Tensor)");
  m.def("layer_norm_bwd(Tensor grad_out, Tensor input, Tensor mean, Tensor rstd, "
        "Tensor? weight, Tensor? bias, bool[3] output_mask, Tensor? grad_extra) "
        "-> (Tensor, Tensor, Tensor)");
  m.def("layer_norm_gelu_fwd(Tensor input, Tensor? weight, Tensor? bias, float eps, "
        "str approximate) -> (Tensor, Tensor, Tensor)");
  m.def("layer_norm_gelu_bwd(Tensor grad_out, Tensor input, Tensor mean, Tensor rstd, "
        "Tensor? weight, Tensor? bias, str approximate, bool[3] output_mask) "
        "-> (Tensor, Tensor, Tensor)");
  m.def("rms_norm_fwd(Tensor input, Tensor? weight, float eps) -> (Tensor, Tensor)");
  m.def("rms_norm_bwd(Tensor grad_out, Tensor input, Tensor rstd, Tensor? weight, "
        "bool[2] output_mask, Tensor? grad_extra) -> (Tensor, Tensor)");
  m.def("add_layer_norm_fwd(Tensor input, Tensor residual, Tensor? weight, Tensor? bias, "
        "float eps) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("add_rms_norm_fwd(Tensor input, Tensor residual, Tensor? weight, float eps) "
        "-> (Tensor, Tensor, Tensor)");
  m.def("layer_norm_fp8_fwd(Tensor input, Tensor? weight, Tensor? bias, float eps) "
        "-> (Tensor, Tensor)");
  m.def("rms_norm_fp8_fwd(Tensor input, Tensor? weight, float eps) -> (Tensor, Tensor)");
  m.def("add_layer_norm_fp8_fwd(Tensor input, Tensor residual, Tensor? weight, Tensor? bias, "
        "float eps) -> (Tensor, Tensor, Tensor)");
  m.def("add_rms_norm_fp8_fwd(Tensor input, Tensor residual, Tensor? weight, float eps) "
        "-> (Tensor, Tensor, Tensor)");
  m.def("layer_norm_mxfp8_fwd(Tensor input, Tensor? weight, Tensor? bias, float eps) "
        "-> (Tensor, Tensor)");
  m.def("rms_norm_mxfp8_fwd(Tensor input, Tensor? weight, float eps) -> (Tensor, Tensor)");
  m.def("add_rms_norm_mxfp8_fwd(Tensor input, Tensor residual, Tensor? weight, float eps) "
        "-> (Tensor, Tensor, Tensor)");
}

// GPU tensors of PyTorch-ROCm carry the CUDA dispatch key.
TORCH_LIBRARY_IMPL(fused_layernorm, CUDA, m) {
  m.impl("layer_norm_fwd", &layer_norm_fwd);
  m.impl("layer_norm_bwd", &layer_norm_bwd);
  m.impl("layer_norm_gelu_fwd", &layer_norm_gelu_fwd);
  m.impl("layer_norm_gelu_bwd", &layer_norm_gelu_bwd);
  m.impl("rms_norm_fwd", &rms_norm_fwd);
  m.impl("rms_norm_bwd", &rms_norm_bwd);
  m.impl("add_layer_norm_fwd", &add_layer_norm_fwd);
  m.impl("add_rms_norm_fwd", &add_rms_norm_fwd);
  m.impl("layer_norm_fp8_fwd", &layer_norm_fp8_fwd);
  m.impl("rms_norm_fp8_fwd", &rms_norm_fp8_fwd);
  m.impl("add_layer_norm_fp8_fwd", &add_layer_norm_fp8_fwd);
  m.impl("add_rms_norm_fp8_fwd", &add_rms_norm_fp8_fwd);
  m.impl("layer_norm_mxfp8_fwd", &layer_norm_mxfp8_fwd);
  m.impl("rms_norm_mxfp8_fwd", &rms_norm_mxfp8_fwd);
  m.impl("add_rms_norm_mxfp8_fwd", &add_rms_norm_mxfp8_fwd);
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Fused LayerNorm / RMSNorm for AMD Instinct MI355X (gfx950), HIP kernels";
  // Built path of the reference (csrc/bindings.cpp:41-44); arguments are named so both the
  // positional style of the reference's scripts and `eps=` keywords work.
  m.def("layernorm", &layernorm, "LayerNorm forward", py::arg("input"), py::arg("gamma"),
        py::arg("beta"), py::arg("eps") = 1e-5);
  m.def("layernorm_gelu", &layernorm_gelu, "LayerNorm + GELU (tanh form by default)",
        py::arg("input"), py::arg("gamma"), py::arg("beta"), py::arg("eps") = 1e-5,
        py::arg("approximate") = "tanh");
  // Training path the reference's Python package calls (csrc/layernorm_cuda.cpp:198-227).
  m.def("forward", &forward, "LayerNorm forward -> [out, mean, rstd]", py::arg("input"),
        py::arg("gamma") = py::none(), py::arg("beta") = py::none(),
        py::arg("epsilon") = 1e-5);
  m.def("backward", &backward, "LayerNorm backward -> [grad_input, grad_gamma, grad_beta]",
        py::arg("grad_output"), py::arg("input"), py::arg("mean"), py::arg("rstd"),
        py::arg("gamma") = py::none(), py::arg("beta") = py::none(),
        py::arg("output_mask") = std::array<bool, 3>{true, true, true});
  m.def("get_memory_usage", &get_memory_usage, "Estimate memory usage",
        py::arg("batch_size"), py::arg("hidden_size"), py::arg("use_mixed_precision") = false);
  m.def("get_performance_hints", &get_performance_hints, "Get performance optimization hints",
        py::arg("batch_size"), py::arg("hidden_size"));
  // New entry points on the same path.
  m.def("rms_norm_forward", &rms_norm_fwd, "RMSNorm forward -> (out, rstd)", py::arg("input"),
        py::arg("weight") = py::none(), py::arg("eps") = 1e-6);
  m.def("rms_norm_backward", &rms_norm_bwd, "RMSNorm backward -> (grad_input, grad_weight)",
        py::arg("grad_output"), py::arg("input"), py::arg("rstd"),
        py::arg("weight") = py::none(),
        py::arg("output_mask") = std::array<bool, 2>{true, true},
        py::arg("grad_extra") = py::none());
  m.def("add_layernorm_forward", &add_layer_norm_fwd,
        "Residual add + LayerNorm -> (out, residual_sum, mean, rstd)", py::arg("input"),
        py::arg("residual"), py::arg("gamma") = py::none(), py::arg("beta") = py::none(),
        py::arg("eps") = 1e-5);
  m.def("add_rmsnorm_forward", &add_rms_norm_fwd,
        "Residual add + RMSNorm -> (out, residual_sum, rstd)", py::arg("input"),
        py::arg("residual"), py::arg("weight") = py::none(), py::arg("eps") = 1e-6);
  m.def("layernorm_fp8_forward", &layer_norm_fp8_fwd,
        "LayerNorm with OCP fp8 e4m3fn output -> (codes, per-row scale)", py::arg("input"),
        py::arg("gamma") = py::none(), py::arg("beta") = py::none(), py::arg("eps") = 1e-5);
  m.def("rmsnorm_fp8_forward", &rms_norm_fp8_fwd,
        "RMSNorm with OCP fp8 e4m3fn output -> (codes, per-row scale)", py::arg("input"),
        py::arg("weight") = py::none(), py::arg("eps") = 1e-6);
  m.def("add_layernorm_fp8_forward", &add_layer_norm_fp8_fwd,
        "Residual add + LayerNorm with fp8 output -> (codes, per-row scale, residual_sum)",
        py::arg("input"), py::arg("residual"), py::arg("gamma") = py::none(),
        py::arg("beta") = py::none(), py::arg("eps") = 1e-5);
  m.def("add_rmsnorm_fp8_forward", &add_rms_norm_fp8_fwd,
        "Residual add + RMSNorm with fp8 output -> (codes, per-row scale, residual_sum)",
        py::arg("input"), py::arg("residual"), py::arg("weight") = py::none(),
        py::arg("eps") = 1e-6);
  m.def("layernorm_mxfp8_forward", &layer_norm_mxfp8_fwd,
        "LayerNorm with OCP MX fp8 (E4M3) output -> (codes, E8M0 block scales)",
        py::arg("input"), py::arg("gamma") = py::none(), py::arg("beta") = py::none(),
        py::arg("eps") = 1e-5);
  m.def("rmsnorm_mxfp8_forward", &rms_norm_mxfp8_fwd,
        "RMSNorm with OCP MX fp8 (E4M3) output -> (codes, E8M0 block scales)",
        py::arg("input"), py::arg("weight") = py::none(), py::arg("eps") = 1e-6);
  m.def("add_rmsnorm_mxfp8_forward", &add_rms_norm_mxfp8_fwd,
        "Residual add + RMSNorm with OCP MX fp8 output -> (codes, block scales, residual_sum)",
        py::arg("input"), py::arg("residual"), py::arg("weight") = py::none(),
        py::arg("eps") = 1e-6);
  m.def("layer_norm_autograd", &layer_norm_autograd,
        "LayerNorm over the last dimension with autograd in C++ (FusedLayerNorm's eager path)",
        py::arg("input"), py::arg("normalized"), py::arg("weight") = py::none(),
        py::arg("bias") = py::none(), py::arg("eps") = 1e-5);
  m.def("rms_norm_autograd", &rms_norm_autograd,
        "RMSNorm over the last dimension with autograd in C++ (FusedRMSNorm's eager path)",
        py::arg("input"), py::arg("normalized"), py::arg("weight") = py::none(),
        py::arg("eps") = 1e-6);
  m.def("forward_plan", &forward_plan,
        "Forward launch plan -> (route, vector_elems, waves_per_row, vectors_per_lane, exact, "
        "threads); dtype / gelu are the C-ABI codes, num_cus 0 = the current device",
        py::arg("rows"), py::arg("cols"), py::arg("dtype"), py::arg("fp8") = 0,
        py::arg("residual") = false, py::arg("gelu") = 0, py::arg("num_cus") = 0);
  m.attr("__version__") = fln_version();
  // The reference exports the CUDA runtime version under this name; here it is HIP's.
  m.attr("__cuda_version__") = fln_hip_version();
  m.attr("__hip_version__") = fln_hip_version();
}
