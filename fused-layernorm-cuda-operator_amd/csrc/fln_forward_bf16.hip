// fln_forward_bf16.hip -- forward instantiations for __bf16 I/O.
#include "fln_forward_impl.h"

namespace fln {
int launch_forward_bf16(const FwdParams& p, bool out_fp8, hipStream_t s) {
  if (!out_fp8) return detail::dispatch_typed<__bf16, 0>(p, s);
  return p.mx ? detail::dispatch_typed<__bf16, 2>(p, s) : detail::dispatch_typed<__bf16, 1>(p, s);
}
int plan_forward_bf16(int64_t rows, int64_t cols, int fp8, bool res, int gelu, int64_t cus,
                      fln_forward_plan_t* out) {
  return detail::plan_query<__bf16>(rows, cols, fp8, res, gelu, cus, out);
}
}  // namespace fln
