// fln_forward_bf16.hip -- forward instantiations for __bf16 I/O.
#include "fln_forward_impl.h"

namespace fln {
int launch_forward_bf16(const FwdParams& p, bool out_fp8, hipStream_t s) {
  if (!out_fp8) return detail::dispatch_typed<__bf16, 0>(p, s);
  return p.mx ? detail::dispatch_typed<__bf16, 2>(p, s) : detail::dispatch_typed<__bf16, 1>(p, s);
}
}  // namespace fln
