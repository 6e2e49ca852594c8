// fln_forward_bf16.hip -- forward instantiations for __bf16 I/O.
#include "fln_forward_impl.h"

namespace fln {
int launch_forward_bf16(const FwdParams& p, bool out_fp8, hipStream_t s) {
  return out_fp8 ? detail::dispatch_typed<__bf16, true>(p, s) : detail::dispatch_typed<__bf16, false>(p, s);
}
}  // namespace fln
