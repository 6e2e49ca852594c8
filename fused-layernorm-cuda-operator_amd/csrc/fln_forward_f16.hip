// fln_forward_f16.hip -- forward instantiations for _Float16 I/O.
#include "fln_forward_impl.h"

namespace fln {
int launch_forward_f16(const FwdParams& p, bool out_fp8, hipStream_t s) {
  return out_fp8 ? detail::dispatch_typed<_Float16, true>(p, s) : detail::dispatch_typed<_Float16, false>(p, s);
}
}  // namespace fln
