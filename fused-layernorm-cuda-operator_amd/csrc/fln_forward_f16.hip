// fln_forward_f16.hip -- forward instantiations for _Float16 I/O.
#include "fln_forward_impl.h"

namespace fln {
int launch_forward_f16(const FwdParams& p, bool out_fp8, hipStream_t s) {
  if (!out_fp8) return detail::dispatch_typed<_Float16, 0>(p, s);
  return p.mx ? detail::dispatch_typed<_Float16, 2>(p, s)
              : detail::dispatch_typed<_Float16, 1>(p, s);
}
}  // namespace fln
