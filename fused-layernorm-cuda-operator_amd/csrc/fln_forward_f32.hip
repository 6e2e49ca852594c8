// fln_forward_f32.hip -- forward instantiations for float I/O.
#include "fln_forward_impl.h"

namespace fln {
int launch_forward_f32(const FwdParams& p, bool out_fp8, hipStream_t s) {
  return out_fp8 ? detail::dispatch_typed<float, true>(p, s) : detail::dispatch_typed<float, false>(p, s);
}
}  // namespace fln
