// fln_forward_f64.hip -- fp64 forward (looped kernel, fp64 accumulation).
#include "fln_forward_impl.h"

namespace fln {
int launch_forward_f64(const FwdParams& p, hipStream_t s) {
  return detail::launch_loop<double, double, 0>(p, s);
}
}  // namespace fln
