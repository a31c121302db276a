// Selective scan forward, method "dirac", fp32 I/O (instantiation unit; the
// reference builds every method for fp32 input only,
// csrc/selective_scan/forward_kernels/*.cu:3).
#include "ss_fwd_impl.h"
namespace lrnnx {
hipError_t ss_fwd_dirac_f32(const lrnnx_selective_scan_args& a, hipStream_t st) {
  return launch_fwd_s<float, LRNNX_DIRAC>(a, ss_geom(a), st);
}
}  // namespace lrnnx
