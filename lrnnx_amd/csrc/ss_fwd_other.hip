// Selective scan forward, methods zoh / bilinear / dirac / s7 / rglru, fp32 I/O
// (the reference instantiates every method for fp32 input only,
// csrc/selective_scan/forward_kernels/*.cu:3).
#include "ss_fwd_impl.h"
namespace lrnnx {
hipError_t ss_fwd_other_f32(const lrnnx_selective_scan_args& a, hipStream_t st) {
  const SSGeom g = ss_geom(a);
  switch (a.method) {
    case LRNNX_ZOH: return launch_fwd_s<float, LRNNX_ZOH>(a, g, st);
    case LRNNX_BILINEAR: return launch_fwd_s<float, LRNNX_BILINEAR>(a, g, st);
    case LRNNX_DIRAC: return launch_fwd_s<float, LRNNX_DIRAC>(a, g, st);
    case LRNNX_S7: return launch_fwd_s<float, LRNNX_S7>(a, g, st);
    case LRNNX_RGLRU: return launch_fwd_s<float, LRNNX_RGLRU>(a, g, st);
  }
  return hipErrorInvalidValue;
}
}  // namespace lrnnx
