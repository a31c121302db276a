// Selective scan backward, method "s7", fp32 I/O (instantiation unit;
// reference: csrc/selective_scan/backward_kernels/*.cu:3, fp32 only).
#include "ss_bwd_impl.h"
namespace lrnnx {
hipError_t ss_bwd_s7_f32(const lrnnx_selective_scan_args& a, float* ws, const float* ckp, hipStream_t st) {
  const SSGeom g = ss_geom(a);
  return launch_bwd_s<float, LRNNX_S7>(a, g, ws, ss_bwd_ws(a, g, a.ckpt == nullptr), ckp, st);
}
}  // namespace lrnnx
