// Selective scan backward, methods zoh / bilinear / dirac / s7 / rglru, fp32 I/O
// (reference: csrc/selective_scan/backward_kernels/*.cu:3, fp32 only).
#include "ss_bwd_impl.h"
namespace lrnnx {
hipError_t ss_bwd_other_f32(const lrnnx_selective_scan_args& a, float* ws, const float* ckp, hipStream_t st) {
  const SSGeom g = ss_geom(a);
  const SSBwdWs wo = ss_bwd_ws(a, g, a.ckpt == nullptr);
  switch (a.method) {
    case LRNNX_ZOH: return launch_bwd_s<float, LRNNX_ZOH>(a, g, ws, wo, ckp, st);
    case LRNNX_BILINEAR: return launch_bwd_s<float, LRNNX_BILINEAR>(a, g, ws, wo, ckp, st);
    case LRNNX_DIRAC: return launch_bwd_s<float, LRNNX_DIRAC>(a, g, ws, wo, ckp, st);
    case LRNNX_S7: return launch_bwd_s<float, LRNNX_S7>(a, g, ws, wo, ckp, st);
    case LRNNX_RGLRU: return launch_bwd_s<float, LRNNX_RGLRU>(a, g, ws, wo, ckp, st);
  }
  return hipErrorInvalidValue;
}
}  // namespace lrnnx
