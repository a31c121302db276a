// Selective scan backward, method "s7", fp32 I/O (instantiation unit;
// reference: csrc/selective_scan/backward_kernels/*.cu:3, fp32 only).
#include "ss_bwd_impl.h"
namespace lrnnx {
bool rgf_ok(const lrnnx_selective_scan_args&);                    // rglru_fast.hip
hipError_t rgf_bwd(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t);

hipError_t ss_bwd_s7_f32(const lrnnx_selective_scan_args& a, float* ws, const float* ckp, hipStream_t st) {
  if (rgf_ok(a)) return rgf_bwd(a, ws, ckp, st);  // one state per channel: lanes along L
  const SSGeom g = ss_geom(a);
  return launch_bwd_s<float, LRNNX_S7>(a, g, ws, ss_bwd_ws(a, g, a.ckpt == nullptr), ckp, st);
}
}  // namespace lrnnx
