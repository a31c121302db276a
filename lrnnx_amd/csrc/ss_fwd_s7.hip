// Selective scan forward, method "s7", fp32 I/O (instantiation unit; the
// reference builds every method for fp32 input only,
// csrc/selective_scan/forward_kernels/*.cu:3).
#include "ss_fwd_impl.h"
namespace lrnnx {
bool rgf_ok(const lrnnx_selective_scan_args&);                    // rglru_fast.hip
hipError_t rgf_fwd(const lrnnx_selective_scan_args&, hipStream_t);

hipError_t ss_fwd_s7_f32(const lrnnx_selective_scan_args& a, hipStream_t st) {
  if (rgf_ok(a)) return rgf_fwd(a, st);  // one state per channel: lanes along L
  return launch_fwd_s<float, LRNNX_S7>(a, ss_geom(a), st);
}
}  // namespace lrnnx
