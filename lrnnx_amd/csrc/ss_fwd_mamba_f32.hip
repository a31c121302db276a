// Selective scan forward, method "mamba", f32 I/O (instantiation unit).
#include "ss_fwd_impl.h"
namespace lrnnx {
hipError_t ss_fwd_mamba_f32(const lrnnx_selective_scan_args& a, hipStream_t st) {
  return launch_fwd_s<float, LRNNX_MAMBA>(a, ss_geom(a), st);
}
}  // namespace lrnnx
