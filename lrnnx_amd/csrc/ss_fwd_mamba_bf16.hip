// Selective scan forward, method "mamba", bf16 I/O (instantiation unit).
#include "ss_fwd_impl.h"
namespace lrnnx {
hipError_t ss_fwd_mamba_bf16(const lrnnx_selective_scan_args& a, hipStream_t st) {
  return launch_fwd_s<bf16, LRNNX_MAMBA>(a, ss_geom(a), st);
}
}  // namespace lrnnx
