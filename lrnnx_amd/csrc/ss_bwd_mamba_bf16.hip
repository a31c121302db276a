// Selective scan backward, method "mamba", bf16 I/O (instantiation unit).
#include "ss_bwd_impl.h"
namespace lrnnx {
hipError_t ss_bwd_mamba_bf16(const lrnnx_selective_scan_args& a, float* ws, const float* ckp, hipStream_t st) {
  const SSGeom g = ss_geom(a);
  return launch_bwd_s<bf16, LRNNX_MAMBA>(a, g, ws, ss_bwd_ws(a, g, a.ckpt == nullptr), ckp, st);
}
}  // namespace lrnnx
