// Selective scan with complex weights: forward (instantiation unit; kernels in ssc_impl.h).
#include "ssc_impl.h"

namespace lrnnx {

hipError_t ssc_fwd_launch(const lrnnx_selective_scan_args& a, hipStream_t st) {
  return ssc::ssc_dispatch<false>(a, ssc::ssc_geom(a), nullptr, nullptr, nullptr, st);
}

int64_t ssc_ckpt_bytes(const lrnnx_selective_scan_args& a) {
  const ssc::SSCGeom g = ssc::ssc_geom(a);
  return a.batch * g.n_ck * a.dstate * a.dim * 2 * (int64_t)sizeof(float);
}

}  // namespace lrnnx
