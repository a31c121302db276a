// Selective scan with complex weights: backward kernels with 2 state(s) per wave
// (instantiation unit; kernels in ssc_impl.h, launched from ssc_bwd.hip).
#include "ssc_impl.h"

namespace lrnnx {
namespace ssc {

hipError_t ssc_bwd_s2(const lrnnx_selective_scan_args& a, const SSCGeom& g, float* ws, const SSCBwdWs* wo,
                       const float* ckp, hipStream_t st) {
  return ssc_dispatch_m<2, true>(a, g, ws, wo, ckp, st);
}

}  // namespace ssc
}  // namespace lrnnx
