// Selective scan forward fast path (ssf_fwd_impl.h), f16 I/O (instantiation unit).
#include "ssf_fwd_impl.h"
namespace lrnnx {
// Launches the fast path when it covers the call; returns false otherwise.
bool ssf_fwd_f16(const lrnnx_selective_scan_args& a, hipStream_t st, hipError_t* err) {
  if (!ssf_fwd_eligible<f16>(a)) return false;
  *err = ssf_fwd_launch<f16>(a, ss_geom(a).n_ck, st);
  return true;
}
}  // namespace lrnnx
