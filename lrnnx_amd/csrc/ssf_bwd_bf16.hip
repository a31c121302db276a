// Selective scan backward fast path (ssf_bwd_impl.h), bf16 I/O (instantiation unit).
#include "ssf_bwd_impl.h"
namespace lrnnx {
// Launches the fast path (kernel + reductions) when it covers the call;
// returns false otherwise.
bool ssf_bwd_bf16(const lrnnx_selective_scan_args& a, float* ws, const float* ckp, hipStream_t st, hipError_t* err) {
  if (!ssf_bwd_eligible<bf16>(a)) return false;
  *err = ssf_bwd_launch<bf16>(a, ws, ckp, st);
  return true;
}
}  // namespace lrnnx
