// Selective scan with complex weights (placeholder until the complex kernels land).
#include "ss_common.h"
namespace lrnnx {
hipError_t ssc_fwd_launch(const lrnnx_selective_scan_args&, hipStream_t) { return hipErrorNotSupported; }
hipError_t ssc_bwd_launch(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t) {
  return hipErrorNotSupported;
}
int64_t ssc_ckpt_bytes(const lrnnx_selective_scan_args&) { return 0; }
int64_t ssc_bwd_ws_bytes(const lrnnx_selective_scan_args&) { return 0; }
}  // namespace lrnnx
