// Selective scan forward, methods zoh / bilinear / dirac / s7 / rglru, fp32 I/O:
// dispatch to the per-method instantiation units (ss_fwd_<method>.hip).
#include "ss_common.h"
namespace lrnnx {
hipError_t ss_fwd_zoh_f32(const lrnnx_selective_scan_args&, hipStream_t);
hipError_t ss_fwd_bilinear_f32(const lrnnx_selective_scan_args&, hipStream_t);
hipError_t ss_fwd_dirac_f32(const lrnnx_selective_scan_args&, hipStream_t);
hipError_t ss_fwd_s7_f32(const lrnnx_selective_scan_args&, hipStream_t);
hipError_t ss_fwd_rglru_f32(const lrnnx_selective_scan_args&, hipStream_t);

hipError_t ss_fwd_other_f32(const lrnnx_selective_scan_args& a, hipStream_t st) {
  switch (a.method) {
    case LRNNX_ZOH: return ss_fwd_zoh_f32(a, st);
    case LRNNX_BILINEAR: return ss_fwd_bilinear_f32(a, st);
    case LRNNX_DIRAC: return ss_fwd_dirac_f32(a, st);
    case LRNNX_S7: return ss_fwd_s7_f32(a, st);
    case LRNNX_RGLRU: return ss_fwd_rglru_f32(a, st);
  }
  return hipErrorInvalidValue;
}
}  // namespace lrnnx
