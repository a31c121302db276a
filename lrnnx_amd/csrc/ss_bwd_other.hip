// Selective scan backward, methods zoh / bilinear / dirac / s7 / rglru, fp32 I/O:
// dispatch to the per-method instantiation units (ss_bwd_<method>.hip).
#include "ss_common.h"
namespace lrnnx {
hipError_t ss_bwd_zoh_f32(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t);
hipError_t ss_bwd_bilinear_f32(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t);
hipError_t ss_bwd_dirac_f32(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t);
hipError_t ss_bwd_s7_f32(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t);
hipError_t ss_bwd_rglru_f32(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t);

hipError_t ss_bwd_other_f32(const lrnnx_selective_scan_args& a, float* ws, const float* ckp, hipStream_t st) {
  switch (a.method) {
    case LRNNX_ZOH: return ss_bwd_zoh_f32(a, ws, ckp, st);
    case LRNNX_BILINEAR: return ss_bwd_bilinear_f32(a, ws, ckp, st);
    case LRNNX_DIRAC: return ss_bwd_dirac_f32(a, ws, ckp, st);
    case LRNNX_S7: return ss_bwd_s7_f32(a, ws, ckp, st);
    case LRNNX_RGLRU: return ss_bwd_rglru_f32(a, ws, ckp, st);
  }
  return hipErrorInvalidValue;
}
}  // namespace lrnnx
