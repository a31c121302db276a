// Selective scan backward fast path (ssf_bwd_impl.h), f32 I/O (instantiation unit).
#include "ssf_bwd_impl.h"
namespace lrnnx {
// Launches the fast path (kernel + reductions) when it covers the call;
// returns false otherwise.
bool ssf_bwd_f32(const lrnnx_selective_scan_args& a, float* ws, const float* ckp, hipStream_t st, hipError_t* err) {
  if (!ssf_bwd_eligible<float>(a)) return false;
  *err = ssf_bwd_launch<float>(a, ws, ckp, st);
  return true;
}

// The backward's geometry for this call (the fast kernel's channel blocks
// when it covers the call), for the workspace layout queries.
SSGeom ssf_bwd_geometry(const lrnnx_selective_scan_args& a) {
  if (a.method == LRNNX_S7 || a.method == LRNNX_RGLRU || a.wtype != LRNNX_F32) return ss_geom(a);
  switch (a.itype) {
    case LRNNX_F32: return ssf_bwd_geom<float>(a);
    case LRNNX_BF16: return ssf_bwd_geom<bf16>(a);
    default: return ssf_bwd_geom<f16>(a);
  }
}

// Segments of the fast backward's split of L for this call (1: no split),
// for the workspace layout queries.
int64_t ssf_bwd_segments(const lrnnx_selective_scan_args& a) {
  if (a.method == LRNNX_S7 || a.method == LRNNX_RGLRU || a.wtype != LRNNX_F32) return 1;
  switch (a.itype) {
    case LRNNX_F32: return ssf_bwd_segs<float>(a);
    case LRNNX_BF16: return ssf_bwd_segs<bf16>(a);
    default: return ssf_bwd_segs<f16>(a);
  }
}
}  // namespace lrnnx
