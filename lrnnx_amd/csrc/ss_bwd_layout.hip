// Workspace layout queries of the real selective-scan backward (host only).
#include "ss_bwd_impl.h"
namespace lrnnx {
int64_t ssf_bwd_segments(const lrnnx_selective_scan_args&);  // ssf_bwd_f32.hip
SSGeom ssf_bwd_geometry(const lrnnx_selective_scan_args&);   // ssf_bwd_f32.hip

// The layout of the fast backward (its split of L, its channel blocks) when
// it covers the call.  The general kernels lay out the same sections with one
// segment and their own channel blocks, which never needs more room; they
// take the checkpoints through their pointer, so a rebuild placed by this
// layout is found either way.
int64_t ss_bwd_ws_bytes(const lrnnx_selective_scan_args& a) {
  return ss_bwd_ws(a, ssf_bwd_geometry(a), a.ckpt == nullptr, ssf_bwd_segments(a)).total * (int64_t)sizeof(float);
}
int64_t ss_bwd_ckpt_offset_bytes(const lrnnx_selective_scan_args& a) {
  return ss_bwd_ws(a, ssf_bwd_geometry(a), true, ssf_bwd_segments(a)).ckpt * (int64_t)sizeof(float);
}
// Section of the checkpoint rebuild's forward split (offset; its size in *bytes, 0 if none).
int64_t ss_bwd_fws_offset_bytes(const lrnnx_selective_scan_args& a, int64_t* bytes) {
  const SSBwdWs w = ss_bwd_ws(a, ssf_bwd_geometry(a), true, ssf_bwd_segments(a));
  *bytes = w.fws_floats * (int64_t)sizeof(float);
  return w.fws * (int64_t)sizeof(float);
}
}  // namespace lrnnx
