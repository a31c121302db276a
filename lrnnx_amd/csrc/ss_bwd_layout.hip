// Workspace layout queries of the real selective-scan backward (host only).
#include "ss_bwd_impl.h"
namespace lrnnx {
int64_t ssf_bwd_segments(const lrnnx_selective_scan_args&);  // ssf_bwd_f32.hip

// The layout of the fast backward's split of L when it applies (the general
// kernels use a prefix of it: the same sections with one segment).
int64_t ss_bwd_ws_bytes(const lrnnx_selective_scan_args& a) {
  return ss_bwd_ws(a, ss_geom(a), a.ckpt == nullptr, ssf_bwd_segments(a)).total * (int64_t)sizeof(float);
}
int64_t ss_bwd_ckpt_offset_bytes(const lrnnx_selective_scan_args& a) {
  return ss_bwd_ws(a, ss_geom(a), true, ssf_bwd_segments(a)).ckpt * (int64_t)sizeof(float);
}
// Section of the checkpoint rebuild's forward split (offset; its size in *bytes, 0 if none).
int64_t ss_bwd_fws_offset_bytes(const lrnnx_selective_scan_args& a, int64_t* bytes) {
  const SSBwdWs w = ss_bwd_ws(a, ss_geom(a), true, ssf_bwd_segments(a));
  *bytes = w.fws_floats * (int64_t)sizeof(float);
  return w.fws * (int64_t)sizeof(float);
}
}  // namespace lrnnx
