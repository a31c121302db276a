// Workspace layout queries of the real selective-scan backward (host only).
#include "ss_bwd_impl.h"
namespace lrnnx {
int64_t ss_bwd_ws_bytes(const lrnnx_selective_scan_args& a) {
  return ss_bwd_ws(a, ss_geom(a), a.ckpt == nullptr).total * (int64_t)sizeof(float);
}
int64_t ss_bwd_ckpt_offset_bytes(const lrnnx_selective_scan_args& a) {
  return ss_bwd_ws(a, ss_geom(a), true).ckpt * (int64_t)sizeof(float);
}
}  // namespace lrnnx
