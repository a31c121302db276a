// Selective scan forward fast path (ssf_fwd_impl.h), f32 I/O (instantiation unit).
#include "ssf_fwd_impl.h"
namespace lrnnx {
// Launches the fast path when it covers the call; returns false otherwise.
bool ssf_fwd_f32(const lrnnx_selective_scan_args& a, hipStream_t st, hipError_t* err) {
  if (!ssf_fwd_eligible<float>(a)) return false;
  *err = ssf_fwd_launch<float>(a, ss_geom(a).n_ck, st);
  return true;
}

// Forward workspace bytes of the fast path's L split (0 when it does not split).
int64_t ssf_fwd_workspace_bytes(const lrnnx_selective_scan_args& a) {
  switch (a.itype) {
    case LRNNX_F32: return ssf_fwd_ws_bytes<float>(a);
    case LRNNX_BF16: return ssf_fwd_ws_bytes<bf16>(a);
    default: return ssf_fwd_ws_bytes<f16>(a);
  }
}

// Checkpoint rebuild of a backward given no checkpoints, on the fast
// forward's states-only kernel: into `ckpt` (the workspace's section), split
// like the forward on small grids (`fws`: the section for its summaries) or
// chunk-parallel from the x carries; returns false when the fast forward does
// not cover the call.
bool ssf_ckpt_rebuild_f32(const lrnnx_selective_scan_args& a, float* ckpt, float* fws, int64_t fws_bytes,
                        const float* x, hipStream_t st, hipError_t* err) {
  if (!ssf::shape_ok<float>(a, ssf::tile_steps<float>(), true)) return false;
  lrnnx_selective_scan_args f = a;
  f.ckpt = ckpt;
  f.out.ptr = nullptr;
  f.out_z.ptr = nullptr;
  f.z.ptr = nullptr;
  f.x = nullptr;
  f.workspace = fws;
  f.workspace_bytes = fws_bytes;
  *err = ssf_fwd_launch<float>(f, ss_geom(a).n_ck, st, true, x);
  return true;
}
}  // namespace lrnnx
