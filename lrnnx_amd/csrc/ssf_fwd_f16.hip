// Selective scan forward fast path (ssf_fwd_impl.h), f16 I/O (instantiation unit).
#include "ssf_fwd_impl.h"
namespace lrnnx {
// Launches the fast path when it covers the call; returns false otherwise.
bool ssf_fwd_f16(const lrnnx_selective_scan_args& a, hipStream_t st, hipError_t* err) {
  if (!ssf_fwd_eligible<f16>(a)) return false;
  *err = ssf_fwd_launch<f16>(a, ss_geom(a).n_ck, st);
  return true;
}

// Checkpoint rebuild of a backward given no checkpoints, on the fast
// forward's states-only kernel: into `ckpt` (the workspace's section), split
// like the forward on small grids (`fws`: the section for its summaries) or
// chunk-parallel from the x carries; returns false when the fast forward does
// not cover the call.
bool ssf_ckpt_rebuild_f16(const lrnnx_selective_scan_args& a, float* ckpt, float* fws, int64_t fws_bytes,
                        const float* x, hipStream_t st, hipError_t* err) {
  if (!ssf::shape_ok<f16>(a, ssf::tile_steps<f16>(), true)) return false;
  lrnnx_selective_scan_args f = a;
  f.ckpt = ckpt;
  f.out.ptr = nullptr;
  f.out_z.ptr = nullptr;
  f.z.ptr = nullptr;
  f.x = nullptr;
  f.workspace = fws;
  f.workspace_bytes = fws_bytes;
  *err = ssf_fwd_launch<f16>(f, ss_geom(a).n_ck, st, true, x);
  return true;
}
}  // namespace lrnnx
