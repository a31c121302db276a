// Selective scan with complex weights: backward (instantiation unit; kernels in ssc_impl.h).
#include "ssc_impl.h"

namespace lrnnx {

hipError_t ssc_fwd_launch(const lrnnx_selective_scan_args& a, hipStream_t st);

int64_t ssc_bwd_ws_bytes(const lrnnx_selective_scan_args& a) {
  return ssc::ssc_bwd_ws(a, ssc::ssc_geom(a), a.ckpt == nullptr).total * (int64_t)sizeof(float);
}

hipError_t ssc_bwd_launch(const lrnnx_selective_scan_args& a, float* ws, const float* ckp, hipStream_t st) {
  const ssc::SSCGeom g = ssc::ssc_geom(a);
  const ssc::SSCBwdWs wo = ssc::ssc_bwd_ws(a, g, ckp == nullptr);
  if (ckp == nullptr) {  // rebuild the checkpoints with a forward that writes nothing else
    lrnnx_selective_scan_args f = a;
    f.out.ptr = nullptr;
    f.out_z.ptr = nullptr;
    f.z.ptr = nullptr;
    f.x = nullptr;
    f.ckpt = ws + wo.ckpt;
    hipError_t e = ssc_fwd_launch(f, st);
    if (e != hipSuccess) return e;
    ckp = ws + wo.ckpt;
  }
  return ssc::ssc_dispatch<true>(a, g, ws, &wo, ckp, st);
}

}  // namespace lrnnx
