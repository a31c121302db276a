// Selective scan with complex weights: backward entry (workspace, checkpoint rebuild); the
// kernels for each number of states per wave are instantiated in ssc_bwd_s<kS>.hip, which
// compile in parallel.
#include "ssc_impl.h"

namespace lrnnx {
namespace ssc {
#define LRNNX_SSC_BWD_DECL(K)                                                                                   \
  hipError_t ssc_bwd_s##K(const lrnnx_selective_scan_args& a, const SSCGeom& g, float* ws, const SSCBwdWs* wo, \
                          const float* ckp, hipStream_t st);
LRNNX_SSC_BWD_DECL(1)
LRNNX_SSC_BWD_DECL(2)
LRNNX_SSC_BWD_DECL(4)
LRNNX_SSC_BWD_DECL(8)
LRNNX_SSC_BWD_DECL(16)
#undef LRNNX_SSC_BWD_DECL
}  // namespace ssc

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
  switch (g.kS) {
    case 1: return ssc::ssc_bwd_s1(a, g, ws, &wo, ckp, st);
    case 2: return ssc::ssc_bwd_s2(a, g, ws, &wo, ckp, st);
    case 4: return ssc::ssc_bwd_s4(a, g, ws, &wo, ckp, st);
    case 8: return ssc::ssc_bwd_s8(a, g, ws, &wo, ckp, st);
    case 16: return ssc::ssc_bwd_s16(a, g, ws, &wo, ckp, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace lrnnx
