// Complex fp32 helpers and the per-element discretisation of the simplified
// (S5 / LRU) scan, shared by the generic and the fast simplified-scan kernels.
#pragma once
#include "common.h"

namespace lrnnx {

struct cf {
  float r, i;
};
__device__ __forceinline__ cf cmake(float r, float i) { return cf{r, i}; }
__device__ __forceinline__ cf cadd(cf a, cf b) { return cf{a.r + b.r, a.i + b.i}; }
__device__ __forceinline__ cf csub(cf a, cf b) { return cf{a.r - b.r, a.i - b.i}; }
__device__ __forceinline__ cf cmul(cf a, cf b) { return cf{a.r * b.r - a.i * b.i, a.r * b.i + a.i * b.r}; }
__device__ __forceinline__ cf cconj(cf a) { return cf{a.r, -a.i}; }
__device__ __forceinline__ cf cscale(cf a, float s) { return cf{a.r * s, a.i * s}; }
// a * b + c
__device__ __forceinline__ cf cfma(cf a, cf b, cf c) {
  return cf{fmaf(a.r, b.r, fmaf(-a.i, b.i, c.r)), fmaf(a.r, b.i, fmaf(a.i, b.r, c.i))};
}
__device__ __forceinline__ cf cdiv(cf a, cf b) {
  const float den = b.r * b.r + b.i * b.i;
  return cf{(a.r * b.r + a.i * b.i) / den, (a.i * b.r - a.r * b.i) / den};
}
__device__ __forceinline__ cf cexp_(cf z) {
  float s, c;
  sincosf(z.i, &s, &c);
  const float e = expf(z.r);
  return cf{e * c, e * s};
}
__device__ __forceinline__ cf ld(const float* p) {
  const float2 v = *reinterpret_cast<const float2*>(p);
  return cf{v.x, v.y};
}
__device__ __forceinline__ void st(float* p, cf v) { *reinterpret_cast<float2*>(p) = make_float2(v.r, v.i); }

// A_bar and beta for one element (simplified_scan.cuh:198-224)
template <int kMethod>
__device__ __forceinline__ void sdisc(float dtA, float dl, cf A, cf& Ab, cf& beta) {
  const cf one = cmake(1.f, 0.f);
  if constexpr (kMethod == LRNNX_BILINEAR) {
    const cf vA = cscale(A, 0.5f * dtA);
    Ab = cdiv(cadd(one, vA), csub(one, vA));
    beta = cdiv(cmake(dl, 0.f), csub(one, cscale(A, 0.5f * dl)));
  } else {
    Ab = cexp_(cscale(A, dtA));
    if constexpr (kMethod == LRNNX_ZOH) beta = cdiv(csub(cexp_(cscale(A, dl)), one), A);
    else beta = one;
  }
}

}  // namespace lrnnx
