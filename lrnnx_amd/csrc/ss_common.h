// Shared pieces of the selective-scan forward and backward kernels.
//
// Work decomposition (both directions):
//   * one workgroup = one batch row b and a block of CB <= 64 channels that
//     lie in a single B/C group (so B/C are wave-uniform);
//   * lane l of every wave owns channel d0 + l;
//   * wave w owns states [w*kS, w*kS + kS) and keeps their fp32 h in VGPRs;
//   * L is walked sequentially in tiles of kT steps staged through LDS
//     (coalesced 16-byte loads of u, delta, deltaA, z; B/C rows of the group).
// The sum over states (y, du, ddelta) crosses waves through LDS; the sum over
// channels (dB, dC) is a wave reduce-scatter followed by a deterministic
// second-stage reduction over channel blocks.
#pragma once

#include "common.h"

namespace lrnnx {

// Checkpoint interval by states per wave; the backward stores kS * kCk values
// of A_bar and h per lane, so kS * kCk <= 64 keeps that at <= 128 VGPRs and
// fits the per-lane dB/dC block into one 64-value reduce-scatter.  kS = 32 is
// the forward's fallback for d_state > 64 without a workspace (ss_geom); it
// writes the interval of the state-block backward (kS = 8) that reads them.
__host__ __device__ constexpr int ck_for(int kS) { return kS == 1 ? 16 : (kS == 32 ? 8 : 64 / kS); }
// forward tile length, sized so that every instantiation fits 160 KB of LDS
// (the backward's, a whole number of checkpoint intervals, is set in ss_bwd_kernel)
__host__ __device__ constexpr int tf_for(int kS) { return kS >= 32 ? 16 : 32; }
constexpr size_t kMaxLds = 160 * 1024;

// launch flags of the selective-scan kernels (computed on the host)
constexpr int kFlagAsyncIn = 1;     // every fetched tensor has 16-byte aligned rows (LDS-DMA usable)
constexpr int kFlagAlignedOut = 2;  // every written sequence tensor has 16-byte aligned rows

inline int pick_kS(int64_t N) {
  if (N <= 4) return 1;
  if (N <= 16) return 4;
  return 8;
}

__host__ __device__ constexpr bool exp_family_m(int m) {
  return m == LRNNX_MAMBA || m == LRNNX_DIRAC || m == LRNNX_ZOH;
}

// expm1(x) given e = exp(x): a degree-5 Taylor polynomial where |x| < 1/16
// (truncation error < 2e-9 relative), e - 1 elsewhere (cancellation costs at
// most ~2e-6 relative at |x| = 1/16, where |e - 1| > 0.06).
__device__ __forceinline__ float expm1_from(float x, float e) {
  const float p = x * fmaf(x, fmaf(x, fmaf(x, fmaf(x, 1.f / 120.f, 1.f / 24.f), 1.f / 6.f), 0.5f), 1.f);
  return fabsf(x) < 0.0625f ? p : e - 1.f;
}

// Per-(t, n) discretisation of a real state.  `dtA` is the step used for
// A_bar (deltaA when kDA, else equal to `dl`), `dl` the post-bias/softplus
// delta', `a2` the per-(d, n) prepared eigenvalue:
//   exp-based methods (mamba, dirac, zoh): A * log2(e);  bilinear: A;
//   rglru: log2(A);  s7: unused.
// `invA` is 1 / A (used by zoh).  Returns A_bar; writes the input factor beta
// so that the increment is beta * B_in * u (selective_scan.cuh:272-302).
// The exponentials are v_exp_f32 on a base-2 argument and the quotients
// v_rcp_f32 products (1 ulp each), well inside the fp32 parity tolerance.
template <int kMethod, bool kDA>
__device__ __forceinline__ float disc_real(float dtA, float dl, float a2, float Araw, float invA, float& beta) {
  if constexpr (kMethod == LRNNX_MAMBA) {
    beta = dl;
    return fast_exp2(dtA * a2);
  } else if constexpr (kMethod == LRNNX_DIRAC) {
    beta = 1.f;
    return fast_exp2(dtA * a2);
  } else if constexpr (kMethod == LRNNX_ZOH) {
    const float ab = fast_exp2(dtA * a2);
    const float eb = kDA ? fast_exp2(dl * a2) : ab;  // exp(delta' A)
    beta = expm1_from(dl * Araw, eb) * invA;
    return ab;
  } else if constexpr (kMethod == LRNNX_BILINEAR) {
    const float vA = 0.5f * dtA * Araw;
    const float rA = __builtin_amdgcn_rcpf(1.f - vA);
    beta = dl * (kDA ? __builtin_amdgcn_rcpf(1.f - 0.5f * dl * Araw) : rA);
    return (1.f + vA) * rA;
  } else if constexpr (kMethod == LRNNX_S7) {
    beta = 1.f;
    return 1.f - __builtin_amdgcn_rcpf(fmaf(dl, dl, 0.5f));
  } else {  // RGLRU: A_bar = A^delta, beta = sqrt(1 - A_bar^2)
    const float ab = fast_exp2(dl * a2);
    beta = __builtin_amdgcn_sqrtf(-expm1_from(dl * a2 * kLn2, ab) * (1.f + ab));  // 1 - ab^2 without cancellation
    return ab;
  }
}

template <int kMethod>
__device__ __forceinline__ float prep_a2(float A) {
  if constexpr (exp_family_m(kMethod)) return A * kLog2e;
  else if constexpr (kMethod == LRNNX_RGLRU) return __log2f(A);
  else return A;
}

// Whether A_bar of this method is exp(dtA * A) (then the running product of
// A_bar over a chunk is exp(A * sum dtA) and needs no per-step multiply).
template <int kMethod>
__host__ __device__ constexpr bool exp_family() {
  return exp_family_m(kMethod);
}

// Whether B (variable or constant) multiplies the input term
// (rglru ignores B on the input side, selective_scan.cuh:296-302).
template <int kMethod>
__host__ __device__ constexpr bool uses_B_input() { return kMethod != LRNNX_RGLRU; }

// Whether deltaA (when given) drives A_bar (s7 and rglru ignore it).
template <int kMethod>
__host__ __device__ constexpr bool uses_deltaA() {
  return kMethod != LRNNX_S7 && kMethod != LRNNX_RGLRU;
}

// Launch geometry shared by forward and backward.  d_state > 64 runs in
// state blocks: nsb workgroups per (channel block, b) along grid z, each with
// nW * kS state slots (the last block's tail is padding).  Their sums over
// states (y; the du / ddelta terms) are fp32 partials in a workspace, added in
// block order by a combine kernel.
struct SSGeom {
  int CB;        // channels per workgroup (<= 64, divides D/G when G > 1)
  int n_cb;      // channel blocks
  int kS, nW;    // states per wave, waves per workgroup
  int nsb;       // state blocks (1 for d_state <= 64)
  int ck;        // checkpoint interval (steps)
  int64_t n_ck;  // checkpoints per (b, d)
};

inline SSGeom ss_geom(const lrnnx_selective_scan_args& a) {
  SSGeom g;
  const int64_t ratio = a.var_B || a.var_C ? a.dim / a.n_groups : a.dim;
  if (a.n_groups <= 1 || !(a.var_B || a.var_C)) {
    g.CB = 64;
  } else {
    int cb = 64;
    while (cb > 1 && ratio % cb != 0) --cb;
    g.CB = cb;
  }
  g.n_cb = (int)((a.dim + g.CB - 1) / g.CB);
  g.kS = pick_kS(a.dstate);
  g.nsb = (int)((a.dstate + 63) / 64);
  const int64_t per_blk = (a.dstate + g.nsb - 1) / g.nsb;   // states per block, balanced
  g.nW = (int)((per_blk + g.kS - 1) / g.kS);
  g.ck = ck_for(g.kS);
  g.n_ck = (a.seqlen + g.ck - 1) / g.ck;
  return g;
}

// Bytes of forward workspace for the state blocks' partial y (0: one block).
inline int64_t ss_fwd_blocks_ws_bytes(const lrnnx_selective_scan_args& a) {
  const SSGeom g = ss_geom(a);
  return g.nsb > 1 ? (int64_t)g.nsb * a.batch * a.dim * a.seqlen * (int64_t)sizeof(float) : 0;
}

}  // namespace lrnnx
