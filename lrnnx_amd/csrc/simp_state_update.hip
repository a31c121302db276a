// One-token S5 decode update (gfx950).
//
// Semantics: reference simplified_state_update_ref
// (lrnnx/ops/triton/simplified_state_update.py:404-469), the pure-PyTorch
// statement of the Triton kernel at :13-251:
//   A_bar = (1 + dtA A / 2) / (1 - dtA A / 2)  (bilinear) | exp(dtA A)  (zoh, dirac)
//   gamma = dt / (1 - dt A / 2) | (exp(dt A) - 1) / A | 1
//   state = A_bar state + gamma (B @ x);  out = s Re(C @ state) + x @ D^T, s = 2 if conj_sym
// The Triton kernel guards the bilinear / zoh denominators with 1e-12 when
// they are exactly zero (:126, :151); the same guards are kept here.  Unlike
// the Triton launch, whose H tiles each re-read and rewrite the shared state
// (a second tile may read the state another tile already updated), every
// state element is updated exactly once.
//
// One workgroup (4 waves) per batch row.  x is staged in LDS; B @ x runs one
// state per wave at a time with lanes along H (coalesced rows of B) and a
// wave sum; the state update runs one state per thread; C @ state and
// x @ D^T run one output per wave at a time with lanes along P (resp. H).
#include "simp_common.h"

namespace lrnnx {

namespace {
constexpr int kSuThreads = 256;
constexpr int kSuWaves = kSuThreads / kWave;

__device__ __forceinline__ cf cdiv_guard(cf a, cf b) {
  float den = b.r * b.r + b.i * b.i;
  den = den == 0.f ? 1e-12f : den;
  return cf{(a.r * b.r + a.i * b.i) / den, (a.i * b.r - a.r * b.i) / den};
}
}  // namespace

__global__ void __launch_bounds__(kSuThreads) simp_state_update_kernel(const lrnnx_simplified_state_update_args a) {
  extern __shared__ float s_mem[];
  const int64_t H = a.H, P = a.P;
  float* s_x = s_mem;                      // [H]
  float* s_st = s_mem + H;                 // [P] complex (the updated state)
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t b = blockIdx.x;
  const float* x = static_cast<const float*>(a.x) + b * a.x_s0;
  for (int64_t h = tid; h < H; h += kSuThreads) s_x[h] = x[h * a.x_s1];
  __syncthreads();
  // B @ x, then the state update, one state per wave
  const float* Bp = static_cast<const float*>(a.B);
  float* stp = static_cast<float*>(a.state) + 2 * b * a.state_s0;
  for (int64_t p = w; p < P; p += kSuWaves) {
    float re = 0.f, im = 0.f;
    for (int64_t h = lane; h < H; h += kWave) {
      const cf bv = ld(Bp + 2 * (p * a.B_s0 + h * a.B_s1));
      re = fmaf(bv.r, s_x[h], re);
      im = fmaf(bv.i, s_x[h], im);
    }
    re = wave_allreduce_sum(re);
    im = wave_allreduce_sum(im);
    if (lane == 0) {
      const cf A = ld(static_cast<const float*>(a.A) + 2 * p * a.A_s0);
      const float dt = static_cast<const float*>(a.dt)[b * a.dt_s0 + p * a.dt_s1];
      const float dtA = a.deltaA ? static_cast<const float*>(a.deltaA)[b * a.dA_s0 + p * a.dA_s1] : dt;
      const cf one = cmake(1.f, 0.f);
      cf Ab, gam;
      if (a.method == LRNNX_BILINEAR) {
        const cf hA = cscale(A, 0.5f * dtA);
        Ab = cdiv_guard(cadd(one, hA), csub(one, hA));
        gam = cdiv_guard(cmake(dt, 0.f), csub(one, cscale(A, 0.5f * dt)));
      } else {
        Ab = cexp_(cscale(A, dtA));
        gam = a.method == LRNNX_ZOH ? cdiv_guard(csub(cexp_(cscale(A, dt)), one), A) : one;
      }
      const cf s_old = ld(stp + 2 * p * a.state_s1);
      const cf s_new = cadd(cmul(Ab, s_old), cmul(gam, cmake(re, im)));
      st(stp + 2 * p * a.state_s1, s_new);
      st(s_st + 2 * p, s_new);
    }
  }
  __syncthreads();
  // out = s Re(C @ state) + x @ D^T, one output per wave
  const float* Cp = static_cast<const float*>(a.C);
  const float* Dp = static_cast<const float*>(a.D);
  float* out = static_cast<float*>(a.out) + b * a.out_s0;
  const float scale = a.conj_sym ? 2.f : 1.f;
  for (int64_t h = w; h < H; h += kSuWaves) {
    float acc = 0.f;
    for (int64_t p = lane; p < P; p += kWave) {
      const cf c = ld(Cp + 2 * (h * a.C_s0 + p * a.C_s1));
      acc = fmaf(c.r, s_st[2 * p], fmaf(-c.i, s_st[2 * p + 1], acc));
    }
    float accD = 0.f;
    if (Dp)
      for (int64_t k = lane; k < H; k += kWave) accD = fmaf(Dp[h * a.D_s0 + k * a.D_s1], s_x[k], accD);
    acc = wave_allreduce_sum(acc);
    accD = wave_allreduce_sum(accD);
    if (lane == 0) out[h * a.out_s1] = fmaf(scale, acc, accD);
  }
}

hipError_t simp_state_update_launch(const lrnnx_simplified_state_update_args& a, hipStream_t st) {
  const size_t lds = (size_t)(a.H + 2 * a.P) * sizeof(float);
  hipLaunchKernelGGL(simp_state_update_kernel, dim3((unsigned)a.batch), dim3(kSuThreads), lds, st, a);
  return hipGetLastError();
}

}  // namespace lrnnx
