// One-token selective state update (decode), gfx950.
//
// Semantics: reference selective_state_update_ref
// (lrnnx/ops/triton/selective_state_update.py:479-599) and its Triton kernel
// (:17-297):  dt' = softplus(dt + dt_bias) (threshold 20);
//   A_bar = A**g (rglru, g = deltaA or dt'), 1 - 1/(dt'^2 + 1/2) (s7),
//           exp(A * (deltaA or dt')) otherwise;
//   B_bar = B dt' (mamba), B (exp(dt' A) - 1)/A (zoh), B dt'/(1 - dt' A/2)
//           (bilinear), B (dirac, s7), B sqrt(1 - A_bar^2) (rglru);
//   state <- state * A_bar + B_bar * x   (stored in the state dtype, in place)
//   out = sum_n state_n C_n (+ D x), times silu(z).
// One thread owns one (batch, head, channel) row of `state` and walks its
// d_state entries; consecutive threads own consecutive channels, so the
// state rows they touch are contiguous in memory.
#include "common.h"

namespace lrnnx {

template <typename T>
__device__ __forceinline__ float ldf(const void* p, int64_t i) { return to_f32(static_cast<const T*>(p)[i]); }

__device__ __forceinline__ float ld_any(const void* p, int64_t i, int ty) {
  switch (ty) {
    case LRNNX_BF16: return ldf<bf16>(p, i);
    case LRNNX_F16: return ldf<f16>(p, i);
    default: return ldf<float>(p, i);
  }
}

template <typename ST, int kMethod>
__global__ void __launch_bounds__(256) state_update_kernel(const lrnnx_state_update_args a) {
  const int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y, hd = blockIdx.z;
  if (d >= a.dim) return;
  const int64_t g = hd / (a.nheads / a.ngroups);
  const int64_t sb = a.state_batch_indices ? (int64_t)a.state_batch_indices[b] : b;
  ST* state = static_cast<ST*>(a.state) + sb * a.state_s0 + hd * a.state_s1 + d * a.state_s2;
  const float x = ld_any(a.x, b * a.x_s0 + hd * a.x_s1 + d * a.x_s2, a.x_type);
  float dt = ld_any(a.dt, b * a.dt_s0 + hd * a.dt_s1 + d * a.dt_s2, a.x_type);
  if (a.dt_bias) dt += static_cast<const float*>(a.dt_bias)[hd * a.dtb_s0 + d * a.dtb_s1];
  if (a.dt_softplus) dt = softplus20(dt);
  const bool has_dA = a.deltaA != nullptr;
  const float dAv = has_dA ? ld_any(a.deltaA, b * a.dA_s0 + hd * a.dA_s1 + d * a.dA_s2, a.x_type) : dt;
  const float* A = static_cast<const float*>(a.A) + hd * a.A_s0 + d * a.A_s1;
  float acc = 0.f;
  for (int64_t n = 0; n < a.dstate; ++n) {
    const float An = A[n * a.A_s2];
    const float Bn = ld_any(a.B, b * a.B_s0 + g * a.B_s1 + n * a.B_s2, a.bc_type);
    const float Cn = ld_any(a.C, b * a.C_s0 + g * a.C_s1 + n * a.C_s2, a.bc_type);
    float Ab, Bb;
    if constexpr (kMethod == LRNNX_RGLRU) {
      const float x = dAv * logf(An);
      Ab = expf(x);
      Bb = Bn * sqrtf(-expm1f(2.f * x));  // sqrt(1 - A_bar^2) without cancellation
    } else if constexpr (kMethod == LRNNX_S7) {
      Ab = 1.f - 1.f / (dt * dt + 0.5f);
      Bb = Bn;
    } else {
      Ab = expf(dAv * An);
      if constexpr (kMethod == LRNNX_ZOH) Bb = Bn * (expf(dt * An) - 1.f) / An;
      else if constexpr (kMethod == LRNNX_BILINEAR) Bb = Bn * (1.f / (1.f - 0.5f * dt * An)) * dt;
      else if constexpr (kMethod == LRNNX_DIRAC) Bb = Bn;
      else Bb = Bn * dt;
    }
    const int64_t si = n * a.state_s3;
    const float s_new = to_f32(state[si]) * Ab + Bb * x;
    const ST stored = from_f32<ST>(s_new);
    state[si] = stored;
    acc = fmaf(to_f32(stored), Cn, acc);
  }
  if (a.D) acc += x * static_cast<const float*>(a.D)[hd * a.D_s0 + d * a.D_s1];
  if (a.z) acc *= silu(ld_any(a.z, b * a.z_s0 + hd * a.z_s1 + d * a.z_s2, a.x_type));
  const int64_t oi = b * a.out_s0 + hd * a.out_s1 + d * a.out_s2;
  switch (a.x_type) {
    case LRNNX_BF16: static_cast<bf16*>(a.out)[oi] = from_f32<bf16>(acc); break;
    case LRNNX_F16: static_cast<f16*>(a.out)[oi] = from_f32<f16>(acc); break;
    default: static_cast<float*>(a.out)[oi] = acc;
  }
}

template <typename ST>
static hipError_t su_m(const lrnnx_state_update_args& a, hipStream_t st) {
  dim3 grid((unsigned)((a.dim + 255) / 256), (unsigned)a.batch, (unsigned)a.nheads);
  switch (a.method) {
    case LRNNX_MAMBA: hipLaunchKernelGGL((state_update_kernel<ST, LRNNX_MAMBA>), grid, dim3(256), 0, st, a); break;
    case LRNNX_ZOH: hipLaunchKernelGGL((state_update_kernel<ST, LRNNX_ZOH>), grid, dim3(256), 0, st, a); break;
    case LRNNX_BILINEAR: hipLaunchKernelGGL((state_update_kernel<ST, LRNNX_BILINEAR>), grid, dim3(256), 0, st, a); break;
    case LRNNX_DIRAC: hipLaunchKernelGGL((state_update_kernel<ST, LRNNX_DIRAC>), grid, dim3(256), 0, st, a); break;
    case LRNNX_S7: hipLaunchKernelGGL((state_update_kernel<ST, LRNNX_S7>), grid, dim3(256), 0, st, a); break;
    case LRNNX_RGLRU: hipLaunchKernelGGL((state_update_kernel<ST, LRNNX_RGLRU>), grid, dim3(256), 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t state_update_launch(const lrnnx_state_update_args& a, hipStream_t st) {
  switch (a.state_type) {
    case LRNNX_BF16: return su_m<bf16>(a, st);
    case LRNNX_F16: return su_m<f16>(a, st);
    case LRNNX_F32: return su_m<float>(a, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace lrnnx
