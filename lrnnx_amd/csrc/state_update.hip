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
// General kernel: one thread owns one (batch, head, channel) row of `state`;
// consecutive threads own consecutive channels.  At d_state 16, 32, 64, 128 or
// 256 with unit-stride aligned rows a row is split over 2 to 16 adjacent
// lanes, each reading and writing 16 to 64 bytes after all its operands are
// loaded.
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

// exp through v_exp_f32 (a few ulp; the state is stored in its own dtype)
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

// Discretised (A_bar, B_bar) of one state entry (the method formulas above).
template <int kMethod>
__device__ __forceinline__ void discretize1(float An, float Bn, float dt, float dAv, float& Ab, float& Bb) {
  if constexpr (kMethod == LRNNX_RGLRU) {
    const float x = dAv * logf(An);
    Ab = expf(x);
    Bb = Bn * sqrtf(-expm1f(2.f * x));  // sqrt(1 - A_bar^2) without cancellation
  } else if constexpr (kMethod == LRNNX_S7) {
    Ab = 1.f - 1.f / (dt * dt + 0.5f);
    Bb = Bn;
  } else {
    Ab = exp_fast(dAv * An);
    if constexpr (kMethod == LRNNX_ZOH) Bb = Bn * (expf(dt * An) - 1.f) / An;
    else if constexpr (kMethod == LRNNX_BILINEAR) Bb = Bn * (1.f / (1.f - 0.5f * dt * An)) * dt;
    else if constexpr (kMethod == LRNNX_DIRAC) Bb = Bn;
    else Bb = Bn * dt;
  }
}

// Row-at-once update for d_state == kN with unit-stride, 16-byte aligned state
// / A rows and unit-stride B / C (checked on the host).  A row is split over
// kSplit = kN / kV adjacent lanes (2 to 16, an aligned group inside one 16-lane
// DPP row), each owning kV entries: 16 bytes of state, or kN / 16 entries when
// that is more (d_state 128 and 256 keep 16 lanes per row), so every state
// access of a wave is contiguous; the lanes' partial outputs are summed with
// DPP (quad xor 1, xor 2, then half-row and row mirrors).  All types are compile-time (ST: state;
// XT: x, dt, z, deltaA, B, C and out), and a lane loads all its operands
// before it computes and stores, so a row costs one round trip to memory.
template <typename ST, typename XT, int kMethod, int kN>
__global__ void __launch_bounds__(256) state_update_rows(const lrnnx_state_update_args a) {
  constexpr int kVB = 16 / (int)sizeof(ST);        // state entries per 16-byte access
  constexpr int kV = kN / 16 > kVB ? kN / 16 : kVB;   // state entries per lane
  constexpr int kSplit = kN / kV;                     // lanes per row
  static_assert(kSplit == 2 || kSplit == 4 || kSplit == 8 || kSplit == 16, "a row spans 2 to 16 lanes");
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t d = t / kSplit;
  const int part = (int)(t % kSplit);
  // the kSplit lanes of a row are one aligned group and share d, so they leave together
  if (d >= a.dim) return;
  const int64_t b = blockIdx.y, hd = blockIdx.z;
  const int64_t g = (int)hd / ((int)a.nheads / (int)a.ngroups);
  const int64_t sb = a.state_batch_indices ? (int64_t)a.state_batch_indices[b] : b;
  ST* __restrict__ state = static_cast<ST*>(a.state) + sb * a.state_s0 + hd * a.state_s1 + d * a.state_s2 + part * kV;
  const float* __restrict__ A = static_cast<const float*>(a.A) + hd * a.A_s0 + d * a.A_s1 + part * kV;
  const XT* __restrict__ Bp = static_cast<const XT*>(a.B) + b * a.B_s0 + g * a.B_s1 + part * kV;
  const XT* __restrict__ Cp = static_cast<const XT*>(a.C) + b * a.C_s0 + g * a.C_s1 + part * kV;
  float sv[kV], Av[kV], Bv[kV], Cv[kV];
#pragma unroll
  for (int c = 0; c < kV / kVB; ++c) {
    const uint4 raw = reinterpret_cast<const uint4*>(state)[c];
    const ST* e = reinterpret_cast<const ST*>(&raw);
#pragma unroll
    for (int v = 0; v < kVB; ++v) sv[c * kVB + v] = to_f32(e[v]);
  }
#pragma unroll
  for (int q = 0; q < kV / 4; ++q) {
    const float4 f = reinterpret_cast<const float4*>(A)[q];
    Av[4 * q] = f.x; Av[4 * q + 1] = f.y; Av[4 * q + 2] = f.z; Av[4 * q + 3] = f.w;
  }
#pragma unroll
  for (int v = 0; v < kV; ++v) {
    Bv[v] = to_f32(Bp[v]);
    Cv[v] = to_f32(Cp[v]);
  }
  // The optional operands are loaded with the others, unconditionally: an
  // absent one reads this row's x (or A) entry instead and is dropped, so the
  // row's loads all issue before the first wait.
  const XT* xp = static_cast<const XT*>(a.x) + b * a.x_s0 + hd * a.x_s1 + d * a.x_s2;
  const float* dtbp = a.dt_bias ? static_cast<const float*>(a.dt_bias) + hd * a.dtb_s0 + d * a.dtb_s1 : A;
  const float* Dp = a.D ? static_cast<const float*>(a.D) + hd * a.D_s0 + d * a.D_s1 : A;
  const XT* zp = a.z ? static_cast<const XT*>(a.z) + b * a.z_s0 + hd * a.z_s1 + d * a.z_s2 : xp;
  const XT* dAp = a.deltaA ? static_cast<const XT*>(a.deltaA) + b * a.dA_s0 + hd * a.dA_s1 + d * a.dA_s2 : xp;
  const float x = to_f32(*xp);
  float dt = to_f32(static_cast<const XT*>(a.dt)[b * a.dt_s0 + hd * a.dt_s1 + d * a.dt_s2]);
  const float dtb = *dtbp, Dv = *Dp, zv = to_f32(*zp), dAraw = to_f32(*dAp);
  if (a.dt_bias) dt += dtb;
  if (a.dt_softplus) dt = softplus20(dt);
  const float dAv = a.deltaA ? dAraw : dt;
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < kV / kVB; ++c) {
    uint4 raw;
    ST* e = reinterpret_cast<ST*>(&raw);
#pragma unroll
    for (int v = 0; v < kVB; ++v) {
      const int i = c * kVB + v;
      float Ab, Bb;
      discretize1<kMethod>(Av[i], Bv[i], dt, dAv, Ab, Bb);
      e[v] = from_f32<ST>(fmaf(sv[i], Ab, Bb * x));
      acc = fmaf(to_f32(e[v]), Cv[i], acc);
    }
    reinterpret_cast<uint4*>(state)[c] = raw;
  }
  // every lane of the group ends with the group's sum: xor 1 and xor 2 sum a
  // quad, the half-row mirror pairs quads 0 / 1, the row mirror halves 0 / 1
  acc += dpp_mov<kDppQuadXor1>(acc);
  if constexpr (kSplit >= 4) acc += dpp_mov<kDppQuadXor2>(acc);
  if constexpr (kSplit >= 8) acc += dpp_mov<kDppRowHalfMirror>(acc);
  if constexpr (kSplit >= 16) acc += dpp_mov<kDppRowMirror>(acc);
  if (part != 0) return;
  if (a.D) acc += x * Dv;
  if (a.z) acc *= silu(zv);
  static_cast<XT*>(a.out)[b * a.out_s0 + hd * a.out_s1 + d * a.out_s2] = from_f32<XT>(acc);
}

// Entry-by-entry update: any strides, runtime dtypes.
template <typename ST, int kMethod>
__global__ void __launch_bounds__(256) state_update_kernel(const lrnnx_state_update_args a) {
  const int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y, hd = blockIdx.z;
  if (d >= a.dim) return;
  const int64_t g = hd / (a.nheads / a.ngroups);
  const int64_t sb = a.state_batch_indices ? (int64_t)a.state_batch_indices[b] : b;
  ST* __restrict__ state = static_cast<ST*>(a.state) + sb * a.state_s0 + hd * a.state_s1 + d * a.state_s2;
  const float* __restrict__ A = static_cast<const float*>(a.A) + hd * a.A_s0 + d * a.A_s1;
  // optional operands load with x and dt (an absent one reads x's entry or A[0]
  // and is dropped), so none of them waits behind a branch or the state loop
  const int64_t xi = b * a.x_s0 + hd * a.x_s1 + d * a.x_s2;
  const float* dtbp = a.dt_bias ? static_cast<const float*>(a.dt_bias) + hd * a.dtb_s0 + d * a.dtb_s1 : A;
  const float* Dp = a.D ? static_cast<const float*>(a.D) + hd * a.D_s0 + d * a.D_s1 : A;
  const void* zb = a.z ? a.z : a.x;
  const int64_t zi = a.z ? b * a.z_s0 + hd * a.z_s1 + d * a.z_s2 : xi;
  const void* dAb = a.deltaA ? a.deltaA : a.x;
  const int64_t dAi = a.deltaA ? b * a.dA_s0 + hd * a.dA_s1 + d * a.dA_s2 : xi;
  const float x = ld_any(a.x, xi, a.x_type);
  float dt = ld_any(a.dt, b * a.dt_s0 + hd * a.dt_s1 + d * a.dt_s2, a.x_type);
  const float dtb = *dtbp, Dv = *Dp, zv = ld_any(zb, zi, a.x_type), dAraw = ld_any(dAb, dAi, a.x_type);
  if (a.dt_bias) dt += dtb;
  if (a.dt_softplus) dt = softplus20(dt);
  const float dAv = a.deltaA ? dAraw : dt;
  float acc = 0.f;
#pragma unroll 4
  for (int64_t n = 0; n < a.dstate; ++n) {
    const float An = A[n * a.A_s2];
    const float Bn = ld_any(a.B, b * a.B_s0 + g * a.B_s1 + n * a.B_s2, a.bc_type);
    const float Cn = ld_any(a.C, b * a.C_s0 + g * a.C_s1 + n * a.C_s2, a.bc_type);
    float Ab, Bb;
    discretize1<kMethod>(An, Bn, dt, dAv, Ab, Bb);
    const int64_t si = n * a.state_s3;
    const ST stored = from_f32<ST>(fmaf(to_f32(state[si]), Ab, Bb * x));
    state[si] = stored;
    acc = fmaf(to_f32(stored), Cn, acc);
  }
  if (a.D) acc += x * Dv;
  if (a.z) acc *= silu(zv);
  const int64_t oi = b * a.out_s0 + hd * a.out_s1 + d * a.out_s2;
  switch (a.x_type) {
    case LRNNX_BF16: static_cast<bf16*>(a.out)[oi] = from_f32<bf16>(acc); break;
    case LRNNX_F16: static_cast<f16*>(a.out)[oi] = from_f32<f16>(acc); break;
    default: static_cast<float*>(a.out)[oi] = acc;
  }
}

// the row-at-once kernel's layout requirements (d_state 16, 32, 64, 128 or 256)
template <typename ST>
static bool su_rows_ok(const lrnnx_state_update_args& a) {
  const int64_t es = sizeof(ST);
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  return (a.dstate == 16 || a.dstate == 32 || a.dstate == 64 || a.dstate == 128 || a.dstate == 256) &&
         a.state_s3 == 1 && a.A_s2 == 1 && a.B_s2 == 1 && a.C_s2 == 1 && al16(a.state) &&
         al16(a.A) && (a.state_s0 * es) % 16 == 0 && (a.state_s1 * es) % 16 == 0 && (a.state_s2 * es) % 16 == 0 &&
         (a.A_s0 * 4) % 16 == 0 && (a.A_s1 * 4) % 16 == 0;
}

// Row-at-once launch at d_state kN; false when the x / B / C type has no
// instantiation (x / B / C of the state's own type, or 16-bit with an fp32 state).
template <typename ST, int kMethod, int kN>
static bool su_rows_launch(const lrnnx_state_update_args& a, dim3 grid, hipStream_t st) {
  // kSplit lanes per row (as in state_update_rows)
  constexpr int64_t kVB = 16 / sizeof(ST);
  constexpr int64_t kSplit = kN / (kN / 16 > kVB ? kN / 16 : kVB);
  const dim3 rg((unsigned)((a.dim * kSplit + 255) / 256), grid.y, grid.z);
  if (a.x_type == a.state_type) {
    hipLaunchKernelGGL((state_update_rows<ST, ST, kMethod, kN>), rg, dim3(256), 0, st, a);
    return true;
  }
  if constexpr (sizeof(ST) == 4) {
    if (a.x_type == LRNNX_BF16) {
      hipLaunchKernelGGL((state_update_rows<ST, bf16, kMethod, kN>), rg, dim3(256), 0, st, a);
      return true;
    }
    if (a.x_type == LRNNX_F16) {
      hipLaunchKernelGGL((state_update_rows<ST, f16, kMethod, kN>), rg, dim3(256), 0, st, a);
      return true;
    }
  }
  return false;
}

template <typename ST, int kMethod>
static void su_launch(const lrnnx_state_update_args& a, dim3 grid, hipStream_t st) {
  if (su_rows_ok<ST>(a) && a.bc_type == a.x_type) {
    const bool done = a.dstate == 16    ? su_rows_launch<ST, kMethod, 16>(a, grid, st)
                      : a.dstate == 32  ? su_rows_launch<ST, kMethod, 32>(a, grid, st)
                      : a.dstate == 64  ? su_rows_launch<ST, kMethod, 64>(a, grid, st)
                      : a.dstate == 128 ? su_rows_launch<ST, kMethod, 128>(a, grid, st)
                                        : su_rows_launch<ST, kMethod, 256>(a, grid, st);
    if (done) return;
  }
  hipLaunchKernelGGL((state_update_kernel<ST, kMethod>), grid, dim3(256), 0, st, a);
}

template <typename ST>
static hipError_t su_m(const lrnnx_state_update_args& a, hipStream_t st) {
  dim3 grid((unsigned)((a.dim + 255) / 256), (unsigned)a.batch, (unsigned)a.nheads);
  switch (a.method) {
    case LRNNX_MAMBA: su_launch<ST, LRNNX_MAMBA>(a, grid, st); break;
    case LRNNX_ZOH: su_launch<ST, LRNNX_ZOH>(a, grid, st); break;
    case LRNNX_BILINEAR: su_launch<ST, LRNNX_BILINEAR>(a, grid, st); break;
    case LRNNX_DIRAC: su_launch<ST, LRNNX_DIRAC>(a, grid, st); break;
    case LRNNX_S7: su_launch<ST, LRNNX_S7>(a, grid, st); break;
    case LRNNX_RGLRU: su_launch<ST, LRNNX_RGLRU>(a, grid, st); break;
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
