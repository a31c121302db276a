// RG-LRU and S7 scans, fast path for one state per channel: the selective
// scan's "rglru" and "s7" discretisations (reference
// csrc/selective_scan/selective_scan.cuh:272-302, backward
// selective_scan_backward.cuh) with constant B / C, fp32,
//   h_t = A_bar_t h_{t-1} + beta_t u_t,  out_t = B C h_t + D u_t,
//   rglru: A_bar_t = A^delta_t, beta_t = sqrt(1 - A_bar_t^2)  (A of shape
//          (D, 1): the RG-LRU layer's `a`, rglru_scan.py:39);
//   s7:    A_bar_t = 1 - 1 / (delta_t^2 + 1/2), beta_t = 1  (S7ScanFn runs one
//          state per S7 state index with the time-varying A as delta,
//          s7_scan.py:49-74).
//
// With one state per channel the general kernels hold one wave per 64
// channels, far fewer waves than the chip has SIMDs at the layers' shapes.
// Here one wave owns one (b, d) sequence and walks it in chunks of 512 steps,
// 8 consecutive steps per lane (coalesced 16-byte accesses):
//   forward   a serial pass over the lane's steps from zero (local state s_j
//             and product P_j of A_bar), an inclusive scan of the lanes'
//             (P, s) pairs across the wave, (a, s) o (a', s') = (a a', a s' + s)
//             in log2(64) stages, then h_j = P_j c + s_j with the lane's
//             carry-in c;
//   backward  the same recomputation from the forward's checkpoint at the
//             chunk start, then the adjoint e_j = A_bar_j (B C dout_j + e_{j+1})
//             by a serial pass right to left and a suffix scan across lanes,
//             and the per-step derivatives of A_bar and beta.
// The forward writes the general path's checkpoint layout (the state after
// every 16th step), so either backward can follow either forward.
#include "ss_bwd_impl.h"

namespace lrnnx {

bool fast_paths_enabled();  // capi.hip

namespace {

constexpr int kE = 8;             // steps per lane
constexpr int kCh = kE * kWave;   // steps per chunk
constexpr int kCk1 = ck_for(1);   // the general path's checkpoint interval at one state
static_assert(kCk1 == 2 * kE, "odd lanes end the checkpoint intervals");

__device__ __forceinline__ float bperm(float v, int src_lane) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute((src_lane & 63) << 2, __float_as_int(v)));
}
__device__ __forceinline__ float rdlane(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// 8 consecutive floats of a row (zero past n); 16-byte accesses when aligned
__device__ __forceinline__ void ld8(const float* q, int n, float* v) {
  if (n >= kE && (reinterpret_cast<uintptr_t>(q) & 15u) == 0) {
    const float4 x = *reinterpret_cast<const float4*>(q);
    const float4 y = *reinterpret_cast<const float4*>(q + 4);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
    v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
  } else {
#pragma unroll
    for (int j = 0; j < kE; ++j) v[j] = j < n ? q[j] : 0.f;
  }
}
__device__ __forceinline__ void st8(float* q, int n, const float* v) {
  if (n >= kE && (reinterpret_cast<uintptr_t>(q) & 15u) == 0) {
    *reinterpret_cast<float4*>(q) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(q + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else {
#pragma unroll
    for (int j = 0; j < kE; ++j)
      if (j < n) q[j] = v[j];
  }
}

// A_bar and beta of one step; la = log2(A) (rglru).  The same operations as
// the general kernels' discretisation (disc_real).
template <int kMethod>
__device__ __forceinline__ void rg_disc(float dl, float la, float& ab, float& beta) {
  if constexpr (kMethod == LRNNX_S7) {
    ab = 1.f - __builtin_amdgcn_rcpf(fmaf(dl, dl, 0.5f));
    beta = 1.f;
  } else {
    const float x = dl * la;
    ab = fast_exp2(x);
    beta = __builtin_amdgcn_sqrtf(-expm1_from(x * kLn2, ab) * (1.f + ab));  // 1 - ab^2 without cancellation
  }
}

// Local pass over the lane's steps and the cross-lane scan: returns the
// state before the lane's first step given `hin`, the state before the chunk;
// P[j] = prod of A_bar over the lane's steps 0..j, s[j] the state from zero.
// Also returns the chunk's total A_bar product (lane 63's inclusive value).
// Steps past L load delta 0 and u 0: for rglru they are the identity
// (A_bar 1, beta 0); for s7 A_bar is -1 there, which only reaches states and
// lanes past L (never stored) and the carry out of the last chunk (unused).
template <int kMethod>
__device__ __forceinline__ float chunk_states(const float* dl, const float* u, float la, float hin, int lane,
                                              float* ab, float* be, float* P, float* h, float& Pchunk,
                                              float& Ain) {
  float s[kE];
#pragma unroll
  for (int j = 0; j < kE; ++j) {
    rg_disc<kMethod>(dl[j], la, ab[j], be[j]);
    const float v = be[j] * u[j];
    s[j] = j == 0 ? v : fmaf(ab[j], s[j - 1], v);
    P[j] = j == 0 ? ab[j] : ab[j] * P[j - 1];
  }
  float Av = P[kE - 1], Sv = s[kE - 1];
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const int d = 1 << k;
    const float ao = bperm(Av, lane - d), so = bperm(Sv, lane - d);
    if (lane >= d) {
      Sv = fmaf(Av, so, Sv);
      Av *= ao;
    }
  }
  Ain = bperm(Av, lane - 1);
  float Sin = bperm(Sv, lane - 1);
  if (lane == 0) {
    Ain = 1.f;
    Sin = 0.f;
  }
  const float cin = fmaf(Ain, hin, Sin);
#pragma unroll
  for (int j = 0; j < kE; ++j) h[j] = fmaf(P[j], cin, s[j]);
  Pchunk = rdlane(Av, 63);
  return cin;
}

}  // namespace

template <int kMethod>
__global__ void __launch_bounds__(256) rgf_fwd_kernel(const lrnnx_selective_scan_args a, int64_t n_ck, int64_t n_x) {
  const int lane = threadIdx.x & 63;
  const int64_t seq = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // b * D + d
  if (seq >= a.batch * a.dim) return;
  const int64_t D = a.dim, b = seq / D, d = seq % D, L = a.seqlen;
  const float la = kMethod == LRNNX_S7 ? 0.f : __log2f(static_cast<const float*>(a.A.ptr)[d * a.A.s0]);
  const float bc = static_cast<const float*>(a.B.ptr)[d * a.B.s0] * static_cast<const float*>(a.C.ptr)[d * a.C.s0];
  const float Dv = a.D.ptr ? static_cast<const float*>(a.D.ptr)[d * a.D.s0] : 0.f;
  const float* u = static_cast<const float*>(a.u.ptr) + b * a.u.s0 + d * a.u.s1;
  const float* dlr = static_cast<const float*>(a.delta.ptr) + b * a.delta.s0 + d * a.delta.s1;
  float* out = a.out.ptr ? static_cast<float*>(a.out.ptr) + b * a.out.s0 + d * a.out.s1 : nullptr;
  float* ck = static_cast<float*>(a.ckpt);
  float* xp = a.x ? static_cast<float*>(a.x) + seq * n_x * 2 : nullptr;
  float hin = 0.f, pc = 1.f;  // state before the chunk, prod A_bar over [0, t0)
  for (int64_t t0 = 0; t0 < L; t0 += kCh) {
    const int64_t tl = t0 + kE * lane;
    const int n = (int)max<int64_t>(0, min<int64_t>(kE, L - tl));
    float uu[kE], dl[kE];
    ld8(u + tl, n, uu);
    ld8(dlr + tl, n, dl);
    float ab[kE], be[kE], P[kE], h[kE], Pc, Ain;
    chunk_states<kMethod>(dl, uu, la, hin, lane, ab, be, P, h, Pc, Ain);
    if (out && n > 0) {
      float y[kE];
#pragma unroll
      for (int j = 0; j < kE; ++j) y[j] = fmaf(bc, h[j], Dv * uu[j]);
      st8(out + tl, n, y);
    }
    // general layout: checkpoint kk holds the state after step 16 kk + 15
    if (ck && (lane & 1) && n == kE) ck[(b * n_ck + (tl + kE) / kCk1 - 1) * D + d] = h[kE - 1];
    if (xp) {  // reference chunk carries (prod A_bar over [0, t], h_t) at t + 1 = 2048 k or t = L - 1
      const float pl = pc * Ain;
#pragma unroll
      for (int j = 0; j < kE; ++j) {
        const int64_t t = tl + j;
        if (j < n && ((t + 1) % kXChunk == 0 || t == L - 1)) {
          float* xr = xp + 2 * (t / kXChunk);
          xr[0] = pl * P[j];
          xr[1] = h[j];
        }
      }
    }
    hin = rdlane(h[kE - 1], 63);
    pc *= Pc;
  }
}

// Per-sequence partials into the general backward's workspace sections
// (dA, constant dB / dC, dD: one value per (b, d)); du, ddelta written.
template <int kMethod>
__global__ void __launch_bounds__(256) rgf_bwd_kernel(const lrnnx_selective_scan_args a, int64_t n_ck,
                                                      const float* __restrict__ ckp, float* __restrict__ ws,
                                                      const SSBwdWs wo) {
  const int lane = threadIdx.x & 63;
  const int64_t seq = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (seq >= a.batch * a.dim) return;
  const int64_t D = a.dim, b = seq / D, d = seq % D, L = a.seqlen;
  const float Araw = static_cast<const float*>(a.A.ptr)[d * a.A.s0];   // unused by s7
  const float la = kMethod == LRNNX_S7 ? 0.f : __log2f(Araw), lnA = la * kLn2, invA = 1.f / Araw;
  const float B0 = static_cast<const float*>(a.B.ptr)[d * a.B.s0];
  const float C0 = static_cast<const float*>(a.C.ptr)[d * a.C.s0];
  const float w = B0 * C0;
  const float Dv = a.D.ptr ? static_cast<const float*>(a.D.ptr)[d * a.D.s0] : 0.f;
  const float* u = static_cast<const float*>(a.u.ptr) + b * a.u.s0 + d * a.u.s1;
  const float* dlr = static_cast<const float*>(a.delta.ptr) + b * a.delta.s0 + d * a.delta.s1;
  const float* dout = static_cast<const float*>(a.dout.ptr) + b * a.dout.s0 + d * a.dout.s1;
  float* du = static_cast<float*>(a.du.ptr) + b * a.du.s0 + d * a.du.s1;
  float* ddl = static_cast<float*>(a.ddelta.ptr) + b * a.ddelta.s0 + d * a.ddelta.s1;
  float dAacc = 0.f, SHd = 0.f, SDu = 0.f;
  float Ech = 0.f;  // adjoint carried into the last step of this chunk from the chunk to the right
  const int64_t n_chunks = (L + kCh - 1) / kCh;
  for (int64_t c = n_chunks - 1; c >= 0; --c) {
    const int64_t t0 = c * kCh, tl = t0 + kE * lane;
    const int n = (int)max<int64_t>(0, min<int64_t>(kE, L - tl));
    float x[kE], dy[kE], dl[kE];
    ld8(u + tl, n, x);
    ld8(dout + tl, n, dy);
    ld8(dlr + tl, n, dl);
    // forward recompute from the state before the chunk (t0 is a multiple of 16)
    const float hin = t0 > 0 ? ckp[(b * n_ck + t0 / kCk1 - 1) * D + d] : 0.f;
    float ab[kE], be[kE], P[kE], h[kE], Pc, Ain;
    const float cin = chunk_states<kMethod>(dl, x, la, hin, lane, ab, be, P, h, Pc, Ain);
    // adjoint: e_j = A_bar_j (w dout_j + e_{j+1}), the gradient carried from
    // step j to j - 1; local values from e = 0 past the lane, Q_j = prod_{i >= j} A_bar_i
    float el[kE], Q[kE];
    el[kE - 1] = ab[kE - 1] * (w * dy[kE - 1]);
    Q[kE - 1] = ab[kE - 1];
#pragma unroll
    for (int j = kE - 2; j >= 0; --j) {
      el[j] = ab[j] * fmaf(w, dy[j], el[j + 1]);
      Q[j] = ab[j] * Q[j + 1];
    }
    float Mv = Q[0], Rv = el[0];
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      const int dd = 1 << k;
      const float mo = bperm(Mv, lane + dd), ro = bperm(Rv, lane + dd);
      if (lane + dd < 64) {
        Rv = fmaf(Mv, ro, Rv);
        Mv *= mo;
      }
    }
    float Mn = bperm(Mv, lane + 1), Rn = bperm(Rv, lane + 1);
    if (lane == 63) {
      Mn = 1.f;
      Rn = 0.f;
    }
    const float Ein = fmaf(Mn, Ech, Rn);  // adjoint entering the lane's last step from the right
    float dx[kE], ddv[kE];
#pragma unroll
    for (int j = 0; j < kE; ++j) {
      const float enext = j == kE - 1 ? Ein : fmaf(Q[j + 1], Ein, el[j + 1]);
      const float g = fmaf(w, dy[j], enext);  // dL/dh_j
      dx[j] = fmaf(be[j], g, Dv * dy[j]);
      const float hp = j > 0 ? h[j - 1] : cin;
      if constexpr (kMethod == LRNNX_S7) {
        // dA_bar/ddelta = 2 delta / (delta^2 + 1/2)^2; A does not enter (dA = 0)
        const float r = __builtin_amdgcn_rcpf(fmaf(dl[j], dl[j], 0.5f));
        ddv[j] = g * hp * (2.f * dl[j] * (r * r));
      } else {
        // dL/dA_bar_j through h_j = A_bar h_{j-1} + beta(A_bar) u_j, dbeta/dA_bar = -A_bar / beta;
        // steps past L are excluded (their beta is 0)
        const float q = j < n ? g * fmaf(-x[j] * ab[j], __builtin_amdgcn_rcpf(be[j]), hp) : 0.f;
        ddv[j] = q * ab[j] * lnA;                          // dA_bar/ddelta = A_bar ln A
        dAacc = fmaf(q, ab[j] * dl[j] * invA, dAacc);     // dA_bar/dA = delta A_bar / A
      }
      SHd = fmaf(h[j], dy[j], SHd);
      SDu = fmaf(x[j], dy[j], SDu);
    }
    if (n > 0) {
      st8(du + tl, n, dx);
      st8(ddl + tl, n, ddv);
    }
    Ech = fmaf(rdlane(Mv, 0), Ech, rdlane(Rv, 0));
  }
  dAacc = wave_allreduce_sum(dAacc);
  SHd = wave_allreduce_sum(SHd);
  SDu = wave_allreduce_sum(SDu);
  if (lane == 0) {
    ws[wo.dA + seq] = dAacc;
    ws[wo.dBc + seq] = C0 * SHd;  // out = B C h + D u
    ws[wo.dCc + seq] = B0 * SHd;
    ws[wo.dD + seq] = SDu;
  }
}

// The fast path covers rglru and s7 with one state, constant B / C, and no z,
// delta bias, softplus or deltaA (RGLRUScanFn's and S7ScanFn's calls,
// rglru_scan.py:39, s7_scan.py:59).
bool rgf_ok(const lrnnx_selective_scan_args& a) {
  return (a.method == LRNNX_RGLRU || a.method == LRNNX_S7) && a.wtype == LRNNX_F32 && a.itype == LRNNX_F32 && a.dstate == 1 && !a.var_B &&
         !a.var_C && a.z.ptr == nullptr && a.delta_bias.ptr == nullptr && a.deltaA.ptr == nullptr &&
         !a.delta_softplus && fast_paths_enabled();
}

hipError_t rgf_fwd(const lrnnx_selective_scan_args& a, hipStream_t st) {
  const SSGeom g = ss_geom(a);
  const int64_t n_x = (a.seqlen + kXChunk - 1) / kXChunk;
  const dim3 grid((unsigned)((a.batch * a.dim + 3) / 4));
  if (a.method == LRNNX_S7) hipLaunchKernelGGL(rgf_fwd_kernel<LRNNX_S7>, grid, dim3(256), 0, st, a, g.n_ck, n_x);
  else hipLaunchKernelGGL(rgf_fwd_kernel<LRNNX_RGLRU>, grid, dim3(256), 0, st, a, g.n_ck, n_x);
  return hipGetLastError();
}

hipError_t rgf_bwd(const lrnnx_selective_scan_args& a, float* ws, const float* ckp, hipStream_t st) {
  const SSGeom g = ss_geom(a);
  const SSBwdWs wo = ss_bwd_ws(a, g, a.ckpt == nullptr);
  const dim3 grid((unsigned)((a.batch * a.dim + 3) / 4));
  if (a.method == LRNNX_S7) hipLaunchKernelGGL(rgf_bwd_kernel<LRNNX_S7>, grid, dim3(256), 0, st, a, g.n_ck, ckp, ws, wo);
  else hipLaunchKernelGGL(rgf_bwd_kernel<LRNNX_RGLRU>, grid, dim3(256), 0, st, a, g.n_ck, ckp, ws, wo);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return ss_bwd_reductions<float, false, false>(a, g, ws, wo, st);
}

}  // namespace lrnnx
