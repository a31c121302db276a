// Simplified complex diagonal scan (S5 / LRU), fast path of the LRU case.
//
// Covers one state per channel (A of shape (P, 1)) with delta (and deltaA)
// constant along L (zero L-stride), which makes A_bar and beta constant per
// (b, p) sequence: h_t = Lambda h_{t-1} + beta u_t, out_t = (B C) h_t
// (reference kernels csrc/simplified_scan/simplified_scan.cuh:85-262,
// simplified_scan_backward.cuh:91-420; discretisation :198-224).
//
// One wave owns one (b, p) sequence and walks it in chunks of 512 steps, 8
// consecutive steps per lane, so every load and store is a coalesced 16-byte
// access.  Per chunk: a serial scan of the lane's 8 steps from zero, an
// inclusive scan of the lanes' end values across the wave (log2(64) stages,
// stage d combining with the value d lanes away through Lambda^(8 d)), and a
// fix-up h_j = s_j + Lambda^(j+1) c with the lane's carry-in c (the previous
// lane's prefix plus Lambda^(8 lane) times the carry from the previous chunk).
// The powers of Lambda are computed once per wave.  The backward runs the
// same machinery right to left for dh (coefficient conj(Lambda)), recomputes
// h from the forward's checkpoints, and accumulates the per-lane sums that
// give dA, dB and dC once multiplied by per-sequence constants.
//
// The forward writes the generic path's checkpoint layout (the state before
// every 32-step chunk), so either backward can follow either forward.
#include "simp_common.h"

namespace lrnnx {

namespace {

constexpr int kE = 8;             // steps per lane
constexpr int kCh = kE * kWave;   // steps per chunk
constexpr int kSC32 = 32;         // the generic path's checkpoint interval

__device__ __forceinline__ cf shfl(cf v, int src_lane) {
  const int addr = (src_lane & 63) << 2;
  return cf{__int_as_float(__builtin_amdgcn_ds_bpermute(addr, __float_as_int(v.r))),
            __int_as_float(__builtin_amdgcn_ds_bpermute(addr, __float_as_int(v.i)))};
}

__device__ __forceinline__ cf readlane(cf v, int l) {
  return cf{__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v.r), l)),
            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v.i), l))};
}

// 8 complex values from / to 64 bytes (16-byte aligned), zero past `n`
__device__ __forceinline__ void load8(const float* p, int n, cf* v) {
  if (n >= kE) {
#pragma unroll
    for (int k = 0; k < kE / 2; ++k) {
      const float4 q = *reinterpret_cast<const float4*>(p + 4 * k);
      v[2 * k] = cf{q.x, q.y};
      v[2 * k + 1] = cf{q.z, q.w};
    }
  } else {
#pragma unroll
    for (int j = 0; j < kE; ++j) v[j] = j < n ? ld(p + 2 * j) : cf{0.f, 0.f};
  }
}
__device__ __forceinline__ void store8(float* p, int n, const cf* v) {
  if (n >= kE) {
#pragma unroll
    for (int k = 0; k < kE / 2; ++k)
      *reinterpret_cast<float4*>(p + 4 * k) = make_float4(v[2 * k].r, v[2 * k].i, v[2 * k + 1].r, v[2 * k + 1].i);
  } else {
#pragma unroll
    for (int j = 0; j < kE; ++j)
      if (j < n) st(p + 2 * j, v[j]);
  }
}

// Powers of Lambda a wave needs: pe[j] = L^(j+1) (j < 8), ps[k] = L^(8 * 2^k),
// pl = L^(8 lane), plr = L^(8 (63 - lane)).
struct Pow {
  cf pe[kE], ps[6], pl, plr;
};
__device__ __forceinline__ void powers(cf lam, int lane, Pow& w) {
  w.pe[0] = lam;
#pragma unroll
  for (int j = 1; j < kE; ++j) w.pe[j] = cmul(w.pe[j - 1], lam);
  w.ps[0] = w.pe[kE - 1];
#pragma unroll
  for (int k = 1; k < 6; ++k) w.ps[k] = cmul(w.ps[k - 1], w.ps[k - 1]);
  w.pl = cmake(1.f, 0.f);
  w.plr = cmake(1.f, 0.f);
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    if ((lane >> k) & 1) w.pl = cmul(w.pl, w.ps[k]);
    if (((63 - lane) >> k) & 1) w.plr = cmul(w.plr, w.ps[k]);
  }
}

// forward chunk: h[j] from the inputs v[j] (already times beta) and the
// carry hin entering the chunk; returns the lane's carry-in (state before
// its first step)
__device__ __forceinline__ cf chunk_fwd(const Pow& w, cf lam, const cf* v, cf hin, int lane, cf* h) {
  cf s[kE];
  s[0] = v[0];
#pragma unroll
  for (int j = 1; j < kE; ++j) s[j] = cfma(lam, s[j - 1], v[j]);
  cf V = s[kE - 1];
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const int d = 1 << k;
    const cf o = shfl(V, lane - d);
    if (lane >= d) V = cfma(w.ps[k], o, V);
  }
  cf cin = shfl(V, lane - 1);
  if (lane == 0) cin = cmake(0.f, 0.f);
  cin = cfma(w.pl, hin, cin);
#pragma unroll
  for (int j = 0; j < kE; ++j) h[j] = cfma(w.pe[j], cin, s[j]);
  return cin;
}

}  // namespace

template <int kMethod>
__global__ void __launch_bounds__(256) simpf_fwd_kernel(const lrnnx_simplified_scan_args a, int64_t nch32,
                                                        int64_t n_x) {
  const int lane = threadIdx.x & 63;
  const int64_t seq = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);   // (b, p)
  if (seq >= a.batch * a.dim) return;
  const int64_t b = seq / a.dim, p = seq % a.dim, L = a.seqlen;
  const cf A = ld(static_cast<const float*>(a.A.ptr) + 2 * p * a.A.s0);
  const float dl = static_cast<const float*>(a.delta.ptr)[b * a.delta.s0 + p * a.delta.s1];
  const float dt = a.deltaA.ptr ? static_cast<const float*>(a.deltaA.ptr)[b * a.deltaA.s0 + p * a.deltaA.s1] : dl;
  cf lam, beta;
  sdisc<kMethod>(dt, dl, A, lam, beta);
  const cf BC = cmul(ld(static_cast<const float*>(a.B.ptr) + 2 * p * a.B.s0),
                     ld(static_cast<const float*>(a.C.ptr) + 2 * p * a.C.s0));
  Pow w;
  powers(lam, lane, w);
  const cf step = cmul(w.ps[5], w.ps[5]);   // Lambda^512
  const float* u = static_cast<const float*>(a.u.ptr) + 2 * (b * a.u.s0 + p * a.u.s1);
  float* out = a.out.ptr ? static_cast<float*>(a.out.ptr) + 2 * (b * a.out.s0 + p * a.out.s1) : nullptr;
  float* ck = a.ckpt ? static_cast<float*>(a.ckpt) + 2 * seq * nch32 : nullptr;
  float* xp = a.x ? static_cast<float*>(a.x) + 2 * seq * n_x * 2 : nullptr;
  cf hin = cmake(0.f, 0.f), pc = cmake(1.f, 0.f);   // carry into the chunk, Lambda^t0
  cf nxt[kE];
  load8(u + 2 * 8 * lane, (int)min<int64_t>(kE, L - 8 * lane), nxt);
  for (int64_t t0 = 0; t0 < L; t0 += kCh) {
    const int64_t tl = t0 + kE * lane;
    const int n = (int)max<int64_t>(0, min<int64_t>(kE, L - tl));
    cf v[kE];
#pragma unroll
    for (int j = 0; j < kE; ++j) v[j] = kMethod == LRNNX_DIRAC ? nxt[j] : cmul(beta, nxt[j]);
    if (t0 + kCh < L)  // prefetch the next chunk
      load8(u + 2 * (tl + kCh), (int)max<int64_t>(0, min<int64_t>(kE, L - tl - kCh)), nxt);
    cf h[kE];
    const cf cin = chunk_fwd(w, lam, v, hin, lane, h);
    if (out) {
      cf y[kE];
#pragma unroll
      for (int j = 0; j < kE; ++j) y[j] = cmul(BC, h[j]);
      if (n > 0) store8(out + 2 * tl, n, y);
    }
    if (ck && (lane & 3) == 0 && n > 0) st(ck + 2 * (tl / kSC32), cin);
    if (xp) {  // reference chunk carries (Lambda^(t+1), h_t) at t + 1 = 2048 k or t = L - 1
#pragma unroll
      for (int j = 0; j < kE; ++j) {
        const int64_t t = tl + j;
        if (j < n && ((t + 1) % kXChunk == 0 || t == L - 1)) {
          float* xr = xp + 4 * (t / kXChunk);
          st(xr, cmul(pc, cmul(w.pl, w.pe[j])));
          st(xr + 2, h[j]);
        }
      }
    }
    hin = readlane(h[kE - 1], 63);
    pc = cmul(pc, step);
  }
}

// dA, dB, dC partials of one sequence: part[seq] = 3 complex
template <int kMethod>
__global__ void __launch_bounds__(256) simpf_bwd_kernel(const lrnnx_simplified_scan_args a, int64_t nch32,
                                                        float* __restrict__ part) {
  const int lane = threadIdx.x & 63;
  const int64_t seq = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (seq >= a.batch * a.dim) return;
  const int64_t b = seq / a.dim, p = seq % a.dim, L = a.seqlen;
  const cf A = ld(static_cast<const float*>(a.A.ptr) + 2 * p * a.A.s0);
  const bool hasdA = a.deltaA.ptr != nullptr;
  const float dl = static_cast<const float*>(a.delta.ptr)[b * a.delta.s0 + p * a.delta.s1];
  const float dt = hasdA ? static_cast<const float*>(a.deltaA.ptr)[b * a.deltaA.s0 + p * a.deltaA.s1] : dl;
  cf lam, beta;
  sdisc<kMethod>(dt, dl, A, lam, beta);
  const cf Bs = ld(static_cast<const float*>(a.B.ptr) + 2 * p * a.B.s0);
  const cf Cs = ld(static_cast<const float*>(a.C.ptr) + 2 * p * a.C.s0);
  const cf wBC = cconj(cmul(Bs, Cs));
  // derivatives of A_bar and beta (constant per sequence; same formulas as the
  // generic backward, simplified_scan.hip)
  const cf one = cmake(1.f, 0.f);
  cf dAb_dt, dAb_dA, gB_dl = cmake(0.f, 0.f), dbeta_dA = cmake(0.f, 0.f);
  if constexpr (kMethod == LRNNX_BILINEAR) {
    const cf om = csub(one, cscale(A, 0.5f * dt));
    const cf inv2 = cdiv(one, cmul(om, om));
    dAb_dt = cmul(A, inv2);
    dAb_dA = cscale(inv2, dt);
    const cf omB = csub(one, cscale(A, 0.5f * dl));
    const cf inv2B = cdiv(one, cmul(omB, omB));
    gB_dl = inv2B;
    dbeta_dA = cscale(inv2B, 0.5f * dl * dl);
  } else {
    dAb_dt = cmul(A, lam);
    dAb_dA = cscale(lam, dt);
    if constexpr (kMethod == LRNNX_ZOH) {
      const cf e = cexp_(cscale(A, dl));
      gB_dl = e;
      dbeta_dA = cdiv(csub(cscale(e, dl), beta), A);
    }
  }
  constexpr bool kGB = kMethod != LRNNX_DIRAC;   // beta depends on delta and A
  Pow w;
  powers(lam, lane, w);
  const float* u = static_cast<const float*>(a.u.ptr) + 2 * (b * a.u.s0 + p * a.u.s1);
  const float* dout = static_cast<const float*>(a.dout.ptr) + 2 * (b * a.dout.s0 + p * a.dout.s1);
  float* du = static_cast<float*>(a.du.ptr) + 2 * (b * a.du.s0 + p * a.du.s1);
  float* ddl = a.need_ddelta ? static_cast<float*>(a.ddelta.ptr) + b * a.ddelta.s0 + p * a.ddelta.s1 : nullptr;
  float* ddA = (a.need_ddelta && hasdA) ? static_cast<float*>(a.ddeltaA.ptr) + b * a.ddeltaA.s0 + p * a.ddeltaA.s1
                                        : nullptr;
  const float* ck = static_cast<const float*>(a.ckpt) + 2 * seq * nch32;
  cf SgA = cmake(0.f, 0.f), SgB = cmake(0.f, 0.f), SHd = cmake(0.f, 0.f);
  cf q = cmake(0.f, 0.f);   // dh at the first step of the chunk to the right
  const int64_t n_chunks = (L + kCh - 1) / kCh;
  for (int64_t c = n_chunks - 1; c >= 0; --c) {
    const int64_t t0 = c * kCh, tl = t0 + kE * lane;
    const int n = (int)max<int64_t>(0, min<int64_t>(kE, L - tl));
    cf x[kE], dy[kE];
    load8(u + 2 * tl, n, x);
    load8(dout + 2 * tl, n, dy);
    // forward recompute from the checkpoint at the chunk start
    cf v[kE], h[kE];
#pragma unroll
    for (int j = 0; j < kE; ++j) v[j] = kMethod == LRNNX_DIRAC ? x[j] : cmul(beta, x[j]);
    const cf cin = chunk_fwd(w, lam, v, ld(ck + 2 * (t0 / kSC32)), lane, h);
    // reverse: g_t = conj(B C) dout_t + conj(Lambda) g_{t+1}
    cf r[kE];
    r[kE - 1] = cmul(wBC, dy[kE - 1]);
#pragma unroll
    for (int j = kE - 2; j >= 0; --j) r[j] = cfma(cconj(lam), r[j + 1], cmul(wBC, dy[j]));
    cf S = r[0];
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      const int d = 1 << k;
      const cf o = shfl(S, lane + d);
      if (lane + d < 64) S = cfma(cconj(w.ps[k]), o, S);
    }
    cf cr = shfl(S, lane + 1);
    if (lane == 63) cr = cmake(0.f, 0.f);
    cr = cfma(cconj(w.plr), q, cr);
    cf g[kE], dx[kE];
#pragma unroll
    for (int j = 0; j < kE; ++j) {
      g[j] = cfma(cconj(w.pe[kE - 1 - j]), cr, r[j]);
      dx[j] = kMethod == LRNNX_DIRAC ? g[j] : cmul(cconj(beta), g[j]);
    }
    if (n > 0) store8(du + 2 * tl, n, dx);
#pragma unroll
    for (int j = 0; j < kE; ++j) {
      const cf hp = j > 0 ? h[j - 1] : cin;
      const cf gA = cmul(cconj(hp), g[j]);
      SgA = cadd(SgA, gA);
      SHd = cfma(cconj(h[j]), dy[j], SHd);
      cf gB = cmake(0.f, 0.f);
      if constexpr (kGB) {
        gB = cmul(cconj(x[j]), g[j]);
        SgB = cadd(SgB, gB);
      }
      if (ddl && j < n) {
        const float tA = dAb_dt.r * gA.r + dAb_dt.i * gA.i;   // Re(conj(dA_bar/dt) gA)
        float dlv = hasdA ? 0.f : tA;
        if constexpr (kGB) dlv += gB_dl.r * gB.r + gB_dl.i * gB.i;
        ddl[tl + j] = dlv;
        if (ddA) ddA[tl + j] = tA;
      }
    }
    q = readlane(g[0], 0);
  }
  // sums over the wave -> one partial per sequence
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const int d = 1 << k;
    SgA = cadd(SgA, shfl(SgA, lane ^ d));
    SHd = cadd(SHd, shfl(SHd, lane ^ d));
    if constexpr (kGB) SgB = cadd(SgB, shfl(SgB, lane ^ d));
  }
  if (lane == 0) {
    cf dA = cmul(cconj(dAb_dA), SgA);
    if constexpr (kGB) dA = cfma(cconj(dbeta_dA), SgB, dA);
    float* pt = part + 6 * seq;
    st(pt, dA);
    st(pt + 2, cmul(cconj(Cs), SHd));   // dB = sum conj(C h) dout
    st(pt + 4, cmul(cconj(Bs), SHd));   // dC = sum conj(B h) dout
  }
}

// dA, dB, dC (p) = sum over b of the per-sequence partials, in batch order
__global__ void __launch_bounds__(256) simpf_bwd_reduce(const lrnnx_simplified_scan_args a,
                                                        const float* __restrict__ part) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= a.dim) return;
  cf s[3] = {cmake(0.f, 0.f), cmake(0.f, 0.f), cmake(0.f, 0.f)};
  for (int64_t b = 0; b < a.batch; ++b)
    for (int k = 0; k < 3; ++k) s[k] = cadd(s[k], ld(part + 6 * (b * a.dim + p) + 2 * k));
  st(static_cast<float*>(a.dA.ptr) + 2 * p * a.dA.s0, s[0]);
  st(static_cast<float*>(a.dB.ptr) + 2 * p * a.dB.s0, s[1]);
  st(static_cast<float*>(a.dC.ptr) + 2 * p * a.dC.s0, s[2]);
}

namespace {
bool rows16(const lrnnx_view& v) {  // complex (b, p, l) rows start on 16-byte boundaries
  return v.ptr == nullptr || ((reinterpret_cast<uintptr_t>(v.ptr) & 15u) == 0 && v.s0 % 2 == 0 && v.s1 % 2 == 0);
}
bool simpf_shape_ok(const lrnnx_simplified_scan_args& a) {
  return a.dstate == 1 && a.delta.s2 == 0 && (a.deltaA.ptr == nullptr || a.deltaA.s2 == 0) && rows16(a.u);
}
int64_t nch32(const lrnnx_simplified_scan_args& a) { return (a.seqlen + kSC32 - 1) / kSC32; }
}  // namespace

// Launch the fast forward when it covers the call; false otherwise.
bool simpf_fwd(const lrnnx_simplified_scan_args& a, hipStream_t st, hipError_t* err) {
  if (!simpf_shape_ok(a) || !rows16(a.out)) return false;
  const dim3 grid((unsigned)((a.batch * a.dim + 3) / 4)), block(256);
  const int64_t n_x = (a.seqlen + kXChunk - 1) / kXChunk;
  switch (a.method) {
    case LRNNX_ZOH: hipLaunchKernelGGL(simpf_fwd_kernel<LRNNX_ZOH>, grid, block, 0, st, a, nch32(a), n_x); break;
    case LRNNX_BILINEAR:
      hipLaunchKernelGGL(simpf_fwd_kernel<LRNNX_BILINEAR>, grid, block, 0, st, a, nch32(a), n_x);
      break;
    default: hipLaunchKernelGGL(simpf_fwd_kernel<LRNNX_DIRAC>, grid, block, 0, st, a, nch32(a), n_x); break;
  }
  *err = hipGetLastError();
  return true;
}

// Launch the fast backward (needs the forward's checkpoints) when it covers the
// call; false otherwise.  `part` holds batch * dim * 6 floats of workspace.
bool simpf_bwd(const lrnnx_simplified_scan_args& a, float* part, hipStream_t st, hipError_t* err) {
  if (!simpf_shape_ok(a) || a.ckpt == nullptr || !rows16(a.dout) || !rows16(a.du)) return false;
  const dim3 grid((unsigned)((a.batch * a.dim + 3) / 4)), block(256);
  switch (a.method) {
    case LRNNX_ZOH: hipLaunchKernelGGL(simpf_bwd_kernel<LRNNX_ZOH>, grid, block, 0, st, a, nch32(a), part); break;
    case LRNNX_BILINEAR:
      hipLaunchKernelGGL(simpf_bwd_kernel<LRNNX_BILINEAR>, grid, block, 0, st, a, nch32(a), part);
      break;
    default: hipLaunchKernelGGL(simpf_bwd_kernel<LRNNX_DIRAC>, grid, block, 0, st, a, nch32(a), part); break;
  }
  hipLaunchKernelGGL(simpf_bwd_reduce, dim3((unsigned)((a.dim + 255) / 256)), block, 0, st, a,
                     static_cast<const float*>(part));
  *err = hipGetLastError();
  return true;
}

}  // namespace lrnnx
