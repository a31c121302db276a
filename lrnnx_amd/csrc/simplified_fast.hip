// Simplified complex diagonal scan (S5 / LRU), fast path for one state per
// channel (A of shape (P, 1)).
//
// Constant time step (delta and deltaA with zero L-stride, the LRU case):
// A_bar and beta are constant per (b, p) sequence,
// h_t = Lambda h_{t-1} + beta u_t, out_t = (B C) h_t
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

// ---------------------------------------------------------------- time-varying delta
// delta (and deltaA) vary along L: A_bar_t and beta_t change every step, so the
// cross-lane stage is a general associative scan of (a, s) pairs,
// (a_l, s_l) then (a_r, s_r) = (a_r a_l, a_r s_l + s_r), with a lane's pair the
// product of its 8 A_bar and its local scan end.  The backward propagates
// e_t = conj(A_bar_t) g_t leftwards (g_{t-1} = conj(B C) dout_{t-1} + e_t), so a
// lane's transfer (prod conj(A_bar), local e) depends on its own steps only,
// and the derivatives of A_bar / beta enter per step.

namespace {
// 8 real values of a row at steps tl .. tl + 7 (L-stride s2 = 0: one value for all)
__device__ __forceinline__ void load8r(const float* row, int64_t s2, int64_t tl, int n, float* v) {
  if (s2 == 0) {
    const float x = row[0];
#pragma unroll
    for (int j = 0; j < kE; ++j) v[j] = x;
    return;
  }
  const float* q = row + tl;
  if (n >= kE && (reinterpret_cast<uintptr_t>(q) & 15u) == 0) {
    const float4 lo = *reinterpret_cast<const float4*>(q), hi = *reinterpret_cast<const float4*>(q + 4);
    v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w; v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
  } else {
#pragma unroll
    for (int j = 0; j < kE; ++j) v[j] = j < n ? q[j] : 0.f;
  }
}
__device__ __forceinline__ void store8r(float* q, int n, const float* v) {
  if (n >= kE && (reinterpret_cast<uintptr_t>(q) & 15u) == 0) {
    *reinterpret_cast<float4*>(q) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(q + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else {
#pragma unroll
    for (int j = 0; j < kE; ++j)
      if (j < n) q[j] = v[j];
  }
}

__device__ __forceinline__ cf crcp(cf z) {   // 1 / z
  const float inv = __builtin_amdgcn_rcpf(z.r * z.r + z.i * z.i);
  return cf{z.r * inv, -z.i * inv};
}

// exp(z) for the per-step discretisation: v_exp_f32 and the branch-free
// sincos_cw (each step has its own A_bar, so per-step rounding does not compound
// the way a constant A_bar's does in A_bar^t)
__device__ __forceinline__ cf cexp_step(cf z) {
  float s, c;
  sincos_cw(z.i, s, c);
  const float e = __builtin_amdgcn_exp2f(z.r * kLog2e);
  return cf{e * c, e * s};
}

// A_bar, beta of one step (simplified_scan.cuh:198-224); dt = deltaA (kDA) or delta
template <int kMethod, bool kDA>
__device__ __forceinline__ void sdisc_tv(float dt, float dl, cf A, cf invA, cf& Ab, cf& beta) {
  const cf one = cmake(1.f, 0.f);
  if constexpr (kMethod == LRNNX_BILINEAR) {
    const cf inv = crcp(csub(one, cscale(A, 0.5f * dt)));
    Ab = cmul(cadd(one, cscale(A, 0.5f * dt)), inv);
    beta = kDA ? cscale(crcp(csub(one, cscale(A, 0.5f * dl))), dl) : cscale(inv, dl);
  } else {
    Ab = cexp_step(cscale(A, dt));
    if constexpr (kMethod == LRNNX_ZOH) beta = cmul(csub(kDA ? cexp_step(cscale(A, dl)) : Ab, one), invA);
    else beta = one;
  }
}
}  // namespace

template <int kMethod, bool kDA>
__global__ void __launch_bounds__(256) simpf_fwd_tv_kernel(const lrnnx_simplified_scan_args a, int64_t nch32,
                                                           int64_t n_x) {
  const int lane = threadIdx.x & 63;
  const int64_t seq = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);   // (b, p)
  if (seq >= a.batch * a.dim) return;
  const int64_t b = seq / a.dim, p = seq % a.dim, L = a.seqlen;
  const cf A = ld(static_cast<const float*>(a.A.ptr) + 2 * p * a.A.s0);
  const cf invA = crcp(A);
  const cf BC = cmul(ld(static_cast<const float*>(a.B.ptr) + 2 * p * a.B.s0),
                     ld(static_cast<const float*>(a.C.ptr) + 2 * p * a.C.s0));
  const float* u = static_cast<const float*>(a.u.ptr) + 2 * (b * a.u.s0 + p * a.u.s1);
  const float* dlr = static_cast<const float*>(a.delta.ptr) + b * a.delta.s0 + p * a.delta.s1;
  const float* dar = kDA ? static_cast<const float*>(a.deltaA.ptr) + b * a.deltaA.s0 + p * a.deltaA.s1 : nullptr;
  float* out = a.out.ptr ? static_cast<float*>(a.out.ptr) + 2 * (b * a.out.s0 + p * a.out.s1) : nullptr;
  float* ck = a.ckpt ? static_cast<float*>(a.ckpt) + 2 * seq * nch32 : nullptr;
  float* xp = a.x ? static_cast<float*>(a.x) + 2 * seq * n_x * 2 : nullptr;
  cf hin = cmake(0.f, 0.f), pc = cmake(1.f, 0.f);   // carry into the chunk, prod A_bar over [0, t0)
  for (int64_t t0 = 0; t0 < L; t0 += kCh) {
    const int64_t tl = t0 + kE * lane;
    const int n = (int)max<int64_t>(0, min<int64_t>(kE, L - tl));
    cf uu[kE];
    float dl[kE], da[kE];
    load8(u + 2 * tl, n, uu);
    load8r(dlr, a.delta.s2, tl, n, dl);
    if constexpr (kDA) load8r(dar, a.deltaA.s2, tl, n, da);
    // steps past L: delta 0 gives A_bar 1, and u 0 adds nothing
    cf s[kE], P[kE];
#pragma unroll
    for (int j = 0; j < kE; ++j) {
      cf ab, be;
      sdisc_tv<kMethod, kDA>(kDA ? da[j] : dl[j], dl[j], A, invA, ab, be);
      const cf v = kMethod == LRNNX_DIRAC ? uu[j] : cmul(be, uu[j]);
      s[j] = j == 0 ? v : cfma(ab, s[j - 1], v);
      P[j] = j == 0 ? ab : cmul(ab, P[j - 1]);
    }
    cf Av = P[kE - 1], Sv = s[kE - 1];
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      const int d = 1 << k;
      const cf ao = shfl(Av, lane - d), so = shfl(Sv, lane - d);
      if (lane >= d) {
        Sv = cfma(Av, so, Sv);
        Av = cmul(Av, ao);
      }
    }
    cf Ain = shfl(Av, lane - 1), Sin = shfl(Sv, lane - 1);
    if (lane == 0) {
      Ain = cmake(1.f, 0.f);
      Sin = cmake(0.f, 0.f);
    }
    const cf cin = cfma(Ain, hin, Sin);   // state before the lane's first step
    cf h[kE];
#pragma unroll
    for (int j = 0; j < kE; ++j) h[j] = cfma(P[j], cin, s[j]);
    if (out) {
      cf y[kE];
#pragma unroll
      for (int j = 0; j < kE; ++j) y[j] = cmul(BC, h[j]);
      if (n > 0) store8(out + 2 * tl, n, y);
    }
    if (ck && (lane & 3) == 0 && n > 0) st(ck + 2 * (tl / kSC32), cin);
    if (xp) {  // reference chunk carries (prod A_bar over [0, t], h_t) at t + 1 = 2048 k or t = L - 1
      const cf pl = cmul(pc, Ain);
#pragma unroll
      for (int j = 0; j < kE; ++j) {
        const int64_t t = tl + j;
        if (j < n && ((t + 1) % kXChunk == 0 || t == L - 1)) {
          float* xr = xp + 4 * (t / kXChunk);
          st(xr, cmul(pl, P[j]));
          st(xr + 2, h[j]);
        }
      }
    }
    hin = readlane(h[kE - 1], 63);
    pc = cmul(pc, readlane(Av, 63));
  }
}

// dA, dB, dC partials of one sequence: part[seq] = 3 complex
template <int kMethod, bool kDA>
__global__ void __launch_bounds__(256) simpf_bwd_tv_kernel(const lrnnx_simplified_scan_args a, int64_t nch32,
                                                           float* __restrict__ part) {
  const int lane = threadIdx.x & 63;
  const int64_t seq = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (seq >= a.batch * a.dim) return;
  const int64_t b = seq / a.dim, p = seq % a.dim, L = a.seqlen;
  const cf A = ld(static_cast<const float*>(a.A.ptr) + 2 * p * a.A.s0);
  const cf invA = crcp(A);
  const cf Bs = ld(static_cast<const float*>(a.B.ptr) + 2 * p * a.B.s0);
  const cf Cs = ld(static_cast<const float*>(a.C.ptr) + 2 * p * a.C.s0);
  const cf wBC = cconj(cmul(Bs, Cs));
  constexpr bool kGB = kMethod != LRNNX_DIRAC;   // beta depends on delta and A
  const cf one = cmake(1.f, 0.f);
  const float* u = static_cast<const float*>(a.u.ptr) + 2 * (b * a.u.s0 + p * a.u.s1);
  const float* dout = static_cast<const float*>(a.dout.ptr) + 2 * (b * a.dout.s0 + p * a.dout.s1);
  const float* dlr = static_cast<const float*>(a.delta.ptr) + b * a.delta.s0 + p * a.delta.s1;
  const float* dar = kDA ? static_cast<const float*>(a.deltaA.ptr) + b * a.deltaA.s0 + p * a.deltaA.s1 : nullptr;
  float* du = static_cast<float*>(a.du.ptr) + 2 * (b * a.du.s0 + p * a.du.s1);
  float* ddl = a.need_ddelta ? static_cast<float*>(a.ddelta.ptr) + b * a.ddelta.s0 + p * a.ddelta.s1 : nullptr;
  float* ddA = (a.need_ddelta && kDA) ? static_cast<float*>(a.ddeltaA.ptr) + b * a.ddeltaA.s0 + p * a.ddeltaA.s1
                                      : nullptr;
  const float* ck = static_cast<const float*>(a.ckpt) + 2 * seq * nch32;
  cf dAacc = cmake(0.f, 0.f), SHd = cmake(0.f, 0.f);
  cf Ech = cmake(0.f, 0.f);   // e at the first step of the chunk to the right
  const int64_t n_chunks = (L + kCh - 1) / kCh;
  for (int64_t c = n_chunks - 1; c >= 0; --c) {
    const int64_t t0 = c * kCh, tl = t0 + kE * lane;
    const int n = (int)max<int64_t>(0, min<int64_t>(kE, L - tl));
    cf x[kE], dy[kE];
    float dl[kE], da[kE];
    load8(u + 2 * tl, n, x);
    load8(dout + 2 * tl, n, dy);
    load8r(dlr, a.delta.s2, tl, n, dl);
    if constexpr (kDA) load8r(dar, a.deltaA.s2, tl, n, da);
    // forward recompute from the checkpoint at the chunk start
    cf Ab[kE], be[kE], h[kE], cin;
    {
      cf s[kE], P[kE];
#pragma unroll
      for (int j = 0; j < kE; ++j) {
        sdisc_tv<kMethod, kDA>(kDA ? da[j] : dl[j], dl[j], A, invA, Ab[j], be[j]);
        const cf v = kMethod == LRNNX_DIRAC ? x[j] : cmul(be[j], x[j]);
        s[j] = j == 0 ? v : cfma(Ab[j], s[j - 1], v);
        P[j] = j == 0 ? Ab[j] : cmul(Ab[j], P[j - 1]);
      }
      cf Av = P[kE - 1], Sv = s[kE - 1];
#pragma unroll
      for (int k = 0; k < 6; ++k) {
        const int d = 1 << k;
        const cf ao = shfl(Av, lane - d), so = shfl(Sv, lane - d);
        if (lane >= d) {
          Sv = cfma(Av, so, Sv);
          Av = cmul(Av, ao);
        }
      }
      cf Ain = shfl(Av, lane - 1), Sin = shfl(Sv, lane - 1);
      if (lane == 0) {
        Ain = one;
        Sin = cmake(0.f, 0.f);
      }
      cin = cfma(Ain, ld(ck + 2 * (t0 / kSC32)), Sin);
#pragma unroll
      for (int j = 0; j < kE; ++j) h[j] = cfma(P[j], cin, s[j]);
    }
    // reverse: e_j = conj(A_bar_j) (w dout_j + e_{j+1}); local from e_8 = 0, with Q_j = prod_{i >= j} conj(A_bar_i)
    cf el[kE], Q[kE];
    el[kE - 1] = cmul(cconj(Ab[kE - 1]), cmul(wBC, dy[kE - 1]));
    Q[kE - 1] = cconj(Ab[kE - 1]);
#pragma unroll
    for (int j = kE - 2; j >= 0; --j) {
      el[j] = cmul(cconj(Ab[j]), cfma(wBC, dy[j], el[j + 1]));
      Q[j] = cmul(cconj(Ab[j]), Q[j + 1]);
    }
    cf Mv = Q[0], Rv = el[0];
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      const int d = 1 << k;
      const cf mo = shfl(Mv, lane + d), ro = shfl(Rv, lane + d);
      if (lane + d < 64) {
        Rv = cfma(Mv, ro, Rv);
        Mv = cmul(Mv, mo);
      }
    }
    cf Mn = shfl(Mv, lane + 1), Rn = shfl(Rv, lane + 1);
    if (lane == 63) {
      Mn = one;
      Rn = cmake(0.f, 0.f);
    }
    const cf Ein = cfma(Mn, Ech, Rn);   // e at the first step of the next lane
    cf dx[kE];
    float ddv[kE], ddav[kE];
#pragma unroll
    for (int j = 0; j < kE; ++j) {
      const cf enext = j == kE - 1 ? Ein : cfma(Q[j + 1], Ein, el[j + 1]);
      const cf g = cfma(wBC, dy[j], enext);
      dx[j] = kMethod == LRNNX_DIRAC ? g : cmul(cconj(be[j]), g);
      const cf hp = j > 0 ? h[j - 1] : cin;
      const cf gA = cmul(cconj(hp), g);
      SHd = cfma(cconj(h[j]), dy[j], SHd);
      const float dt = kDA ? da[j] : dl[j];
      // derivatives of A_bar (w.r.t. its time step and A) and of beta (w.r.t. delta and A)
      cf dAb_dt, dAb_dA, db_dl = cmake(0.f, 0.f), db_dA = cmake(0.f, 0.f);
      if constexpr (kMethod == LRNNX_BILINEAR) {
        const cf inv = crcp(csub(one, cscale(A, 0.5f * dt)));
        const cf inv2 = cmul(inv, inv);
        dAb_dt = cmul(A, inv2);
        dAb_dA = cscale(inv2, dt);
        const cf invB = kDA ? crcp(csub(one, cscale(A, 0.5f * dl[j]))) : inv;
        const cf inv2B = cmul(invB, invB);
        db_dl = inv2B;
        db_dA = cscale(inv2B, 0.5f * dl[j] * dl[j]);
      } else {
        dAb_dt = cmul(A, Ab[j]);
        dAb_dA = cscale(Ab[j], dt);
        if constexpr (kMethod == LRNNX_ZOH) {
          const cf e = kDA ? cexp_step(cscale(A, dl[j])) : Ab[j];
          db_dl = e;
          db_dA = cmul(csub(cscale(e, dl[j]), be[j]), invA);
        }
      }
      dAacc = cfma(cconj(dAb_dA), gA, dAacc);
      const float tA = dAb_dt.r * gA.r + dAb_dt.i * gA.i;   // Re(conj(dA_bar/dt) gA)
      float dlv = kDA ? 0.f : tA;
      if constexpr (kGB) {
        const cf gB = cmul(cconj(x[j]), g);
        dAacc = cfma(cconj(db_dA), gB, dAacc);
        dlv += db_dl.r * gB.r + db_dl.i * gB.i;
      }
      ddv[j] = dlv;
      ddav[j] = tA;
    }
    if (n > 0) {
      store8(du + 2 * tl, n, dx);
      if (ddl) store8r(ddl + tl, n, ddv);
      if (ddA) store8r(ddA + tl, n, ddav);
    }
    // e at the first step of this chunk (lane 0's inclusive suffix through the carry)
    Ech = cfma(readlane(Mv, 0), Ech, readlane(Rv, 0));
  }
  // sums over the wave -> one partial per sequence
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const int d = 1 << k;
    dAacc = cadd(dAacc, shfl(dAacc, lane ^ d));
    SHd = cadd(SHd, shfl(SHd, lane ^ d));
  }
  if (lane == 0) {
    float* pt = part + 6 * seq;
    st(pt, dAacc);
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
// constant time step: delta (and deltaA) broadcast along L
bool simpf_const(const lrnnx_simplified_scan_args& a) {
  return a.delta.s2 == 0 && (a.deltaA.ptr == nullptr || a.deltaA.s2 == 0);
}
bool simpf_shape_ok(const lrnnx_simplified_scan_args& a) {
  const bool s2_ok = (a.delta.s2 == 0 || a.delta.s2 == 1) && (a.deltaA.ptr == nullptr || a.deltaA.s2 == 0 ||
                                                              a.deltaA.s2 == 1);
  return a.dstate == 1 && s2_ok && rows16(a.u);
}
int64_t nch32(const lrnnx_simplified_scan_args& a) { return (a.seqlen + kSC32 - 1) / kSC32; }

template <int kMethod>
void launch_fwd_m(const lrnnx_simplified_scan_args& a, dim3 grid, hipStream_t st, int64_t n_x) {
  const dim3 block(256);
  if (simpf_const(a)) hipLaunchKernelGGL(simpf_fwd_kernel<kMethod>, grid, block, 0, st, a, nch32(a), n_x);
  else if (a.deltaA.ptr) hipLaunchKernelGGL((simpf_fwd_tv_kernel<kMethod, true>), grid, block, 0, st, a, nch32(a), n_x);
  else hipLaunchKernelGGL((simpf_fwd_tv_kernel<kMethod, false>), grid, block, 0, st, a, nch32(a), n_x);
}
template <int kMethod>
void launch_bwd_m(const lrnnx_simplified_scan_args& a, dim3 grid, hipStream_t st, float* part) {
  const dim3 block(256);
  if (simpf_const(a)) hipLaunchKernelGGL(simpf_bwd_kernel<kMethod>, grid, block, 0, st, a, nch32(a), part);
  else if (a.deltaA.ptr) hipLaunchKernelGGL((simpf_bwd_tv_kernel<kMethod, true>), grid, block, 0, st, a, nch32(a), part);
  else hipLaunchKernelGGL((simpf_bwd_tv_kernel<kMethod, false>), grid, block, 0, st, a, nch32(a), part);
}
}  // namespace

// Launch the fast forward when it covers the call; false otherwise.
bool simpf_fwd(const lrnnx_simplified_scan_args& a, hipStream_t st, hipError_t* err) {
  if (!simpf_shape_ok(a) || !rows16(a.out)) return false;
  const dim3 grid((unsigned)((a.batch * a.dim + 3) / 4));
  const int64_t n_x = (a.seqlen + kXChunk - 1) / kXChunk;
  switch (a.method) {
    case LRNNX_ZOH: launch_fwd_m<LRNNX_ZOH>(a, grid, st, n_x); break;
    case LRNNX_BILINEAR: launch_fwd_m<LRNNX_BILINEAR>(a, grid, st, n_x); break;
    default: launch_fwd_m<LRNNX_DIRAC>(a, grid, st, n_x); break;
  }
  *err = hipGetLastError();
  return true;
}

// Launch the fast backward when it covers the call; false otherwise.  `part`
// holds batch * dim * 6 floats of workspace; `ckpt_ws`, used when the caller
// passes no checkpoints, holds batch * dim * ceil(L / 32) complex values: the
// fast forward rebuilds the checkpoints there first.
bool simpf_bwd(const lrnnx_simplified_scan_args& a, float* part, float* ckpt_ws, hipStream_t st, hipError_t* err) {
  if (!simpf_shape_ok(a) || !rows16(a.dout) || !rows16(a.du)) return false;
  if (a.ckpt == nullptr && ckpt_ws == nullptr) return false;
  const dim3 grid((unsigned)((a.batch * a.dim + 3) / 4)), block(256);
  lrnnx_simplified_scan_args b = a;
  if (b.ckpt == nullptr) {   // rebuild the checkpoints (no out, no x)
    lrnnx_simplified_scan_args f = a;
    f.out = lrnnx_view{};
    f.x = nullptr;
    f.ckpt = ckpt_ws;
    hipError_t e = hipSuccess;
    simpf_fwd(f, st, &e);
    if (e != hipSuccess) {
      *err = e;
      return true;
    }
    b.ckpt = ckpt_ws;
  }
  switch (b.method) {
    case LRNNX_ZOH: launch_bwd_m<LRNNX_ZOH>(b, grid, st, part); break;
    case LRNNX_BILINEAR: launch_bwd_m<LRNNX_BILINEAR>(b, grid, st, part); break;
    default: launch_bwd_m<LRNNX_DIRAC>(b, grid, st, part); break;
  }
  hipLaunchKernelGGL(simpf_bwd_reduce, dim3((unsigned)((b.dim + 255) / 256)), block, 0, st, b,
                     static_cast<const float*>(part));
  *err = hipGetLastError();
  return true;
}

}  // namespace lrnnx
