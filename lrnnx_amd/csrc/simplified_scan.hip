// Simplified complex diagonal scan (S5 / LRU), forward and backward, gfx950.
//
// Semantics: reference kernels csrc/simplified_scan/simplified_scan.cuh:85-262
// and simplified_scan_backward.cuh:91-420:
//   h_{t,s} = A_bar_{t,s} h_{t-1,s} + beta_{t,s} u_t      (B does not enter here)
//   out_t   = sum_s (B_s C_s) h_{t,s}
// with A_bar, beta from zoh / bilinear / dirac (deltaA, when given, drives A_bar).
//
// Design.  The practical shape has one state per channel and few channels
// (config 1: 8 x 256 channels, L = 4096), so parallelism comes from L: each
// (b, p) sequence is cut into chunks of kSC steps and one lane owns one
// (b, p, chunk).  Three launches per direction:
//   1. chunk aggregates  (prod A_bar over the chunk, local end state from 0),
//   2. carry scan over the chunks of each (b, p, s)  -> chunk start states
//      (kept in `ckpt` for the backward) and the reference's x carries,
//   3. rescan of every chunk from its start state, writing the outputs.
// The backward mirrors this right-to-left for dh (carry q = conj(A_bar) dh),
// recomputes h inside each chunk from the forward's start states, and writes
// per-thread partials of dA, dB, dC that a last kernel sums in a fixed order.
// When delta (and deltaA) has zero stride along L, A_bar and beta are
// computed once per (b, p, s) instead of per element.
#include "simp_common.h"

namespace lrnnx {

constexpr int kSC = 32;  // chunk length along L

struct SView {  // (b, p, l) real or complex sequence view
  const float* p;
  int64_t s0, s1, s2;
};

struct SimpParams {
  lrnnx_simplified_scan_args a;
  int64_t nch;       // chunks per sequence
  int64_t n_x;       // reference x chunks
  float* agg;        // [b][p][s][nch] x 4 floats
  float* carry;      // [b][p][s][nch] complex  (forward: h start; backward: q in)
  float* ckpt;       // forward chunk-start states (== carry in the forward)
  float* part;       // backward partials [b][nch][p][s] x 3 complex
  bool dl_const, dtA_const;
};

__device__ __forceinline__ float seq_real(const lrnnx_view& v, int64_t b, int64_t p, int64_t t) {
  return static_cast<const float*>(v.ptr)[b * v.s0 + p * v.s1 + t * v.s2];
}

// ---------------------------------------------------------------- forward
template <int kMethod>
__global__ void __launch_bounds__(256) simp_fwd_agg(SimpParams P) {
  const auto& a = P.a;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = a.batch * a.dim * P.nch;
  if (gid >= total) return;
  const int64_t c = gid % P.nch, bp = gid / P.nch, p = bp % a.dim, b = bp / a.dim;
  const int64_t t0 = c * kSC;
  const int len = (int)min<int64_t>(kSC, a.seqlen - t0);
  const float* u = static_cast<const float*>(a.u.ptr) + 2 * (b * a.u.s0 + p * a.u.s1);
  const bool hasdA = a.deltaA.ptr != nullptr;
  for (int64_t s = 0; s < a.dstate; ++s) {
    const cf A = ld(static_cast<const float*>(a.A.ptr) + 2 * (p * a.A.s0 + s * a.A.s1));
    cf h = cmake(0.f, 0.f), prod = cmake(1.f, 0.f);
    float sumdt = 0.f;
    cf Ab, beta;
    if (P.dl_const) {
      const float dl = seq_real(a.delta, b, p, 0);
      const float dt = hasdA ? seq_real(a.deltaA, b, p, 0) : dl;
      sdisc<kMethod>(dt, dl, A, Ab, beta);
    }
    for (int j = 0; j < len; ++j) {
      const int64_t t = t0 + j;
      if (!P.dl_const) {
        const float dl = seq_real(a.delta, b, p, t);
        const float dt = hasdA ? seq_real(a.deltaA, b, p, t) : dl;
        sdisc<kMethod>(dt, dl, A, Ab, beta);
        sumdt += dt;
      }
      const cf x = ld(u + 2 * t);
      h = cfma(Ab, h, kMethod == LRNNX_DIRAC ? x : cmul(beta, x));
      if (kMethod == LRNNX_BILINEAR || P.dl_const) prod = cmul(prod, Ab);
    }
    if (kMethod != LRNNX_BILINEAR && !P.dl_const) prod = cexp_(cscale(A, sumdt));
    float* ag = P.agg + 4 * ((bp * a.dstate + s) * P.nch + c);
    *reinterpret_cast<float4*>(ag) = make_float4(prod.r, prod.i, h.r, h.i);
  }
}

// carry scan over chunks (forward): start state of every chunk + reference x
__global__ void __launch_bounds__(256) simp_fwd_carry(SimpParams P) {
  const auto& a = P.a;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= a.batch * a.dim * a.dstate) return;
  const int64_t s = gid % a.dstate, bp = gid / a.dstate;
  cf h = cmake(0.f, 0.f), pc = cmake(1.f, 0.f);
  float* x = static_cast<float*>(a.x);
  for (int64_t c = 0; c < P.nch; ++c) {
    const int64_t o = gid * P.nch + c;
    st(P.carry + 2 * o, h);
    const float4 g = *reinterpret_cast<const float4*>(P.agg + 4 * o);
    h = cfma(cmake(g.x, g.y), h, cmake(g.z, g.w));
    pc = cmul(pc, cmake(g.x, g.y));
    const int64_t tend = min<int64_t>((c + 1) * kSC, a.seqlen);  // exclusive
    if (x != nullptr && (tend % kXChunk == 0 || tend == a.seqlen)) {
      const int64_t xc = (tend - 1) / kXChunk;
      float* xr = x + 2 * ((bp * P.n_x + xc) * 2 * a.dstate);
      st(xr + 2 * (2 * s), pc);
      st(xr + 2 * (2 * s + 1), h);
    }
  }
}

template <int kMethod>
__global__ void __launch_bounds__(256) simp_fwd_out(SimpParams P) {
  const auto& a = P.a;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= a.batch * a.dim * P.nch) return;
  const int64_t c = gid % P.nch, bp = gid / P.nch, p = bp % a.dim, b = bp / a.dim;
  const int64_t t0 = c * kSC;
  const int len = (int)min<int64_t>(kSC, a.seqlen - t0);
  const float* u = static_cast<const float*>(a.u.ptr) + 2 * (b * a.u.s0 + p * a.u.s1);
  float* out = static_cast<float*>(a.out.ptr) + 2 * (b * a.out.s0 + p * a.out.s1);
  const bool hasdA = a.deltaA.ptr != nullptr;
  for (int64_t s = 0; s < a.dstate; ++s) {
    const cf A = ld(static_cast<const float*>(a.A.ptr) + 2 * (p * a.A.s0 + s * a.A.s1));
    const cf BC = cmul(ld(static_cast<const float*>(a.B.ptr) + 2 * (p * a.B.s0 + s * a.B.s1)),
                       ld(static_cast<const float*>(a.C.ptr) + 2 * (p * a.C.s0 + s * a.C.s1)));
    cf h = ld(P.carry + 2 * ((bp * a.dstate + s) * P.nch + c));
    cf Ab, beta;
    if (P.dl_const) {
      const float dl = seq_real(a.delta, b, p, 0);
      sdisc<kMethod>(hasdA ? seq_real(a.deltaA, b, p, 0) : dl, dl, A, Ab, beta);
    }
    for (int j = 0; j < len; ++j) {
      const int64_t t = t0 + j;
      if (!P.dl_const) {
        const float dl = seq_real(a.delta, b, p, t);
        sdisc<kMethod>(hasdA ? seq_real(a.deltaA, b, p, t) : dl, dl, A, Ab, beta);
      }
      const cf x = ld(u + 2 * t);
      h = cfma(Ab, h, kMethod == LRNNX_DIRAC ? x : cmul(beta, x));
      const cf y = cmul(BC, h);
      st(out + 2 * t, s == 0 ? y : cadd(ld(out + 2 * t), y));
    }
  }
}

// ---------------------------------------------------------------- backward
// chunk aggregate of the reverse recurrence g_t = conj(A_bar_{t+1}) g_{t+1} + w_t,
// w_t = conj(B_s C_s) dout_t.  With q = conj(A_bar_{t1+1}) g_{t1+1} entering
// from the right, the carry leaving to the left is Q q + R with
// Q = conj(prod A_bar over the chunk), R = conj(A_bar_{t0}) g_{t0}|_{q=0}.
template <int kMethod>
__global__ void __launch_bounds__(256) simp_bwd_agg(SimpParams P) {
  const auto& a = P.a;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= a.batch * a.dim * P.nch) return;
  const int64_t c = gid % P.nch, bp = gid / P.nch, p = bp % a.dim, b = bp / a.dim;
  const int64_t t0 = c * kSC;
  const int len = (int)min<int64_t>(kSC, a.seqlen - t0);
  const float* dout = static_cast<const float*>(a.dout.ptr) + 2 * (b * a.dout.s0 + p * a.dout.s1);
  const bool hasdA = a.deltaA.ptr != nullptr;
  for (int64_t s = 0; s < a.dstate; ++s) {
    const cf A = ld(static_cast<const float*>(a.A.ptr) + 2 * (p * a.A.s0 + s * a.A.s1));
    const cf wBC = cconj(cmul(ld(static_cast<const float*>(a.B.ptr) + 2 * (p * a.B.s0 + s * a.B.s1)),
                              ld(static_cast<const float*>(a.C.ptr) + 2 * (p * a.C.s0 + s * a.C.s1))));
    cf g = cmake(0.f, 0.f), carry = cmake(0.f, 0.f), prod = cmake(1.f, 0.f);
    cf Ab, beta;
    if (P.dl_const) {
      const float dl = seq_real(a.delta, b, p, 0);
      sdisc<kMethod>(hasdA ? seq_real(a.deltaA, b, p, 0) : dl, dl, A, Ab, beta);
    }
    for (int j = len - 1; j >= 0; --j) {
      const int64_t t = t0 + j;
      if (!P.dl_const) {
        const float dl = seq_real(a.delta, b, p, t);
        sdisc<kMethod>(hasdA ? seq_real(a.deltaA, b, p, t) : dl, dl, A, Ab, beta);
      }
      g = cfma(wBC, ld(dout + 2 * t), carry);
      carry = cmul(cconj(Ab), g);
      prod = cmul(prod, Ab);
    }
    const cf Q = cconj(prod);
    float* ag = P.agg + 4 * ((bp * a.dstate + s) * P.nch + c);
    *reinterpret_cast<float4*>(ag) = make_float4(Q.r, Q.i, carry.r, carry.i);
  }
}

__global__ void __launch_bounds__(256) simp_bwd_carry(SimpParams P) {
  const auto& a = P.a;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= a.batch * a.dim * a.dstate) return;
  cf q = cmake(0.f, 0.f);
  for (int64_t c = P.nch - 1; c >= 0; --c) {
    const int64_t o = gid * P.nch + c;
    st(P.carry + 2 * o, q);
    const float4 g = *reinterpret_cast<const float4*>(P.agg + 4 * o);
    q = cfma(cmake(g.x, g.y), q, cmake(g.z, g.w));
  }
}

template <int kMethod>
__global__ void __launch_bounds__(256) simp_bwd_main(SimpParams P) {
  const auto& a = P.a;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= a.batch * a.dim * P.nch) return;
  const int64_t c = gid % P.nch, bp = gid / P.nch, p = bp % a.dim, b = bp / a.dim;
  const int64_t t0 = c * kSC;
  const int len = (int)min<int64_t>(kSC, a.seqlen - t0);
  const float* u = static_cast<const float*>(a.u.ptr) + 2 * (b * a.u.s0 + p * a.u.s1);
  const float* dout = static_cast<const float*>(a.dout.ptr) + 2 * (b * a.dout.s0 + p * a.dout.s1);
  float* du = static_cast<float*>(a.du.ptr) + 2 * (b * a.du.s0 + p * a.du.s1);
  float* ddl = a.need_ddelta ? static_cast<float*>(a.ddelta.ptr) + b * a.ddelta.s0 + p * a.ddelta.s1 : nullptr;
  const bool hasdA = a.deltaA.ptr != nullptr;
  float* ddA = (a.need_ddelta && hasdA) ? static_cast<float*>(a.ddeltaA.ptr) + b * a.ddeltaA.s0 + p * a.ddeltaA.s1
                                        : nullptr;
  for (int64_t s = 0; s < a.dstate; ++s) {
    const cf A = ld(static_cast<const float*>(a.A.ptr) + 2 * (p * a.A.s0 + s * a.A.s1));
    const cf Bs = ld(static_cast<const float*>(a.B.ptr) + 2 * (p * a.B.s0 + s * a.B.s1));
    const cf Cs = ld(static_cast<const float*>(a.C.ptr) + 2 * (p * a.C.s0 + s * a.C.s1));
    const cf wBC = cconj(cmul(Bs, Cs));
    const int64_t o = (bp * a.dstate + s) * P.nch + c;
    // recompute h inside the chunk from the forward's start state
    cf H[kSC];
    {
      cf h = ld(P.ckpt + 2 * o);
      cf Ab, beta;
      if (P.dl_const) {
        const float dl = seq_real(a.delta, b, p, 0);
        sdisc<kMethod>(hasdA ? seq_real(a.deltaA, b, p, 0) : dl, dl, A, Ab, beta);
      }
#pragma unroll
      for (int j = 0; j < kSC; ++j) {
        if (j < len) {
          const int64_t t = t0 + j;
          if (!P.dl_const) {
            const float dl = seq_real(a.delta, b, p, t);
            sdisc<kMethod>(hasdA ? seq_real(a.deltaA, b, p, t) : dl, dl, A, Ab, beta);
          }
          const cf x = ld(u + 2 * t);
          h = cfma(Ab, h, kMethod == LRNNX_DIRAC ? x : cmul(beta, x));
          H[j] = h;
        }
      }
    }
    const cf h_start = ld(P.ckpt + 2 * o);
    cf carry = ld(P.carry + 2 * o);
    cf dA = cmake(0.f, 0.f), dB = cmake(0.f, 0.f), dC = cmake(0.f, 0.f);
#pragma unroll
    for (int j = kSC - 1; j >= 0; --j) {
      if (j < len) {
        const int64_t t = t0 + j;
        const float dl = P.dl_const ? seq_real(a.delta, b, p, 0) : seq_real(a.delta, b, p, t);
        const float dt = hasdA ? (P.dtA_const ? seq_real(a.deltaA, b, p, 0) : seq_real(a.deltaA, b, p, t)) : dl;
        cf Ab, beta;
        sdisc<kMethod>(dt, dl, A, Ab, beta);
        const cf dy = ld(dout + 2 * t);
        const cf g = cfma(wBC, dy, carry);        // dh_t
        carry = cmul(cconj(Ab), g);
        const cf hp = j > 0 ? H[j - 1] : h_start;
        const cf x = ld(u + 2 * t);
        // du (PyTorch convention: grad_in = conj(d out / d in) * grad_out)
        const cf dx = kMethod == LRNNX_DIRAC ? g : cmul(cconj(beta), g);
        st(du + 2 * t, s == 0 ? dx : cadd(ld(du + 2 * t), dx));
        const cf gA = cmul(cconj(hp), g);        // grad wrt A_bar
        const cf gB = cmul(cconj(x), g);         // grad wrt beta
        // dA_bar / d(dtA) and dA_bar / dA
        cf dAb_dt, dAb_dA;
        if constexpr (kMethod == LRNNX_BILINEAR) {
          const cf one = cmake(1.f, 0.f);
          const cf om = csub(one, cscale(A, 0.5f * dt));
          const cf inv2 = cdiv(one, cmul(om, om));
          dAb_dt = cmul(A, inv2);
          dAb_dA = cscale(inv2, dt);
        } else {
          dAb_dt = cmul(A, Ab);
          dAb_dA = cscale(Ab, dt);
        }
        float ddl_v = 0.f, ddA_v = 0.f;
        const float tA = dAb_dt.r * gA.r + dAb_dt.i * gA.i;  // Re(conj(dAb/dt) gA)
        if (hasdA) ddA_v = tA; else ddl_v = tA;
        cf dAcontrib = cmul(cconj(dAb_dA), gA);
        if constexpr (kMethod == LRNNX_ZOH) {
          const cf e = cexp_(cscale(A, dl));
          ddl_v += e.r * gB.r + e.i * gB.i;
          const cf dbeta_dA = cdiv(csub(cscale(e, dl), beta), A);
          dAcontrib = cadd(dAcontrib, cmul(cconj(dbeta_dA), gB));
        } else if constexpr (kMethod == LRNNX_BILINEAR) {
          const cf one = cmake(1.f, 0.f);
          const cf om = csub(one, cscale(A, 0.5f * dl));
          const cf inv2 = cdiv(one, cmul(om, om));
          ddl_v += inv2.r * gB.r + inv2.i * gB.i;
          dAcontrib = cadd(dAcontrib, cmul(cconj(cscale(inv2, 0.5f * dl * dl)), gB));
        }
        dA = cadd(dA, dAcontrib);
        if (ddl) ddl[t] = s == 0 ? ddl_v : ddl[t] + ddl_v;
        if (ddA) ddA[t] = s == 0 ? ddA_v : ddA[t] + ddA_v;
        // out = sum_s B_s C_s h_s
        dB = cadd(dB, cmul(cconj(cmul(Cs, H[j])), dy));
        dC = cadd(dC, cmul(cconj(cmul(Bs, H[j])), dy));
      }
    }
    float* pt = P.part + 6 * (((b * P.nch + c) * a.dim + p) * a.dstate + s);
    st(pt, dA);
    st(pt + 2, dB);
    st(pt + 4, dC);
  }
}

// dA, dB, dC (p, s) = sum over (b, chunk) of the partials, in a fixed order
__global__ void __launch_bounds__(256) simp_bwd_reduce(SimpParams P) {
  const auto& a = P.a;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (p, s)
  if (i >= a.dim * a.dstate) return;
  const int64_t p = i / a.dstate, s = i % a.dstate;
  cf sA = cmake(0.f, 0.f), sB = cmake(0.f, 0.f), sC = cmake(0.f, 0.f);
  const int64_t rows = a.batch * P.nch;
  for (int64_t r = 0; r < rows; ++r) {
    const float* pt = P.part + 6 * (r * a.dim * a.dstate + i);
    sA = cadd(sA, ld(pt));
    sB = cadd(sB, ld(pt + 2));
    sC = cadd(sC, ld(pt + 4));
  }
  st(static_cast<float*>(a.dA.ptr) + 2 * (p * a.dA.s0 + s * a.dA.s1), sA);
  st(static_cast<float*>(a.dB.ptr) + 2 * (p * a.dB.s0 + s * a.dB.s1), sB);
  st(static_cast<float*>(a.dC.ptr) + 2 * (p * a.dC.s0 + s * a.dC.s1), sC);
}

// ---------------------------------------------------------------- host side
static int64_t simp_nch(const lrnnx_simplified_scan_args& a) { return (a.seqlen + kSC - 1) / kSC; }

int64_t simp_ckpt_bytes(const lrnnx_simplified_scan_args& a) {
  return a.batch * a.dim * a.dstate * simp_nch(a) * 8;
}

// fp32 element offsets in the workspace
static void simp_ws(const lrnnx_simplified_scan_args& a, bool bwd, bool need_ckpt, int64_t& agg, int64_t& carry,
                    int64_t& ck, int64_t& part, int64_t& total) {
  const int64_t nseq = a.batch * a.dim * a.dstate * simp_nch(a);
  int64_t o = 0;
  agg = o; o += (nseq * 4 + 63) / 64 * 64;
  carry = o; o += (nseq * 2 + 63) / 64 * 64;
  ck = o; if (need_ckpt) o += (nseq * 2 + 63) / 64 * 64;
  part = o; if (bwd) o += (a.batch * simp_nch(a) * a.dim * a.dstate * 6 + 63) / 64 * 64;
  total = o;
}

int64_t simp_ws_bytes(const lrnnx_simplified_scan_args& a, int bwd) {
  int64_t agg, carry, ck, part, total;
  simp_ws(a, bwd != 0, bwd != 0 && a.ckpt == nullptr, agg, carry, ck, part, total);
  return total * 4;
}

template <int kMethod>
static hipError_t simp_fwd_t(SimpParams P, hipStream_t st) {
  const int64_t n1 = P.a.batch * P.a.dim * P.nch, n2 = P.a.batch * P.a.dim * P.a.dstate;
  hipLaunchKernelGGL(simp_fwd_agg<kMethod>, dim3((unsigned)((n1 + 255) / 256)), dim3(256), 0, st, P);
  hipLaunchKernelGGL(simp_fwd_carry, dim3((unsigned)((n2 + 255) / 256)), dim3(256), 0, st, P);
  if (P.a.out.ptr)
    hipLaunchKernelGGL(simp_fwd_out<kMethod>, dim3((unsigned)((n1 + 255) / 256)), dim3(256), 0, st, P);
  return hipGetLastError();
}

static SimpParams simp_params(const lrnnx_simplified_scan_args& a) {
  SimpParams P;
  P.a = a;
  P.nch = simp_nch(a);
  P.n_x = (a.seqlen + kXChunk - 1) / kXChunk;
  P.dl_const = a.delta.s2 == 0 && (a.deltaA.ptr == nullptr || a.deltaA.s2 == 0);
  P.dtA_const = a.deltaA.ptr != nullptr && a.deltaA.s2 == 0;
  return P;
}

bool simpf_fwd(const lrnnx_simplified_scan_args& a, hipStream_t st, hipError_t* err);
bool simpf_bwd(const lrnnx_simplified_scan_args& a, float* part, float* ckpt_ws, hipStream_t st, hipError_t* err);
bool fast_paths_enabled();

hipError_t simp_fwd_launch(const lrnnx_simplified_scan_args& a, hipStream_t st) {
  hipError_t e = hipSuccess;
  if (fast_paths_enabled() && simpf_fwd(a, st, &e)) return e;
  SimpParams P = simp_params(a);
  int64_t agg, carry, ck, part, total;
  simp_ws(a, false, false, agg, carry, ck, part, total);
  float* ws = static_cast<float*>(a.workspace);
  P.agg = ws + agg;
  P.carry = a.ckpt ? static_cast<float*>(a.ckpt) : ws + carry;
  P.ckpt = P.carry;
  P.part = nullptr;
  switch (a.method) {
    case LRNNX_ZOH: return simp_fwd_t<LRNNX_ZOH>(P, st);
    case LRNNX_BILINEAR: return simp_fwd_t<LRNNX_BILINEAR>(P, st);
    case LRNNX_DIRAC: return simp_fwd_t<LRNNX_DIRAC>(P, st);
  }
  return hipErrorInvalidValue;
}

template <int kMethod>
static hipError_t simp_bwd_t(SimpParams P, hipStream_t st) {
  const int64_t n1 = P.a.batch * P.a.dim * P.nch, n2 = P.a.batch * P.a.dim * P.a.dstate;
  const dim3 g1((unsigned)((n1 + 255) / 256)), g2((unsigned)((n2 + 255) / 256));
  if (P.a.ckpt == nullptr) {  // rebuild the forward chunk-start states
    SimpParams F = P;
    F.carry = P.ckpt;
    F.a.out.ptr = nullptr;
    F.a.x = nullptr;
    hipLaunchKernelGGL(simp_fwd_agg<kMethod>, g1, dim3(256), 0, st, F);
    hipLaunchKernelGGL(simp_fwd_carry, g2, dim3(256), 0, st, F);
  }
  hipLaunchKernelGGL(simp_bwd_agg<kMethod>, g1, dim3(256), 0, st, P);
  hipLaunchKernelGGL(simp_bwd_carry, g2, dim3(256), 0, st, P);
  hipLaunchKernelGGL(simp_bwd_main<kMethod>, g1, dim3(256), 0, st, P);
  const int64_t n3 = P.a.dim * P.a.dstate;
  hipLaunchKernelGGL(simp_bwd_reduce, dim3((unsigned)((n3 + 255) / 256)), dim3(256), 0, st, P);
  return hipGetLastError();
}

hipError_t simp_bwd_launch(const lrnnx_simplified_scan_args& a, hipStream_t st) {
  SimpParams P = simp_params(a);
  int64_t agg, carry, ck, part, total;
  simp_ws(a, true, a.ckpt == nullptr, agg, carry, ck, part, total);
  float* ws = static_cast<float*>(a.workspace);
  hipError_t e = hipSuccess;
  if (fast_paths_enabled() && simpf_bwd(a, ws + part, a.ckpt ? nullptr : ws + ck, st, &e)) return e;
  P.agg = ws + agg;
  P.carry = ws + carry;
  P.ckpt = a.ckpt ? static_cast<float*>(a.ckpt) : ws + ck;
  P.part = ws + part;
  switch (a.method) {
    case LRNNX_ZOH: return simp_bwd_t<LRNNX_ZOH>(P, st);
    case LRNNX_BILINEAR: return simp_bwd_t<LRNNX_BILINEAR>(P, st);
    case LRNNX_DIRAC: return simp_bwd_t<LRNNX_DIRAC>(P, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace lrnnx
