// Selective scan backward (real weights), gfx950.
//
// Semantics: reference kernel csrc/selective_scan/selective_scan_backward.cuh:86-845
// (gradients of the forward defined in ss_fwd_impl.h; softplus backward =
// sigmoid, :797-799; dz = dout * out * sigma(z) (1 + z (1 - sigma(z))), :218-219).
//
// Per workgroup (b, channel block), tiles of kTB steps are processed from the
// end of the sequence to the start; each tile holds kTB / kCk checkpoint
// intervals ("sub-chunks").  Per sub-chunk a wave
//   1. reloads h at the sub-chunk start from the forward's fp32 checkpoints,
//   2. recomputes A_bar and h for the kCk steps and keeps them in VGPRs,
//   3. walks the steps backwards: dh_t = A_bar_{t+1} dh_{t+1} + C_t dy_t, and
//      accumulates the per-step partials of du / ddelta / ddeltaA (summed
//      over its kS states; crossed over waves in LDS), dA (per lane), and the
//      kS * kCk per-lane values of dB / dC,
//   4. reduce-scatters the dB / dC values over the 64 channels of the wave
//      and writes one fp32 partial per (channel block, b, n, t) to the
//      workspace.  A second kernel sums the partials over channel blocks in
//      a fixed order, so the result is deterministic (the reference uses one
//      global atomic per element and channel block,
//      selective_scan_backward.cuh:483-502).
#pragma once
#include "ss_common.h"

namespace lrnnx {

template <int kMethod>
__host__ __device__ constexpr bool needs_p3() {
  return kMethod == LRNNX_ZOH || kMethod == LRNNX_BILINEAR || kMethod == LRNNX_RGLRU;
}
inline bool needs_p3_rt(int m) { return m == LRNNX_ZOH || m == LRNNX_BILINEAR || m == LRNNX_RGLRU; }

struct SSBwdWs {  // fp32 workspace sections (element offsets)
  int64_t dBv, dCv, dA, dBc, dCc, dD, dbias, ckpt, total;
};

inline int64_t align64(int64_t x) { return (x + 63) / 64 * 64; }

inline SSBwdWs ss_bwd_ws(const lrnnx_selective_scan_args& a, const SSGeom& g, bool need_ckpt) {
  SSBwdWs w;
  int64_t o = 0;
  const int64_t B = a.batch, D = a.dim, N = a.dstate, L = a.seqlen;
  w.dBv = o; if (a.var_B) o += align64((int64_t)g.n_cb * B * N * L);
  w.dCv = o; if (a.var_C) o += align64((int64_t)g.n_cb * B * N * L);
  w.dA = o; o += align64(B * D * N);
  w.dBc = o; if (!a.var_B) o += align64(B * D * N);
  w.dCc = o; if (!a.var_C) o += align64(B * D * N);
  w.dD = o; o += align64(B * D);
  w.dbias = o; o += align64(B * D);
  w.ckpt = o; if (need_ckpt) o += align64(B * g.n_ck * N * D);
  w.total = o;
  return w;
}

template <typename IT, int kS, int kMethod, bool kVarB, bool kVarC>
__global__ void __launch_bounds__(512)
ss_bwd_kernel(const lrnnx_selective_scan_args a, const int CB, const int64_t n_ck, float* __restrict__ ws,
              const SSBwdWs wo, const float* __restrict__ ckp) {
  constexpr int kCk = ck_for(kS);
  constexpr int kTB = tb_for(kS);
  constexpr int kP = kTB + 4;
  constexpr int V = Vec<IT>::n;
  constexpr int kNV = kS * kCk;       // dB/dC values per lane per sub-chunk (<= 64)
  constexpr bool kP3 = needs_p3<kMethod>();
  extern __shared__ float smem[];

  const int nW = blockDim.x / kWave;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int64_t b = blockIdx.y;
  const int64_t D = a.dim, L = a.seqlen, N = a.dstate;
  const int64_t cb = blockIdx.x;
  const int64_t d0 = cb * CB;
  const int64_t d = d0 + lane;
  const bool lane_ok = lane < CB && d < D;
  const int64_t grp = (a.var_B || a.var_C) ? d0 / (D / a.n_groups) : 0;
  const int n0 = w * kS;
  const bool has_dA_in = a.deltaA.ptr != nullptr;
  const bool has_dA = has_dA_in && uses_deltaA<kMethod>();
  const bool has_bias = a.delta_bias.ptr != nullptr;
  const bool has_D = a.D.ptr != nullptr;
  const bool has_z = a.z.ptr != nullptr;

  float* sDl = smem;               // [64][kP] delta'
  float* sU = sDl + kWave * kP;    // [64][kP] u
  float* sDy = sU + kWave * kP;    // [64][kP] dy = dout * silu(z)
  float* sDt = sDy + kWave * kP;   // [64][kP] deltaA
  float* sB = sDt + kWave * kP;    // [nW*kS][kTB] (rows >= N are zero)
  float* sC = sB + nW * kS * kTB;  // [nW*kS][kTB]
  float* sP1 = sC + nW * kS * kTB;       // [nW][64][kP]
  float* sP2 = sP1 + nW * kWave * kP;
  float* sP3 = sP2 + nW * kWave * kP;  // only if kP3
  if (!has_dA) sDt = sDl;

  float a2[kS], Araw[kS], bcst[kS], ccst[kS], cout_c[kS];
  float dh[kS], Anext[kS], dA_acc[kS], dBc_acc[kS], dCc_acc[kS];
  const float* Ap = static_cast<const float*>(a.A.ptr);
  const float* Bp = static_cast<const float*>(a.B.ptr);
  const float* Cp = static_cast<const float*>(a.C.ptr);
#pragma unroll
  for (int k = 0; k < kS; ++k) {
    const int n = n0 + k;
    const bool ok = lane_ok && n < N;
    const float Av = ok ? Ap[d * a.A.s0 + n * a.A.s1] : (kMethod == LRNNX_RGLRU ? 0.5f : -1.f);
    Araw[k] = Av;
    a2[k] = prep_a2<kMethod>(Av);
    bcst[k] = (!kVarB && ok) ? Bp[d * a.B.s0 + n * a.B.s1] : 1.f;
    ccst[k] = (!kVarC && ok) ? Cp[d * a.C.s0 + n * a.C.s1] : 1.f;
    cout_c[k] = ok ? (kVarB ? 1.f : bcst[k]) * (kVarC ? 1.f : ccst[k]) : 0.f;
    dh[k] = 0.f; Anext[k] = 0.f; dA_acc[k] = 0.f; dBc_acc[k] = 0.f; dCc_acc[k] = 0.f;
  }
  float dD_acc = 0.f, dbias_acc = 0.f;  // wave 0, per channel

  const IT* Pu = static_cast<const IT*>(a.u.ptr);
  const IT* Pd = static_cast<const IT*>(a.delta.ptr);
  const IT* PdA = static_cast<const IT*>(a.deltaA.ptr);
  const IT* Pz = static_cast<const IT*>(a.z.ptr);
  const IT* Pdo = static_cast<const IT*>(a.dout.ptr);
  const IT* Pos = static_cast<const IT*>(a.out_saved.ptr);
  const IT* VBp = static_cast<const IT*>(a.B.ptr);
  const IT* VCp = static_cast<const IT*>(a.C.ptr);
  IT* Pdu = static_cast<IT*>(a.du.ptr);
  IT* Pddl = static_cast<IT*>(a.ddelta.ptr);
  IT* PddA = static_cast<IT*>(a.ddeltaA.ptr);
  IT* Pdz = static_cast<IT*>(a.dz.ptr);

  const int vpr = kTB / V;
  const int rows = CB;
  const int64_t n_tiles = (L + kTB - 1) / kTB;
  for (int64_t tile = n_tiles - 1; tile >= 0; --tile) {
    const int64_t t0 = tile * kTB;
    const int Tv = (int)((L - t0) < kTB ? (L - t0) : kTB);
    __syncthreads();
    // ---- tile load; dz is finished here (it needs only dout, out, z)
    for (int e = tid; e < rows * vpr; e += blockDim.x) {
      const int r = e / vpr, c = (e % vpr) * V;
      const int64_t dr = d0 + r;
      const int nv = Tv - c;
      float vu[V], vd[V], vdy[V], va[V];
      if (dr < D && nv > 0) {
        const int n_ = nv < V ? nv : V;
        load_vec(Pu + b * a.u.s0 + dr * a.u.s1 + t0 + c, n_, vu);
        load_vec(Pd + b * a.delta.s0 + dr * a.delta.s1 + t0 + c, n_, vd);
        load_vec(Pdo + b * a.dout.s0 + dr * a.dout.s1 + t0 + c, n_, vdy);
        const float bias = has_bias ? static_cast<const float*>(a.delta_bias.ptr)[dr * a.delta_bias.s0] : 0.f;
#pragma unroll
        for (int i = 0; i < V; ++i) {
          const float x = vd[i] + bias;
          vd[i] = a.delta_softplus ? softplus20(x) : x;
        }
        if (has_z) {
          float vz[V], vo[V], dzv[V];
          load_vec(Pz + b * a.z.s0 + dr * a.z.s1 + t0 + c, n_, vz);
          load_vec(Pos + b * a.out_saved.s0 + dr * a.out_saved.s1 + t0 + c, n_, vo);
#pragma unroll
          for (int i = 0; i < V; ++i) {
            const float sg = 1.f / (1.f + expf(-vz[i]));
            dzv[i] = vdy[i] * vo[i] * sg * (1.f + vz[i] * (1.f - sg));
            vdy[i] = vdy[i] * vz[i] * sg;
          }
          store_vec(Pdz + b * a.dz.s0 + dr * a.dz.s1 + t0 + c, n_, dzv);
        }
        if (has_dA) load_vec(PdA + b * a.deltaA.s0 + dr * a.deltaA.s1 + t0 + c, n_, va);
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i) { vu[i] = 0.f; vd[i] = 0.f; vdy[i] = 0.f; va[i] = 0.f; }
      }
#pragma unroll
      for (int i = 0; i < V; ++i) {
        sU[r * kP + c + i] = vu[i];
        sDl[r * kP + c + i] = vd[i];
        sDy[r * kP + c + i] = vdy[i];
        if (has_dA) sDt[r * kP + c + i] = va[i];
      }
    }
    if constexpr (kVarB || kVarC) {
      for (int e = tid; e < nW * kS * vpr; e += blockDim.x) {
        const int n = e / vpr, c = (e % vpr) * V;
        const int nv = n < N ? Tv - c : 0;  // padded states get B = C = 0
        const int n_ = nv < V ? (nv > 0 ? nv : 0) : V;
        float vb[V], vc[V];
        if constexpr (kVarB) {
          load_vec(VBp + b * a.B.s0 + grp * a.B.s1 + n * a.B.s2 + t0 + c, n_, vb);
#pragma unroll
          for (int i = 0; i < V; ++i) sB[n * kTB + c + i] = vb[i];
        }
        if constexpr (kVarC) {
          load_vec(VCp + b * a.C.s0 + grp * a.C.s1 + n * a.C.s2 + t0 + c, n_, vc);
#pragma unroll
          for (int i = 0; i < V; ++i) sC[n * kTB + c + i] = vc[i];
        }
      }
    }
    __syncthreads();

    // ---- sub-chunks of this tile, last first
    const int n_sub = (Tv + kCk - 1) / kCk;
    for (int s = n_sub - 1; s >= 0; --s) {
      const int ts = s * kCk;                       // tile-local start
      const int Ls = (Tv - ts) < kCk ? (Tv - ts) : kCk;
      const int64_t kk = (t0 + ts) / kCk;           // global checkpoint interval index
      float h0[kS];
#pragma unroll
      for (int k = 0; k < kS; ++k)
        h0[k] = (kk > 0 && lane_ok && n0 + k < N) ? ckp[((b * n_ck + kk - 1) * N + n0 + k) * D + d] : 0.f;

      float Ab[kCk][kS], H[kCk][kS];
      // recompute
      {
        float hc[kS];
#pragma unroll
        for (int k = 0; k < kS; ++k) hc[k] = h0[k];
#pragma unroll
        for (int j = 0; j < kCk; ++j) {
          if (j < Ls) {
            const int t = ts + j;
            const float dl = sDl[lane * kP + t], uu = sU[lane * kP + t], dt = sDt[lane * kP + t];
            const float du_ = dl * uu;
#pragma unroll
            for (int k = 0; k < kS; ++k) {
              float beta;
              const float ab = disc_real<kMethod>(dt, dl, a2[k], Araw[k], beta);
              float bin = 1.f;
              if constexpr (kVarB) bin = sB[(n0 + k) * kTB + t];
              float inc;
              if constexpr (kMethod == LRNNX_MAMBA) inc = du_ * bin;
              else if constexpr (uses_B_input<kMethod>()) inc = beta * uu * bin;
              else inc = beta * uu;
              hc[k] = fmaf(ab, hc[k], inc);
              Ab[j][k] = ab;
              H[j][k] = hc[k];
            }
          }
        }
      }
      // reverse walk.  dB/dC: for kS >= 4 the two cross-half reduce-scatter
      // steps (index bits 5, 4 = the top bits of k) are applied right after
      // each step, leaving 16 values per quantity (index bits 3..0).
      constexpr int kAcc = kS >= 4 ? 16 : kNV;
      float accB[kAcc], accC[kAcc];
#pragma unroll
      for (int j = kCk - 1; j >= 0; --j) {
        if (j < Ls) {
          const int t = ts + j;
          const float dl = sDl[lane * kP + t], uu = sU[lane * kP + t], dt = sDt[lane * kP + t];
          const float dy = sDy[lane * kP + t];
          const float du_ = dl * uu;
          float p1 = 0.f, p2 = 0.f, p3 = 0.f;
          float vB[kS], vC[kS];
#pragma unroll
          for (int k = 0; k < kS; ++k) {
            // effective output weight: (C_t or C_const) * (B_const when B is constant)
            float cvar = 0.f, cc = cout_c[k];
            float bin = 1.f;
            if constexpr (kVarC) {
              cvar = sC[(n0 + k) * kTB + t];
              cc = kVarB ? cvar : cvar * cout_c[k];
            }
            if constexpr (kVarB) bin = sB[(n0 + k) * kTB + t];
            dh[k] = fmaf(Anext[k], dh[k], dy * cc);
            const float ab = Ab[j][k];
            const float hp = j > 0 ? H[j - 1][k] : h0[k];
            const float hcur = H[j][k];
            Anext[k] = ab;
            // contribution through A_bar: dh * hp * dA_bar/d(.)
            if constexpr (kMethod == LRNNX_MAMBA || kMethod == LRNNX_DIRAC || kMethod == LRNNX_ZOH) {
              const float wv = dh[k] * (ab * hp);
              p2 = fmaf(wv, Araw[k], p2);
              dA_acc[k] = fmaf(wv, dt, dA_acc[k]);
            } else if constexpr (kMethod == LRNNX_BILINEAR) {
              const float vA = 0.5f * dt * Araw[k];
              const float q = dh[k] * hp / ((1.f - vA) * (1.f - vA));
              p2 = fmaf(q, Araw[k], p2);
              dA_acc[k] = fmaf(q, dt, dA_acc[k]);
            } else if constexpr (kMethod == LRNNX_S7) {
              const float den = dl * dl + 0.5f;
              p2 = fmaf(dh[k] * hp, 2.f * dl / (den * den), p2);
            } else {  // RGLRU: dA_bar/ddelta = A_bar ln A, dA_bar/dA = delta A_bar / A
              const float wv = dh[k] * (ab * hp);
              const float lnA = a2[k] * kLn2;
              p2 = fmaf(wv, lnA, p2);
              dA_acc[k] = fmaf(wv, dl / Araw[k], dA_acc[k]);
            }
            // contribution through the input term
            if constexpr (kMethod == LRNNX_MAMBA) {
              p1 = fmaf(dh[k], bin, p1);                 // du = delta' * p1, ddelta' += u * p1
              if constexpr (kVarB) vB[k] = dh[k] * du_;
            } else if constexpr (kMethod == LRNNX_DIRAC || kMethod == LRNNX_S7) {
              p1 = fmaf(dh[k], bin, p1);
              if constexpr (kVarB) vB[k] = dh[k] * uu;
            } else if constexpr (kMethod == LRNNX_ZOH) {
              const float e1 = expf(dl * Araw[k]);
              const float beta = expm1f(dl * Araw[k]) / Araw[k];
              const float g = dh[k] * bin;
              p1 = fmaf(g, beta, p1);
              p3 = fmaf(g * uu, e1, p3);
              dA_acc[k] = fmaf(g * uu, (dl * e1 - beta) / Araw[k], dA_acc[k]);
              if constexpr (kVarB) vB[k] = dh[k] * beta * uu;
            } else if constexpr (kMethod == LRNNX_BILINEAR) {
              const float vB_ = 0.5f * dl * Araw[k];
              const float inv = 1.f / (1.f - vB_);
              const float beta = dl * inv;
              const float g = dh[k] * bin;
              p1 = fmaf(g, beta, p1);
              p3 = fmaf(g * uu, inv * inv, p3);
              dA_acc[k] = fmaf(g * uu, 0.5f * dl * dl * inv * inv, dA_acc[k]);
              if constexpr (kVarB) vB[k] = dh[k] * beta * uu;
            } else {  // RGLRU: beta = sqrt(1 - ab^2), B unused on the input side
              const float beta = sqrtf(-expm1f(dl * a2[k] * kLn2) * (1.f + ab));
              const float g = dh[k];
              p1 = fmaf(g, beta, p1);
              const float dbeta_dab = -ab / beta;
              const float lnA = a2[k] * kLn2;
              p3 = fmaf(g * uu * dbeta_dab, ab * lnA, p3);
              dA_acc[k] = fmaf(g * uu * dbeta_dab, ab * dl / Araw[k], dA_acc[k]);
              if constexpr (kVarB) vB[k] = 0.f;
            }
            // output side: y = sum_n cout h  (cout = C * B_const)
            const float dyh = dy * hcur;
            if constexpr (kVarC) vC[k] = kVarB ? dyh : dyh * bcst[k];
            if constexpr (!kVarB) dBc_acc[k] = fmaf(dyh, kVarC ? cvar : ccst[k], dBc_acc[k]);
            if constexpr (!kVarC) dCc_acc[k] = fmaf(dyh, kVarB ? 1.f : bcst[k], dCc_acc[k]);
          }
          sP1[(w * kWave + lane) * kP + t] = p1;
          sP2[(w * kWave + lane) * kP + t] = p2;
          if constexpr (kP3) sP3[(w * kWave + lane) * kP + t] = p3;
          if constexpr (kVarB || kVarC) {
            if (!lane_ok) {
#pragma unroll
              for (int k = 0; k < kS; ++k) { vB[k] = 0.f; vC[k] = 0.f; }
            }
            if constexpr (kS >= 4) {
              if constexpr (kVarB) { rs_step32<kS / 2>(vB); rs_step16<kS / 4>(vB); }
              if constexpr (kVarC) { rs_step32<kS / 2>(vC); rs_step16<kS / 4>(vC); }
#pragma unroll
              for (int k = 0; k < kS / 4; ++k) {
                if constexpr (kVarB) accB[k * kCk + j] = vB[k];
                if constexpr (kVarC) accC[k * kCk + j] = vC[k];
              }
            } else {
              if constexpr (kVarB) accB[j] = vB[0];
              if constexpr (kVarC) accC[j] = vC[0];
            }
          }
        } else {
          if constexpr (kS >= 4) {
#pragma unroll
            for (int k = 0; k < kS / 4; ++k) { accB[k * kCk + j] = 0.f; accC[k * kCk + j] = 0.f; }
          } else {
            accB[j] = 0.f; accC[j] = 0.f;
          }
        }
      }
      // dB / dC over the wave's channels -> one partial per (cb, b, n, t)
      if constexpr (kVarB || kVarC) {
        const int kq = lane / kCk, jq = lane % kCk;  // lane now owns index v = k * kCk + j
        const bool wr = lane < kNV && n0 + kq < N && jq < Ls;
        const int64_t tg = t0 + ts + jq;
        if constexpr (kVarB) {
          float r;
          if constexpr (kS >= 4) { rs_tail16(accB, lane); r = accB[0]; }
          else { float r64[64];
#pragma unroll
                 for (int i = 0; i < 64; ++i) r64[i] = i < kNV ? accB[i] : 0.f;
                 r = reduce_scatter64(r64, lane); }
          if (wr) ws[wo.dBv + ((cb * a.batch + b) * N + n0 + kq) * L + tg] = r;
        }
        if constexpr (kVarC) {
          float r;
          if constexpr (kS >= 4) { rs_tail16(accC, lane); r = accC[0]; }
          else { float r64[64];
#pragma unroll
                 for (int i = 0; i < 64; ++i) r64[i] = i < kNV ? accC[i] : 0.f;
                 r = reduce_scatter64(r64, lane); }
          if (wr) ws[wo.dCv + ((cb * a.batch + b) * N + n0 + kq) * L + tg] = r;
        }
      }
    }
    __syncthreads();

    // ---- epilogue over the tile: cross-wave sums, du / ddelta / ddeltaA
    for (int e = tid; e < rows * vpr; e += blockDim.x) {
      const int r = e / vpr, c = (e % vpr) * V;
      const int64_t dr = d0 + r;
      const int nv = Tv - c;
      if (dr >= D || nv <= 0) continue;
      const int n_ = nv < V ? nv : V;
      const float Dv = has_D ? static_cast<const float*>(a.D.ptr)[dr * a.D.s0] : 0.f;
      float vdu[V], vdd[V], vda[V], q1[V], q2[V];
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const int t = c + i;
        float P1 = 0.f, P2 = 0.f, P3 = 0.f;
        for (int ww = 0; ww < nW; ++ww) {
          P1 += sP1[(ww * kWave + r) * kP + t];
          P2 += sP2[(ww * kWave + r) * kP + t];
          if constexpr (kP3) P3 += sP3[(ww * kWave + r) * kP + t];
        }
        const float dl = sDl[r * kP + t], uu = sU[r * kP + t], dy = sDy[r * kP + t];
        float ddl;
        if constexpr (kMethod == LRNNX_MAMBA) {
          vdu[i] = dl * P1 + Dv * dy;
          ddl = uu * P1;
        } else {
          vdu[i] = P1 + Dv * dy;
          ddl = P3;
        }
        if (has_dA) { vda[i] = P2; } else { ddl += P2; vda[i] = 0.f; }
        // d softplus(x)/dx = sigmoid(x) = 1 - exp(-softplus(x))
        const float dd = a.delta_softplus ? ddl * (-expm1f(-dl)) : ddl;
        vdd[i] = dd;
        q1[i] = dy * uu;
        q2[i] = dd;
      }
      store_vec(Pdu + b * a.du.s0 + dr * a.du.s1 + t0 + c, n_, vdu);
      store_vec(Pddl + b * a.ddelta.s0 + dr * a.ddelta.s1 + t0 + c, n_, vdd);
      if (has_dA_in) store_vec(PddA + b * a.ddeltaA.s0 + dr * a.ddeltaA.s1 + t0 + c, n_, vda);
      // per-element contributions to dD and ddelta_bias, summed below in t order
#pragma unroll
      for (int i = 0; i < V; ++i) {
        sP1[r * kP + c + i] = i < n_ ? q1[i] : 0.f;
        sP2[r * kP + c + i] = i < n_ ? q2[i] : 0.f;
      }
    }
    __syncthreads();
    if (w == 0 && lane_ok) {
      for (int t = 0; t < Tv; ++t) {
        dD_acc += sP1[lane * kP + t];
        dbias_acc += sP2[lane * kP + t];
      }
    }
  }

  // per-(b, d, n) and per-(b, d) partials; summed over b by ss_reduce_kernel
#pragma unroll
  for (int k = 0; k < kS; ++k) {
    if (lane_ok && n0 + k < N) {
      const int64_t o = (b * D + d) * N + n0 + k;
      ws[wo.dA + o] = dA_acc[k];
      if constexpr (!kVarB) ws[wo.dBc + o] = dBc_acc[k];
      if constexpr (!kVarC) ws[wo.dCc + o] = dCc_acc[k];
    }
  }
  if (w == 0 && lane_ok) {
    ws[wo.dD + b * D + d] = dD_acc;
    ws[wo.dbias + b * D + d] = dbias_acc;
  }
}

inline size_t ss_bwd_smem_bytes(int kS, int kMethod, int64_t N, int nW) {
  const int kTB = tb_for(kS), kP = kTB + 4;
  const int np = needs_p3_rt(kMethod) ? 3 : 2;
  return sizeof(float) * ((size_t)4 * kWave * kP + (size_t)2 * nW * kS * kTB + (size_t)np * nW * kWave * kP);
}

// Sum of the dB / dC partials over the channel blocks of each group, in
// block order; written in the input dtype with the caller's strides.
template <typename OT>
__global__ void __launch_bounds__(256)
ss_reduce_bc_kernel(const float* __restrict__ part, lrnnx_view out, int64_t B, int64_t G, int64_t N, int64_t L,
                    int64_t ncpg) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = blockIdx.y;  // (b, g, n)
  if (t >= L) return;
  const int64_t n = row % N, g = (row / N) % G, b = row / (N * G);
  float acc = 0.f;
  for (int64_t j = 0; j < ncpg; ++j) acc += part[(((g * ncpg + j) * B + b) * N + n) * L + t];
  static_cast<OT*>(out.ptr)[b * out.s0 + g * out.s1 + n * out.s2 + t] = from_f32<OT>(acc);
}

// out[d, n] = sum_b part[b, d, n]  (fp32; n == 1 for per-channel vectors)
template <typename OT>
__global__ void __launch_bounds__(256)
ss_reduce_batch_kernel(const float* __restrict__ part, lrnnx_view out, int64_t B, int64_t D, int64_t N) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= D * N) return;
  float acc = 0.f;
  for (int64_t b = 0; b < B; ++b) acc += part[b * D * N + i];
  const int64_t d = i / N, n = i % N;
  static_cast<OT*>(out.ptr)[d * out.s0 + n * out.s1] = acc;
}

template <typename IT, int kS, int kMethod, bool kVarB, bool kVarC>
static hipError_t launch_bwd_t(const lrnnx_selective_scan_args& a, const SSGeom& g, float* ws, const SSBwdWs& wo,
                               const float* ckp, hipStream_t st) {
  dim3 grid(g.n_cb, (unsigned)a.batch);
  dim3 block(g.nW * kWave);
  const size_t sm = ss_bwd_smem_bytes(kS, kMethod, a.dstate, g.nW);
  if (sm > kMaxLds) return hipErrorInvalidConfiguration;
  auto kfn = ss_bwd_kernel<IT, kS, kMethod, kVarB, kVarC>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kfn),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)sm);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kfn, grid, block, sm, st, a, g.CB, g.n_ck, ws, wo, ckp);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t B = a.batch, D = a.dim, N = a.dstate, L = a.seqlen, G = a.n_groups;
  if constexpr (kVarB || kVarC) {
    const int64_t ncpg = g.n_cb / G;
    dim3 rg((unsigned)((L + 255) / 256), (unsigned)(B * G * N));
    if constexpr (kVarB) hipLaunchKernelGGL(ss_reduce_bc_kernel<IT>, rg, dim3(256), 0, st, ws + wo.dBv, a.dB, B, G, N, L, ncpg);
    if constexpr (kVarC) hipLaunchKernelGGL(ss_reduce_bc_kernel<IT>, rg, dim3(256), 0, st, ws + wo.dCv, a.dC, B, G, N, L, ncpg);
  }
  const unsigned gdn = (unsigned)((D * N + 255) / 256), gd = (unsigned)((D + 255) / 256);
  hipLaunchKernelGGL(ss_reduce_batch_kernel<float>, dim3(gdn), dim3(256), 0, st, ws + wo.dA, a.dA, B, D, N);
  if constexpr (!kVarB) hipLaunchKernelGGL(ss_reduce_batch_kernel<float>, dim3(gdn), dim3(256), 0, st, ws + wo.dBc, a.dB, B, D, N);
  if constexpr (!kVarC) hipLaunchKernelGGL(ss_reduce_batch_kernel<float>, dim3(gdn), dim3(256), 0, st, ws + wo.dCc, a.dC, B, D, N);
  if (a.dD.ptr) {
    lrnnx_view v = a.dD; v.s1 = 0;
    hipLaunchKernelGGL(ss_reduce_batch_kernel<float>, dim3(gd), dim3(256), 0, st, ws + wo.dD, v, B, D, (int64_t)1);
  }
  if (a.ddelta_bias.ptr) {
    lrnnx_view v = a.ddelta_bias; v.s1 = 0;
    hipLaunchKernelGGL(ss_reduce_batch_kernel<float>, dim3(gd), dim3(256), 0, st, ws + wo.dbias, v, B, D, (int64_t)1);
  }
  return hipGetLastError();
}

template <typename IT, int kS, int kMethod>
static hipError_t launch_bwd_bc(const lrnnx_selective_scan_args& a, const SSGeom& g, float* ws, const SSBwdWs& wo,
                                const float* ckp, hipStream_t st) {
  if (a.var_B && a.var_C) return launch_bwd_t<IT, kS, kMethod, true, true>(a, g, ws, wo, ckp, st);
  if (a.var_B) return launch_bwd_t<IT, kS, kMethod, true, false>(a, g, ws, wo, ckp, st);
  if (a.var_C) return launch_bwd_t<IT, kS, kMethod, false, true>(a, g, ws, wo, ckp, st);
  return launch_bwd_t<IT, kS, kMethod, false, false>(a, g, ws, wo, ckp, st);
}

template <typename IT, int kMethod>
static hipError_t launch_bwd_s(const lrnnx_selective_scan_args& a, const SSGeom& g, float* ws, const SSBwdWs& wo,
                               const float* ckp, hipStream_t st) {
  switch (g.kS) {
    case 1: return launch_bwd_bc<IT, 1, kMethod>(a, g, ws, wo, ckp, st);
    case 4: return launch_bwd_bc<IT, 4, kMethod>(a, g, ws, wo, ckp, st);
    case 8: return launch_bwd_bc<IT, 8, kMethod>(a, g, ws, wo, ckp, st);
    case 32: return launch_bwd_bc<IT, 32, kMethod>(a, g, ws, wo, ckp, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace lrnnx
