/* Float64 CPU restatement of the selective scan, "mamba" discretisation,
 * forward and backward.  TEST INFRASTRUCTURE ONLY: the GPU parity tests call
 * it (through oracle/fast.py) as the checker at shapes where the PyTorch
 * restatement (oracle/scan_ref.py) is too slow; nothing in the product links
 * or loads it.
 *
 * Forward, per (b, d), as selective_scan_ref (lrnnx/ops/selective_scan.py:
 * 200-360) with discretization "mamba":
 *   delta' = softplus(delta + delta_bias)   (threshold 20, F.softplus;
 *            csrc/selective_scan/selective_scan.cuh:172-174) or delta + bias
 *   A_bar  = exp(delta' A), B_bar u = delta' B u      (selective_scan.py:247-263)
 *   h_t    = A_bar_t h_{t-1} + B_bar_t u_t, h_{-1} = 0   (:330-332)
 *   y_t    = sum_n C_t h_t + D u_t; out = y silu(z)       (:333-357)
 *   last_state = h_{L-1} (:343-344); for a constant B this is the state
 *   the reference wrapper returns after multiplying the kernel's B-free
 *   state by B (:87-92).
 * Backward: the exact gradient of that function, written as the reference
 * kernel's adjoint recurrence (csrc/selective_scan/selective_scan_backward.cuh:
 * 429-442 for this method, :216-219 for the z gate, :788-801 for softplus):
 *   dy_t   = dout_t silu(z_t);  dz_t = dout_t (y_t + D u_t) s (1 + z (1 - s)),
 *            s = sigmoid(z_t)
 *   dh_t   = A_bar_{t+1} dh_{t+1} + C_t dy_t
 *   du_t   = D dy_t + delta'_t sum_n dh_t B_t
 *   ddelta'_t = u_t sum_n dh_t B_t + sum_n dh_t A A_bar_t h_{t-1}
 *   ddelta_t  = ddelta'_t sigmoid(delta + bias)   (1 above the threshold)
 *   dA     = sum_{b,t} dh_t delta'_t A_bar_t h_{t-1}
 *   dB_t   = sum_d dh_t delta'_t u_t,  dC_t = sum_d dy_t h_t  (variable B / C;
 *            constant: summed over b, t per (d, n))
 *   dD     = sum_{b,t} dy_t u_t,  ddelta_bias = sum_{b,t} ddelta_t.
 *
 * Layouts (all contiguous): u, delta, z, dout (B, D, L) float32; A (D, N);
 * variable B / C (B, G, N, L), constant (D, N); D, delta_bias (D).  Outputs
 * float64: out (B, D, L) (the z-gated output when z is given), out_pre (the
 * output before the gate, optional), last (B, D, N); gradients with the shapes
 * of their inputs.  dout == NULL runs the forward only.
 *
 * Threads split the (b, d) rows; each thread sums its rows' contributions to
 * dA, dB, dC, dD, ddelta_bias in a private buffer, and the buffers are added
 * in thread order, so results depend only on the thread count.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static double softplus20(double x) { return x > 20.0 ? x : log1p(exp(x)); }
static double dsoftplus20(double x) { return x > 20.0 ? 1.0 : 1.0 / (1.0 + exp(-x)); }
static double sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); }

int lrnnx_oracle_ss_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Returns 0 on success, 1 on an allocation failure. */
int lrnnx_oracle_ss_mamba(int64_t Bt, int64_t D, int64_t L, int64_t N, int64_t G, const float* u,
                          const float* delta, const float* z, const float* dout, const float* A, const float* Bm,
                          const float* Cm, int varB, int varC, const float* Dv, const float* delta_bias,
                          int softplus, int nthreads, double* out, double* out_pre, double* last, double* du,
                          double* ddelta, double* dA, double* dB, double* dC, double* dD, double* ddelta_bias,
                          double* dz) {
  const int bwd = dout != NULL;
  const int64_t dpg = D / G;                      /* channels per group */
  const int64_t nB = varB ? Bt * G * N * L : D * N; /* elements of dB */
  const int64_t nC = varC ? Bt * G * N * L : D * N;
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = omp_get_max_threads();
#else
  nthreads = 1;
#endif
  /* per-thread partial sums: dA (D N), dB, dC, dD (D), ddelta_bias (D) */
  const int64_t part = bwd ? D * N + nB + nC + 2 * D : 0;
  double* parts = NULL;
  if (bwd) {
    parts = (double*)calloc((size_t)(part * nthreads), sizeof(double));
    if (!parts) return 1;
  }
  int fail = 0;
#ifdef _OPENMP
#pragma omp parallel num_threads(nthreads)
#endif
  {
#ifdef _OPENMP
    const int tid = omp_get_thread_num();
    const int nt = omp_get_num_threads();
#else
    const int tid = 0, nt = 1;
#endif
    double* H = (double*)malloc((size_t)(L * N) * sizeof(double));   /* h_t */
    double* AB = (double*)malloc((size_t)(L * N) * sizeof(double));  /* A_bar_t */
    double* dl = (double*)malloc((size_t)L * sizeof(double));        /* delta' */
    double* dy = (double*)malloc((size_t)L * sizeof(double));
    double* g = (double*)malloc((size_t)N * sizeof(double));
    if (!H || !AB || !dl || !dy || !g) {
#ifdef _OPENMP
#pragma omp atomic write
#endif
      fail = 1;
    } else {
      double* pA = bwd ? parts + (int64_t)tid * part : NULL;
      double* pB = bwd ? pA + D * N : NULL;
      double* pC = bwd ? pB + nB : NULL;
      double* pD = bwd ? pC + nC : NULL;
      double* pbias = bwd ? pD + D : NULL;
      /* rows (b, d) in contiguous blocks per thread */
      const int64_t rows = Bt * D;
      const int64_t r0 = rows * tid / nt, r1 = rows * (tid + 1) / nt;
      for (int64_t r = r0; r < r1; ++r) {
        const int64_t b = r / D, d = r % D, grp = d / dpg;
        const int64_t o = r * L;
        const float* ur = u + o;
        const float* dr = delta + o;
        const float* zr = z ? z + o : NULL;
        const double bias = delta_bias ? (double)delta_bias[d] : 0.0;
        const double Dd = Dv ? (double)Dv[d] : 0.0;
        const float* Arow = A + d * N;
        /* B_t[n] / C_t[n]: variable (b, grp, n, t) or constant (d, n) */
        const float* Bvar = varB ? Bm + ((b * G + grp) * N) * L : NULL;
        const float* Cvar = varC ? Cm + ((b * G + grp) * N) * L : NULL;
        for (int64_t t = 0; t < L; ++t) {
          const double x = (double)dr[t] + bias;
          dl[t] = softplus ? softplus20(x) : x;
        }
        /* forward */
        for (int64_t n = 0; n < N; ++n) g[n] = 0.0; /* g holds h here */
        for (int64_t t = 0; t < L; ++t) {
          const double x = dl[t] * (double)ur[t];
          double y = 0.0;
          for (int64_t n = 0; n < N; ++n) {
            const double a = exp(dl[t] * (double)Arow[n]);
            const double bn = varB ? (double)Bvar[n * L + t] : (double)Bm[d * N + n];
            const double cn = varC ? (double)Cvar[n * L + t] : (double)Cm[d * N + n];
            g[n] = a * g[n] + x * bn;
            AB[t * N + n] = a;
            H[t * N + n] = g[n];
            y += cn * g[n];
          }
          const double pre = y + Dd * (double)ur[t];
          if (out_pre) out_pre[o + t] = pre;
          out[o + t] = zr ? pre * (double)zr[t] * sigmoid((double)zr[t]) : pre;
          /* dy (backward) */
          if (bwd) {
            const double dout_t = (double)dout[o + t];
            if (zr) {
              const double zt = (double)zr[t], s = sigmoid(zt);
              dy[t] = dout_t * zt * s;
              dz[o + t] = dout_t * pre * s * (1.0 + zt * (1.0 - s));
            } else {
              dy[t] = dout_t;
            }
          }
        }
        for (int64_t n = 0; n < N; ++n) last[r * N + n] = g[n];
        if (!bwd) continue;
        /* backward */
        for (int64_t n = 0; n < N; ++n) g[n] = 0.0; /* g = A_bar_{t+1} dh_{t+1} */
        double sD = 0.0, sbias = 0.0;
        for (int64_t t = L - 1; t >= 0; --t) {
          const double ut = (double)ur[t], dlt = dl[t], dyt = dy[t];
          double sB = 0.0, sAh = 0.0;
          for (int64_t n = 0; n < N; ++n) {
            const double bn = varB ? (double)Bvar[n * L + t] : (double)Bm[d * N + n];
            const double cn = varC ? (double)Cvar[n * L + t] : (double)Cm[d * N + n];
            const double dh = g[n] + cn * dyt;
            const double a = AB[t * N + n];
            const double hprev = t > 0 ? H[(t - 1) * N + n] : 0.0;
            const double w = dh * a * hprev; /* dh A_bar h_{t-1} */
            sB += dh * bn;
            sAh += w * (double)Arow[n];
            pA[d * N + n] += w * dlt;
            if (varB) pB[((b * G + grp) * N + n) * L + t] += dh * dlt * ut;
            else pB[d * N + n] += dh * dlt * ut;
            if (varC) pC[((b * G + grp) * N + n) * L + t] += dyt * H[t * N + n];
            else pC[d * N + n] += dyt * H[t * N + n];
            g[n] = dh * a;
          }
          du[o + t] = Dd * dyt + dlt * sB;
          double dd = ut * sB + sAh;
          if (softplus) dd *= dsoftplus20((double)dr[t] + bias);
          ddelta[o + t] = dd;
          sD += dyt * ut;
          sbias += dd;
        }
        pD[d] += sD;
        pbias[d] += sbias;
      }
    }
    free(H);
    free(AB);
    free(dl);
    free(dy);
    free(g);
  }
  if (fail) {
    free(parts);
    return 1;
  }
  if (bwd) {
    /* thread partials, added in thread order */
    memset(dA, 0, (size_t)(D * N) * sizeof(double));
    memset(dB, 0, (size_t)nB * sizeof(double));
    memset(dC, 0, (size_t)nC * sizeof(double));
    if (dD) memset(dD, 0, (size_t)D * sizeof(double));
    if (ddelta_bias) memset(ddelta_bias, 0, (size_t)D * sizeof(double));
    for (int t = 0; t < nthreads; ++t) {
      const double* p = parts + (int64_t)t * part;
      for (int64_t i = 0; i < D * N; ++i) dA[i] += p[i];
      p += D * N;
      for (int64_t i = 0; i < nB; ++i) dB[i] += p[i];
      p += nB;
      for (int64_t i = 0; i < nC; ++i) dC[i] += p[i];
      p += nC;
      if (dD)
        for (int64_t i = 0; i < D; ++i) dD[i] += p[i];
      p += D;
      if (ddelta_bias)
        for (int64_t i = 0; i < D; ++i) ddelta_bias[i] += p[i];
    }
    free(parts);
  }
  return 0;
}
