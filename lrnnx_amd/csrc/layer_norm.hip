// Fused residual-add + LayerNorm / RMSNorm, forward and backward (gfx950).
//
// Semantics: reference lrnnx/ops/triton/layer_norm.py (_layer_norm_fwd_1pass_kernel
// :202-322, _layer_norm_bwd_kernel :490-649; pure-PyTorch statements
// layer_norm_ref :23-82, rms_norm_ref :84-142) for the options lrnnx uses
// (lrnnx/layers/block.py:77-87, lrnnx/architectures/language_model.py:378-445):
//   s = x + residual (fp32),  residual_out = s (stored in the residual dtype),
//   LayerNorm: mu = mean(s), rstd = 1 / sqrt(mean((s - mu)^2) + eps), xhat = (s - mu) rstd
//   RMSNorm:   rstd = 1 / sqrt(mean(s^2) + eps),                        xhat = s rstd
//   y = xhat w (+ b)
// Backward (wdy = w dy):  dx = rstd (wdy - xhat mean(xhat wdy) - mean(wdy)) (the last
// term for LayerNorm only) + dresidual;  dw = sum_rows dy xhat,  db = sum_rows dy.
//
// Two kernel families:
// * fast (cols % 4 == 0, cols <= 4096, 4-element aligned rows): a row is held in
//   registers by 1, 2 or 4 waves (at most 16 elements per lane, as 4-element
//   8- or 16-byte accesses); row sums are wave reductions plus, for split rows,
//   an LDS exchange; x / residual types are template parameters.  The backward
//   keeps dw / db per lane in registers over the rows it visits, sums the
//   workgroup's row groups through LDS and writes one partial per workgroup.
// * generic (any cols up to the 64 KiB row limit, any alignment): one wave per
//   row, element-strided, re-reading the row per pass (from L2); dw / db come
//   from a column kernel (thread per column, rows split over blockIdx.y).
// Both finish dw / db with the same two-stage reduce over the partials, in a
// fixed order (deterministic).  The row loops' grids are sized to the number of
// workgroups resident on the device (occupancy query), so the chip is filled
// once with no partial second round.
#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "common.h"

namespace lrnnx {

namespace {
constexpr int kLnThreads = 256;
constexpr int kLnWaves = kLnThreads / kWave;
constexpr int kLnBwdMaxWG = 1024;     // fast backward: at most this many dw / db partials
constexpr int kLnColRowSplit = 64;   // generic dw / db: row blocks per column
constexpr int kLnRedSplit = 16;      // first stage of the dw / db reduce: partial-row blocks

template <typename T>
__device__ __forceinline__ float ld_f(const void* p, int64_t i) {
  return to_f32(static_cast<const T*>(p)[i]);
}
template <typename T>
__device__ __forceinline__ void st_f(void* p, int64_t i, float v) {
  static_cast<T*>(p)[i] = from_f32<T>(v);
}
__device__ __forceinline__ float ld_any(int dt, const void* p, int64_t i) {
  switch (dt) {
    case LRNNX_F32: return ld_f<float>(p, i);
    case LRNNX_BF16: return ld_f<bf16>(p, i);
    default: return ld_f<f16>(p, i);
  }
}
__device__ __forceinline__ void st_any(int dt, void* p, int64_t i, float v) {
  switch (dt) {
    case LRNNX_F32: st_f<float>(p, i, v); break;
    case LRNNX_BF16: st_f<bf16>(p, i, v); break;
    default: st_f<f16>(p, i, v); break;
  }
}

// 4 consecutive elements as one 16-byte (fp32) or 8-byte (16-bit) access
template <typename T> struct Raw4 { using type = uint2; };
template <> struct Raw4<float> { using type = uint4; };

template <typename T>
__device__ __forceinline__ void ld4(const T* p, int i, float* o) {
  const auto raw = *reinterpret_cast<const typename Raw4<T>::type*>(p + i);
  const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
  for (int v = 0; v < 4; ++v) o[v] = to_f32(e[v]);
}
template <typename T>
__device__ __forceinline__ void st4(T* p, int i, const float* o) {
  typename Raw4<T>::type raw;
  T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
  for (int v = 0; v < 4; ++v) e[v] = from_f32<T>(o[v]);
  *reinterpret_cast<typename Raw4<T>::type*>(p + i) = raw;
}
}  // namespace

// ------------------------------------------------------------------ fast path
// A row is split over kWPR waves (a "row group"); wave q of the group owns the
// 4-element chunks i kWPR + q (i < kNPL) of 256 columns each, lane l the
// elements 4 l .. 4 l + 3 of a chunk.  cols <= 256 kNPL kWPR.  The workgroup's
// 4 / kWPR row groups take consecutive rows; every wave of the workgroup runs
// the same number of iterations (rows past the end are skipped inside), so the
// barriers of the cross-wave row sums are uniform.

// Row sums over the kWPR waves of a row group: wave-level sum, then (kWPR > 1)
// through LDS slot `slot` (the caller alternates slots so that a slot is
// rewritten only after a barrier that follows its last read).
template <int kWPR>
__device__ __forceinline__ float2 group_sum2(float2 v, float2 (*red)[kLnWaves], int slot, int wid) {
  v.x = wave_allreduce_sum(v.x);
  v.y = wave_allreduce_sum(v.y);
  if constexpr (kWPR > 1) {
    if ((threadIdx.x & 63) == 0) red[slot][wid] = v;
    __syncthreads();
    const int g0 = wid - wid % kWPR;
    float2 t = red[slot][g0];
#pragma unroll
    for (int q = 1; q < kWPR; ++q) {
      t.x += red[slot][g0 + q].x;
      t.y += red[slot][g0 + q].y;
    }
    v = t;
  }
  return v;
}

template <typename XT, typename RT, int kNPL, int kWPR, bool kRms>
__global__ void __launch_bounds__(kLnThreads) ln_fwd_fast(const lrnnx_layer_norm_args a) {
  constexpr int kGroups = kLnWaves / kWPR;
  __shared__ float2 red[4][kLnWaves];
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int q = wid % kWPR;
  const int N = (int)a.cols;
  const float invN = 1.f / (float)N;
  float w[kNPL][4], bb[kNPL][4];
#pragma unroll
  for (int i = 0; i < kNPL; ++i) {
    const int e0 = ((i * kWPR + q) * 64 + lane) * 4;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      w[i][v] = e0 < N ? ld_any(a.wtype, a.weight.ptr, e0 + v) : 0.f;
      bb[i][v] = (e0 < N && a.bias.ptr) ? ld_any(a.wtype, a.bias.ptr, e0 + v) : 0.f;
    }
  }
  int it = 0;
  for (int64_t base = (int64_t)blockIdx.x * kGroups; base < a.rows; base += (int64_t)gridDim.x * kGroups, ++it) {
    const int64_t r = base + wid / kWPR;
    const bool live = r < a.rows;
    const XT* xr = static_cast<const XT*>(a.x.ptr) + r * a.x.s0;
    const RT* rr = static_cast<const RT*>(a.residual.ptr) + r * a.residual.s0;
    float s[kNPL][4];
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < kNPL; ++i) {
      const int e0 = ((i * kWPR + q) * 64 + lane) * 4;
#pragma unroll
      for (int v = 0; v < 4; ++v) s[i][v] = 0.f;
      if (live && e0 < N) {
        ld4<XT>(xr, e0, s[i]);
        if (a.residual.ptr) {
          float rv[4];
          ld4<RT>(rr, e0, rv);
#pragma unroll
          for (int v = 0; v < 4; ++v) s[i][v] += rv[v];
        }
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) sum += s[i][v];
    }
    float mu = 0.f;
    if constexpr (!kRms) mu = group_sum2<kWPR>(make_float2(sum, 0.f), red, 2 * (it & 1), wid).x * invN;
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < kNPL; ++i) {
      const bool ok = ((i * kWPR + q) * 64 + lane) * 4 < N;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float c = ok ? s[i][v] - mu : 0.f;
        sq = fmaf(c, c, sq);
      }
    }
    const float var = group_sum2<kWPR>(make_float2(sq, 0.f), red, 2 * (it & 1) + 1, wid).x * invN;
    const float rstd = 1.f / sqrtf(var + a.eps);
    if (!live) continue;
    XT* yr = static_cast<XT*>(a.y.ptr) + r * a.y.s0;
    RT* ror = static_cast<RT*>(a.residual_out.ptr) + r * a.residual_out.s0;
#pragma unroll
    for (int i = 0; i < kNPL; ++i) {
      const int e0 = ((i * kWPR + q) * 64 + lane) * 4;
      if (e0 < N) {
        float y[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) y[v] = fmaf((s[i][v] - mu) * rstd, w[i][v], bb[i][v]);
        st4<XT>(yr, e0, y);
        if (a.residual_out.ptr) st4<RT>(ror, e0, s[i]);
      }
    }
    if (q == 0 && lane == 0) {
      if constexpr (!kRms) a.mean[r] = mu;
      a.rstd[r] = rstd;
    }
  }
}

// x_saved (the pre-norm sum, stored in RT) and dresidual / dresidual_in are RT;
// dy and dx are XT.  part: (gridDim.x, 2, cols) fp32 partials of dw, db.
template <typename XT, typename RT, int kNPL, int kWPR, bool kRms>
__global__ void __launch_bounds__(kLnThreads) ln_bwd_fast(const lrnnx_layer_norm_args a, float* __restrict__ part) {
  constexpr int kGroups = kLnWaves / kWPR;
  __shared__ float2 red[4][kLnWaves];
  __shared__ float col[kLnWaves][256];
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int q = wid % kWPR;
  const int N = (int)a.cols;
  const float invN = 1.f / (float)N;
  float w[kNPL][4], dw[kNPL][4], db[kNPL][4];
#pragma unroll
  for (int i = 0; i < kNPL; ++i) {
    const int e0 = ((i * kWPR + q) * 64 + lane) * 4;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      w[i][v] = e0 < N ? ld_any(a.wtype, a.weight.ptr, e0 + v) : 0.f;
      dw[i][v] = 0.f;
      db[i][v] = 0.f;
    }
  }
  int it = 0;
  for (int64_t base = (int64_t)blockIdx.x * kGroups; base < a.rows; base += (int64_t)gridDim.x * kGroups, ++it) {
    const int64_t r = base + wid / kWPR;
    const bool live = r < a.rows;
    const float rstd = live ? a.rstd[r] : 0.f;
    const float mu = (kRms || !live) ? 0.f : a.mean[r];
    const RT* xr = static_cast<const RT*>(a.x_saved.ptr) + r * a.x_saved.s0;
    const XT* dyr = static_cast<const XT*>(a.dy.ptr) + r * a.dy.s0;
    float xh[kNPL][4], wdy[kNPL][4];
    float c1 = 0.f, c2 = 0.f;
#pragma unroll
    for (int i = 0; i < kNPL; ++i) {
      const int e0 = ((i * kWPR + q) * 64 + lane) * 4;
      const bool ok = live && e0 < N;
      float xv[4] = {0.f, 0.f, 0.f, 0.f}, dy[4] = {0.f, 0.f, 0.f, 0.f};
      if (ok) {
        ld4<RT>(xr, e0, xv);
        ld4<XT>(dyr, e0, dy);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        xh[i][v] = ok ? (xv[v] - mu) * rstd : 0.f;
        wdy[i][v] = w[i][v] * dy[v];
        dw[i][v] = fmaf(dy[v], xh[i][v], dw[i][v]);
        db[i][v] += dy[v];
        c1 = fmaf(xh[i][v], wdy[i][v], c1);
        c2 += wdy[i][v];
      }
    }
    const float2 cs = group_sum2<kWPR>(make_float2(c1, c2), red, it & 1, wid);
    c1 = cs.x * invN;
    c2 = kRms ? 0.f : cs.y * invN;
    if (!live) continue;
    const RT* drr = static_cast<const RT*>(a.dresidual.ptr) + r * a.dresidual.s0;
    XT* dxr = static_cast<XT*>(a.dx.ptr) + r * a.dx.s0;
    RT* dri = static_cast<RT*>(a.dresidual_in.ptr) + r * a.dresidual_in.s0;
#pragma unroll
    for (int i = 0; i < kNPL; ++i) {
      const int e0 = ((i * kWPR + q) * 64 + lane) * 4;
      if (e0 < N) {
        float dx[4], dr[4] = {0.f, 0.f, 0.f, 0.f};
        if (a.dresidual.ptr) ld4<RT>(drr, e0, dr);
#pragma unroll
        for (int v = 0; v < 4; ++v) dx[v] = fmaf(wdy[i][v] - fmaf(xh[i][v], c1, c2), rstd, dr[v]);
        st4<XT>(dxr, e0, dx);
        if (a.dresidual_in.ptr) st4<RT>(dri, e0, dx);
      }
    }
  }
  // sum dw, db over the workgroup's row groups through LDS, one local chunk
  // (kWPR chunks of 256 columns) at a time
#pragma unroll
  for (int i = 0; i < kNPL; ++i) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      __syncthreads();
#pragma unroll
      for (int v = 0; v < 4; ++v) col[wid][lane * 4 + v] = h ? db[i][v] : dw[i][v];
      __syncthreads();
#pragma unroll
      for (int qq = 0; qq < kWPR; ++qq) {
        const int e = (i * kWPR + qq) * 256 + threadIdx.x;
        if (e < N) {
          float t = col[qq][threadIdx.x];
#pragma unroll
          for (int g = 1; g < kGroups; ++g) t += col[g * kWPR + qq][threadIdx.x];
          part[((int64_t)blockIdx.x * 2 + h) * N + e] = t;
        }
      }
    }
  }
}

// ------------------------------------------------------------------ generic path
template <bool kRms>
__global__ void __launch_bounds__(kLnThreads) ln_fwd_generic(const lrnnx_layer_norm_args a) {
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t)blockIdx.x * kLnWaves + (threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * kLnWaves;
  const int64_t N = a.cols;
  const float invN = 1.f / (float)N;
  for (int64_t r = wave0; r < a.rows; r += nw) {
    auto sval = [&](int64_t e) {
      float v = ld_any(a.xtype, a.x.ptr, r * a.x.s0 + e);
      if (a.residual.ptr) v += ld_any(a.rtype, a.residual.ptr, r * a.residual.s0 + e);
      return v;
    };
    float mu = 0.f;
    if constexpr (!kRms) {
      float sum = 0.f;
      for (int64_t e = lane; e < N; e += 64) sum += sval(e);
      mu = wave_allreduce_sum(sum) * invN;
    }
    float sq = 0.f;
    for (int64_t e = lane; e < N; e += 64) {
      const float c = sval(e) - mu;
      sq = fmaf(c, c, sq);
    }
    const float rstd = 1.f / sqrtf(wave_allreduce_sum(sq) * invN + a.eps);
    for (int64_t e = lane; e < N; e += 64) {
      const float s = sval(e);
      const float b = a.bias.ptr ? ld_any(a.wtype, a.bias.ptr, e) : 0.f;
      st_any(a.xtype, a.y.ptr, r * a.y.s0 + e, fmaf((s - mu) * rstd, ld_any(a.wtype, a.weight.ptr, e), b));
      if (a.residual_out.ptr) st_any(a.rtype, a.residual_out.ptr, r * a.residual_out.s0 + e, s);
    }
    if (lane == 0) {
      if constexpr (!kRms) a.mean[r] = mu;
      a.rstd[r] = rstd;
    }
  }
}

template <bool kRms>
__global__ void __launch_bounds__(kLnThreads) ln_bwd_generic(const lrnnx_layer_norm_args a) {
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t)blockIdx.x * kLnWaves + (threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * kLnWaves;
  const int64_t N = a.cols;
  const float invN = 1.f / (float)N;
  for (int64_t r = wave0; r < a.rows; r += nw) {
    const float rstd = a.rstd[r];
    const float mu = kRms ? 0.f : a.mean[r];
    float c1 = 0.f, c2 = 0.f;
    for (int64_t e = lane; e < N; e += 64) {
      const float xh = (ld_any(a.rtype, a.x_saved.ptr, r * a.x_saved.s0 + e) - mu) * rstd;
      const float wdy = ld_any(a.wtype, a.weight.ptr, e) * ld_any(a.xtype, a.dy.ptr, r * a.dy.s0 + e);
      c1 = fmaf(xh, wdy, c1);
      c2 += wdy;
    }
    c1 = wave_allreduce_sum(c1) * invN;
    if constexpr (!kRms) c2 = wave_allreduce_sum(c2) * invN;
    for (int64_t e = lane; e < N; e += 64) {
      const float xh = (ld_any(a.rtype, a.x_saved.ptr, r * a.x_saved.s0 + e) - mu) * rstd;
      const float wdy = ld_any(a.wtype, a.weight.ptr, e) * ld_any(a.xtype, a.dy.ptr, r * a.dy.s0 + e);
      const float dr = a.dresidual.ptr ? ld_any(a.rtype, a.dresidual.ptr, r * a.dresidual.s0 + e) : 0.f;
      const float dx = fmaf(wdy - fmaf(xh, c1, kRms ? 0.f : c2), rstd, dr);
      st_any(a.xtype, a.dx.ptr, r * a.dx.s0 + e, dx);
      if (a.dresidual_in.ptr) st_any(a.rtype, a.dresidual_in.ptr, r * a.dresidual_in.s0 + e, dx);
    }
  }
}

// dw, db partials of row block blockIdx.y (rows y, y + gridDim.y, ...), one
// thread per column: part[(y * 2 + {0, 1}) * cols + col]
template <bool kRms>
__global__ void __launch_bounds__(kLnThreads) ln_wb_cols(const lrnnx_layer_norm_args a, float* __restrict__ part) {
  const int64_t col = (int64_t)blockIdx.x * kLnThreads + threadIdx.x;
  const int64_t N = a.cols;
  if (col >= N) return;
  float dw = 0.f, db = 0.f;
  for (int64_t r = blockIdx.y; r < a.rows; r += gridDim.y) {
    const float mu = kRms ? 0.f : a.mean[r];
    const float xh = (ld_any(a.rtype, a.x_saved.ptr, r * a.x_saved.s0 + col) - mu) * a.rstd[r];
    const float dy = ld_any(a.xtype, a.dy.ptr, r * a.dy.s0 + col);
    dw = fmaf(dy, xh, dw);
    db += dy;
  }
  part[((int64_t)blockIdx.y * 2) * N + col] = dw;
  part[((int64_t)blockIdx.y * 2 + 1) * N + col] = db;
}

// First stage of the dw / db reduce: workgroup (x, y) sums, for the 64
// columns 64 x .. 64 x + 63, the partial rows g = 4 y + k, 4 y + k + 4 S, ...
// (wave k, S = gridDim.y), adds its 4 waves in order and writes
// out[(y * 2 + {0, 1}) * cols + col].
__global__ void __launch_bounds__(kLnThreads) ln_wb_stage1(const lrnnx_layer_norm_args a, const float* __restrict__ part,
                                                           int64_t G, float* __restrict__ out) {
  __shared__ float red[2][kLnWaves][64];
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int64_t N = a.cols;
  const int64_t col = (int64_t)blockIdx.x * 64 + lane;
  float sw = 0.f, sb = 0.f;
  if (col < N) {
    for (int64_t g = (int64_t)blockIdx.y * kLnWaves + wid; g < G; g += (int64_t)gridDim.y * kLnWaves) {
      sw += part[(g * 2) * N + col];
      sb += part[(g * 2 + 1) * N + col];
    }
  }
  red[0][wid][lane] = sw;
  red[1][wid][lane] = sb;
  __syncthreads();
  if (wid < 2 && col < N)
    out[((int64_t)blockIdx.y * 2 + wid) * N + col] =
        (red[wid][0][lane] + red[wid][1][lane]) + (red[wid][2][lane] + red[wid][3][lane]);
}

// dweight[col], dbias[col] = sum of the S first-stage rows, in order.
__global__ void __launch_bounds__(kLnThreads) ln_wb_stage2(const lrnnx_layer_norm_args a, const float* __restrict__ part,
                                                           int64_t S) {
  const int64_t col = (int64_t)blockIdx.x * kLnThreads + threadIdx.x;
  const int64_t N = a.cols;
  if (col >= N) return;
  float sw = 0.f, sb = 0.f;
  for (int64_t g = 0; g < S; ++g) {
    sw += part[(g * 2) * N + col];
    sb += part[(g * 2 + 1) * N + col];
  }
  st_any(a.wtype, a.dweight.ptr, col, sw);
  if (a.dbias.ptr) st_any(a.wtype, a.dbias.ptr, col, sb);
}

// ------------------------------------------------------------------ host side
namespace {
int64_t esize(int32_t t) { return t == LRNNX_F32 ? 4 : 2; }

bool al4(const lrnnx_view& v, int32_t t) {
  return v.ptr == nullptr || ((reinterpret_cast<uintptr_t>(v.ptr) % (4 * esize(t))) == 0 && v.s0 % 4 == 0);
}

// waves per row of the fast kernels (matches launch_fast's cases)
int64_t fast_wpr(int64_t cols) {
  const int64_t nch = (cols + 255) / 256;
  return nch <= 4 ? 1 : (nch <= 8 ? 2 : 4);
}

bool fast_ok(const lrnnx_layer_norm_args& a, bool bwd) {
  if (a.cols % 4 != 0 || a.cols > 4096) return false;
  if (!(a.rtype == a.xtype || a.rtype == LRNNX_F32)) return false;
  if (!bwd) return al4(a.x, a.xtype) && al4(a.y, a.xtype) && al4(a.residual, a.rtype) && al4(a.residual_out, a.rtype);
  return al4(a.x_saved, a.rtype) && al4(a.dy, a.xtype) && al4(a.dx, a.xtype) && al4(a.dresidual, a.rtype) &&
         al4(a.dresidual_in, a.rtype);
}

// Workgroups of `kernel` (256 threads) resident on the current device at once:
// the grid of the row loops is sized to fill the chip exactly once, so that
// no partial second round of workgroups runs at the end.  Cached per device.
int64_t resident_wgs(const void* kernel) {
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, int64_t> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1024;
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find({dev, kernel});
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  int64_t n = 1024;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kLnThreads, 0) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && per_cu > 0 &&
      cus > 0)
    n = (int64_t)per_cu * cus;
  cache[{dev, kernel}] = n;
  return n;
}

// row-group units of work (one workgroup iteration each)
int64_t units(int64_t rows, int64_t per_wg) { return (rows + per_wg - 1) / per_wg; }

int64_t clamp_grid(int64_t u, int64_t cap) { return u < 1 ? 1 : (u < cap ? u : cap); }

// Partials of the fast backward: one per workgroup, at most kLnBwdMaxWG (an
// upper bound independent of the device; the launch may use fewer).
int64_t fast_bwd_partials_max(const lrnnx_layer_norm_args& a) {
  return clamp_grid(units(a.rows, kLnWaves / fast_wpr(a.cols)), kLnBwdMaxWG);
}

int64_t generic_partials(const lrnnx_layer_norm_args& a) {
  return a.rows < kLnColRowSplit ? (a.rows < 1 ? 1 : a.rows) : kLnColRowSplit;
}

int64_t partial_rows_max(const lrnnx_layer_norm_args& a) {
  return fast_ok(a, true) ? fast_bwd_partials_max(a) : generic_partials(a);
}

template <typename XT, typename RT, bool kRms>
int64_t launch_fast(const lrnnx_layer_norm_args& a, bool bwd, float* part, hipStream_t st) {
  const int64_t nch = (a.cols + 255) / 256;   // 256-column chunks per row
  const dim3 blk(kLnThreads);
#define LN_CASE(K, W)                                                                                 \
  if (nch <= K * W) {                                                                                 \
    const int64_t u = units(a.rows, kLnWaves / W);                                                    \
    if (bwd) {                                                                                        \
      auto k = ln_bwd_fast<XT, RT, K, W, kRms>;                                                       \
      const int64_t g = clamp_grid(u, std::min<int64_t>(kLnBwdMaxWG, resident_wgs((const void*)k))); \
      hipLaunchKernelGGL(k, dim3((unsigned)g), blk, 0, st, a, part);                                  \
      return g;                                                                                       \
    }                                                                                                 \
    auto k = ln_fwd_fast<XT, RT, K, W, kRms>;                                                         \
    const int64_t g = clamp_grid(u, resident_wgs((const void*)k));                                    \
    hipLaunchKernelGGL(k, dim3((unsigned)g), blk, 0, st, a);                                          \
    return g;                                                                                         \
  }
  LN_CASE(1, 1) LN_CASE(2, 1) LN_CASE(4, 1) LN_CASE(4, 2) LN_CASE(4, 4)
#undef LN_CASE
  return 0;
}

template <bool kRms>
int64_t launch_fast_t(const lrnnx_layer_norm_args& a, bool bwd, float* part, hipStream_t st) {
  const bool same = a.rtype == a.xtype;
  switch (a.xtype) {
    case LRNNX_F32: return launch_fast<float, float, kRms>(a, bwd, part, st);
    case LRNNX_BF16:
      return same ? launch_fast<bf16, bf16, kRms>(a, bwd, part, st) : launch_fast<bf16, float, kRms>(a, bwd, part, st);
    default:
      return same ? launch_fast<f16, f16, kRms>(a, bwd, part, st) : launch_fast<f16, float, kRms>(a, bwd, part, st);
  }
}

template <bool kRms>
hipError_t ln_launch_r(const lrnnx_layer_norm_args& a, bool bwd, float* part, hipStream_t st) {
  const dim3 blk(kLnThreads);
  int64_t G = 0;   // dw / db partial rows written by the backward
  if (fast_ok(a, bwd)) {
    G = launch_fast_t<kRms>(a, bwd, part, st);
  } else if (!bwd) {
    auto k = ln_fwd_generic<kRms>;
    hipLaunchKernelGGL(k, dim3((unsigned)clamp_grid(units(a.rows, kLnWaves), resident_wgs((const void*)k))), blk,
                       0, st, a);
  } else {
    auto k = ln_bwd_generic<kRms>;
    hipLaunchKernelGGL(k, dim3((unsigned)clamp_grid(units(a.rows, kLnWaves), resident_wgs((const void*)k))), blk,
                       0, st, a);
    G = generic_partials(a);
    hipLaunchKernelGGL(ln_wb_cols<kRms>, dim3((unsigned)((a.cols + kLnThreads - 1) / kLnThreads), (unsigned)G),
                       blk, 0, st, a, part);
  }
  if (bwd) {
    // two-stage fixed-order reduce; the first stage's rows follow the partials
    const int64_t S = std::min<int64_t>(kLnRedSplit, (G + kLnWaves - 1) / kLnWaves);
    float* part2 = part + partial_rows_max(a) * 2 * a.cols;
    hipLaunchKernelGGL(ln_wb_stage1, dim3((unsigned)((a.cols + 63) / 64), (unsigned)S), blk, 0, st, a,
                       static_cast<const float*>(part), G, part2);
    hipLaunchKernelGGL(ln_wb_stage2, dim3((unsigned)((a.cols + kLnThreads - 1) / kLnThreads)), blk, 0, st, a,
                       static_cast<const float*>(part2), S);
  }
  return hipGetLastError();
}
}  // namespace

int64_t ln_workspace_bytes(const lrnnx_layer_norm_args& a) {
  return (partial_rows_max(a) + kLnRedSplit) * 2 * a.cols * (int64_t)sizeof(float);
}

hipError_t ln_launch(const lrnnx_layer_norm_args& a, bool bwd, float* part, hipStream_t st) {
  return a.is_rms_norm ? ln_launch_r<true>(a, bwd, part, st) : ln_launch_r<false>(a, bwd, part, st);
}

}  // namespace lrnnx
