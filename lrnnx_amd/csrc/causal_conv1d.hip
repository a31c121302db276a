// Depthwise causal conv1d (the short convolution in front of the Mamba scan),
// forward, backward and one-step decode update, gfx950.
//
// Semantics (the reference's own fallbacks for the causal-conv1d package,
// lrnnx/models/ltv/mamba.py:271 and :398-410):
//   out[b, d, t] = act(bias[d] + sum_{k < W} w[d, k] x[b, d, t - W + 1 + k]),  x[t < 0] = 0,
//   act = identity or silu.
// Backward: g = dout act'(pre); dx[t] = sum_k w[k] g[t + W - 1 - k];
// dw[k] = sum_{b, t} g[t] x[t - W + 1 + k]; dbias = sum_{b, t} g[t].
//
// One wave per (b, d) row; the row is walked in chunks of 512 steps, 8
// consecutive steps per lane (16-byte loads / stores for 16-bit types when
// the row is aligned), several chunks loaded together ahead of their compute.  The W - 1 steps of history a lane needs come from the
// previous lane through ds_bpermute, and lane 0 takes them from the previous
// chunk (forward) or from a few extra loads (backward, which walks right to
// left so that the W - 1 steps of g to the right come from the chunk just
// processed).  dw / dbias are per-row partials (workspace) summed over the
// batch in a fixed order by a second kernel.
#include "tile_io.h"

namespace lrnnx {

namespace {
constexpr int kCE = 8;                 // steps per lane
constexpr int kCCh = kCE * kWave;      // steps per chunk

__device__ __forceinline__ float shfl_f(float v, int src) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute((src & 63) << 2, __float_as_int(v)));
}
// sigmoid through v_exp_f32 and v_rcp_f32 (<= 1 ulp each) instead of an IEEE
// division; exp(-p) = inf for p << 0 gives sigmoid 0, silu -0 and silu' 0.
__device__ __forceinline__ float sigmoid_f(float p) { return __builtin_amdgcn_rcpf(1.f + __expf(-p)); }
__device__ __forceinline__ float silu_f(float p) { return p * sigmoid_f(p); }
// d silu(p) / dp = s (1 + p (1 - s)), s = sigmoid(p)
__device__ __forceinline__ float silu_grad(float p) {
  const float s = sigmoid_f(p);
  return s * (1.f + p * (1.f - s));
}

template <typename IT>
__device__ __forceinline__ void load_row8(const IT* p, int64_t t, int64_t L, bool vec, float* v) {
  if (vec && t + kCE <= L) {
    if constexpr (sizeof(IT) == 4) {
      const float4 a = *reinterpret_cast<const float4*>(p + t);
      const float4 b = *reinterpret_cast<const float4*>(p + t + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      raw_to_f32<IT>(*reinterpret_cast<const uint4*>(p + t), v);
    }
  } else {
#pragma unroll
    for (int j = 0; j < kCE; ++j) {
      v[j] = 0.f;
      if (t + j < L && t + j >= 0) v[j] = to_f32(p[t + j]);
    }
  }
}

template <typename IT>
__device__ __forceinline__ void store_row8(IT* p, int64_t t, int64_t L, bool vec, const float* v) {
  if (vec && t + kCE <= L) {
    if constexpr (sizeof(IT) == 4) {
      *reinterpret_cast<float4*>(p + t) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(p + t + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      uint4 raw;
      IT* e = reinterpret_cast<IT*>(&raw);
#pragma unroll
      for (int j = 0; j < kCE; ++j) e[j] = from_f32<IT>(v[j]);
      *reinterpret_cast<uint4*>(p + t) = raw;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kCE; ++j)
      if (t + j < L) p[t + j] = from_f32<IT>(v[j]);
  }
}
}  // namespace

// 8 consecutive elements as raw 16-byte words (one for 16-bit types, two for fp32)
template <typename IT>
struct Raw8 {
  uint4 v[sizeof(IT) == 4 ? 2 : 1];
};
template <typename IT>
__device__ __forceinline__ Raw8<IT> ld_raw8(const IT* p) {
  Raw8<IT> r;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(r.v) / sizeof(uint4)); ++i) r.v[i] = reinterpret_cast<const uint4*>(p)[i];
  return r;
}
template <typename IT>
__device__ __forceinline__ void cvt_raw8(const Raw8<IT>& r, float* v) {
  if constexpr (sizeof(IT) == 4) {
    const uint32_t* u = reinterpret_cast<const uint32_t*>(r.v);
#pragma unroll
    for (int j = 0; j < kCE; ++j) v[j] = __uint_as_float(u[j]);
  } else {
    raw_to_f32<IT>(r.v[0], v);
  }
}

// 8 elements starting at t with those outside [0, L) as zero, element by element
template <typename IT>
__device__ __forceinline__ Raw8<IT> ld_raw8_guarded(const IT* p, int64_t t, int64_t L) {
  Raw8<IT> r;
  IT* e = reinterpret_cast<IT*>(r.v);
#pragma unroll
  for (int j = 0; j < kCE; ++j) {
    e[j] = from_f32<IT>(0.f);
    if (t + j >= 0 && t + j < L) e[j] = p[t + j];
  }
  return r;
}

// A chunk that is not wholly inside the row: per lane, 16-byte words when the
// lane's 8 elements are, element by element otherwise (only the lane holding
// the row's end, and lanes before the row's start, take that path)
template <typename IT>
__device__ __forceinline__ Raw8<IT> ld_raw8_part(const IT* p, int64_t t, int64_t L, bool vec) {
  if (vec && t >= 0 && t + kCE <= L) return ld_raw8<IT>(p + t);
  return ld_raw8_guarded<IT>(p, t, L);
}

// Chunks of a row loaded together before any of them is used: bytes in flight
// per wave against registers (occupancy).  Measured at B 8, D 4096, L 4096,
// W 4, bf16: the forward is fastest at 8, the backward (two arrays, more
// registers per chunk) at 1.
constexpr int kCUf = 8;
constexpr int kCUb = 1;

template <typename IT, int W, bool kSilu>
__global__ void __launch_bounds__(256) cconv_fwd_kernel(const lrnnx_causal_conv1d_args a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.batch * a.dim) return;
  const int64_t b = row / a.dim, d = row % a.dim, L = a.seqlen;
  float w[W];
  const float* wp = static_cast<const float*>(a.weight.ptr);
#pragma unroll
  for (int k = 0; k < W; ++k) w[k] = wp[d * a.weight.s0 + k * a.weight.s1];
  const float bias = a.bias.ptr ? static_cast<const float*>(a.bias.ptr)[d * a.bias.s0] : 0.f;
  const IT* x = static_cast<const IT*>(a.x.ptr) + b * a.x.s0 + d * a.x.s1;
  IT* out = static_cast<IT*>(a.out.ptr) + b * a.out.s0 + d * a.out.s1;
  const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
  float prev[W > 1 ? W - 1 : 1];   // the W - 1 inputs before the chunk
#pragma unroll
  for (int i = 0; i < W - 1; ++i) prev[i] = 0.f;
  for (int64_t t0 = 0; t0 < L; t0 += kCUf * kCCh) {
    // raw 16-byte words of the group's chunks, converted only when used
    // a chunk wholly inside the row loads as 16-byte words, a partial one element by element
    // (the condition is uniform over the wave)
    Raw8<IT> raw[kCUf];
#pragma unroll
    for (int u = 0; u < kCUf; ++u) {
      const int64_t t = t0 + u * kCCh + kCE * lane;
      if (vec && t0 + (u + 1) * kCCh <= L) raw[u] = ld_raw8<IT>(x + t);
      else raw[u] = ld_raw8_part<IT>(x, t, L, vec);
    }
#pragma unroll
    for (int u = 0; u < kCUf; ++u) {
      if (t0 + u * kCCh >= L) break;
      const int64_t t = t0 + u * kCCh + kCE * lane;
      float xx[W - 1 + kCE];
      cvt_raw8<IT>(raw[u], xx + W - 1);
#pragma unroll
      for (int i = 0; i < W - 1; ++i) {
        const float h = shfl_f(xx[W - 1 + kCE - (W - 1) + i], lane - 1);
        xx[i] = lane == 0 ? prev[i] : h;
      }
      float y[kCE];
#pragma unroll
      for (int j = 0; j < kCE; ++j) {
        float acc = bias;
#pragma unroll
        for (int k = 0; k < W; ++k) acc = fmaf(w[k], xx[j + k], acc);
        y[j] = kSilu ? silu_f(acc) : acc;
      }
      if (t < L) store_row8<IT>(out, t, L, vec, y);
#pragma unroll
      for (int i = 0; i < W - 1; ++i)
        prev[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xx[W - 1 + kCE - (W - 1) + i]), 63));
    }
  }
}

// dx (row) and per-row partials of dw[W], dbias -> part[row * (W + 1) + k].
// Walks the row right to left, kCUb chunks per group (loaded together).
template <typename IT, int W, bool kSilu>
__global__ void __launch_bounds__(256) cconv_bwd_kernel(const lrnnx_causal_conv1d_args a, float* __restrict__ part) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.batch * a.dim) return;
  const int64_t b = row / a.dim, d = row % a.dim, L = a.seqlen;
  float w[W];
  const float* wp = static_cast<const float*>(a.weight.ptr);
#pragma unroll
  for (int k = 0; k < W; ++k) w[k] = wp[d * a.weight.s0 + k * a.weight.s1];
  const float bias = a.bias.ptr ? static_cast<const float*>(a.bias.ptr)[d * a.bias.s0] : 0.f;
  const IT* x = static_cast<const IT*>(a.x.ptr) + b * a.x.s0 + d * a.x.s1;
  const IT* dout = static_cast<const IT*>(a.dout.ptr) + b * a.dout.s0 + d * a.dout.s1;
  IT* dx = static_cast<IT*>(a.dx.ptr) + b * a.dx.s0 + d * a.dx.s1;
  const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(dout) & 15u) == 0 &&
                   (reinterpret_cast<uintptr_t>(dx) & 15u) == 0;
  float gnext[W > 1 ? W - 1 : 1];   // g of the W - 1 steps after the chunk
#pragma unroll
  for (int i = 0; i < W - 1; ++i) gnext[i] = 0.f;
  float dw[W], db = 0.f;
#pragma unroll
  for (int k = 0; k < W; ++k) dw[k] = 0.f;
  const int64_t n_chunks = (L + kCCh - 1) / kCCh;
  for (int64_t c = n_chunks - 1; c >= 0; c -= kCUb) {
    // group: chunks c, c - 1, ..., c - kCUb + 1 (those >= 0), processed in that order
    // raw 16-byte words of the group's chunks, converted only when used
    Raw8<IT> rx[kCUb], rg[kCUb];
    float hist[kCUb][W > 1 ? W - 1 : 1];
    // a chunk wholly inside the row loads as 16-byte words, a partial one (or one
    // before the row, c - u < 0: zeros) element by element; uniform over the wave
#pragma unroll
    for (int u = 0; u < kCUb; ++u) {
      const int64_t t = (c - u) * kCCh + kCE * lane;
      if (vec && c - u >= 0 && (c - u + 1) * kCCh <= L) {
        rx[u] = ld_raw8<IT>(x + t);
        rg[u] = ld_raw8<IT>(dout + t);
      } else {
        rx[u] = ld_raw8_part<IT>(x, t, L, vec);
        rg[u] = ld_raw8_part<IT>(dout, t, L, vec);
      }
    }
    // lane 0: the W - 1 inputs before each chunk
#pragma unroll
    for (int u = 0; u < kCUb; ++u) {
#pragma unroll
      for (int i = 0; i < W - 1; ++i) {
        const int64_t tt = (c - u) * kCCh - (W - 1) + i;
        hist[u][i] = 0.f;
        if (lane == 0 && tt >= 0 && tt < L) hist[u][i] = to_f32(x[tt]);
      }
    }
#pragma unroll
    for (int u = 0; u < kCUb; ++u) {
      if (c - u < 0) break;
      const int64_t t = (c - u) * kCCh + kCE * lane;
      float xx[W - 1 + kCE], go[kCE];
      cvt_raw8<IT>(rx[u], xx + W - 1);
      cvt_raw8<IT>(rg[u], go);
#pragma unroll
      for (int i = 0; i < W - 1; ++i) {
        const float h = shfl_f(xx[W - 1 + kCE - (W - 1) + i], lane - 1);
        xx[i] = lane == 0 ? hist[u][i] : h;
      }
      // g = dout act'(pre) (zero past L: dout loads as zero there)
      float g[kCE + (W > 1 ? W - 1 : 0)];
#pragma unroll
      for (int j = 0; j < kCE; ++j) {
        float gj = go[j];
        if constexpr (kSilu) {
          float pre = bias;
#pragma unroll
          for (int k = 0; k < W; ++k) pre = fmaf(w[k], xx[j + k], pre);
          gj *= silu_grad(pre);
        }
        g[j] = gj;
        db += gj;
#pragma unroll
        for (int k = 0; k < W; ++k) dw[k] = fmaf(gj, xx[j + k], dw[k]);
      }
      // the W - 1 values of g after the lane's steps: the next lane's first ones
#pragma unroll
      for (int i = 0; i < W - 1; ++i) {
        const float h = shfl_f(g[i], lane + 1);
        g[kCE + i] = lane == 63 ? gnext[i] : h;
      }
      float dxv[kCE];
#pragma unroll
      for (int j = 0; j < kCE; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < W; ++k) acc = fmaf(w[k], g[j + W - 1 - k], acc);
        dxv[j] = acc;
      }
      if (t < L) store_row8<IT>(dx, t, L, vec, dxv);
#pragma unroll
      for (int i = 0; i < W - 1; ++i) gnext[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g[i]), 0));
    }
  }
#pragma unroll
  for (int k = 0; k < W; ++k) dw[k] = wave_allreduce_sum(dw[k]);
  db = wave_allreduce_sum(db);
  if (lane == 0) {
    float* p = part + row * (W + 1);
#pragma unroll
    for (int k = 0; k < W; ++k) p[k] = dw[k];
    p[W] = db;
  }
}

// dweight[d, k], dbias[d] (fp32) = sum over b of the per-row partials, in batch order
__global__ void __launch_bounds__(256) cconv_bwd_reduce(const lrnnx_causal_conv1d_args a, const float* __restrict__ part) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // (d, k), k <= W
  const int64_t W = a.width;
  if (i >= a.dim * (W + 1)) return;
  const int64_t d = i / (W + 1), k = i % (W + 1);
  float s = 0.f;
  for (int64_t b = 0; b < a.batch; ++b) s += part[(b * a.dim + d) * (W + 1) + k];
  if (k < W) static_cast<float*>(a.dweight.ptr)[d * a.dweight.s0 + k * a.dweight.s1] = s;
  else if (a.dbias.ptr) static_cast<float*>(a.dbias.ptr)[d * a.dbias.s0] = s;
}

// One decode step (or a few new steps): conv_state (b, d, S), S >= W - 1,
// holds the last S inputs; x (b, d, Lx) new inputs; out (b, d, Lx).
//   x_all = [state, x];  state <- last S of x_all;  out[j] = act(bias + sum_k w[k] x_all[S + j - W + 1 + k])
template <typename IT, int W, bool kSilu>
__global__ void __launch_bounds__(256) cconv_update_kernel(const lrnnx_causal_conv1d_args a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // (b, d)
  if (i >= a.batch * a.dim) return;
  const int64_t b = i / a.dim, d = i % a.dim, S = a.state_len, Lx = a.seqlen;
  float w[W];
  const float* wp = static_cast<const float*>(a.weight.ptr);
#pragma unroll
  for (int k = 0; k < W; ++k) w[k] = wp[d * a.weight.s0 + k * a.weight.s1];
  const float bias = a.bias.ptr ? static_cast<const float*>(a.bias.ptr)[d * a.bias.s0] : 0.f;
  IT* st = static_cast<IT*>(a.conv_state.ptr) + b * a.conv_state.s0 + d * a.conv_state.s1;
  const int64_t ss = a.conv_state.s2;
  const IT* x = static_cast<const IT*>(a.x.ptr) + b * a.x.s0 + d * a.x.s1;
  IT* out = static_cast<IT*>(a.out.ptr) + b * a.out.s0 + d * a.out.s1;
  for (int64_t j = 0; j < Lx; ++j) {
    const float xn = to_f32(x[j * a.x.s2]);
    float acc = fmaf(w[W - 1], xn, bias);
#pragma unroll
    for (int k = 0; k < W - 1; ++k) acc = fmaf(w[k], to_f32(st[(S - (W - 1) + k) * ss]), acc);
    for (int64_t s = 0; s + 1 < S; ++s) st[s * ss] = st[(s + 1) * ss];
    st[(S - 1) * ss] = from_f32<IT>(xn);
    out[j * a.out.s2] = from_f32<IT>(kSilu ? silu_f(acc) : acc);
  }
}

namespace {
template <typename IT, int W>
hipError_t cconv_launch_w(const lrnnx_causal_conv1d_args& a, int which, float* part, hipStream_t st) {
  const int64_t rows = a.batch * a.dim;
  const dim3 gr((unsigned)((rows + 3) / 4)), blk(256), gt((unsigned)((rows + 255) / 256));
  if (which == 0) {
    if (a.silu) hipLaunchKernelGGL((cconv_fwd_kernel<IT, W, true>), gr, blk, 0, st, a);
    else hipLaunchKernelGGL((cconv_fwd_kernel<IT, W, false>), gr, blk, 0, st, a);
  } else if (which == 1) {
    if (a.silu) hipLaunchKernelGGL((cconv_bwd_kernel<IT, W, true>), gr, blk, 0, st, a, part);
    else hipLaunchKernelGGL((cconv_bwd_kernel<IT, W, false>), gr, blk, 0, st, a, part);
    const int64_t n = a.dim * (a.width + 1);
    hipLaunchKernelGGL(cconv_bwd_reduce, dim3((unsigned)((n + 255) / 256)), blk, 0, st, a,
                       static_cast<const float*>(part));
  } else {
    if (a.silu) hipLaunchKernelGGL((cconv_update_kernel<IT, W, true>), gt, blk, 0, st, a);
    else hipLaunchKernelGGL((cconv_update_kernel<IT, W, false>), gt, blk, 0, st, a);
  }
  return hipGetLastError();
}

template <typename IT>
hipError_t cconv_launch_t(const lrnnx_causal_conv1d_args& a, int which, float* part, hipStream_t st) {
  switch (a.width) {
    case 1: return cconv_launch_w<IT, 1>(a, which, part, st);
    case 2: return cconv_launch_w<IT, 2>(a, which, part, st);
    case 3: return cconv_launch_w<IT, 3>(a, which, part, st);
    case 4: return cconv_launch_w<IT, 4>(a, which, part, st);
    case 5: return cconv_launch_w<IT, 5>(a, which, part, st);
    case 6: return cconv_launch_w<IT, 6>(a, which, part, st);
    case 7: return cconv_launch_w<IT, 7>(a, which, part, st);
    case 8: return cconv_launch_w<IT, 8>(a, which, part, st);
  }
  return hipErrorInvalidValue;
}
}  // namespace

// which: 0 forward, 1 backward (part = workspace), 2 decode update
hipError_t cconv_launch(const lrnnx_causal_conv1d_args& a, int which, float* part, hipStream_t st) {
  switch (a.itype) {
    case LRNNX_F32: return cconv_launch_t<float>(a, which, part, st);
    case LRNNX_BF16: return cconv_launch_t<bf16>(a, which, part, st);
    case LRNNX_F16: return cconv_launch_t<f16>(a, which, part, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace lrnnx
