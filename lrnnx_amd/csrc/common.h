// Device-side helpers shared by the gfx950 scan kernels.
//
// Written for CDNA4 (wave64).  Nothing here is a compatibility layer: the
// kernels use AMDGCN builtins directly (v_exp_f32, DPP, permlane swaps).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lrnnx_scan.h"

namespace lrnnx {

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kXChunk = 2048;  // reference chunk of the `x` carries (selective_scan_cpu.cpp:380)

// ---------------------------------------------------------------- element types
struct bf16 { uint16_t bits; };
using f16 = _Float16;

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(f16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f32(bf16 v) { return __uint_as_float(static_cast<uint32_t>(v.bits) << 16); }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) { return static_cast<f16>(v); }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) {
  // round to nearest even (gfx950 v_cvt_pk_bf16_f32; NaN stays NaN)
  bf16 r;
  r.bits = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
  return r;
}

// Load / store `n` (<= 8) consecutive elements as float; vector path when the
// pointer is 16-byte aligned and n is the full vector width.
template <typename T> struct Vec;      // elements per 16-byte vector
template <> struct Vec<float> { static constexpr int n = 4; };
template <> struct Vec<f16> { static constexpr int n = 8; };
template <> struct Vec<bf16> { static constexpr int n = 8; };

template <typename T>
__device__ __forceinline__ void load_vec(const T* __restrict__ p, int n, float* out) {
  constexpr int V = Vec<T>::n;
  if (n == V && (reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
    uint4 raw = *reinterpret_cast<const uint4*>(p);
    const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int i = 0; i < V; ++i) out[i] = to_f32(e[i]);
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) out[i] = i < n ? to_f32(p[i]) : 0.f;
  }
}

template <typename T>
__device__ __forceinline__ void store_vec(T* __restrict__ p, int n, const float* v) {
  constexpr int V = Vec<T>::n;
  if (n == V && (reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
    uint4 raw;
    T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
    for (int i = 0; i < V; ++i) e[i] = from_f32<T>(v[i]);
    *reinterpret_cast<uint4*>(p) = raw;
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (i < n) p[i] = from_f32<T>(v[i]);
  }
}

// ---------------------------------------------------------------- math
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// An empty asm that takes and returns v in a VGPR: the computation of v
// cannot move past this point.  Used to keep an accumulation chain at its
// step when only its final value is read later: machine sinking would
// otherwise move the chain to that read and keep every step's operands live.
__device__ __forceinline__ void pin_vgpr(float& v) { asm volatile("" : "+v"(v)); }

// sin and cos of x without branches.  Cody-Waite reduction to r = x - k pi/2,
// |r| <= pi/4, with pi/2 split into three parts (the leading ones short, so
// the products k * part are exact for |k| < 2^15); then the minimax
// polynomials of the Cephes library (S. L. Moshier) for sin and cos on
// [-pi/4, pi/4] (about 1 ulp), and the quadrant k mod 4 selects and signs them.
__device__ __forceinline__ void sincos_cw(float x, float& sn, float& cs) {
  const float k = __builtin_rintf(x * 0.63661977236758134f);  // 2 / pi
  float r = fmaf(-k, 1.5703125f, x);
  r = fmaf(-k, 4.837512969970703125e-4f, r);
  r = fmaf(-k, 7.54978995489188216e-8f, r);
  const float z = r * r;
  const float sp = fmaf(z, fmaf(z, -1.9515295891e-4f, 8.3321608736e-3f), -1.6666654611e-1f);
  const float s = fmaf(r * z, sp, r);
  const float cp = fmaf(z, fmaf(z, 2.443315711809948e-5f, -1.388731625493765e-3f), 4.166664568298827e-2f);
  const float c = fmaf(z * z, cp, fmaf(-0.5f, z, 1.f));
  const int q = (int)k;
  const float S = (q & 1) ? c : s;
  const float C = (q & 1) ? s : c;
  sn = (q & 2) ? -S : S;
  cs = ((q + 1) & 2) ? -C : C;
}

// softplus with the reference's threshold: identity above 20
// (selective_scan.cuh:172-174; F.softplus default threshold).
__device__ __forceinline__ float softplus20(float x) { return x <= 20.f ? log1pf(expf(x)) : x; }

__device__ __forceinline__ float silu(float z) { return z / (1.f + expf(-z)); }

// ---------------------------------------------------------------- wave reductions
__device__ __forceinline__ float dpp_f32(float v, int ctrl);

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), CTRL, 0xf, 0xf, false));
}

// The same with no old value (every lane of these patterns reads a lane of
// its own row): nothing to initialise, so the move can fold into an FMA's
// addend or a VOP2 operand without an extra v_mov.
template <int CTRL>
__device__ __forceinline__ float dpp_get(float v) {
  return __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), CTRL, 0xf, 0xf, true));
}

// DPP control words (GFX9 encoding)
constexpr int kDppQuadXor1 = 0xb1;        // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4e;        // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;  // lane i <-> 7-i within each 8
constexpr int kDppRowMirror = 0x140;      // lane i <-> 15-i within each 16

// Sum over all 64 lanes; every lane receives the total.
__device__ __forceinline__ float wave_allreduce_sum(float v) {
  v += dpp_mov<kDppQuadXor1>(v);
  v += dpp_mov<kDppQuadXor2>(v);
  v += dpp_mov<kDppRowHalfMirror>(v);
  v += dpp_mov<kDppRowMirror>(v);
  {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  return v;
}

// Reduce-scatter over the 64 lanes of a wave.  Conceptually every lane holds
// 64 values v[0..63] (v[i] = this lane's contribution to output i); on exit
// lane l holds the 64-lane sum of output l.  The index bits are consumed
// from the top:
//   bit 5  xor-32 lane pairing, v_permlane32_swap (gfx950) + add,
//   bit 4  xor-16 pairing inside each half, v_permlane16_swap + add,
//   bits 3..0  pairings inside a 16-lane row through DPP row_mirror,
//   row_half_mirror and two quad permutations (select what to send, add the
//   partner's value through the DPP operand).
// The first two steps are exposed separately (rs_step32 / rs_step16) so a
// caller can apply them as soon as the paired values exist, which keeps only
// 16 values per quantity live.

// v[0..n) paired with v[n..2n): lanes < 32 keep index k, lanes >= 32 keep k + n.
template <int n>
__device__ __forceinline__ void rs_step32(float* v) {
#pragma unroll
  for (int k = 0; k < n; ++k) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[k]), __float_as_uint(v[k + n]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// v[0..n) paired with v[n..2n): even 16-lane rows keep k, odd rows keep k + n.
template <int n>
__device__ __forceinline__ void rs_step16(float* v) {
#pragma unroll
  for (int k = 0; k < n; ++k) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]), __float_as_uint(v[k + n]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// One reduce-scatter pairing of index bit 3 (kBit = 8: lanes i <-> 15 - i of
// a 16-lane row) or bit 2 (kBit = 4: i <-> 7 - i of each 8): lanes whose bit
// is clear return lo + the partner's lo, the others hi + the partner's hi.
// The two halves are DPP bank groups (bit 3: banks 0-1 / 2-3; bit 2: banks
// 0, 2 / 1, 3), so two v_add_f32_dpp with complementary bank masks do it,
// with no selects: each writes only its banks.  Inline asm, because the
// compiler does not form bank-masked DPP adds that keep the other lanes;
// the s_nop covers the wait states a DPP read needs after a VALU write.
template <int kBit>
__device__ __forceinline__ float rs_pair_banked(float lo, float hi) {
  static_assert(kBit == 8 || kBit == 4, "bank-group pairings are index bits 3 and 2");
  float r;
#if defined(__HIP_DEVICE_COMPILE__)
  if constexpr (kBit == 8) {
    asm volatile(
        "s_nop 1\n\t"
        "v_add_f32_dpp %0, %1, %1 row_mirror row_mask:0xf bank_mask:0x3\n\t"
        "v_add_f32_dpp %0, %2, %2 row_mirror row_mask:0xf bank_mask:0xc"
        : "=&v"(r)
        : "v"(lo), "v"(hi));
  } else {
    asm volatile(
        "s_nop 1\n\t"
        "v_add_f32_dpp %0, %1, %1 row_half_mirror row_mask:0xf bank_mask:0x5\n\t"
        "v_add_f32_dpp %0, %2, %2 row_half_mirror row_mask:0xf bank_mask:0xa"
        : "=&v"(r)
        : "v"(lo), "v"(hi));
  }
#else
  r = lo + hi;
#endif
  return r;
}

// Last four steps on 16 values (index bits 3..0); result in v[0].
__device__ __forceinline__ void rs_tail16(float (&v)[16], int lane) {
  const bool b1 = lane & 2, b0 = lane & 1;
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = rs_pair_banked<8>(v[k], v[k + 8]);
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = rs_pair_banked<4>(v[k], v[k + 4]);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const float keep = b1 ? v[k + 2] : v[k];
    const float send = b1 ? v[k] : v[k + 2];
    v[k] = keep + dpp_mov<kDppQuadXor2>(send);
  }
  const float keep = b0 ? v[1] : v[0];
  const float send = b0 ? v[0] : v[1];
  v[0] = keep + dpp_mov<kDppQuadXor1>(send);
}

__device__ __forceinline__ float reduce_scatter64(float (&v)[64], int lane) {
  rs_step32<32>(v);
  rs_step16<16>(v);
  float t[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) t[k] = v[k];
  rs_tail16(t, lane);
  return t[0];
}

// Output index owned by `lane` after reduce_scatter64.
__host__ __device__ __forceinline__ int reduce_scatter64_index(int lane) {
  int k = 0;
  if (lane & 32) k += 32;
  if (lane & 16) k += 16;
  if (lane & 8) k += 8;
  if (lane & 4) k += 4;
  if (lane & 2) k += 2;
  if (lane & 1) k += 1;
  return k;
}

}  // namespace lrnnx
