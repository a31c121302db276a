// Tile staging through LDS for the selective-scan kernels.
//
// A "raw tile" is a [rows][kT] block of one sequence tensor (element type IT,
// rows = channels or states), copied byte-for-byte into LDS in row-major
// order: row r occupies kQ 16-byte blocks, kQ = kT * sizeof(IT) / 16.
//
// Full tiles of suitably aligned tensors are fetched with gfx950's
// global_load_lds_dwordx4: one wave instruction moves 64 blocks (1 KiB)
// straight into LDS without passing through VGPRs, so the fetch of tile k+1
// is issued before tile k is computed and completes in the background (the
// consumer waits with s_waitcnt vmcnt(0) + a workgroup barrier).  Block j of
// the tile (row j / kQ, block j % kQ) lands at LDS byte offset 16 j; lane l of
// the instruction that covers blocks [64 i, 64 i + 64) moves block 64 i + l,
// so consecutive lanes read consecutive 16-byte pieces of a row (coalesced).
// Partial tiles and misaligned tensors take the synchronous path, which
// writes the same layout (zero-filled outside the valid rows / steps).
#pragma once

#include <type_traits>

#include "common.h"

namespace lrnnx {

using lds_void = __attribute__((address_space(3))) void;

__device__ __forceinline__ lds_void* to_lds(void* p) {
  return reinterpret_cast<lds_void*>(reinterpret_cast<uintptr_t>(p));
}

// One global_load_lds_dwordx4: every active lane copies the 16 bytes at its
// `g` to LDS address lds_wave_base + 16 * lane.  Issued through inline asm
// so that the compiler does not model the LDS write: it would otherwise make
// every later LDS read of the workgroup wait (s_waitcnt vmcnt(0)) for the
// fetch, which would serialise the fetch with the compute it is meant to
// overlap.  The consumer therefore waits explicitly (kWaitVm0 + barrier).
// Extra loads unknown to the compiler only make its own vmcnt waits
// stricter (loads retire in order), never weaker.
// M0 is listed as clobbered; clang warns that it is a reserved register whose
// value it may not preserve around the statement.  The kernels of this
// library give the compiler no other use of M0 (no LDS-DMA builtins, no
// indirect register indexing, no message/interpolation instructions); the
// built code objects are checked for that by the test suite.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma_16(const void* g, char* lds_wave_base) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(to_lds(lds_wave_base)));
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off"
      :
      : "s"(m0), "v"(g)
      : "memory", "m0");
#endif
}
#pragma clang diagnostic pop

// The same copy in the scalar-base form: lane l copies the 16 bytes at
// base + voff (base uniform, held in SGPRs; voff a per-lane 32-bit byte
// offset).  A kernel that moves a tile window along L keeps voff fixed and
// moves only the scalar base, so a fetch costs no VALU address arithmetic.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma_16_s(const void* base, uint32_t voff, char* lds_wave_base) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t m0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
      static_cast<int>(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(to_lds(lds_wave_base))))));
  // readfirstlane returns int: both halves go through uint32_t so that the
  // low half is zero-extended (a sign extension would set the high 32 bits)
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(b))));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(b >> 32))));
  const uint64_t sb = (static_cast<uint64_t>(hi) << 32) | static_cast<uint64_t>(lo);
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2"
      :
      : "s"(m0), "v"(voff), "s"(sb)
      : "memory", "m0");
#endif
}
#pragma clang diagnostic pop

// Byte offset of the block that lane `lane` moves in instruction `instr` of
// a [rows][kQ] raw-tile fetch (block j = 64 instr + lane: row j / kQ, 16-byte
// piece j % kQ), for rows `g_stride` elements apart.
template <typename IT, int kQ>
__device__ __forceinline__ uint32_t dma_lane_offset(uint32_t g_stride, int instr, int lane) {
  const uint32_t j = static_cast<uint32_t>(instr * kWave + lane);
  return ((j / kQ) * g_stride + (j % kQ) * (16 / sizeof(IT))) * static_cast<uint32_t>(sizeof(IT));
}

// Instruction `instr` of the asynchronous fetch of a [rows][kQ] raw tile whose
// row 0 starts at `base`, with the lane offsets of dma_lane_offset: lanes past
// the tile's rows * kQ blocks stay idle.  Tiles of at most 64 * (number of
// waves) blocks are fetched with one instruction per wave (instr = wave).
template <int kQ>
__device__ __forceinline__ void tile_fetch_async_s(const void* base, uint32_t voff, int rows, char* lds, int instr,
                                                   int lane) {
  const int nblk = rows * kQ;
  if (instr * kWave < nblk && instr * kWave + lane < nblk) lds_dma_16_s(base, voff, lds + instr * 1024);
}

// Whether a tile fetch with the scalar-base form reaches every block: the
// largest lane offset of a [rows][kQ] tile of row stride `stride` elements
// fits the 32-bit offset.
inline bool dma_offsets_fit(int64_t stride, int64_t rows, int64_t row_bytes, int64_t elem_bytes) {
  return (rows - 1) * stride * elem_bytes + row_bytes <= 0xffffffffll;
}

// Asynchronous full-tile fetch.  `rows` valid rows (rows * kQ blocks), row r
// at g_base + r * g_stride (elements).  Instructions are dealt round-robin
// to the nW waves of the workgroup.
template <typename IT, int kQ>
__device__ __forceinline__ void tile_fetch_async(const IT* __restrict__ g_base, uint32_t g_stride, int rows,
                                                 char* lds, int w, int nW, int lane) {
  constexpr int kEl = 16 / sizeof(IT);
  const int nblk = rows * kQ;
  for (int i = w; i * kWave < nblk; i += nW) {
    const int j = i * kWave + lane;
    if (j < nblk) {
      const int r = j / kQ, q = j % kQ;
      const IT* g = g_base + r * g_stride + q * kEl;
      lds_dma_16(g, lds + i * 1024);
    }
  }
}

// Synchronous fetch into the same layout; steps >= nt and rows >= rows_valid
// are zero.  All threads of the workgroup take part.
template <typename IT, int kQ>
__device__ __forceinline__ void tile_fetch_sync(const IT* __restrict__ g_base, uint32_t g_stride, int rows,
                                                int rows_valid, int nt, char* lds, int tid, int nthreads) {
  constexpr int kEl = 16 / sizeof(IT);
  for (int j = tid; j < rows * kQ; j += nthreads) {
    const int r = j / kQ, q = j % kQ;
    uint4 v = make_uint4(0, 0, 0, 0);
    IT* e = reinterpret_cast<IT*>(&v);
    const int n = nt - q * kEl;
    if (r < rows_valid && n > 0) {
      const IT* g = g_base + r * g_stride + q * kEl;
      if (n >= kEl && (reinterpret_cast<uintptr_t>(g) & 15u) == 0) {
        v = *reinterpret_cast<const uint4*>(g);
      } else {
#pragma unroll
        for (int i = 0; i < kEl; ++i)
          if (i < n) e[i] = g[i];
      }
    }
    *reinterpret_cast<uint4*>(lds + 16 * j) = v;
  }
}

// s_waitcnt encodings (gfx9 family): vmcnt bits [3:0]+[15:14], expcnt [6:4], lgkmcnt [11:8]
constexpr int kWaitVm0 = 0x0f70;   // vmcnt(0): global loads (incl. LDS-DMA) and stores done
constexpr int kWaitLgkm0 = 0xc07f; // lgkmcnt(0): LDS / scalar-memory ops done

// Workgroup barrier that orders LDS only: it does not wait for outstanding
// global loads / stores (the fetch of the next tile keeps running).
__device__ __forceinline__ void barrier_lds() {
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_s_barrier();
}

// Wait for this wave's outstanding global memory operations (the async tile
// fetch), then barrier so every wave's part of the tile is in LDS.
__device__ __forceinline__ void barrier_after_fetch() {
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_s_barrier();
}

// 16 raw bytes -> floats (kEl = 4 for f32, 8 for 16-bit types)
template <typename IT>
__device__ __forceinline__ void raw_to_f32(const uint4& raw, float* out) {
  const IT* e = reinterpret_cast<const IT*>(&raw);
#pragma unroll
  for (int i = 0; i < (int)(16 / sizeof(IT)); ++i) out[i] = to_f32(e[i]);
}

template <typename IT>
__device__ __forceinline__ uint4 f32_to_raw(const float* v) {
  uint4 raw;
  if constexpr (sizeof(IT) == 2 && !std::is_same<IT, f16>::value) {
    // bf16: one v_cvt_pk_bf16_f32 per adjacent pair (round to nearest even)
    using f2 = float __attribute__((ext_vector_type(2)));
    using b2 = __bf16 __attribute__((ext_vector_type(2)));
    uint32_t* w = reinterpret_cast<uint32_t*>(&raw);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const b2 p = __builtin_convertvector((f2){v[2 * i], v[2 * i + 1]}, b2);
      w[i] = __builtin_bit_cast(uint32_t, p);
    }
  } else {
    IT* e = reinterpret_cast<IT*>(&raw);
#pragma unroll
    for (int i = 0; i < (int)(16 / sizeof(IT)); ++i) e[i] = from_f32<IT>(v[i]);
  }
  return raw;
}

// 4 consecutive elements at LDS byte address p (8-byte aligned for 16-bit
// types, 16-byte for f32) -> floats
template <typename IT>
__device__ __forceinline__ void raw4_to_f32(const char* p, float* out) {
  if constexpr (sizeof(IT) == 4) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  } else {
    const uint2 raw = *reinterpret_cast<const uint2*>(p);
    const IT* e = reinterpret_cast<const IT*>(&raw);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = to_f32(e[i]);
  }
}

// 2 consecutive elements at LDS byte address p (4-byte aligned for 16-bit
// types, 8-byte for f32) -> floats
template <typename IT>
__device__ __forceinline__ void raw2_to_f32(const char* p, float* out) {
  if constexpr (sizeof(IT) == 4) {
    const float2 v = *reinterpret_cast<const float2*>(p);
    out[0] = v.x; out[1] = v.y;
  } else {
    const uint32_t raw = *reinterpret_cast<const uint32_t*>(p);
    const IT* e = reinterpret_cast<const IT*>(&raw);
    out[0] = to_f32(e[0]);
    out[1] = to_f32(e[1]);
  }
}

// kN (4 or 2) consecutive raw elements at LDS byte address p -> floats
template <typename IT, int kN>
__device__ __forceinline__ void rawn_to_f32(const char* p, float* out) {
  if constexpr (kN == 4) raw4_to_f32<IT>(p, out);
  else raw2_to_f32<IT>(p, out);
}

// 2 floats -> 2 consecutive elements at global address p (one 4- or 8-byte store)
template <typename IT>
__device__ __forceinline__ void store2(IT* p, const float* v) {
  if constexpr (sizeof(IT) == 4) {
    *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
  } else {
    float w8[8] = {v[0], v[1], 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const uint4 raw = f32_to_raw<IT>(w8);
    *reinterpret_cast<uint32_t*>(p) = raw.x;
  }
}

// 4 floats -> 4 consecutive elements at global address p (one 8- or 16-byte store)
template <typename IT>
__device__ __forceinline__ void store4(IT* p, const float* v) {
  if constexpr (sizeof(IT) == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    float w8[8] = {v[0], v[1], v[2], v[3], 0.f, 0.f, 0.f, 0.f};
    const uint4 raw = f32_to_raw<IT>(w8);
    *reinterpret_cast<uint2*>(p) = make_uint2(raw.x, raw.y);
  }
}

template <typename IT, int kN>
__device__ __forceinline__ void storen(IT* p, const float* v) {
  if constexpr (kN == 4) store4<IT>(p, v);
  else store2<IT>(p, v);
}

// fast transcendental helpers (v_exp_f32 / v_log_f32 / v_rcp_f32)
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ __forceinline__ float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }

// softplus with the reference's threshold (identity above 20); log1p(e) by a
// 4-term series below 1/32 (relative error < 3e-7), else log(1 + e).
__device__ __forceinline__ float softplus_fast(float x) {
  const float e = exp_fast(x);
  const float small = e * (1.f - e * (0.5f - e * (0.33333334f - e * 0.25f)));
  const float big = __builtin_amdgcn_logf(1.f + e) * kLn2;
  const float r = e < 0.03125f ? small : big;
  return x > 20.f ? x : r;
}

__device__ __forceinline__ float sigmoid_fast(float z) { return rcp_fast(1.f + exp_fast(-z)); }

// sigmoid(x) from d = softplus(x) >= 0: 1 - exp(-d), by its 4-term series
// below 1/32 (relative error < 1e-8) so that small d loses no digits.
__device__ __forceinline__ float one_minus_exp_neg(float d) {
  const float small = d * (1.f - d * (0.5f - d * (0.16666667f - d * 0.041666668f)));
  const float big = 1.f - exp_fast(-d);
  return d < 0.03125f ? small : big;
}

}  // namespace lrnnx
