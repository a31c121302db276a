// Selective scan backward (real weights), gfx950.
//
// Semantics: reference kernel csrc/selective_scan/selective_scan_backward.cuh:86-845
// (gradients of the forward in ss_fwd_impl.h; softplus backward = sigmoid,
// :797-799; dz = dout * out * sigma(z) (1 + z (1 - sigma(z))), :218-219).
//
// Same decomposition as the forward (lane = channel, wave = kS states).
// Tiles of kTB steps are processed from the end of the sequence to the start;
// a tile holds kTB / kCk checkpoint intervals ("sub-chunks").  Per sub-chunk a
// wave takes h at the sub-chunk start from the forward's fp32 checkpoints,
// recomputes h (and A_bar where kAbLive) for the kCk steps into VGPRs, then
// walks the steps backwards:
//   dh_t = A_bar_{t+1} dh_{t+1} + C_t dy_t
// accumulating the per-step partials of du / ddelta / ddeltaA (summed over
// its kS states; crossed over waves in LDS), dA (per lane) and the values of
// dB / dC.  dB / dC are reduce-scattered over the 64 channels of the wave
// (the two cross-half steps right after each step, so only 16 values per
// quantity stay live) and one fp32 partial per (channel block, b, n, t) goes
// to the workspace; a second kernel sums the partials over channel blocks in
// a fixed order, so the result is deterministic (the reference uses one
// global atomic per element and channel block, selective_scan_backward.cuh:483-502).
//
// Phases per tile k, as in the forward:
//   compute(k)  issue the asynchronous LDS fetch of raw tile k-1 (u, delta,
//               dout, z, out, deltaA, B/C rows and, when a tile is one
//               checkpoint interval, the checkpoint rows), then the
//               sub-chunks of tile k;
//   finish(k)   wait + barrier; epilogue of tile k (du, ddelta, ddeltaA and
//               the per-element dD / ddelta_bias terms) and conversion of raw
//               tile k-1 (delta' = softplus(delta + bias), dy = dout silu(z),
//               dz written here, B/C to fp32).
// The fp32 operands of a tile (delta', u, dy) are double buffered because the
// epilogue of tile k and the conversion of tile k-1 share a phase.
#pragma once
#include <type_traits>

#include "ss_common.h"
#include "ss_fwd_impl.h"
#include "tile_io.h"

namespace lrnnx {

__host__ __device__ constexpr bool needs_p3_m(int m) {
  return m == LRNNX_ZOH || m == LRNNX_BILINEAR || m == LRNNX_RGLRU;
}
template <int kMethod>
__host__ __device__ constexpr bool needs_p3() { return needs_p3_m(kMethod); }

struct SSBwdWs {  // fp32 workspace sections (element offsets)
  int64_t dBv, dCv, dA, dBc, dCc, dD, dbias, ckpt, total;
  // state blocks (SSGeom::nsb > 1): the blocks' sums over their states of the
  // du / ddelta / ddeltaA terms, fp32 [block][term][b][d][L], n_terms of them
  int64_t pp, n_terms;
  // split of L (fast path, small grids): S segments; the per-(b, ...) partials
  // dA / dD / ddelta_bias are per (segment, b); the adjoint buffers
  // g_loc, g_init [seg][b][n][d] and dsum [seg][b][d]
  int64_t S, g_loc, g_init, dsum;
  // checkpoint rebuild on a split grid: the forward split's summaries and
  // carries (h_end, h_init [seg][b][n][d], dsum_seg, dsum_pre [seg][b][d])
  int64_t fws, fws_floats;
};

inline int64_t align64(int64_t x) { return (x + 63) / 64 * 64; }

inline SSBwdWs ss_bwd_ws(const lrnnx_selective_scan_args& a, const SSGeom& g, bool need_ckpt, int64_t S = 1) {
  SSBwdWs w;
  int64_t o = 0;
  const int64_t B = a.batch, D = a.dim, N = a.dstate, L = a.seqlen;
  const int64_t Bp = B * S;  // rows of the per-(segment, b) partials
  w.S = S;
  w.dBv = o; if (a.var_B) o += align64((int64_t)g.n_cb * B * N * L);
  w.dCv = o; if (a.var_C) o += align64((int64_t)g.n_cb * B * N * L);
  w.dA = o; o += align64(Bp * D * N);
  w.dBc = o; if (!a.var_B) o += align64(Bp * D * N);
  w.dCc = o; if (!a.var_C) o += align64(Bp * D * N);
  w.dD = o; o += align64(Bp * D);
  w.dbias = o; o += align64(Bp * D);
  w.g_loc = o; if (S > 1) o += align64(S * B * N * D);
  w.g_init = o; if (S > 1) o += align64(S * B * N * D);
  w.dsum = o; if (S > 1) o += align64(S * B * D);
  w.n_terms = needs_p3_m(a.method) ? 3 : 2;
  w.pp = o; if (g.nsb > 1) o += align64((int64_t)g.nsb * w.n_terms * B * D * L);
  w.ckpt = o; if (need_ckpt) o += align64(B * g.n_ck * N * D);
  w.fws = o;
  w.fws_floats = (need_ckpt && S > 1) ? 2 * S * B * N * D + 2 * S * B * D : 0;
  o += align64(w.fws_floats);
  w.total = o;
  return w;
}

// kV consecutive floats from LDS (kV = 4 or 2, naturally aligned)
template <int kV>
__device__ __forceinline__ void lds_ldv(const float* p, float* o) {
  if constexpr (kV == 4) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  } else {
    const float2 v = *reinterpret_cast<const float2*>(p);
    o[0] = v.x; o[1] = v.y;
  }
}
template <int kV>
__device__ __forceinline__ void lds_stv(float* p, const float* o) {
  if constexpr (kV == 4) *reinterpret_cast<float4*>(p) = make_float4(o[0], o[1], o[2], o[3]);
  else *reinterpret_cast<float2*>(p) = make_float2(o[0], o[1]);
}

// Scheduling fence between groups of steps: keeps the compiler from hoisting
// the LDS operand loads of later steps above the arithmetic of earlier ones
// (which raises register pressure past 256 VGPRs and forces spills).
__device__ __forceinline__ void kSchedFence() { __builtin_amdgcn_sched_barrier(0); }

// the kS consecutive floats of a wave's states (16-byte aligned when kS >= 4)
template <int kS>
__device__ __forceinline__ void lds_states(const float* p, float* o) {
  if constexpr (kS == 1) {
    o[0] = p[0];
  } else {
#pragma unroll
    for (int k = 0; k < kS; k += 4) lds_ldv<4>(p + k, o + k);
  }
}

// kNWm: most waves of a launch (as in the forward).
template <typename IT, int kS, int kMethod, bool kVarB, bool kVarC, bool kDA, int kNWm = fwd_nw_max(kS)>
__global__ void __launch_bounds__(512)
ss_bwd_kernel(const lrnnx_selective_scan_args a, const int CB, const int64_t n_ck, float* __restrict__ ws,
              const SSBwdWs wo, const float* __restrict__ ckp, const int flags, const int nsb) {
  constexpr int kCk = ck_for(kS);
  // steps per tile: 16, or 8 at 8 states per wave with fp32 I/O where 16 would not fit: two
  // 4-wave workgroups per CU need 80 KB, and one 8-wave workgroup of zoh / bilinear (their
  // third partial sum) more than 160 KB
  constexpr int kTB = (kS >= 8 && sizeof(IT) == 4 && (kNWm <= 4 || needs_p3_m(kMethod))) ? 8 : 16;
  constexpr int kEl = 16 / sizeof(IT);  // elements per 16-byte block
  constexpr int kQ = kTB / kEl;         // 16-byte blocks per raw row
  constexpr int kG = kTB / 4;           // groups of 4 steps
  constexpr int kNV = kS * kCk;         // dB/dC values per lane per sub-chunk (<= 64)
  constexpr int kV = kCk < 4 ? kCk : 4; // steps per LDS vector access
  constexpr bool kP3 = needs_p3<kMethod>();
  // A_bar of the interval kept in VGPRs (s7's is one value per step; mamba
  // and dirac keep it up to kS = 4 and re-derive it, one exp, above)
  constexpr bool kAbLive = kMethod == LRNNX_S7 || (!kP3 && kS <= 4);
  constexpr int kNWmax = kNWm;
  constexpr int kNPmax = kNWmax * kS;
  constexpr int kRawArr = kWave * kTB * (int)sizeof(IT);
  constexpr int kRawBC = kNPmax * kTB * (int)sizeof(IT);
  constexpr bool kCkLds = kTB == kCk;   // one checkpoint interval per tile: stage its rows in LDS
  static_assert(kTB % kCk == 0, "tile must hold whole checkpoint intervals");
  static_assert(kCk % kV == 0 && kTB % 4 == 0, "vector access must not straddle groups");

  // separate LDS objects (see the forward): the asynchronous fetches write
  // only s_raw_* and s_ck
  __shared__ __attribute__((aligned(16))) char s_raw_u[kRawArr];
  __shared__ __attribute__((aligned(16))) char s_raw_d[kRawArr];
  __shared__ __attribute__((aligned(16))) char s_raw_do[kRawArr];
  __shared__ __attribute__((aligned(16))) char s_raw_z[kRawArr];
  __shared__ __attribute__((aligned(16))) char s_raw_os[kRawArr];
  __shared__ __attribute__((aligned(16))) char s_raw_dA[kDA ? kRawArr : 16];
  __shared__ __attribute__((aligned(16))) char s_raw_bc[(kVarB || kVarC) ? 2 * kRawBC : 16];
  __shared__ __attribute__((aligned(16))) float s_ck[kCkLds ? 2 * kNPmax * kWave : 4];  // [buf][NP][64]
  __shared__ __attribute__((aligned(16))) float s_dl[2][kWave * kTB];  // [buf][kG][64][4] delta'
  __shared__ __attribute__((aligned(16))) float s_u[2][kWave * kTB];   // u
  __shared__ __attribute__((aligned(16))) float s_dy[2][kWave * kTB];  // dout * silu(z)
  __shared__ __attribute__((aligned(16))) float s_dt[kDA ? kWave * kTB : 4];  // deltaA
  __shared__ __attribute__((aligned(16))) float s_B[kVarB ? kTB * kNPmax : 4];  // [kTB][NPmax] (step-major)
  __shared__ __attribute__((aligned(16))) float s_C[kVarC ? kTB * kNPmax : 4];
  __shared__ __attribute__((aligned(16))) float s_P1[kNWmax * kWave * kTB];  // [w][kG][64][4]
  __shared__ __attribute__((aligned(16))) float s_P2[kNWmax * kWave * kTB];
  __shared__ __attribute__((aligned(16))) float s_P3[kP3 ? kNWmax * kWave * kTB : 4];
  __shared__ float s_Dv[kWave], s_bias[kWave];

  const int nW = blockDim.x / kWave;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int64_t b = blockIdx.y;
  const int64_t D = a.dim, L = a.seqlen;
  const int N = (int)a.dstate;                 // all states (layout of the checkpoints, dA, dB, dC)
  const int64_t cb = blockIdx.x;
  const int64_t d0 = cb * CB;
  const int rows = (int)((D - d0) < CB ? (D - d0) : CB);
  const int64_t d = d0 + lane;
  const bool lane_ok = lane < rows;
  const int64_t grp = (a.var_B || a.var_C) ? d0 / (D / a.n_groups) : 0;
  const int n0 = w * kS;
  const int NP = nW * kS;
  const int nb = (int)blockIdx.z * NP;               // first state of this state block
  const int Nb = N - nb < NP ? N - nb : NP;          // its real states
  // state blocks: the epilogue writes the block's du / ddelta terms here (a
  // combine kernel finishes them, with dD and ddelta_bias)
  float* gpp = nsb > 1 ? ws + wo.pp + (((int64_t)blockIdx.z * wo.n_terms * a.batch + b) * D + d0) * L : nullptr;
  const int64_t pp_term = a.batch * D * L;           // between the terms of one block
  const bool has_dA_in = a.deltaA.ptr != nullptr;
  const bool has_bias = a.delta_bias.ptr != nullptr;
  const bool has_D = a.D.ptr != nullptr;
  const bool has_z = a.z.ptr != nullptr;
  const bool async_ok = flags & kFlagAsyncIn;   // fetched tensors allow 16-byte LDS-DMA rows
  const bool out_al = flags & kFlagAlignedOut;  // du / ddelta / ddeltaA / dz rows are 16-byte aligned

  const IT* gu = static_cast<const IT*>(a.u.ptr) + b * a.u.s0 + d0 * a.u.s1;
  const IT* gd = static_cast<const IT*>(a.delta.ptr) + b * a.delta.s0 + d0 * a.delta.s1;
  const IT* gdo = static_cast<const IT*>(a.dout.ptr) + b * a.dout.s0 + d0 * a.dout.s1;
  const IT* gz = has_z ? static_cast<const IT*>(a.z.ptr) + b * a.z.s0 + d0 * a.z.s1 : nullptr;
  const IT* gos =
      has_z ? static_cast<const IT*>(a.out_saved.ptr) + b * a.out_saved.s0 + d0 * a.out_saved.s1 : nullptr;
  const IT* gdA = kDA ? static_cast<const IT*>(a.deltaA.ptr) + b * a.deltaA.s0 + d0 * a.deltaA.s1 : nullptr;
  const IT* gB = kVarB ? static_cast<const IT*>(a.B.ptr) + b * a.B.s0 + grp * a.B.s1 + nb * a.B.s2 : nullptr;
  const IT* gC = kVarC ? static_cast<const IT*>(a.C.ptr) + b * a.C.s0 + grp * a.C.s1 + nb * a.C.s2 : nullptr;
  IT* gdu = static_cast<IT*>(a.du.ptr) + b * a.du.s0 + d0 * a.du.s1;
  IT* gddl = static_cast<IT*>(a.ddelta.ptr) + b * a.ddelta.s0 + d0 * a.ddelta.s1;
  IT* gddA = has_dA_in ? static_cast<IT*>(a.ddeltaA.ptr) + b * a.ddeltaA.s0 + d0 * a.ddeltaA.s1 : nullptr;
  IT* gdz = has_z ? static_cast<IT*>(a.dz.ptr) + b * a.dz.s0 + d0 * a.dz.s1 : nullptr;
  const uint32_t su = (uint32_t)a.u.s1, sd = (uint32_t)a.delta.s1, sdo = (uint32_t)a.dout.s1;
  const uint32_t sz = (uint32_t)a.z.s1, sos = (uint32_t)a.out_saved.s1, sdA = (uint32_t)a.deltaA.s1;
  const uint32_t sBn = (uint32_t)a.B.s2, sCn = (uint32_t)a.C.s2;
  const uint32_t sdu = (uint32_t)a.du.s1, sddl = (uint32_t)a.ddelta.s1, sddA = (uint32_t)a.ddeltaA.s1;
  const uint32_t sdz = (uint32_t)a.dz.s1;
  // checkpoint rows: state n of interval kk at ckp[((b * n_ck + kk) * N + n) * D + d]
  const float* gck = ckp + b * n_ck * N * D + nb * D + d0;

  float a2[kS], Araw[kS], invA[kS], bcst[kS], ccst[kS], cout_c[kS];
  // dh: gradient of the state at the current step; gn: A_bar_{t+1} dh_{t+1}
  float dh[kS], gn[kS], dA_acc[kS], dBc_acc[kS], dCc_acc[kS];
  {
    const float* Ap = static_cast<const float*>(a.A.ptr);
    const float* Bp = static_cast<const float*>(a.B.ptr);
    const float* Cp = static_cast<const float*>(a.C.ptr);
#pragma unroll
    for (int k = 0; k < kS; ++k) {
      const int n = n0 + k;
      const bool ok = lane_ok && n < Nb;
      const int64_t ng = nb + n;
      const float Av = ok ? Ap[d * a.A.s0 + ng * a.A.s1] : (kMethod == LRNNX_RGLRU ? 0.5f : -1.f);
      Araw[k] = Av;
      invA[k] = 1.f / Av;
      a2[k] = prep_a2<kMethod>(Av);
      bcst[k] = (!kVarB && ok) ? Bp[d * a.B.s0 + ng * a.B.s1] : 1.f;
      ccst[k] = (!kVarC && ok) ? Cp[d * a.C.s0 + ng * a.C.s1] : 1.f;
      cout_c[k] = ok ? (kVarB ? 1.f : bcst[k]) * (kVarC ? 1.f : ccst[k]) : 0.f;
      dh[k] = 0.f; gn[k] = 0.f; dA_acc[k] = 0.f; dBc_acc[k] = 0.f; dCc_acc[k] = 0.f;
    }
  }
  float dD_acc = 0.f, dbias_acc = 0.f;  // wave 0, per channel
  if (tid < kWave) {
    s_Dv[tid] = (has_D && tid < rows) ? static_cast<const float*>(a.D.ptr)[(d0 + tid) * a.D.s0] : 0.f;
    s_bias[tid] = (has_bias && tid < rows) ? static_cast<const float*>(a.delta_bias.ptr)[(d0 + tid) * a.delta_bias.s0]
                                           : 0.f;
  }

  const int64_t n_tiles = (L + kTB - 1) / kTB;

  // ---- fetch of raw tile `tile` (checkpoint rows into buffer `buf`).  As in
  // the forward, the synchronous form runs in the finish phase only.
  auto async_tile = [&](int64_t tile) __attribute__((always_inline)) {
    return async_ok && (L - tile * kTB) >= kTB && rows == CB && CB == kWave;
  };
  auto fetch_async = [&](int64_t tile, int buf) __attribute__((always_inline)) {
    const int64_t t0 = tile * kTB;
    tile_fetch_async<IT, kQ>(gu + t0, su, CB, s_raw_u, w, nW, lane);
    tile_fetch_async<IT, kQ>(gd + t0, sd, CB, s_raw_d, w, nW, lane);
    tile_fetch_async<IT, kQ>(gdo + t0, sdo, CB, s_raw_do, w, nW, lane);
    if (has_z) {
      tile_fetch_async<IT, kQ>(gz + t0, sz, CB, s_raw_z, w, nW, lane);
      tile_fetch_async<IT, kQ>(gos + t0, sos, CB, s_raw_os, w, nW, lane);
    }
    if constexpr (kDA) tile_fetch_async<IT, kQ>(gdA + t0, sdA, CB, s_raw_dA, w, nW, lane);
    if constexpr (kVarB) tile_fetch_async<IT, kQ>(gB + t0, sBn, Nb, s_raw_bc, w, nW, lane);
    if constexpr (kVarC) tile_fetch_async<IT, kQ>(gC + t0, sCn, Nb, s_raw_bc + kRawBC, w, nW, lane);
    if constexpr (kCkLds) {
      if (tile > 0)  // h at the tile start = checkpoint of interval tile - 1 (64 channels x Nb states)
        tile_fetch_async<float, kWave * 4 / 16>(gck + (tile - 1) * N * D, (uint32_t)D, Nb,
                                                 reinterpret_cast<char*>(s_ck + buf * kNPmax * kWave), w, nW, lane);
    }
  };
  auto fetch_sync = [&](int64_t tile, int buf) __attribute__((always_inline)) {
    const int64_t t0 = tile * kTB;
    const int nt = (int)((L - t0) < kTB ? (L - t0) : kTB);
    tile_fetch_sync<IT, kQ>(gu + t0, su, kWave, rows, nt, s_raw_u, tid, blockDim.x);
    tile_fetch_sync<IT, kQ>(gd + t0, sd, kWave, rows, nt, s_raw_d, tid, blockDim.x);
    tile_fetch_sync<IT, kQ>(gdo + t0, sdo, kWave, rows, nt, s_raw_do, tid, blockDim.x);
    if (has_z) {
      tile_fetch_sync<IT, kQ>(gz + t0, sz, kWave, rows, nt, s_raw_z, tid, blockDim.x);
      tile_fetch_sync<IT, kQ>(gos + t0, sos, kWave, rows, nt, s_raw_os, tid, blockDim.x);
    }
    if constexpr (kDA) tile_fetch_sync<IT, kQ>(gdA + t0, sdA, kWave, rows, nt, s_raw_dA, tid, blockDim.x);
    if constexpr (kVarB) tile_fetch_sync<IT, kQ>(gB + t0, sBn, NP, Nb, nt, s_raw_bc, tid, blockDim.x);
    if constexpr (kVarC) tile_fetch_sync<IT, kQ>(gC + t0, sCn, NP, Nb, nt, s_raw_bc + kRawBC, tid, blockDim.x);
    if constexpr (kCkLds) {
      if (tile > 0) {
        const float* src = gck + (tile - 1) * N * D;
        float* dst = s_ck + buf * kNPmax * kWave;
        for (int j = tid; j < Nb * kWave; j += blockDim.x) {
          const int n = j / kWave, c = j % kWave;
          dst[j] = c < rows ? src[(int64_t)n * D + c] : 0.f;
        }
      }
    }
  };

  // a tile whose kTB steps and 64 channels are all valid
  auto full_tile = [&](int64_t tile) __attribute__((always_inline)) {
    return (L - tile * kTB) >= kTB && rows == kWave;
  };

  // ---- raw tile -> fp32 operands of buffer `p`; dz is finished here
  auto convert = [&](auto full_tag, int64_t tile, int p) __attribute__((always_inline)) {
    constexpr bool kFull = decltype(full_tag)::value;
    const int64_t t0 = tile * kTB;
    const int nt = (int)((L - t0) < kTB ? (L - t0) : kTB);
    for (int j = tid; j < kWave * kQ; j += blockDim.x) {
      const int r = j / kQ, q = j % kQ;
      float vu[kEl], vd[kEl], vdo[kEl], vz[kEl], vo[kEl], vda[kEl], dzv[kEl];
      raw_to_f32<IT>(*reinterpret_cast<const uint4*>(s_raw_u + 16 * j), vu);
      raw_to_f32<IT>(*reinterpret_cast<const uint4*>(s_raw_d + 16 * j), vd);
      raw_to_f32<IT>(*reinterpret_cast<const uint4*>(s_raw_do + 16 * j), vdo);
      if constexpr (kDA) raw_to_f32<IT>(*reinterpret_cast<const uint4*>(s_raw_dA + 16 * j), vda);
      if (has_z) {
        raw_to_f32<IT>(*reinterpret_cast<const uint4*>(s_raw_z + 16 * j), vz);
        raw_to_f32<IT>(*reinterpret_cast<const uint4*>(s_raw_os + 16 * j), vo);
      }
      const float bias = s_bias[r];
#pragma unroll
      for (int i = 0; i < kEl; ++i) {
        const bool valid = kFull || (r < rows && q * kEl + i < nt);
        const float x = vd[i] + bias;
        const float dl = a.delta_softplus ? softplus_fast(x) : x;
        float dy = vdo[i];
        if (has_z) {
          const float sg = sigmoid_fast(vz[i]);
          dzv[i] = dy * vo[i] * sg * (1.f + vz[i] * (1.f - sg));
          dy = dy * vz[i] * sg;
        }
        vd[i] = valid ? dl : 0.f;
        vu[i] = valid ? vu[i] : 0.f;
        vdo[i] = valid ? dy : 0.f;
        if constexpr (kDA) vda[i] = valid ? vda[i] : 0.f;
      }
      const int n_ = kFull ? kEl : nt - q * kEl;
      if (has_z && blockIdx.z == 0 && (kFull || (r < rows && n_ > 0))) {   // one state block writes dz
        IT* pz = gdz + r * sdz + t0 + q * kEl;
        if ((kFull && out_al) || (n_ >= kEl && (reinterpret_cast<uintptr_t>(pz) & 15u) == 0))
          *reinterpret_cast<uint4*>(pz) = f32_to_raw<IT>(dzv);
        else
          for (int i = 0; i < (n_ < kEl ? n_ : kEl); ++i) pz[i] = from_f32<IT>(dzv[i]);
      }
      // step s = q * kEl + i goes to group s / 4, slot s % 4 of row r
#pragma unroll
      for (int i = 0; i < kEl; i += 4) {
        const int o = (((q * kEl + i) / 4) * kWave + r) * 4;
        lds_stv<4>(&s_dl[p][o], vd + i);
        lds_stv<4>(&s_u[p][o], vu + i);
        lds_stv<4>(&s_dy[p][o], vdo + i);
        if constexpr (kDA) lds_stv<4>(&s_dt[o], vda + i);
      }
    }
    if constexpr (kVarB || kVarC) {
      for (int j = tid; j < NP * kQ; j += blockDim.x) {
        const bool st_ok = j / kQ < Nb;  // padded states read B = C = 0
        float v[kEl];
        const int n = j / kQ, s0 = (j % kQ) * kEl;
        if constexpr (kVarB) {
          raw_to_f32<IT>(*reinterpret_cast<const uint4*>(s_raw_bc + 16 * j), v);
#pragma unroll
          for (int i = 0; i < kEl; ++i) s_B[(s0 + i) * kNPmax + n] = st_ok ? v[i] : 0.f;
        }
        if constexpr (kVarC) {
          raw_to_f32<IT>(*reinterpret_cast<const uint4*>(s_raw_bc + kRawBC + 16 * j), v);
#pragma unroll
          for (int i = 0; i < kEl; ++i) s_C[(s0 + i) * kNPmax + n] = st_ok ? v[i] : 0.f;
        }
      }
    }
  };

  // ---- epilogue of tile `tile` (fp32 buffer p): cross-wave sums -> du, ddelta,
  // ddeltaA; the per-element terms of dD (dy u) and ddelta_bias (ddelta) are
  // left in wave 0's partial slots
  auto epilogue = [&](auto full_tag, int64_t tile, int p) __attribute__((always_inline)) {
    constexpr bool kFull = decltype(full_tag)::value;
    const int64_t t0 = tile * kTB;
    const int nt = (int)((L - t0) < kTB ? (L - t0) : kTB);
    for (int j = tid; j < kWave * kQ; j += blockDim.x) {
      const int r = j / kQ, q = j % kQ;
      const float Dv = s_Dv[r];
      float vdu[kEl], vdd[kEl], vda[kEl];
#pragma unroll
      for (int i = 0; i < kEl; i += 4) {
        const int g = (q * kEl + i) / 4;
        const int o = (g * kWave + r) * 4;
        float P1[4], P2[4], P3[4] = {0.f, 0.f, 0.f, 0.f}, x[4];
        lds_ldv<4>(&s_P1[o], P1);
        lds_ldv<4>(&s_P2[o], P2);
        if constexpr (kP3) lds_ldv<4>(&s_P3[o], P3);
        for (int ww = 1; ww < nW; ++ww) {
          const int ow = ((ww * kG + g) * kWave + r) * 4;
          lds_ldv<4>(&s_P1[ow], x);
#pragma unroll
          for (int m = 0; m < 4; ++m) P1[m] += x[m];
          lds_ldv<4>(&s_P2[ow], x);
#pragma unroll
          for (int m = 0; m < 4; ++m) P2[m] += x[m];
          if constexpr (kP3) {
            lds_ldv<4>(&s_P3[ow], x);
#pragma unroll
            for (int m = 0; m < 4; ++m) P3[m] += x[m];
          }
        }
        if (gpp) {  // state block: its sums of the terms, fp32 (the combine kernel finishes them)
          if (!kFull && (r >= rows || q * kEl + i >= nt)) continue;
          float* pp = gpp + r * L + t0 + q * kEl + i;
          const int nv = kFull ? 4 : (nt - (q * kEl + i) < 4 ? nt - (q * kEl + i) : 4);
          auto put4 = [&](float* dst, const float* v) __attribute__((always_inline)) {
            if (nv == 4 && (L & 3) == 0) *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
            else for (int m = 0; m < nv; ++m) dst[m] = v[m];
          };
          put4(pp, P1);
          put4(pp + pp_term, P2);
          if constexpr (kP3) put4(pp + 2 * pp_term, P3);
          continue;
        }
        float dlv[4], uv[4], dyv[4], q1[4], q2[4];
        lds_ldv<4>(&s_dl[p][o], dlv);
        lds_ldv<4>(&s_u[p][o], uv);
        lds_ldv<4>(&s_dy[p][o], dyv);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          float ddl;
          if constexpr (kMethod == LRNNX_MAMBA) {
            vdu[i + m] = fmaf(dlv[m], P1[m], Dv * dyv[m]);
            ddl = uv[m] * P1[m];
          } else {
            vdu[i + m] = fmaf(Dv, dyv[m], P1[m]);
            ddl = P3[m];
          }
          if constexpr (kDA) {
            vda[i + m] = P2[m];
          } else {
            ddl += P2[m];
            vda[i + m] = 0.f;
          }
          // d softplus(x)/dx = sigmoid(x) = 1 - exp(-softplus(x))
          const float dd = a.delta_softplus ? ddl * one_minus_exp_neg(dlv[m]) : ddl;
          vdd[i + m] = dd;
          q1[m] = dyv[m] * uv[m];
          q2[m] = dd;
        }
        lds_stv<4>(&s_P1[o], q1);
        lds_stv<4>(&s_P2[o], q2);
      }
      if (gpp) continue;
      const int n_ = kFull ? kEl : nt - q * kEl;
      if (!kFull && (r >= rows || n_ <= 0)) continue;
      auto put = [&](IT* pp, const float* v) __attribute__((always_inline)) {
        if ((kFull && out_al) || (n_ >= kEl && (reinterpret_cast<uintptr_t>(pp) & 15u) == 0))
          *reinterpret_cast<uint4*>(pp) = f32_to_raw<IT>(v);
        else
          for (int i = 0; i < (n_ < kEl ? n_ : kEl); ++i) pp[i] = from_f32<IT>(v[i]);
      };
      put(gdu + r * sdu + t0 + q * kEl, vdu);
      put(gddl + r * sddl + t0 + q * kEl, vdd);
      if (has_dA_in) put(gddA + r * sddA + t0 + q * kEl, vda);
    }
  };

  // ---- one checkpoint interval: steps [ts, ts + Ls) of tile `tile` (fp32 buffer p).
  // kFull: Ls == kCk, no per-step guards.  Steps past Ls hold zero operands
  // and are skipped; their partial slots are written as zero.
  auto sub_chunk = [&](auto full_tag, int64_t tile, int p, int ts, int Ls) __attribute__((always_inline)) {
    constexpr bool kFull = decltype(full_tag)::value;
    const int64_t kk = (tile * kTB + ts) / kCk;  // global checkpoint interval
    float h0[kS];
#pragma unroll
    for (int k = 0; k < kS; ++k) {
      if constexpr (kCkLds) {
        h0[k] = (kk > 0 && n0 + k < Nb) ? s_ck[(p * kNPmax + n0 + k) * kWave + lane] : 0.f;
      } else {
        h0[k] = (kk > 0 && lane_ok && n0 + k < Nb) ? ckp[((b * n_ck + kk - 1) * N + nb + n0 + k) * D + d] : 0.f;
      }
    }
    // recompute h (and, where kAbLive, A_bar) over the interval.  Otherwise
    // the reverse walk re-derives A_bar (zoh, bilinear and rglru recompute
    // the same discretisation there for their input-term gradients anyway);
    // keeping it live as well would take kS * kCk more VGPRs and spill.
    float Ab[kAbLive ? kCk : 1][kS], H[kCk][kS];
    {
      float hc[kS];
#pragma unroll
      for (int k = 0; k < kS; ++k) hc[k] = h0[k];
#pragma unroll
      for (int jg = 0; jg < kCk; jg += kV) {
        kSchedFence();
        const int t = ts + jg;
        const int o = ((t >> 2) * kWave + lane) * 4 + (t & 3);
        float dlv[kV], uvv[kV], dtv[kV];
        lds_ldv<kV>(&s_dl[p][o], dlv);
        lds_ldv<kV>(&s_u[p][o], uvv);
        if constexpr (kDA) lds_ldv<kV>(&s_dt[o], dtv);
#pragma unroll
        for (int i = 0; i < kV; ++i) {
          const int j = jg + i;
          if (kFull || j < Ls) {
            const float dt = kDA ? dtv[i] : dlv[i];
            const float du_ = dlv[i] * uvv[i];
            float bv[kS];
            if constexpr (kVarB) lds_states<kS>(&s_B[(t + i) * kNPmax + n0], bv);
#pragma unroll
            for (int k = 0; k < kS; ++k) {
              float beta;
              const float ab = disc_real<kMethod, kDA>(dt, dlv[i], a2[k], Araw[k], invA[k], beta);
              const float bin = kVarB ? bv[k] : 1.f;
              float inc;
              if constexpr (kMethod == LRNNX_MAMBA) inc = du_ * bin;
              else if constexpr (uses_B_input<kMethod>()) inc = beta * uvv[i] * bin;
              else inc = beta * uvv[i];
              hc[k] = fmaf(ab, hc[k], inc);
              if constexpr (kAbLive) Ab[j][k] = ab;
              H[j][k] = hc[k];
            }
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
    for (int jg = kCk - kV; jg >= 0; jg -= kV) {
      kSchedFence();
      const int t = ts + jg;
      const int o = ((t >> 2) * kWave + lane) * 4 + (t & 3);
      float dlv[kV], uvv[kV], dtv[kV], dyv[kV];
      float p1v[kV], p2v[kV], p3v[kV];
      lds_ldv<kV>(&s_dl[p][o], dlv);
      lds_ldv<kV>(&s_u[p][o], uvv);
      lds_ldv<kV>(&s_dy[p][o], dyv);
      if constexpr (kDA) lds_ldv<kV>(&s_dt[o], dtv);
#pragma unroll
      for (int i = kV - 1; i >= 0; --i) {
        const int j = jg + i;
        p1v[i] = 0.f; p2v[i] = 0.f; p3v[i] = 0.f;
        if (kFull || j < Ls) {
          const float dl = dlv[i], uu = uvv[i], dt = kDA ? dtv[i] : dlv[i], dy = dyv[i];
          const float du_ = dl * uu;
          float p1 = 0.f, p2 = 0.f, p3 = 0.f;
          float vB[kS], vC[kS], bv[kS], cv[kS];
          if constexpr (kVarB) lds_states<kS>(&s_B[(t + i) * kNPmax + n0], bv);
          if constexpr (kVarC) lds_states<kS>(&s_C[(t + i) * kNPmax + n0], cv);
#pragma unroll
          for (int k = 0; k < kS; ++k) {
            // effective output weight: (C_t or C_const) * (B_const when B is constant)
            float cvar = 0.f, cc = cout_c[k];
            if constexpr (kVarC) {
              cvar = cv[k];
              cc = kVarB ? cvar : cvar * cout_c[k];
            }
            const float bin = kVarB ? bv[k] : 1.f;
            dh[k] = fmaf(dy, cc, gn[k]);
            float beta_r = 0.f;  // input factor of this step (methods that re-derive A_bar)
            float ab;
            if constexpr (kAbLive) ab = Ab[j][k];
            else ab = disc_real<kMethod, kDA>(dt, dl, a2[k], Araw[k], invA[k], beta_r);
            const float hp = j > 0 ? H[j - 1][k] : h0[k];
            const float hcur = H[j][k];
            const float gk = ab * dh[k];  // carried to step t-1
            gn[k] = gk;
            float rA = 0.f;  // bilinear: 1 / (1 - dtA A / 2)
            // through A_bar: dh * hp * dA_bar/d(.)
            if constexpr (kMethod == LRNNX_MAMBA || kMethod == LRNNX_DIRAC || kMethod == LRNNX_ZOH) {
              const float wv = gk * hp;
              p2 = fmaf(wv, Araw[k], p2);
              dA_acc[k] = fmaf(wv, dt, dA_acc[k]);
            } else if constexpr (kMethod == LRNNX_BILINEAR) {
              // dA_bar/d(dtA A) = 1 / (1 - dtA A / 2)^2
              rA = __builtin_amdgcn_rcpf(1.f - 0.5f * dt * Araw[k]);
              const float qv = dh[k] * hp * (rA * rA);
              p2 = fmaf(qv, Araw[k], p2);
              dA_acc[k] = fmaf(qv, dt, dA_acc[k]);
            } else if constexpr (kMethod == LRNNX_S7) {
              const float r = __builtin_amdgcn_rcpf(fmaf(dl, dl, 0.5f));
              p2 = fmaf(dh[k] * hp, 2.f * dl * (r * r), p2);
            } else {  // RGLRU: dA_bar/ddelta = A_bar ln A, dA_bar/dA = delta A_bar / A
              const float wv = gk * hp;
              const float lnA = a2[k] * kLn2;
              p2 = fmaf(wv, lnA, p2);
              dA_acc[k] = fmaf(wv, dl * invA[k], dA_acc[k]);
            }
            // through the input term
            if constexpr (kMethod == LRNNX_MAMBA) {
              p1 = fmaf(dh[k], bin, p1);  // du = delta' p1, ddelta' += u p1
              if constexpr (kVarB) vB[k] = dh[k] * du_;
            } else if constexpr (kMethod == LRNNX_DIRAC || kMethod == LRNNX_S7) {
              p1 = fmaf(dh[k], bin, p1);
              if constexpr (kVarB) vB[k] = dh[k] * uu;
            } else if constexpr (kMethod == LRNNX_ZOH) {
              // beta = expm1(delta' A) / A; without deltaA, exp(delta' A) is A_bar
              const float e1 = kDA ? fast_exp2(dl * a2[k]) : ab;
              const float beta = beta_r;
              const float g = dh[k] * bin;
              p1 = fmaf(g, beta, p1);
              p3 = fmaf(g * uu, e1, p3);
              dA_acc[k] = fmaf(g * uu, (dl * e1 - beta) * invA[k], dA_acc[k]);
              if constexpr (kVarB) vB[k] = dh[k] * beta * uu;
            } else if constexpr (kMethod == LRNNX_BILINEAR) {
              // beta = delta' / (1 - delta' A / 2); without deltaA the same reciprocal as A_bar's
              const float inv = kDA ? __builtin_amdgcn_rcpf(1.f - 0.5f * dl * Araw[k]) : rA;
              const float beta = dl * inv;
              const float g = dh[k] * bin;
              p1 = fmaf(g, beta, p1);
              p3 = fmaf(g * uu, inv * inv, p3);
              dA_acc[k] = fmaf(g * uu, 0.5f * dl * dl * inv * inv, dA_acc[k]);
              if constexpr (kVarB) vB[k] = dh[k] * beta * uu;
            } else {  // RGLRU: beta = sqrt(1 - ab^2), B unused on the input side
              const float beta = beta_r;
              const float g = dh[k];
              p1 = fmaf(g, beta, p1);
              const float dbeta_dab = -ab * __builtin_amdgcn_rcpf(beta);
              const float lnA = a2[k] * kLn2;
              p3 = fmaf(g * uu * dbeta_dab, ab * lnA, p3);
              dA_acc[k] = fmaf(g * uu * dbeta_dab, ab * dl * invA[k], dA_acc[k]);
              if constexpr (kVarB) vB[k] = 0.f;
            }
            // output side: y = sum_n cout h  (cout = C * B_const)
            const float dyh = dy * hcur;
            if constexpr (kVarC) vC[k] = kVarB ? dyh : dyh * bcst[k];
            if constexpr (!kVarB) dBc_acc[k] = fmaf(dyh, kVarC ? cvar : ccst[k], dBc_acc[k]);
            if constexpr (!kVarC) dCc_acc[k] = fmaf(dyh, kVarB ? 1.f : bcst[k], dCc_acc[k]);
          }
          p1v[i] = p1; p2v[i] = p2; p3v[i] = p3;
          // lanes past the last channel hold zero operands (convert) and a zero
          // checkpoint, so their dh and h, hence vB and vC, are exactly zero
          if constexpr (kVarB || kVarC) {
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
        // keep the per-lane accumulations at their step: only their final
        // values are read after the walk, and sinking the chains there keeps
        // every step's operands live across the walk (spills past 256 VGPRs)
#pragma unroll
        for (int k = 0; k < kS; ++k) {
          pin_vgpr(dA_acc[k]);
          if constexpr (!kVarB) pin_vgpr(dBc_acc[k]);
          if constexpr (!kVarC) pin_vgpr(dCc_acc[k]);
        }
      }
      const int op = ((w * kG + (t >> 2)) * kWave + lane) * 4 + (t & 3);
      lds_stv<kV>(&s_P1[op], p1v);
      lds_stv<kV>(&s_P2[op], p2v);
      if constexpr (kP3) lds_stv<kV>(&s_P3[op], p3v);
    }
    // dB / dC over the wave's channels -> one partial per (cb, b, n, t)
    if constexpr (kVarB || kVarC) {
      const int kq = lane / kCk, jq = lane % kCk;  // lane now owns index v = k * kCk + j
      const bool wr = lane < kNV && n0 + kq < Nb && (kFull || jq < Ls);
      const int64_t tg = tile * kTB + ts + jq;
      if constexpr (kVarB) {
        float r;
        if constexpr (kS >= 4) {
          rs_tail16(accB, lane);
          r = accB[0];
        } else {
          float r64[64];
#pragma unroll
          for (int i = 0; i < 64; ++i) r64[i] = i < kNV ? accB[i] : 0.f;
          r = reduce_scatter64(r64, lane);
        }
        if (wr) ws[wo.dBv + ((cb * a.batch + b) * N + nb + n0 + kq) * L + tg] = r;
      }
      if constexpr (kVarC) {
        float r;
        if constexpr (kS >= 4) {
          rs_tail16(accC, lane);
          r = accC[0];
        } else {
          float r64[64];
#pragma unroll
          for (int i = 0; i < 64; ++i) r64[i] = i < kNV ? accC[i] : 0.f;
          r = reduce_scatter64(r64, lane);
        }
        if (wr) ws[wo.dCv + ((cb * a.batch + b) * N + nb + n0 + kq) * L + tg] = r;
      }
    }
  };

  // ---- prologue: last tile
  {
    const int64_t tl = n_tiles - 1;
    if (async_tile(tl)) fetch_async(tl, (int)(tl & 1));
    else fetch_sync(tl, (int)(tl & 1));
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    if (full_tile(tl)) convert(std::true_type{}, tl, (int)(tl & 1));
    else convert(std::false_type{}, tl, (int)(tl & 1));
    __syncthreads();
  }
  for (int64_t tile = n_tiles - 1; tile >= 0; --tile) {
    const int p = (int)(tile & 1);
    const int64_t t0 = tile * kTB;
    const int Tv = (int)((L - t0) < kTB ? (L - t0) : kTB);
    const bool prev = tile > 0;
    const bool prev_async = prev && async_tile(tile - 1);
    if (prev_async) fetch_async(tile - 1, p ^ 1);

    // ---- compute(tile): checkpoint intervals, last first
    if (Tv == kTB) {
      // 8-wave workgroups keep one copy of the interval body (unrolled per interval, the
      // 16-step tiles double the compile time for no measured gain); the 4-wave ones unroll
      // (2 % faster at d_state 24)
      if constexpr (kNWm <= 4) {
#pragma unroll
        for (int s = kTB / kCk - 1; s >= 0; --s) sub_chunk(std::true_type{}, tile, p, s * kCk, kCk);
      } else {
#pragma unroll 1
        for (int s = kTB / kCk - 1; s >= 0; --s) sub_chunk(std::true_type{}, tile, p, s * kCk, kCk);
      }
    } else {
      for (int s = (Tv + kCk - 1) / kCk - 1; s >= 0; --s) {
        const int ts = s * kCk;
        sub_chunk(std::false_type{}, tile, p, ts, (Tv - ts) < kCk ? (Tv - ts) : kCk);
      }
    }

    // ---- finish(tile): tile-1 in LDS, epilogue(tile), convert(tile-1)
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    if (prev && !prev_async) {
      fetch_sync(tile - 1, p ^ 1);
      __syncthreads();
    }
    if (full_tile(tile)) epilogue(std::true_type{}, tile, p);
    else epilogue(std::false_type{}, tile, p);
    if (prev) {
      if (full_tile(tile - 1)) convert(std::true_type{}, tile - 1, p ^ 1);
      else convert(std::false_type{}, tile - 1, p ^ 1);
    }
    __syncthreads();
    if (w == 0 && !gpp) {  // dD / ddelta_bias terms of this tile, in step order
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        float q1[4], q2[4];
        lds_ldv<4>(&s_P1[(g * kWave + lane) * 4], q1);
        lds_ldv<4>(&s_P2[(g * kWave + lane) * 4], q2);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          if (4 * g + m < Tv) {
            dD_acc += q1[m];
            dbias_acc += q2[m];
          }
        }
      }
    }
  }

  // per-(b, d, n) and per-(b, d) partials; summed over b by ss_reduce_batch_kernel
#pragma unroll
  for (int k = 0; k < kS; ++k) {
    if (lane_ok && n0 + k < Nb) {
      const int64_t o = (b * D + d) * N + nb + n0 + k;
      ws[wo.dA + o] = dA_acc[k];
      if constexpr (!kVarB) ws[wo.dBc + o] = dBc_acc[k];
      if constexpr (!kVarC) ws[wo.dCc + o] = dCc_acc[k];
    }
  }
  if (w == 0 && lane_ok && !gpp) {
    ws[wo.dD + b * D + d] = dD_acc;
    ws[wo.dbias + b * D + d] = dbias_acc;
  }
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

// Vector form of ss_reduce_bc_kernel for dB and dC in one launch (blockIdx.z
// selects the quantity): each thread sums 4 consecutive steps with 16-byte
// loads, the channel blocks in the same fixed order.  Needs L % 4 == 0 and
// output rows aligned to 4 elements (checked by the caller).
template <typename OT>
__global__ void __launch_bounds__(256)
ss_reduce_bc4_kernel(const float* __restrict__ part_b, const float* __restrict__ part_c, lrnnx_view out_b,
                     lrnnx_view out_c, int64_t B, int64_t G, int64_t N, int64_t L, int64_t ncpg) {
  const int64_t t = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
  const int64_t row = blockIdx.y;  // (b, g, n)
  if (t >= L) return;
  const bool isC = blockIdx.z != 0;
  const float* part = isC ? part_c : part_b;
  const lrnnx_view out = isC ? out_c : out_b;
  const int64_t n = row % N, g = (row / N) % G, b = row / (N * G);
  const int64_t step = B * N * L;  // between consecutive channel blocks
  const float* p = part + ((g * ncpg * B + b) * N + n) * L + t;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
  for (int64_t j = 0; j < ncpg; ++j) {
    const float4 v = *reinterpret_cast<const float4*>(p + j * step);
    acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
  }
  const float r[4] = {acc.x, acc.y, acc.z, acc.w};
  store4<OT>(static_cast<OT*>(out.ptr) + b * out.s0 + g * out.s1 + n * out.s2 + t, r);
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

template <typename IT, bool kVarB, bool kVarC>
static hipError_t ss_bwd_reductions(const lrnnx_selective_scan_args& a, const SSGeom& g, float* ws,
                                    const SSBwdWs& wo, hipStream_t st, bool batch_only = false);

// State blocks: du, ddelta, ddeltaA from the blocks' term sums (added in block
// order), by the formulas of ss_bwd_kernel's epilogue, and the per-(b, d) dD
// (sum of dy u) and ddelta_bias (sum of ddelta) terms for ss_bwd_reductions.
// One wave per (b, d) row, lanes along L; the lane sums are added across the
// wave in a fixed order.
template <typename IT>
__global__ void __launch_bounds__(256)
ss_bwd_combine_kernel(const lrnnx_selective_scan_args a, float* __restrict__ ws, const SSBwdWs wo, const int nsb) {
  const int64_t L = a.seqlen, D = a.dim, BD = a.batch * a.dim;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t r = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;   // b * D + d
  if (r >= BD) return;
  const int64_t b = r / D, d = r % D;
  const bool mamba = a.method == LRNNX_MAMBA;
  const bool p3 = wo.n_terms == 3;
  const bool has_dA = a.deltaA.ptr != nullptr;
  const bool dA_on = has_dA && a.method != LRNNX_S7 && a.method != LRNNX_RGLRU;   // deltaA drives A_bar
  const bool has_z = a.z.ptr != nullptr;
  const float Dv = a.D.ptr ? static_cast<const float*>(a.D.ptr)[d * a.D.s0] : 0.f;
  const float bias = a.delta_bias.ptr ? static_cast<const float*>(a.delta_bias.ptr)[d * a.delta_bias.s0] : 0.f;
  const IT* pu = static_cast<const IT*>(a.u.ptr) + b * a.u.s0 + d * a.u.s1;
  const IT* pd = static_cast<const IT*>(a.delta.ptr) + b * a.delta.s0 + d * a.delta.s1;
  const IT* pdo = static_cast<const IT*>(a.dout.ptr) + b * a.dout.s0 + d * a.dout.s1;
  const IT* pz = has_z ? static_cast<const IT*>(a.z.ptr) + b * a.z.s0 + d * a.z.s1 : nullptr;
  IT* pdu = static_cast<IT*>(a.du.ptr) + b * a.du.s0 + d * a.du.s1;
  IT* pddl = static_cast<IT*>(a.ddelta.ptr) + b * a.ddelta.s0 + d * a.ddelta.s1;
  IT* pddA = has_dA ? static_cast<IT*>(a.ddeltaA.ptr) + b * a.ddeltaA.s0 + d * a.ddeltaA.s1 : nullptr;
  const float* pp = ws + wo.pp + r * L;
  const int64_t term = BD * L, blk = wo.n_terms * term;
  float dD = 0.f, dbias = 0.f;
  for (int64_t t = lane; t < L; t += kWave) {
    float P1 = 0.f, P2 = 0.f, P3 = 0.f;
    for (int z = 0; z < nsb; ++z) {
      P1 += pp[z * blk + t];
      P2 += pp[z * blk + term + t];
      if (p3) P3 += pp[z * blk + 2 * term + t];
    }
    const float x = to_f32(pd[t]) + bias;
    const float dl = a.delta_softplus ? softplus_fast(x) : x;
    const float uu = to_f32(pu[t]);
    float dy = to_f32(pdo[t]);
    if (has_z) {
      const float zv = to_f32(pz[t]);
      dy = dy * zv * sigmoid_fast(zv);
    }
    float du, ddl;
    if (mamba) {
      du = fmaf(dl, P1, Dv * dy);
      ddl = uu * P1;
    } else {
      du = fmaf(Dv, dy, P1);
      ddl = P3;
    }
    if (!dA_on) ddl += P2;
    const float dd = a.delta_softplus ? ddl * one_minus_exp_neg(dl) : ddl;
    pdu[t] = from_f32<IT>(du);
    pddl[t] = from_f32<IT>(dd);
    if (has_dA) pddA[t] = from_f32<IT>(dA_on ? P2 : 0.f);
    dD = fmaf(dy, uu, dD);
    dbias += dd;
  }
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) {
    dD += __shfl_xor(dD, m);
    dbias += __shfl_xor(dbias, m);
  }
  if (lane == 0) {
    ws[wo.dD + r] = dD;
    ws[wo.dbias + r] = dbias;
  }
}

template <typename IT, int kS, int kMethod, bool kVarB, bool kVarC, bool kDA, int kNWm>
static hipError_t launch_bwd_t(const lrnnx_selective_scan_args& a, const SSGeom& g, float* ws, const SSBwdWs& wo,
                               const float* ckp, hipStream_t st) {
  dim3 grid(g.n_cb, (unsigned)a.batch, (unsigned)g.nsb);
  dim3 block(g.nW * kWave);
  if (g.nW > kNWm) return hipErrorInvalidConfiguration;
  // async LDS fetches need 16-byte aligned row starts for every fetched tensor
  auto al = [](const void* p, int64_t s_batch, int64_t s_row) {
    return p == nullptr || ((reinterpret_cast<uintptr_t>(p) & 15u) == 0 && ((s_batch * sizeof(IT)) & 15) == 0 &&
                            ((s_row * sizeof(IT)) & 15) == 0);
  };
  const bool has_z = a.z.ptr != nullptr;
  const bool in_ok = al(a.u.ptr, a.u.s0, a.u.s1) && al(a.delta.ptr, a.delta.s0, a.delta.s1) &&
                     al(a.dout.ptr, a.dout.s0, a.dout.s1) && (!has_z || al(a.z.ptr, a.z.s0, a.z.s1)) &&
                     (!has_z || al(a.out_saved.ptr, a.out_saved.s0, a.out_saved.s1)) &&
                     (!kDA || al(a.deltaA.ptr, a.deltaA.s0, a.deltaA.s1)) &&
                     (!kVarB || (al(a.B.ptr, a.B.s0, a.B.s2) && ((a.B.s1 * sizeof(IT)) & 15) == 0)) &&
                     (!kVarC || (al(a.C.ptr, a.C.s0, a.C.s2) && ((a.C.s1 * sizeof(IT)) & 15) == 0)) &&
                     (reinterpret_cast<uintptr_t>(ckp) & 15u) == 0 && (a.dim % 4) == 0;
  const bool out_ok = al(a.du.ptr, a.du.s0, a.du.s1) && al(a.ddelta.ptr, a.ddelta.s0, a.ddelta.s1) &&
                      al(a.ddeltaA.ptr, a.ddeltaA.s0, a.ddeltaA.s1) && (!has_z || al(a.dz.ptr, a.dz.s0, a.dz.s1));
  const int flags = (in_ok ? kFlagAsyncIn : 0) | (out_ok ? kFlagAlignedOut : 0);
  hipLaunchKernelGGL((ss_bwd_kernel<IT, kS, kMethod, kVarB, kVarC, kDA, kNWm>), grid, block, 0, st, a, g.CB, g.n_ck, ws,
                     wo, ckp, flags, g.nsb);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (g.nsb > 1) {
    const int64_t rows = a.batch * a.dim;
    hipLaunchKernelGGL(ss_bwd_combine_kernel<IT>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, a, ws, wo,
                       g.nsb);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return ss_bwd_reductions<IT, kVarB, kVarC>(a, g, ws, wo, st);
}

// Second-stage reductions of the backward: dB / dC partials over channel
// blocks (variable B / C), dA, constant dB / dC, dD, ddelta_bias over the batch.
template <typename IT, bool kVarB, bool kVarC>
static hipError_t ss_bwd_reductions(const lrnnx_selective_scan_args& a, const SSGeom& g, float* ws,
                                    const SSBwdWs& wo, hipStream_t st, bool batch_only) {
  const int64_t B = a.batch, D = a.dim, N = a.dstate, L = a.seqlen, G = a.n_groups;
  if constexpr (kVarB && kVarC) {
    auto al4 = [](const lrnnx_view& v) {
      const int64_t s = sizeof(IT);
      return (reinterpret_cast<uintptr_t>(v.ptr) % (4 * s)) == 0 && v.s0 % 4 == 0 && v.s1 % 4 == 0 && v.s2 % 4 == 0;
    };
    if (L % 4 == 0 && al4(a.dB) && al4(a.dC)) {
      const int64_t ncpg = g.n_cb / G;
      dim3 rg((unsigned)((L / 4 + 255) / 256), (unsigned)(B * G * N), 2);
      hipLaunchKernelGGL(ss_reduce_bc4_kernel<IT>, rg, dim3(256), 0, st, ws + wo.dBv, ws + wo.dCv, a.dB, a.dC, B, G,
                         N, L, ncpg);
      return ss_bwd_reductions<IT, false, false>(a, g, ws, wo, st, /*batch_only=*/true);
    }
  }
  if constexpr (kVarB || kVarC) {
    const int64_t ncpg = g.n_cb / G;
    dim3 rg((unsigned)((L + 255) / 256), (unsigned)(B * G * N));
    if constexpr (kVarB)
      hipLaunchKernelGGL(ss_reduce_bc_kernel<IT>, rg, dim3(256), 0, st, ws + wo.dBv, a.dB, B, G, N, L, ncpg);
    if constexpr (kVarC)
      hipLaunchKernelGGL(ss_reduce_bc_kernel<IT>, rg, dim3(256), 0, st, ws + wo.dCv, a.dC, B, G, N, L, ncpg);
  }
  const unsigned gdn = (unsigned)((D * N + 255) / 256), gd = (unsigned)((D + 255) / 256);
  hipLaunchKernelGGL(ss_reduce_batch_kernel<float>, dim3(gdn), dim3(256), 0, st, ws + wo.dA, a.dA, B * wo.S, D, N);
  if (!kVarB && !batch_only)
    hipLaunchKernelGGL(ss_reduce_batch_kernel<float>, dim3(gdn), dim3(256), 0, st, ws + wo.dBc, a.dB, B * wo.S, D, N);
  if (!kVarC && !batch_only)
    hipLaunchKernelGGL(ss_reduce_batch_kernel<float>, dim3(gdn), dim3(256), 0, st, ws + wo.dCc, a.dC, B * wo.S, D, N);
  if (a.dD.ptr) {
    lrnnx_view v = a.dD;
    v.s1 = 0;
    hipLaunchKernelGGL(ss_reduce_batch_kernel<float>, dim3(gd), dim3(256), 0, st, ws + wo.dD, v, B * wo.S, D, (int64_t)1);
  }
  if (a.ddelta_bias.ptr) {
    lrnnx_view v = a.ddelta_bias;
    v.s1 = 0;
    hipLaunchKernelGGL(ss_reduce_batch_kernel<float>, dim3(gd), dim3(256), 0, st, ws + wo.dbias, v, B * wo.S, D, (int64_t)1);
  }
  return hipGetLastError();
}

template <typename IT, int kS, int kMethod, bool kVarB, bool kVarC, int kNWm>
static hipError_t launch_bwd_da(const lrnnx_selective_scan_args& a, const SSGeom& g, float* ws, const SSBwdWs& wo,
                                const float* ckp, hipStream_t st) {
  if constexpr (uses_deltaA<kMethod>()) {
    if (a.deltaA.ptr != nullptr) return launch_bwd_t<IT, kS, kMethod, kVarB, kVarC, true, kNWm>(a, g, ws, wo, ckp, st);
  }
  return launch_bwd_t<IT, kS, kMethod, kVarB, kVarC, false, kNWm>(a, g, ws, wo, ckp, st);
}

template <typename IT, int kS, int kMethod, int kNWm = fwd_nw_max(kS)>
static hipError_t launch_bwd_bc(const lrnnx_selective_scan_args& a, const SSGeom& g, float* ws, const SSBwdWs& wo,
                                const float* ckp, hipStream_t st) {
  if (a.var_B && a.var_C) return launch_bwd_da<IT, kS, kMethod, true, true, kNWm>(a, g, ws, wo, ckp, st);
  if (a.var_B) return launch_bwd_da<IT, kS, kMethod, true, false, kNWm>(a, g, ws, wo, ckp, st);
  if (a.var_C) return launch_bwd_da<IT, kS, kMethod, false, true, kNWm>(a, g, ws, wo, ckp, st);
  return launch_bwd_da<IT, kS, kMethod, false, false, kNWm>(a, g, ws, wo, ckp, st);
}

template <typename IT, int kMethod>
static hipError_t launch_bwd_s(const lrnnx_selective_scan_args& a, const SSGeom& g, float* ws, const SSBwdWs& wo,
                               const float* ckp, hipStream_t st) {
  switch (g.kS) {
    case 1: return launch_bwd_bc<IT, 1, kMethod>(a, g, ws, wo, ckp, st);
    case 4: return launch_bwd_bc<IT, 4, kMethod>(a, g, ws, wo, ckp, st);
    case 8:   // d_state 17..32: at most 4 waves, half the LDS (as in the forward)
      return g.nW <= 4 ? launch_bwd_bc<IT, 8, kMethod, 4>(a, g, ws, wo, ckp, st)
                       : launch_bwd_bc<IT, 8, kMethod>(a, g, ws, wo, ckp, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace lrnnx
