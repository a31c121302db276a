// Selective scan forward (real weights), gfx950.
//
// Semantics: reference kernel csrc/selective_scan/selective_scan.cuh:73-382
// (per (b, d): delta' = softplus(delta + bias); h_t = A_bar h_{t-1} + beta B u;
// y = sum_n C h (+ D u); out_z = y * silu(z); chunk carries x every 2048 steps).
//
// Work decomposition (ss_common.h): one workgroup = one batch row and CB <= 64
// channels of one B/C group; lane = channel; wave w owns kS states and keeps
// their fp32 h in VGPRs; L is walked in tiles of kT steps.
//
// Per tile k the workgroup runs two phases separated by barriers:
//   compute(k)  issue the asynchronous LDS fetch of raw tile k+1 (u, delta,
//               z, deltaA, B/C rows; tile_io.h), then walk the kT steps of
//               tile k for the wave's kS states and write per-wave partial
//               sums of y to LDS;
//   finish(k)   wait for the fetch, barrier; epilogue of tile k (sum of the
//               wave partials + D u, out and out_z = out silu(z), written as
//               16-byte stores) and conversion of raw tile k+1 into the fp32
//               operands of compute(k+1): delta' = softplus(delta + bias),
//               delta' u, B and C.
// So the HBM fetch of the next tile overlaps the arithmetic of the current
// one and every per-element transcendental outside the recurrence (softplus,
// silu) is computed once per element, not once per state.
#pragma once
#include <type_traits>

#include "ss_common.h"
#include "tile_io.h"

namespace lrnnx {

// tile length: 64 bytes of each input row (4 x 16-byte blocks), fewer steps
// when the state rows of B/C would not fit LDS
template <typename IT, int kS>
__host__ __device__ constexpr int fwd_tile() {
  return (int)(64 / sizeof(IT)) < tf_for(kS) ? (int)(64 / sizeof(IT)) : tf_for(kS);
}

// most waves a workgroup can have for a given kS (ceil(256 / kS) capped at 8)
__host__ __device__ constexpr int fwd_nw_max(int kS) { return (kS == 8 || kS == 32) ? 8 : 4; }

// ypart: with state blocks (grid z > 1) and outputs, the block's partial y
// (sum over its states of C h, fp32, [block][b][d][L]) instead of out / out_z.
// kNWm: most waves of a launch (LDS is sized for it; fewer waves than
// fwd_nw_max(kS) halve it for d_state 17..32).
template <typename IT, int kS, int kMethod, bool kVarB, bool kVarC, bool kDA, int kNWm = fwd_nw_max(kS)>
__global__ void __launch_bounds__(512)
ss_fwd_kernel(const lrnnx_selective_scan_args a, const int CB, const int64_t n_ck, const int flags,
              float* __restrict__ ypart) {
  constexpr int kCk = ck_for(kS);
  // fp32 8-wave workgroups (one per CU) of the exp-family methods without deltaA have the LDS
  // for 32-step tiles: fewer barriers per step (bilinear and rglru would spill more)
  constexpr int kT = (sizeof(IT) == 4 && kS == 8 && kNWm == 8 && !kDA && exp_family<kMethod>()) ? 32 : fwd_tile<IT, kS>();
  constexpr int kEl = 16 / sizeof(IT);   // elements per 16-byte block
  constexpr int kQ = kT / kEl;           // blocks per row
  constexpr int kG = kT / 4;             // groups of 4 steps
  static_assert(kT % kCk == 0 || kCk % kT == 0, "tile / checkpoint interval mismatch");
  constexpr int kNWmax = kNWm;
  constexpr int kNPmax = kNWmax * kS;
  constexpr int kRawArr = kWave * kT * (int)sizeof(IT);   // one [64][kT] raw tile (bytes)
  constexpr int kRawBC = kNPmax * kT * (int)sizeof(IT);   // one [NP][kT] raw B or C tile
  // Separate LDS objects: the asynchronous fetches write only s_raw_*, so the
  // compiler needs no wait on them before the compute loop reads s_dl / s_x /
  // s_B / s_C (it cannot prove that for offsets into one array).
  __shared__ __attribute__((aligned(16))) char s_raw_u[2][kRawArr];   // u, double buffered (epilogue reads D u)
  __shared__ __attribute__((aligned(16))) char s_raw_z[2][kRawArr];   // z, double buffered (epilogue)
  __shared__ __attribute__((aligned(16))) char s_raw_d[kRawArr];      // delta (consumed by the conversion)
  __shared__ __attribute__((aligned(16))) char s_raw_bc[(kVarB || kVarC) ? 2 * kRawBC : 16];
  __shared__ __attribute__((aligned(16))) float s_dl[kWave * kT];     // [kG][64][4] delta'
  __shared__ __attribute__((aligned(16))) float s_x[kWave * kT];      // [kG][64][4] delta' u (mamba) or u
  __shared__ __attribute__((aligned(16))) float s_B[(kVarB ? kNPmax * kT : 4)];  // [NP][kT]
  __shared__ __attribute__((aligned(16))) float s_C[(kVarC ? kNPmax * kT : 4)];  // [NP][kT]
  __shared__ __attribute__((aligned(16))) float s_Y[kNWmax * kWave * kT];         // [nW][kG][64][4]
  __shared__ __attribute__((aligned(16))) char s_raw_dA[kDA ? kRawArr : 16];    // deltaA (consumed by the conversion)
  __shared__ __attribute__((aligned(16))) float s_dt[kDA ? kWave * kT : 4];      // [kG][64][4] deltaA

  const int nW = blockDim.x / kWave;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int64_t b = blockIdx.y;
  const int64_t D = a.dim, L = a.seqlen;
  const int N = (int)a.dstate;                 // all states (layout of x and the checkpoints)
  const int64_t d0 = (int64_t)blockIdx.x * CB;
  const int rows = (int)((D - d0) < CB ? (D - d0) : CB);   // valid channels of this block
  const int64_t d = d0 + lane;
  const bool lane_ok = lane < rows;
  const int64_t grp = (a.var_B || a.var_C) ? d0 / (D / a.n_groups) : 0;
  const int n0 = w * kS;
  const int NP = nW * kS;
  const int nb = (int)blockIdx.z * NP;               // first state of this state block
  const int Nb = N - nb < NP ? N - nb : NP;          // its real states
  constexpr bool has_dA = kDA;  // deltaA drives A_bar (never for s7 / rglru)
  const bool has_bias = a.delta_bias.ptr != nullptr;
  const bool has_D = a.D.ptr != nullptr;
  const bool has_z = a.z.ptr != nullptr;
  const bool async_ok = flags & kFlagAsyncIn;   // fetched tensors allow 16-byte LDS-DMA rows
  const bool out_al = flags & kFlagAlignedOut;  // out / out_z rows are 16-byte aligned

  // per-workgroup row bases (64-bit) and row strides (32-bit)
  const IT* gu = static_cast<const IT*>(a.u.ptr) + b * a.u.s0 + d0 * a.u.s1;
  const IT* gd = static_cast<const IT*>(a.delta.ptr) + b * a.delta.s0 + d0 * a.delta.s1;
  const IT* gz = has_z ? static_cast<const IT*>(a.z.ptr) + b * a.z.s0 + d0 * a.z.s1 : nullptr;
  const IT* gdA = has_dA ? static_cast<const IT*>(a.deltaA.ptr) + b * a.deltaA.s0 + d0 * a.deltaA.s1 : nullptr;
  const IT* gB = kVarB ? static_cast<const IT*>(a.B.ptr) + b * a.B.s0 + grp * a.B.s1 + nb * a.B.s2 : nullptr;
  const IT* gC = kVarC ? static_cast<const IT*>(a.C.ptr) + b * a.C.s0 + grp * a.C.s1 + nb * a.C.s2 : nullptr;
  IT* go = (a.out.ptr && !ypart) ? static_cast<IT*>(a.out.ptr) + b * a.out.s0 + d0 * a.out.s1 : nullptr;
  IT* goz = (a.out_z.ptr && !ypart) ? static_cast<IT*>(a.out_z.ptr) + b * a.out_z.s0 + d0 * a.out_z.s1 : nullptr;
  float* gyp = ypart ? ypart + (((int64_t)blockIdx.z * a.batch + b) * D + d0) * L : nullptr;
  const uint32_t su = (uint32_t)a.u.s1, sd = (uint32_t)a.delta.s1, sz = (uint32_t)a.z.s1;
  const uint32_t sdA = (uint32_t)a.deltaA.s1, sBn = (uint32_t)a.B.s2, sCn = (uint32_t)a.C.s2;
  const uint32_t so = (uint32_t)a.out.s1, soz = (uint32_t)a.out_z.s1;

  // per-lane constants
  float a2[kS], Araw[kS], invA[kS], cout_c[kS], h[kS], prodA[kS];
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
      const float bc = (!kVarB && ok) ? Bp[d * a.B.s0 + ng * a.B.s1] : 1.f;
      const float cc = (!kVarC && ok) ? Cp[d * a.C.s0 + ng * a.C.s1] : 1.f;
      cout_c[k] = ok ? (kVarB ? 1.f : bc) * (kVarC ? 1.f : cc) : 0.f;
      h[k] = 0.f;
      prodA[k] = 1.f;
    }
  }
  // D and delta_bias of channel `lane` in a VGPR; the per-element phases take
  // their row's value with a cross-lane read (ds_bpermute: no LDS allocated,
  // which keeps the 4-wave d_state 17..32 forward at two workgroups per CU)
  const float lane_D = (has_D && lane_ok) ? static_cast<const float*>(a.D.ptr)[d * a.D.s0] : 0.f;
  const float lane_bias = (has_bias && lane_ok) ? static_cast<const float*>(a.delta_bias.ptr)[d * a.delta_bias.s0] : 0.f;
  float sumdt = 0.f;  // running sum of the A step (exp-family chunk products)
  float* ckp = static_cast<float*>(a.ckpt);
  float* xp = static_cast<float*>(a.x);
  const int64_t n_xc = (L + kXChunk - 1) / kXChunk;

  float* sDl = s_dl;
  float* sX = s_x;
  float* sB = s_B;
  float* sC = s_C;
  float* sY = s_Y;
  float* sDt = s_dt;

  const int64_t n_tiles = (L + kT - 1) / kT;

  // ---- fetch of raw tile `tile` (u, z into buffer `buf`).  The asynchronous form is
  // issued at the start of a compute phase; the synchronous fallback (partial
  // tile, misaligned tensors) runs inside the finish phase, so that the compute
  // phase never has a compiler-visible global load outstanding (any such load
  // would make the compiler wait on the whole vmcnt, i.e. on the prefetch).
  auto async_tile = [&](int64_t tile) __attribute__((always_inline)) {
    const int64_t t0 = tile * kT;
    return async_ok && (L - t0) >= kT && rows == CB && (CB * kQ) % kWave == 0;
  };
  auto fetch_async = [&](int64_t tile, int buf) __attribute__((always_inline)) {
    const int64_t t0 = tile * kT;
    tile_fetch_async<IT, kQ>(gu + t0, su, CB, s_raw_u[buf], w, nW, lane);
    tile_fetch_async<IT, kQ>(gd + t0, sd, CB, s_raw_d, w, nW, lane);
    if (has_z) tile_fetch_async<IT, kQ>(gz + t0, sz, CB, s_raw_z[buf], w, nW, lane);
    if constexpr (kVarB) tile_fetch_async<IT, kQ>(gB + t0, sBn, Nb, s_raw_bc, w, nW, lane);
    if constexpr (kVarC) tile_fetch_async<IT, kQ>(gC + t0, sCn, Nb, s_raw_bc + kRawBC, w, nW, lane);
    if constexpr (kDA) tile_fetch_async<IT, kQ>(gdA + t0, sdA, CB, s_raw_dA, w, nW, lane);
  };
  auto fetch_sync = [&](int64_t tile, int buf) __attribute__((always_inline)) {
    const int64_t t0 = tile * kT;
    const int nt = (int)((L - t0) < kT ? (L - t0) : kT);
    tile_fetch_sync<IT, kQ>(gu + t0, su, kWave, rows, nt, s_raw_u[buf], tid, blockDim.x);
    tile_fetch_sync<IT, kQ>(gd + t0, sd, kWave, rows, nt, s_raw_d, tid, blockDim.x);
    if (has_z) tile_fetch_sync<IT, kQ>(gz + t0, sz, kWave, rows, nt, s_raw_z[buf], tid, blockDim.x);
    if constexpr (kVarB) tile_fetch_sync<IT, kQ>(gB + t0, sBn, NP, Nb, nt, s_raw_bc, tid, blockDim.x);
    if constexpr (kVarC) tile_fetch_sync<IT, kQ>(gC + t0, sCn, NP, Nb, nt, s_raw_bc + kRawBC, tid, blockDim.x);
    if constexpr (kDA) tile_fetch_sync<IT, kQ>(gdA + t0, sdA, kWave, rows, nt, s_raw_dA, tid, blockDim.x);
  };

  // a tile whose kT steps and 64 channels are all valid
  auto full_tile = [&](int64_t tile) __attribute__((always_inline)) {
    return (L - tile * kT) >= kT && rows == kWave;
  };

  // ---- raw tile in buffer `buf` -> fp32 operands (delta', x, deltaA, B, C)
  auto convert = [&](auto full_tag, int64_t tile, int buf) __attribute__((always_inline)) {
    constexpr bool kFull = decltype(full_tag)::value;
    const int64_t t0 = tile * kT;
    const int nt = (int)((L - t0) < kT ? (L - t0) : kT);
    for (int j = tid; j < kWave * kQ; j += blockDim.x) {
      const int r = j / kQ, q = j % kQ;
      float vu[kEl], vd[kEl];
      raw_to_f32<IT>(*reinterpret_cast<const uint4*>(s_raw_u[buf] + 16 * j), vu);
      raw_to_f32<IT>(*reinterpret_cast<const uint4*>(s_raw_d + 16 * j), vd);
      const float bias = __shfl(lane_bias, r);
      float vdt[kEl];
      if constexpr (kDA) raw_to_f32<IT>(*reinterpret_cast<const uint4*>(s_raw_dA + 16 * j), vdt);
#pragma unroll
      for (int i = 0; i < kEl; ++i) {
        const float x = vd[i] + bias;
        float dl = a.delta_softplus ? softplus_fast(x) : x;
        const bool valid = kFull || (r < rows && q * kEl + i < nt);
        dl = valid ? dl : 0.f;
        vd[i] = dl;
        vu[i] = valid ? (kMethod == LRNNX_MAMBA ? dl * vu[i] : vu[i]) : 0.f;
        if constexpr (kDA) vdt[i] = valid ? vdt[i] : 0.f;
      }
      // step s = q * kEl + i goes to group s / 4, slot s % 4 of row r
#pragma unroll
      for (int i = 0; i < kEl; i += 4) {
        const int g = (q * kEl + i) / 4;
        *reinterpret_cast<float4*>(sDl + (g * kWave + r) * 4) = make_float4(vd[i], vd[i + 1], vd[i + 2], vd[i + 3]);
        *reinterpret_cast<float4*>(sX + (g * kWave + r) * 4) = make_float4(vu[i], vu[i + 1], vu[i + 2], vu[i + 3]);
        if constexpr (kDA)
          *reinterpret_cast<float4*>(sDt + (g * kWave + r) * 4) =
              make_float4(vdt[i], vdt[i + 1], vdt[i + 2], vdt[i + 3]);
      }
    }
    if constexpr (kVarB || kVarC) {
      const char* rbc = s_raw_bc;
      for (int j = tid; j < NP * kQ; j += blockDim.x) {
        const bool st_ok = j / kQ < Nb;  // padded states read B = C = 0
        float v[kEl];
        if constexpr (kVarB) {
          raw_to_f32<IT>(*reinterpret_cast<const uint4*>(rbc + 16 * j), v);
#pragma unroll
          for (int i = 0; i < kEl; ++i) sB[j * kEl + i] = st_ok ? v[i] : 0.f;
        }
        if constexpr (kVarC) {
          raw_to_f32<IT>(*reinterpret_cast<const uint4*>(rbc + kRawBC + 16 * j), v);
#pragma unroll
          for (int i = 0; i < kEl; ++i) sC[j * kEl + i] = st_ok ? v[i] : 0.f;
        }
      }
    }
  };

  // ---- epilogue of tile `tile` (raw buffer `buf`): y = sum of wave partials + D u
  auto epilogue = [&](auto full_tag, int64_t tile, int buf) __attribute__((always_inline)) {
    constexpr bool kFull = decltype(full_tag)::value;
    const int64_t t0 = tile * kT;
    const int nt = (int)((L - t0) < kT ? (L - t0) : kT);
    for (int j = tid; j < kWave * kQ; j += blockDim.x) {
      const int r = j / kQ, q = j % kQ;
      const float Dv = __shfl(lane_D, r);   // before the divergent exits: every lane of the wave
      if (!kFull && r >= rows) continue;
      if (gyp) {  // state block: its partial y, fp32 (D u and the gate come in the combine)
        float y[kEl];
#pragma unroll
        for (int i = 0; i < kEl; i += 4) {
          const int g = (q * kEl + i) / 4;
          float4 acc = *reinterpret_cast<const float4*>(sY + (g * kWave + r) * 4);
          for (int ww = 1; ww < nW; ++ww) {
            const float4 p = *reinterpret_cast<const float4*>(sY + ((ww * kG + g) * kWave + r) * 4);
            acc.x += p.x; acc.y += p.y; acc.z += p.z; acc.w += p.w;
          }
          y[i] = acc.x; y[i + 1] = acc.y; y[i + 2] = acc.z; y[i + 3] = acc.w;
        }
        float* p = gyp + r * L + t0 + q * kEl;
        const int n_ = kFull ? kEl : nt - q * kEl;
        if (n_ >= kEl && (L & 3) == 0) {
#pragma unroll
          for (int i = 0; i < kEl; i += 4) *reinterpret_cast<float4*>(p + i) = make_float4(y[i], y[i + 1], y[i + 2], y[i + 3]);
        } else {
          for (int i = 0; i < (n_ < kEl ? n_ : kEl); ++i) p[i] = y[i];
        }
        continue;
      }
      float vu[kEl], y[kEl];
      raw_to_f32<IT>(*reinterpret_cast<const uint4*>(s_raw_u[buf] + 16 * j), vu);
#pragma unroll
      for (int i = 0; i < kEl; i += 4) {
        const int g = (q * kEl + i) / 4;
        float4 acc = *reinterpret_cast<const float4*>(sY + (g * kWave + r) * 4);
        for (int ww = 1; ww < nW; ++ww) {
          const float4 p = *reinterpret_cast<const float4*>(sY + ((ww * kG + g) * kWave + r) * 4);
          acc.x += p.x; acc.y += p.y; acc.z += p.z; acc.w += p.w;
        }
        y[i] = fmaf(Dv, vu[i], acc.x);
        y[i + 1] = fmaf(Dv, vu[i + 1], acc.y);
        y[i + 2] = fmaf(Dv, vu[i + 2], acc.z);
        y[i + 3] = fmaf(Dv, vu[i + 3], acc.w);
      }
      const int n_ = kFull ? kEl : nt - q * kEl;
      if (!kFull && n_ <= 0) continue;
      auto put = [&](IT* p) __attribute__((always_inline)) {
        if ((kFull && out_al) || (n_ >= kEl && (reinterpret_cast<uintptr_t>(p) & 15u) == 0))
          *reinterpret_cast<uint4*>(p) = f32_to_raw<IT>(y);
        else
          for (int i = 0; i < (n_ < kEl ? n_ : kEl); ++i) p[i] = from_f32<IT>(y[i]);
      };
      if (go) put(go + r * so + t0 + q * kEl);
      if (has_z && goz) {
        float vz[kEl];
        raw_to_f32<IT>(*reinterpret_cast<const uint4*>(s_raw_z[buf] + 16 * j), vz);
#pragma unroll
        for (int i = 0; i < kEl; ++i) y[i] *= vz[i] * sigmoid_fast(vz[i]);
        put(goz + r * soz + t0 + q * kEl);
      }
    }
  };

  // ---- one step of the recurrence for the wave's kS states
  auto step = [&](float dl, float xx, float dt, const float* bin, const float* cc) __attribute__((always_inline)) {
    float y = 0.f;
#pragma unroll
    for (int k = 0; k < kS; ++k) {
      float beta;
      const float ab = disc_real<kMethod, kDA>(dt, dl, a2[k], Araw[k], invA[k], beta);
      float inc;
      if constexpr (kMethod == LRNNX_MAMBA) inc = xx * bin[k];           // xx = delta' u
      else if constexpr (uses_B_input<kMethod>()) inc = beta * xx * bin[k];
      else inc = beta * xx;
      h[k] = fmaf(ab, h[k], inc);
      y = fmaf(cc[k], h[k], y);
      if constexpr (!exp_family<kMethod>()) prodA[k] *= ab;
    }
    if constexpr (exp_family<kMethod>()) sumdt += dt;
    return y;
  };

  // this lane's real states (0 past the last channel): one per-lane bound
  // instead of a predicate per state, and one row address per checkpoint
  // (the lane's states are D apart), keep the stores' index math out of SGPRs
  const int n_real = lane_ok ? (Nb - n0 < kS ? Nb - n0 : kS) : 0;
  auto store_ckpt = [&](int64_t tg) __attribute__((always_inline)) {  // state after step tg
    float* p = ckp + ((b * n_ck + tg / kCk) * N + nb + n0) * D + d;
    // bound and stride opaque here: compared and stepped at each store, not
    // hoisted out of the tile loop as per-state masks and offsets (SGPRs the
    // loop cannot keep: they spill to VGPR lanes)
    int nr = n_real;
    int64_t ds = D;
    asm volatile("" : "+v"(nr), "+s"(ds));
#pragma unroll
    for (int k = 0; k < kS; ++k) {
      if (k < nr) *p = h[k];
      p += ds;
    }
  };
  auto store_x = [&](int64_t tg) __attribute__((always_inline)) {  // reference chunk carry at step tg
    const int64_t c = tg / kXChunk;
#pragma unroll
    for (int k = 0; k < kS; ++k) {
      if (lane_ok && n0 + k < Nb) {
        float ac;
        if constexpr (exp_family<kMethod>())
          ac = fast_exp2(a2[k] * sumdt);
        else
          ac = prodA[k];
        float* xr = xp + ((b * D + d) * n_xc + c) * 2 * N;
        xr[2 * (nb + n0 + k)] = ac;
        xr[2 * (nb + n0 + k) + 1] = h[k];
      }
    }
  };

  // ---- prologue: per-channel constants, tile 0
  if (async_tile(0)) fetch_async(0, 0);
  else fetch_sync(0, 0);
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  __syncthreads();
  if (full_tile(0)) convert(std::true_type{}, 0, 0);
  else convert(std::false_type{}, 0, 0);
  __syncthreads();

  for (int64_t tile = 0; tile < n_tiles; ++tile) {
    const int buf = (int)(tile & 1);
    const int64_t t0 = tile * kT;
    const int nt = (int)((L - t0) < kT ? (L - t0) : kT);
    const bool next = tile + 1 < n_tiles;
    const bool next_async = next && async_tile(tile + 1);
    if (next_async) fetch_async(tile + 1, buf ^ 1);

    // ---- compute(tile)
    if (nt == kT) {
      float bin[kS], cc[kS];
#pragma unroll
      for (int k = 0; k < kS; ++k) { bin[k] = 1.f; cc[k] = cout_c[k]; }
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        const float4 dl4 = *reinterpret_cast<const float4*>(sDl + (g * kWave + lane) * 4);
        const float4 x4 = *reinterpret_cast<const float4*>(sX + (g * kWave + lane) * 4);
        float4 dt4 = dl4;
        if constexpr (kDA) dt4 = *reinterpret_cast<const float4*>(sDt + (g * kWave + lane) * 4);
        float4 b4[kS], c4[kS];
#pragma unroll
        for (int k = 0; k < kS; ++k) {
          if constexpr (kVarB) b4[k] = *reinterpret_cast<const float4*>(sB + (n0 + k) * kT + 4 * g);
          if constexpr (kVarC) c4[k] = *reinterpret_cast<const float4*>(sC + (n0 + k) * kT + 4 * g);
        }
        float y[4];
        const float dlv[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
        const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
        const float dtv[4] = {dt4.x, dt4.y, dt4.z, dt4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int k = 0; k < kS; ++k) {
            if constexpr (kVarB) bin[k] = (&b4[k].x)[i];
            if constexpr (kVarC) cc[k] = kVarB ? (&c4[k].x)[i] : (&c4[k].x)[i] * cout_c[k];
          }
          y[i] = step(dlv[i], xv[i], dtv[i], bin, cc);
          const int s = 4 * g + i;
          if (ckp != nullptr && (s + 1) % kCk == 0) store_ckpt(t0 + s);
        }
        *reinterpret_cast<float4*>(sY + ((w * kG + g) * kWave + lane) * 4) = make_float4(y[0], y[1], y[2], y[3]);
      }
      if (xp != nullptr && (((t0 + kT) % kXChunk) == 0 || t0 + kT == L)) store_x(t0 + kT - 1);
    } else {
      for (int s = 0; s < nt; ++s) {
        const int g = s / 4, i = s % 4;
        const float dl = sDl[(g * kWave + lane) * 4 + i];
        const float xx = sX[(g * kWave + lane) * 4 + i];
        const float dt = kDA ? sDt[(g * kWave + lane) * 4 + i] : dl;
        float bin[kS], cc[kS];
#pragma unroll
        for (int k = 0; k < kS; ++k) {
          bin[k] = kVarB ? sB[(n0 + k) * kT + s] : 1.f;
          cc[k] = kVarC ? (kVarB ? sC[(n0 + k) * kT + s] : sC[(n0 + k) * kT + s] * cout_c[k]) : cout_c[k];
        }
        sY[((w * kG + g) * kWave + lane) * 4 + i] = step(dl, xx, dt, bin, cc);
        if (ckp != nullptr && ((t0 + s + 1) % kCk) == 0) store_ckpt(t0 + s);
        if (xp != nullptr && (((t0 + s + 1) % kXChunk) == 0 || t0 + s == L - 1)) store_x(t0 + s);
      }
    }

    // ---- finish(tile): tile+1 in LDS, epilogue(tile), convert(tile+1)
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    if (next && !next_async) {
      fetch_sync(tile + 1, buf ^ 1);
      __syncthreads();
    }
    if (full_tile(tile)) epilogue(std::true_type{}, tile, buf);
    else epilogue(std::false_type{}, tile, buf);
    if (next) {
      if (full_tile(tile + 1)) convert(std::true_type{}, tile + 1, buf ^ 1);
      else convert(std::false_type{}, tile + 1, buf ^ 1);
    }
    __syncthreads();
  }
}

// State blocks: out = sum over the blocks' partial y in block order + D u,
// out_z = out silu(z).  One thread per (b, d, t), consecutive threads along t.
template <typename IT>
__global__ void __launch_bounds__(256)
ss_fwd_combine_kernel(const lrnnx_selective_scan_args a, const float* __restrict__ ypart, const int nsb) {
  const int64_t L = a.seqlen, D = a.dim, BD = a.batch * a.dim;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= BD * L) return;
  const int64_t t = i % L, r = i / L, b = r / D, d = r % D;
  float y = 0.f;
  for (int z = 0; z < nsb; ++z) y += ypart[(z * BD + r) * L + t];
  if (a.D.ptr) {
    const float u = to_f32(static_cast<const IT*>(a.u.ptr)[b * a.u.s0 + d * a.u.s1 + t]);
    y = fmaf(static_cast<const float*>(a.D.ptr)[d * a.D.s0], u, y);
  }
  if (a.out.ptr) static_cast<IT*>(a.out.ptr)[b * a.out.s0 + d * a.out.s1 + t] = from_f32<IT>(y);
  if (a.z.ptr && a.out_z.ptr) {
    const float z = to_f32(static_cast<const IT*>(a.z.ptr)[b * a.z.s0 + d * a.z.s1 + t]);
    static_cast<IT*>(a.out_z.ptr)[b * a.out_z.s0 + d * a.out_z.s1 + t] = from_f32<IT>(y * (z * sigmoid_fast(z)));
  }
}

template <typename IT, int kS, int kMethod, bool kVarB, bool kVarC, bool kDA, int kNWm>
static hipError_t launch_fwd_t(const lrnnx_selective_scan_args& a, const SSGeom& g, hipStream_t st) {
  // state blocks write partial y to the workspace when there are outputs (ss_fwd_blocks_ws_bytes;
  // launch_fwd_s falls back to one block when the workspace is missing)
  float* ypart = (g.nsb > 1 && (a.out.ptr || a.out_z.ptr)) ? static_cast<float*>(a.workspace) : nullptr;
  dim3 grid(g.n_cb, (unsigned)a.batch, (unsigned)g.nsb);
  dim3 block(g.nW * kWave);
  if (g.nW > kNWm) return hipErrorInvalidConfiguration;
  // async LDS fetches need 16-byte aligned row starts for every fetched tensor
  auto al = [](const void* p, int64_t s_batch, int64_t s_row) {
    return p == nullptr || ((reinterpret_cast<uintptr_t>(p) & 15u) == 0 && ((s_batch * sizeof(IT)) & 15) == 0 &&
                            ((s_row * sizeof(IT)) & 15) == 0);
  };
  const bool in_ok = al(a.u.ptr, a.u.s0, a.u.s1) && al(a.delta.ptr, a.delta.s0, a.delta.s1) &&
                     al(a.z.ptr, a.z.s0, a.z.s1) && (!kDA || al(a.deltaA.ptr, a.deltaA.s0, a.deltaA.s1)) &&
                     (!kVarB || (al(a.B.ptr, a.B.s0, a.B.s2) && ((a.B.s1 * sizeof(IT)) & 15) == 0)) &&
                     (!kVarC || (al(a.C.ptr, a.C.s0, a.C.s2) && ((a.C.s1 * sizeof(IT)) & 15) == 0));
  const bool out_ok = al(a.out.ptr, a.out.s0, a.out.s1) && al(a.out_z.ptr, a.out_z.s0, a.out_z.s1);
  const int flags = (in_ok ? kFlagAsyncIn : 0) | (out_ok ? kFlagAlignedOut : 0);
  hipLaunchKernelGGL((ss_fwd_kernel<IT, kS, kMethod, kVarB, kVarC, kDA, kNWm>), grid, block, 0, st, a, g.CB, g.n_ck,
                     flags, ypart);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || ypart == nullptr) return e;
  const int64_t n = a.batch * a.dim * a.seqlen;
  hipLaunchKernelGGL(ss_fwd_combine_kernel<IT>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a,
                     static_cast<const float*>(ypart), g.nsb);
  return hipGetLastError();
}

template <typename IT, int kS, int kMethod, bool kVarB, bool kVarC, int kNWm>
static hipError_t launch_fwd_da(const lrnnx_selective_scan_args& a, const SSGeom& g, hipStream_t st) {
  if constexpr (uses_deltaA<kMethod>()) {
    if (a.deltaA.ptr != nullptr) return launch_fwd_t<IT, kS, kMethod, kVarB, kVarC, true, kNWm>(a, g, st);
  }
  return launch_fwd_t<IT, kS, kMethod, kVarB, kVarC, false, kNWm>(a, g, st);
}

template <typename IT, int kS, int kMethod, int kNWm = fwd_nw_max(kS)>
static hipError_t launch_fwd_bc(const lrnnx_selective_scan_args& a, const SSGeom& g, hipStream_t st) {
  if (a.var_B && a.var_C) return launch_fwd_da<IT, kS, kMethod, true, true, kNWm>(a, g, st);
  if (a.var_B) return launch_fwd_da<IT, kS, kMethod, true, false, kNWm>(a, g, st);
  if (a.var_C) return launch_fwd_da<IT, kS, kMethod, false, true, kNWm>(a, g, st);
  return launch_fwd_da<IT, kS, kMethod, false, false, kNWm>(a, g, st);
}

template <typename IT, int kMethod>
static hipError_t launch_fwd_s(const lrnnx_selective_scan_args& a, const SSGeom& g, hipStream_t st) {
  if (g.nsb > 1 && (a.out.ptr || a.out_z.ptr) &&
      (a.workspace == nullptr || a.workspace_bytes < ss_fwd_blocks_ws_bytes(a) ||
       (reinterpret_cast<uintptr_t>(a.workspace) & 15u) != 0)) {
    // no room for the blocks' partial y: every state in one workgroup, 32 per
    // wave (slower: it spills), with the checkpoint interval of the blocks
    SSGeom g1 = g;
    g1.kS = 32;
    g1.nW = (int)((a.dstate + 31) / 32);
    g1.nsb = 1;
    return launch_fwd_bc<IT, 32, kMethod>(a, g1, st);
  }
  switch (g.kS) {
    case 1: return launch_fwd_bc<IT, 1, kMethod>(a, g, st);
    case 4: return launch_fwd_bc<IT, 4, kMethod>(a, g, st);
    case 8:   // d_state 17..32: at most 4 waves, 80 KB of LDS without deltaA (two workgroups per CU)
      return g.nW <= 4 ? launch_fwd_bc<IT, 8, kMethod, 4>(a, g, st) : launch_fwd_bc<IT, 8, kMethod>(a, g, st);
    case 32: return launch_fwd_bc<IT, 32, kMethod>(a, g, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace lrnnx
