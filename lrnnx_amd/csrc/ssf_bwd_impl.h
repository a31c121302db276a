// Selective scan backward, fast path of the headline case (gfx950).
//
// The fast forward's coverage (ssf_fwd_eligible): method "mamba" (f32 / bf16
// / f16 I/O), "dirac", "zoh" and "bilinear" (f32 I/O; zoh and bilinear in
// 32-channel workgroups, unsplit), variable B and C, d_state <= 16, 64
// channels per group block, L a multiple of 16, 16-byte aligned rows; deltaA
// (mamba), as Mamba's event mode passes it.
// Gradients of the reference kernel
// csrc/selective_scan/selective_scan_backward.cuh:86-845 for this method:
//   dh_t  = A_bar_{t+1} dh_{t+1} + C_t dy_t      (dy = dout silu(z))
//   du    = delta' sum_n dh B + D dy
//   ddelta' = u sum_n dh B + sum_n A A_bar h_{t-1} dh, times sigmoid(delta + bias)
//   dA    = sum_t delta' A_bar h_{t-1} dh,  dB_t = sum_d dh delta' u,
//   dC_t  = sum_d dy h_t,  dD = sum dy u,  ddelta_bias = sum ddelta,
//   dz    = dout out sigma(z) (1 + z (1 - sigma(z)))      (:218-219)
// With deltaA, A_bar = exp(deltaA A): the A term goes to ddeltaA instead of
// ddelta', and dA sums deltaA A_bar h_{t-1} dh.
// For "dirac" (input term B u) delta' drops out of du and dB, and ddelta'
// keeps the A term only.  For "zoh" and "bilinear" (input factor beta per
// state) du = sum_n dh beta B, dB_t = sum_d dh beta u, and
//   ddelta' = sum_n dh dA_bar/ddelta' (A h_{t-1} + u B),
// since dbeta/ddelta' = dA_bar/ddelta' / A: A_bar for zoh, r^2 for bilinear
// (r = 1 / (1 - delta' A / 2) = (A_bar + 1) / 2); dA adds the input term
// dh u B dbeta/dA: (delta' A_bar - beta) / A (zoh), delta'^2 r^2 / 2 (bilinear).
//
// Decomposition as in the forward (ssf_fwd_impl.h): one workgroup = one batch
// row and 64 channels, wave w owns states 4w..4w+3, lane = channel.  The
// sequence is walked from the end in tiles of 16 steps = one checkpoint
// interval of the forward (fp32 states every 16 steps, layout (B, n_ck, N, D)).
// Per tile k:
//   compute(k)  issue the LDS-DMA fetch of the checkpoint row that starts
//               tile k-1 and, when tile k-1 lies in the next raw tile, of
//               that raw tile (u, delta, dout, z, out, B, C over one or two
//               16-step tiles, kRT);
//               recompute A_bar and h over the 16 steps of tile k from its
//               checkpoint into VGPRs; walk the steps backwards accumulating
//               dA (per lane), the per-step sums over the wave's states of
//               dh B and A A_bar h_{t-1} dh (to LDS, summed over waves in the
//               epilogue) and the dB / dC values, reduce-scattered over the
//               64 channels of the wave (one fp32 partial per channel block,
//               summed over blocks in a fixed order by ss_reduce_bc_kernel).
//   finish(k)   wait + barrier; epilogue of tile k (du, ddelta; the dD and
//               ddelta_bias terms stay in per-thread registers) and
//               conversion of tile k-1 from its raw tile (delta' = softplus(delta + bias),
//               u, dy = dout silu(z) to fp32, dz written here, B / C rows).
// The fp32 operands have one buffer: in the finish phase every thread reads
// its own slots of tile k (epilogue) before it writes the same slots with
// tile k-1 (conversion), and the compute phases read them only between the
// barriers.  (Keeping the LDS under 80 KB also for fp32 I/O with z lets two
// workgroups share a CU.)
#pragma once
#include <type_traits>

#include "ss_bwd_impl.h"
#include "ssf_fwd_impl.h"

namespace lrnnx {

namespace ssf {
// softplus20_fast(x) and its derivative from the same exp: sigmoid(x) =
// e / (1 + e), e = exp(x) (relative precision kept for small e), and 1 past
// the threshold 20, where softplus is the identity
__device__ __forceinline__ float softplus20_sig(float x, float& sg) {
  const float e = __builtin_amdgcn_exp2f(x * kLog2e);
  const float t = 1.f + e;
  const float small = e * fmaf(e, fmaf(e, fmaf(e, -0.25f, 0.33333334f), -0.5f), 1.f);
  const float big = __builtin_amdgcn_logf(t) * kLn2;
  const float r = e < 0.03125f ? small : big;
  sg = x > 20.f ? 1.f : e * __builtin_amdgcn_rcpf(t);
  return x > 20.f ? x : r;
}
}  // namespace ssf

// kRT: steps of one raw-tile fetch, one tile (16) or two (32: 16-bit I/O,
// L a multiple of 32).  A two-tile fetch reads 64 bytes of each row, half a
// 128-byte line instead of a quarter, so each line is fetched from memory
// about half as often; its 11 KB more LDS keep two workgroups per CU.
// kCh: channels per workgroup, as in the forward.  64: lane = channel, 4
// states per lane.  32: lane = channel + 32 half, 2 states per lane (the
// lower half of wave w holds states 4w, 4w+1, the upper half 4w+2, 4w+3);
// a grid of at most 256 64-channel workgroups then runs twice as many, two
// per CU.  The channel reductions lose their cross-half stage (the halves
// hold different states), and the per-element phases take 2 elements per
// thread.
// kDA: deltaA given (mamba).  The operand tile s_x then holds deltaA (the
// step of A_bar) and the compute phases form delta' u from s_dl and s_u; the
// raw deltaA tile takes the LDS that sigmoid(delta + bias) has with softplus
// (the epilogue re-derives it from delta').
// kM: the method (LRNNX_MAMBA, DIRAC, ZOH or BILINEAR), compile-time; zoh and
// bilinear re-derive their input factor beta from A_bar in the reverse walk,
// whose extra terms fit the registers of the 32-channel form only.
template <typename IT, bool kSP, bool kZ, int kRT, int kCh = kWave, int kM = LRNNX_MAMBA, bool kDA = false>
__global__ void __launch_bounds__(ssf::kNT) __attribute__((amdgpu_waves_per_eu(2, 2)))
ssf_bwd_kernel(const lrnnx_selective_scan_args a, const int64_t n_ck, float* __restrict__ ws, const SSBwdWs wo,
               const float* __restrict__ ckp, const int64_t seg_tiles) {
  using namespace ssf;
  constexpr int kT = 16;                  // steps per tile = checkpoint interval
  static_assert(kT == kCk, "one checkpoint interval per tile");
  static_assert(kRT == kT || kRT == 2 * kT, "a raw fetch covers one or two tiles");
  static_assert(kCh == kWave || kCh == kWave / 2, "64 or 32 channels per workgroup");
  constexpr bool kDi = kM == LRNNX_DIRAC;
  constexpr bool kBeta = kM == LRNNX_ZOH || kM == LRNNX_BILINEAR;   // input factor per state
  static_assert(kM == LRNNX_MAMBA || kDi || kBeta, "method");
  static_assert(kM == LRNNX_MAMBA || sizeof(IT) == 4, "methods other than mamba take fp32 input only");
  static_assert(!kDA || kM == LRNNX_MAMBA, "deltaA on the fast backward: mamba only");
  static_assert(!kBeta || kCh == kWave / 2, "zoh / bilinear: 32-channel workgroups");
  constexpr int kH = kWave / kCh;         // lane halves per wave
  constexpr int kS = 4 / kH;              // states per lane
  constexpr int kPair = kRT / kT;         // tiles per raw fetch
  constexpr int kG = kT / 4;              // groups of 4 steps
  constexpr int kRow = kT * (int)sizeof(IT);    // bytes of one tile's part of a raw row
  constexpr int kRowR = kRT * (int)sizeof(IT);  // bytes of one raw row
  constexpr int kQ = kRowR / 16;          // 16-byte blocks per raw row
  constexpr int kRaw = kCh * kRowR;       // [kCh][kRT] raw tile
  constexpr int kRawS = 16 * kRowR;       // [16][kRT] raw B or C tile
  constexpr int kOp = kG * kCh * 4;       // floats of one [g][ch][4] operand tile
  constexpr int kNP = kNW * kH;           // per-step partial sums per element (waves x halves)
  constexpr int kEt = kCh * kT / kNT;     // elements per thread in the per-element phases (4 or 2)
  constexpr int kP = kT / kEt;            // threads per row
  constexpr int kQck = kCh * 4 / 16;      // 16-byte blocks of one checkpoint row (kCh fp32)
  static_assert(kCh * kQ <= kNW * kWave && 16 * kQ <= kWave, "one fetch instruction per wave and tensor");

  __shared__ __attribute__((aligned(16))) char s_raw_u[kRaw];
  __shared__ __attribute__((aligned(16))) char s_raw_d[kRaw];
  __shared__ __attribute__((aligned(16))) char s_raw_do[kRaw];
  __shared__ __attribute__((aligned(16))) char s_raw_z[kZ ? kRaw : 16];
  __shared__ __attribute__((aligned(16))) char s_raw_o[kZ ? kRaw : 16];
  __shared__ __attribute__((aligned(16))) char s_raw_b[kRawS];
  __shared__ __attribute__((aligned(16))) char s_raw_c[kRawS];
  __shared__ __attribute__((aligned(16))) char s_raw_a[kDA ? kRaw : 16];  // deltaA
  __shared__ __attribute__((aligned(16))) float s_ck[16 * kCh];        // [n][ch] h at the tile start
  __shared__ __attribute__((aligned(16))) float s_dl[kOp];             // [g][ch][4] delta'
  __shared__ __attribute__((aligned(16))) float s_u[kOp];              // u (epilogue)
  __shared__ __attribute__((aligned(16))) float s_x[kOp];              // delta' u (compute phases; deltaA: deltaA)
  __shared__ __attribute__((aligned(16))) float s_dy[kOp];             // dout silu(z)
  // sigmoid(delta + bias); with deltaA the epilogue re-derives it as 1 - exp(-delta'), and its
  // 4 KB hold the raw deltaA tile
  __shared__ __attribute__((aligned(16))) float s_sg[kSP && !kDA ? kOp : 4];
  __shared__ __attribute__((aligned(16))) float s_B[kT * 16];          // [t][n]
  __shared__ __attribute__((aligned(16))) float s_C[kT * 16];
  __shared__ __attribute__((aligned(16))) float s_P1[kNP * kOp];       // [w, half][g][ch][4] sum_k dh B
  __shared__ __attribute__((aligned(16))) float s_P2[kNP * kOp];       // sum_k A log2(e) A_bar h_{t-1} dh

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ch = lane & (kCh - 1), hf = lane / kCh;   // the lane's channel and lane half
  const int64_t b = blockIdx.y;
  const int64_t D = a.dim, L = a.seqlen;
  const int N = (int)a.dstate;
  const int64_t cb = blockIdx.x;
  const int64_t d0 = cb * kCh;
  const int64_t grp = d0 / (D / a.n_groups);
  const int n0w = w * 4;                 // the wave's first state
  const int n0 = n0w + hf * kS;          // the lane's first state
  // State order of the lane's registers: register k holds state n0 + (k ^ sm)
  // with sm from lane bits 3 and 2 (4 states: 2 b3 + (b2 ^ b3)) or bit 3 (2
  // states).  The DPP row mirror (lane i <-> 15 - i) flips sm's bit 1 (bit 0
  // with 2 states) and the half-row mirror (i <-> 7 - i) its bit 0, so the
  // first dB / dC reduce-scatter stages, over lane bits 3 and 2, pair
  // registers that hold the same state in both lanes: one DPP add per pair.
  const int lb2 = (lane >> 2) & 1, lb3 = (lane >> 3) & 1;
  const int sm = kS == 4 ? 2 * lb3 + (lb2 ^ lb3) : lb3;
  int ns[kS];
#pragma unroll
  for (int k = 0; k < kS; ++k) ns[k] = n0 + (k ^ sm);
  // thread -> (row er, piece eq of kEt elements) of the per-element phases
  const int er = tid / kP, eq = tid % kP;
  constexpr int kEb = kEt * (int)sizeof(IT);  // bytes of a thread's raw elements
  // the piece's slot in the [g][ch][4] operand tiles
  const int eo = op_off<0, kCh>((eq * kEt) >> 2, er) + ((eq * kEt) & 3);

  const IT* gu = static_cast<const IT*>(a.u.ptr) + b * a.u.s0 + d0 * a.u.s1;
  const IT* gd = static_cast<const IT*>(a.delta.ptr) + b * a.delta.s0 + d0 * a.delta.s1;
  const IT* gdo = static_cast<const IT*>(a.dout.ptr) + b * a.dout.s0 + d0 * a.dout.s1;
  const IT* gz = kZ ? static_cast<const IT*>(a.z.ptr) + b * a.z.s0 + d0 * a.z.s1 : nullptr;
  const IT* gos = kZ ? static_cast<const IT*>(a.out_saved.ptr) + b * a.out_saved.s0 + d0 * a.out_saved.s1 : nullptr;
  const IT* gB = static_cast<const IT*>(a.B.ptr) + b * a.B.s0 + grp * a.B.s1;
  const IT* gC = static_cast<const IT*>(a.C.ptr) + b * a.C.s0 + grp * a.C.s1;
  IT* gdu = static_cast<IT*>(a.du.ptr) + b * a.du.s0 + (d0 + er) * a.du.s1 + kEt * eq;
  IT* gddl = static_cast<IT*>(a.ddelta.ptr) + b * a.ddelta.s0 + (d0 + er) * a.ddelta.s1 + kEt * eq;
  IT* gdz = kZ ? static_cast<IT*>(a.dz.ptr) + b * a.dz.s0 + (d0 + er) * a.dz.s1 + kEt * eq : nullptr;
  const IT* gA = kDA ? static_cast<const IT*>(a.deltaA.ptr) + b * a.deltaA.s0 + d0 * a.deltaA.s1 : nullptr;
  IT* gddA = kDA ? static_cast<IT*>(a.ddeltaA.ptr) + b * a.ddeltaA.s0 + (d0 + er) * a.ddeltaA.s1 + kEt * eq : nullptr;
  const uint32_t su = (uint32_t)a.u.s1, sd = (uint32_t)a.delta.s1, sdo = (uint32_t)a.dout.s1;
  const uint32_t sz = (uint32_t)a.z.s1, sos = (uint32_t)a.out_saved.s1;
  const uint32_t sBn = (uint32_t)a.B.s2, sCn = (uint32_t)a.C.s2;
  const float* gck = ckp + b * n_ck * N * D + d0;   // checkpoint kk, state n: gck[(kk * N + n) * D + ch]
  // after the reduce-scatters lane l holds state ns[0] = n0 + sm and step
  // rs_step(l) of the tile, summed over the block's channels
  const int rs_n = ns[0];
  const int rs_t = kH == 1 ? 8 * ((lane >> 4) & 1) + 4 * ((lane >> 5) & 1) + (lane & 3)
                           : 8 * lb2 + 4 * ((lane >> 4) & 1) + (lane & 3);
  float* wsB = ws + wo.dBv + ((cb * a.batch + b) * N + rs_n) * L + rs_t;
  float* wsC = ws + wo.dCv + ((cb * a.batch + b) * N + rs_n) * L + rs_t;
  const bool wr_bc = rs_n < N;

  float a2[kS], gn[kS], dA_acc[kS];
  float Ar[kBeta ? kS : 1], iA[kM == LRNNX_ZOH ? kS : 1];   // A, 1 / A (zoh / bilinear)
  // zoh: the input term of dA, sum dh u B (delta' A_bar - beta), times 1 / A at the end
  float dAz[kM == LRNNX_ZOH ? kS : 1];
#pragma unroll
  for (int k = 0; k < kS; ++k) {
    const int n = ns[k];
    const float A_ = n < N ? static_cast<const float*>(a.A.ptr)[(d0 + ch) * a.A.s0 + n * a.A.s1] : -1.f;
    a2[k] = A_ * kLog2e;
    if constexpr (kBeta) Ar[k] = A_;
    if constexpr (kM == LRNNX_ZOH) {
      iA[k] = 1.f / A_;
      dAz[k] = 0.f;
    }
    // split of L: the adjoint entering this segment from the right
    gn[k] = (wo.S > 1 && n < N) ? ws[wo.g_init + ((blockIdx.z * a.batch + b) * N + n) * D + d0 + ch] : 0.f;
    dA_acc[k] = 0.f;
  }
  const float e_bias = a.delta_bias.ptr ? static_cast<const float*>(a.delta_bias.ptr)[(d0 + er) * a.delta_bias.s0] : 0.f;
  const float e_D = a.D.ptr ? static_cast<const float*>(a.D.ptr)[(d0 + er) * a.D.s0] : 0.f;
  float e_dD = 0.f, e_dbias = 0.f;  // this thread's share of dD and ddelta_bias (channel d0 + er)

  const int64_t n_tiles = L / kT;
  const int64_t tb = (int64_t)blockIdx.z * seg_tiles;   // this segment's tiles [tb, te)
  const int64_t te = tb + seg_tiles < n_tiles ? tb + seg_tiles : n_tiles;
  const int64_t prow = (int64_t)blockIdx.z * a.batch + b;  // row of the (segment, b) partials

  // Tile fetches: at most one LDS-DMA instruction per wave and tensor (kCh
  // rows x kQ blocks), with per-lane byte offsets fixed along L; per tile
  // only the scalar base moves.  B on wave 2, C on wave 3 (N * kQ <= 64
  // blocks each).  The checkpoint row: wave w fetches the 4 state rows it
  // reads itself (4 kQck blocks).
  const uint32_t off_u = dma_lane_offset<IT, kQ>(su, w, lane);
  const uint32_t off_d = dma_lane_offset<IT, kQ>(sd, w, lane);
  const uint32_t off_do = dma_lane_offset<IT, kQ>(sdo, w, lane);
  const uint32_t off_z = kZ ? dma_lane_offset<IT, kQ>(sz, w, lane) : 0u;
  const uint32_t off_os = kZ ? dma_lane_offset<IT, kQ>(sos, w, lane) : 0u;
  const uint32_t off_a = kDA ? dma_lane_offset<IT, kQ>((uint32_t)a.deltaA.s1, w, lane) : 0u;
  const uint32_t off_bc = dma_lane_offset<IT, kQ>(w == 2 ? sBn : sCn, 0, lane);
  const int ck_row = n0w + lane / kQck;                       // state row of this lane's checkpoint block
  const bool ck_on = lane < 4 * kQck && ck_row < N;
  const uint32_t off_ck = ((uint32_t)ck_row * (uint32_t)D + (uint32_t)(lane % kQck) * 4u) * 4u;
  // raw tile r: steps [r kRT, (r + 1) kRT) of every input row
  auto fetch_raw = [&](int64_t r) __attribute__((always_inline)) {
    const int64_t t0 = r * kRT;
    tile_fetch_async_s<kQ>(gu + t0, off_u, kCh, s_raw_u, w, lane);
    tile_fetch_async_s<kQ>(gd + t0, off_d, kCh, s_raw_d, w, lane);
    tile_fetch_async_s<kQ>(gdo + t0, off_do, kCh, s_raw_do, w, lane);
    if constexpr (kZ) {
      tile_fetch_async_s<kQ>(gz + t0, off_z, kCh, s_raw_z, w, lane);
      tile_fetch_async_s<kQ>(gos + t0, off_os, kCh, s_raw_o, w, lane);
    }
    if constexpr (kDA) tile_fetch_async_s<kQ>(gA + t0, off_a, kCh, s_raw_a, w, lane);
    if (w == 2) tile_fetch_async_s<kQ>(gB + t0, off_bc, N, s_raw_b, 0, lane);
    if (w == 3) tile_fetch_async_s<kQ>(gC + t0, off_bc, N, s_raw_c, 0, lane);
  };
  // h at the start of `tile` = checkpoint tile - 1 (none for tile 0)
  auto fetch_ck = [&](int64_t tile) __attribute__((always_inline)) {
    if (tile > 0 && ck_on)
      lds_dma_16_s(gck + (tile - 1) * N * D, off_ck, reinterpret_cast<char*>(s_ck) + w * 64 * kQck);
  };

  // tile's part of its raw tile -> fp32 operands; dz is written here
  auto convert = [&](int64_t tile) __attribute__((always_inline)) {
    float vu[kEt], vd[kEt], vdo[kEt];
    const int half = (int)(tile % kPair) * kRow;   // the tile's bytes within a raw row
    const int ro = er * kRowR + half + eq * kEb;   // byte offset of this thread's raw elements
    rawn_to_f32<IT, kEt>(s_raw_u + ro, vu);
    rawn_to_f32<IT, kEt>(s_raw_d + ro, vd);
    rawn_to_f32<IT, kEt>(s_raw_do + ro, vdo);
    float dy[kEt], sg[kEt], xu[kEt];
#pragma unroll
    for (int i = 0; i < kEt; ++i) {
      const float x = vd[i] + e_bias;
      vd[i] = kSP ? softplus20_sig(x, sg[i]) : x;
      dy[i] = vdo[i];
      xu[i] = (kDi || kBeta) ? vu[i] : vd[i] * vu[i];
    }
    if constexpr (kZ) {
      float vz[kEt], vo[kEt], dz[kEt];
      rawn_to_f32<IT, kEt>(s_raw_z + ro, vz);
      rawn_to_f32<IT, kEt>(s_raw_o + ro, vo);
#pragma unroll
      for (int i = 0; i < kEt; ++i) {
        const float sgz = sigmoidf_fast(vz[i]);
        const float zs = vz[i] * sgz;
        dz[i] = vdo[i] * vo[i] * fmaf(zs, 1.f - sgz, sgz);   // sg (1 + z (1 - sg))
        dy[i] = vdo[i] * zs;
      }
      storen<IT, kEt>(gdz + tile * kT, dz);
    }
    lds_stv<kEt>(&s_dl[eo], vd);
    lds_stv<kEt>(&s_u[eo], vu);
    if constexpr (kDA) {
      float va[kEt];
      rawn_to_f32<IT, kEt>(s_raw_a + ro, va);
      lds_stv<kEt>(&s_x[eo], va);
    } else {
      lds_stv<kEt>(&s_x[eo], xu);
    }
    lds_stv<kEt>(&s_dy[eo], dy);
    // read back by this thread only, in the epilogue
    if constexpr (kSP && !kDA) lds_stv<kEt>(&s_sg[eo], sg);
    // B / C rows, transposed to step-major: threads [0, 64) B, [64, 128) C,
    // 4 steps of one state each; states >= N are zero
    if (tid < 2 * 16 * 4) {
      const bool isC = tid >= 64;
      const int j = tid & 63;
      const int n = j >> 2, s4 = (j & 3) * 4;
      float v[4];
      raw4_to_f32<IT>((isC ? s_raw_c : s_raw_b) + n * kRowR + half + s4 * (int)sizeof(IT), v);
      float* dst = (isC ? s_C : s_B) + s4 * 16 + n;
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i * 16] = n < N ? v[i] : 0.f;
    }
  };

  // epilogue of tile: du, ddelta; dD / ddelta_bias terms
  auto epilogue = [&](int64_t tile) __attribute__((always_inline)) {
    float p1[kEt], p2[kEt];
    lds_ldv<kEt>(&s_P1[eo], p1);
    lds_ldv<kEt>(&s_P2[eo], p2);
#pragma unroll
    for (int p = 1; p < kNP; ++p) {
      float q1[kEt], q2[kEt];
      lds_ldv<kEt>(&s_P1[p * kOp + eo], q1);
      lds_ldv<kEt>(&s_P2[p * kOp + eo], q2);
#pragma unroll
      for (int i = 0; i < kEt; ++i) {
        p1[i] += q1[i];
        p2[i] += q2[i];
      }
    }
    float dl[kEt], uu[kEt], dy[kEt], sg[kEt];
    lds_ldv<kEt>(&s_dl[eo], dl);
    lds_ldv<kEt>(&s_u[eo], uu);
    lds_ldv<kEt>(&s_dy[eo], dy);
    if constexpr (kSP && !kDA) lds_ldv<kEt>(&s_sg[eo], sg);
    if constexpr (kSP && kDA) {
#pragma unroll
      for (int i = 0; i < kEt; ++i) sg[i] = one_minus_exp_neg(dl[i]);   // sigmoid(delta + bias)
    }
    float du[kEt], dd[kEt], dda[kEt];
#pragma unroll
    for (int i = 0; i < kEt; ++i) {
      du[i] = (kDi || kBeta) ? fmaf(e_D, dy[i], p1[i]) : fmaf(dl[i], p1[i], e_D * dy[i]);
      const float ddl = kBeta ? p2[i] : kDi ? kLn2 * p2[i] : kDA ? uu[i] * p1[i] : fmaf(uu[i], p1[i], kLn2 * p2[i]);
      dda[i] = kLn2 * p2[i];
      dd[i] = kSP ? ddl * sg[i] : ddl;
      e_dD = fmaf(dy[i], uu[i], e_dD);
      e_dbias += dd[i];
    }
    storen<IT, kEt>(gdu + tile * kT, du);
    storen<IT, kEt>(gddl + tile * kT, dd);
    if constexpr (kDA) storen<IT, kEt>(gddA + tile * kT, dda);
  };

  // ---- prologue: the segment's last tile (segment bounds are multiples of kPair tiles)
  fetch_raw((te - 1) / kPair);
  fetch_ck(te - 1);
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  __syncthreads();
  convert(te - 1);
  __syncthreads();

  for (int64_t tile = te - 1; tile >= tb; --tile) {
    // ---- compute(tile).  The state at the tile start first: the checkpoint
    // rows a wave reads are the rows its own fetch writes (states 4w..4w+3),
    // so once its reads have returned (lgkmcnt(0)) the wave can fetch the
    // next tile's rows into the same buffer.
    float h0[kS];
#pragma unroll
    for (int k = 0; k < kS; ++k) h0[k] = (tile > 0 && ns[k] < N) ? s_ck[ns[k] * kCh + ch] : 0.f;
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    if (tile > tb) {
      // tile - 1 starts a new raw tile when `tile` is the first of its own
      if (tile % kPair == 0) fetch_raw((tile - 1) / kPair);
      fetch_ck(tile - 1);
    }
    // Reduce-scatter of the dB / dC values over the block's channels (the
    // lanes, with 32 channels each lane half on its own).  Stage 1, per step:
    // the lane's kS states over lane bits 3 (row mirror) and 2 (half-row
    // mirror, 4 states only), one DPP add per pair thanks to the register
    // order above; the lane keeps state ns[0].  Stage 2, streamed over the
    // tile's 16 steps as they exist: step bit 3 pairs t with t + 8 over lane
    // bit 4 (32 channels: bit 2, bank-masked DPP), step bit 2 t with t + 4
    // over lane bit 5 (32 channels: bit 4), then step bits 1 and 0 over lane
    // bits 1 and 0 (quad DPP), so at most 8 partials live; the lane ends with
    // step rs_t.
    auto rs_states = [&](const float (&v)[kS]) __attribute__((always_inline)) {
      if constexpr (kS == 4) {
        const float a0 = v[0] + dpp_get<kDppRowMirror>(v[2]);
        const float a1 = v[1] + dpp_get<kDppRowMirror>(v[3]);
        return a0 + dpp_get<kDppRowHalfMirror>(a1);
      } else {
        return v[0] + dpp_get<kDppRowMirror>(v[1]);
      }
    };
    auto rs_pair = [&](float lo, float hi, bool bit, auto ctrl) __attribute__((always_inline)) {
      const float keep = bit ? hi : lo;
      const float send = bit ? lo : hi;
      return keep + dpp_mov<decltype(ctrl)::value>(send);
    };
    auto swap_add16 = [&](float lo, float hi) __attribute__((always_inline)) {   // even rows keep lo
      auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
      return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    };
    auto swap_add32 = [&](float lo, float hi) __attribute__((always_inline)) {   // lanes < 32 keep lo
      auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
      return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    };
    auto rs_b3 = [&](float lo, float hi) __attribute__((always_inline)) {
      if constexpr (kH == 1) return swap_add16(lo, hi);
      else return rs_pair_banked<4>(lo, hi);
    };
    auto rs_b2 = [&](float lo, float hi) __attribute__((always_inline)) {
      if constexpr (kH == 1) return swap_add32(lo, hi);
      else return swap_add16(lo, hi);
    };
    auto rs_b1 = [&](float lo, float hi) __attribute__((always_inline)) {
      return rs_pair(lo, hi, lane & 2, std::integral_constant<int, kDppQuadXor2>{});
    };
    auto rs_b0 = [&](float lo, float hi) __attribute__((always_inline)) {
      return rs_pair(lo, hi, lane & 1, std::integral_constant<int, kDppQuadXor1>{});
    };
    // operands of 4 steps: the step of A_bar (delta', or deltaA) and the input factor x (delta' u)
    auto step_ops = [&](int og, float (&dt)[4], float (&xx)[4]) __attribute__((always_inline)) {
      const float4 d4 = *reinterpret_cast<const float4*>(&s_dl[og]);
      const float4 x4 = *reinterpret_cast<const float4*>(&s_x[og]);
      if constexpr (kDA) {
        const float4 u4 = *reinterpret_cast<const float4*>(&s_u[og]);
        dt[0] = x4.x; dt[1] = x4.y; dt[2] = x4.z; dt[3] = x4.w;
        xx[0] = d4.x * u4.x; xx[1] = d4.y * u4.y; xx[2] = d4.z * u4.z; xx[3] = d4.w * u4.w;
      } else {
        dt[0] = d4.x; dt[1] = d4.y; dt[2] = d4.z; dt[3] = d4.w;
        xx[0] = x4.x; xx[1] = x4.y; xx[2] = x4.z; xx[3] = x4.w;
      }
    };
    // recompute A_bar and h over the tile; dC_t = sum_d dy_t h_t is complete
    // here, so its reduce-scatter runs with it (steps in increasing order)
    float AB[kT][kS], H[kT][kS];
    // the input factor beta of zoh / bilinear from A_bar: expm1(delta' A) / A
    // (zoh; A_bar = exp(delta' A)), delta' r with r = (A_bar + 1) / 2 (bilinear)
    auto beta_of = [&](float ab, float dlt, int k) __attribute__((always_inline)) {
      if constexpr (kM == LRNNX_ZOH) return expm1_from(dlt * Ar[k], ab) * iA[k];
      else return dlt * (0.5f * (ab + 1.f));
    };
    float c8[8], c4[4], c2[2], c1 = 0.f, dC_part = 0.f;
    auto stream_dC = [&](int t, float v) __attribute__((always_inline)) {
      if (t < 8) { c8[t] = v; return; }
      const int j = t - 8;
      const float x3 = rs_b3(c8[j], v);
      if (j < 4) { c4[j] = x3; return; }
      const int k = j - 4;
      const float x2 = rs_b2(c4[k], x3);
      if (k < 2) { c2[k] = x2; return; }
      const int q = k - 2;
      const float x1 = rs_b1(c2[q], x2);
      if (q == 0) { c1 = x1; return; }
      dC_part = rs_b0(c1, x1);
    };
    {
      float hc[kS];
#pragma unroll
      for (int k = 0; k < kS; ++k) hc[k] = h0[k];
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        // scheduling fence: the LDS operand loads of later groups are not
        // hoisted above this group's arithmetic (that would exceed 256 VGPRs)
        __builtin_amdgcn_sched_barrier(0);
        const int og = op_off<0, kCh>(g, ch);
        float dl[4], xx[4];
        step_ops(og, dl, xx);
        const float4 dy4 = *reinterpret_cast<const float4*>(&s_dy[og]);
        const float dy[4] = {dy4.x, dy4.y, dy4.z, dy4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 4 * g + i;
          float bv[kS];
#pragma unroll
          for (int k = 0; k < kS; ++k) bv[k] = s_B[t * 16 + ns[k]];
          const float x = xx[i];
          float vC[kS];
#pragma unroll
          for (int k = 0; k < kS; ++k) {
            float ab, xk = x;   // A_bar and the input factor times u
            if constexpr (kM == LRNNX_BILINEAR) {
              const float v = 0.5f * dl[i] * Ar[k];
              const float r = __builtin_amdgcn_rcpf(1.f - v);
              ab = (1.f + v) * r;
              xk = dl[i] * r * x;
            } else {
              ab = __builtin_amdgcn_exp2f(dl[i] * a2[k]);
              if constexpr (kM == LRNNX_ZOH) xk = beta_of(ab, dl[i], k) * x;
            }
            hc[k] = fmaf(ab, hc[k], xk * bv[k]);
            AB[t][k] = ab;
            H[t][k] = hc[k];
            vC[k] = dy[i] * hc[k];
          }
          stream_dC(t, rs_states(vC));
        }
      }
    }

    // reverse walk; dB's reduce-scatter as dC's, steps in decreasing order
    float r8[8], r4[4], r2[2], r1 = 0.f, dB_part = 0.f;
    auto stream_dB = [&](int t, float v) __attribute__((always_inline)) {
      if (t >= 8) { r8[t - 8] = v; return; }
      const float x3 = rs_b3(v, r8[t]);
      if (t >= 4) { r4[t - 4] = x3; return; }
      const float x2 = rs_b2(x3, r4[t]);
      if (t >= 2) { r2[t - 2] = x2; return; }
      const float x1 = rs_b1(x2, r2[t]);
      if (t == 1) { r1 = x1; return; }
      dB_part = rs_b0(x1, r1);
    };
    float* sP1w = s_P1 + (w * kH + hf) * kOp;   // this lane's partial slots
    float* sP2w = s_P2 + (w * kH + hf) * kOp;
#pragma unroll
    for (int g = kG - 1; g >= 0; --g) {
      __builtin_amdgcn_sched_barrier(0);
      const int og = op_off<0, kCh>(g, ch);
      float dl[4], xx[4];
      step_ops(og, dl, xx);
      const float4 dy4 = *reinterpret_cast<const float4*>(&s_dy[og]);
      const float dy[4] = {dy4.x, dy4.y, dy4.z, dy4.w};
      float p1v[4], p2v[4];
#pragma unroll
      for (int i = 3; i >= 0; --i) {
        const int t = 4 * g + i;
        float bv[kS], cv[kS];
#pragma unroll
        for (int k = 0; k < kS; ++k) {
          bv[k] = s_B[t * 16 + ns[k]];
          cv[k] = s_C[t * 16 + ns[k]];
        }
        const float x = xx[i];
        float p1 = 0.f, p2 = 0.f, vB[kS];
#pragma unroll
        for (int k = 0; k < kS; ++k) {
          const float dh = fmaf(dy[i], cv[k], gn[k]);
          const float gk = AB[t][k] * dh;
          gn[k] = gk;
          const float hp = t > 0 ? H[t - 1][k] : h0[k];
          if constexpr (kBeta) {
            // natural units: the epilogue takes p2 as ddelta' unscaled
            const float be = beta_of(AB[t][k], dl[i], k);
            const float g2 = dh * bv[k];                 // dh B
            const float q = fmaf(Ar[k], hp, x * bv[k]);  // A h_{t-1} + u B
            p1 = fmaf(g2, be, p1);
            if constexpr (kM == LRNNX_ZOH) {
              p2 = fmaf(gk, q, p2);
              dA_acc[k] = fmaf(gk * hp, dl[i], dA_acc[k]);
              dAz[k] = fmaf(g2 * x, fmaf(dl[i], AB[t][k], -be), dAz[k]);
              // accumulate at this step: sinking the chains to the end of the
              // walk keeps every step's operands live (spills past 256 VGPRs)
              pin_vgpr(dA_acc[k]);
              pin_vgpr(dAz[k]);
            } else {
              const float rr = 0.5f * (AB[t][k] + 1.f);
              const float dr = dh * (rr * rr);           // dh r^2
              p2 = fmaf(dr, q, p2);
              dA_acc[k] = fmaf(dr * dl[i], fmaf(0.5f * dl[i], x * bv[k], hp), dA_acc[k]);
            }
            vB[k] = dh * be * x;
          } else {
            const float wv = gk * hp;
            p2 = fmaf(wv, a2[k], p2);   // A log2(e) units; the epilogue multiplies by ln 2
            dA_acc[k] = fmaf(wv, dl[i], dA_acc[k]);
            p1 = fmaf(dh, bv[k], p1);
            vB[k] = dh * x;
          }
        }
        p1v[i] = p1;
        p2v[i] = p2;
        stream_dB(t, rs_states(vB));
      }
      *reinterpret_cast<float4*>(&sP1w[og]) = make_float4(p1v[0], p1v[1], p1v[2], p1v[3]);
      *reinterpret_cast<float4*>(&sP2w[og]) = make_float4(p2v[0], p2v[1], p2v[2], p2v[3]);
    }

    // ---- finish(tile).  The wait covers the fetch of tile - 1 and the stores
    // of the previous finish phase; this tile's partials are stored after it.
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    if (wr_bc) {
      wsB[tile * kT] = dB_part;
      wsC[tile * kT] = dC_part;
    }
    epilogue(tile);
    if (tile > tb) convert(tile - 1);
    __syncthreads();
  }

  // per-((segment, b), d, n) and per-((segment, b), d) partials, summed over
  // the rows by ss_reduce_batch_kernel
#pragma unroll
  for (int k = 0; k < kS; ++k) {
    if constexpr (kM == LRNNX_ZOH) dA_acc[k] = fmaf(dAz[k], iA[k], dA_acc[k]);
    if (ns[k] < N) ws[wo.dA + (prow * D + d0 + ch) * N + ns[k]] = dA_acc[k];
  }
  // dD / ddelta_bias: the kP threads of a channel are consecutive lanes
  e_dD += dpp_mov<kDppQuadXor1>(e_dD);
  e_dD += dpp_mov<kDppQuadXor2>(e_dD);
  e_dbias += dpp_mov<kDppQuadXor1>(e_dbias);
  e_dbias += dpp_mov<kDppQuadXor2>(e_dbias);
  if constexpr (kP == 8) {
    e_dD += __shfl_xor(e_dD, 4);
    e_dbias += __shfl_xor(e_dbias, 4);
  }
  if (eq == 0) {
    ws[wo.dD + prow * D + d0 + er] = e_dD;
    ws[wo.dbias + prow * D + d0 + er] = e_dbias;
  }
}

// Split of L, adjoint summaries: for each segment s >= 1 and state n, the
// adjoint it carries out of its first step when it starts from zero at its
// last step, g <- A_bar_t (C_t dy_t + g) with dy = dout silu(z) (the recurrence
// of the kernel above without the states), and the segment's sum of delta'.
// One thread per (segment, b, d, n), 16 consecutive lanes per channel (lanes
// past d_state idle); 8 steps per 16-byte (bf16) or 32-byte (fp32) load.
template <typename IT>
__device__ __forceinline__ void ld8_f32(const IT* p, float* o) {
  if constexpr (sizeof(IT) == 4) {
    raw_to_f32<IT>(*reinterpret_cast<const uint4*>(p), o);
    raw_to_f32<IT>(*reinterpret_cast<const uint4*>(p + 4), o + 4);
  } else {
    raw_to_f32<IT>(*reinterpret_cast<const uint4*>(p), o);
  }
}

template <typename IT, bool kSP, bool kZ, bool kDA>
__global__ void __launch_bounds__(256)
ssf_bwd_adj_summary_kernel(const lrnnx_selective_scan_args a, const int64_t seg_steps, const int n_seg, float* ws,
                           const SSBwdWs wo) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t B = a.batch, D = a.dim, L = a.seqlen;
  const int N = (int)a.dstate;
  if (i >= (int64_t)(n_seg - 1) * B * D * 16) return;
  const int n = (int)(i & 15);
  const int64_t d = (i >> 4) % D, b = ((i >> 4) / D) % B, s = (i >> 4) / (B * D) + 1;
  const bool on = n < N;
  const int64_t grp = d / (D / a.n_groups);
  const int64_t t0 = s * seg_steps, t1 = t0 + seg_steps < L ? t0 + seg_steps : L;  // multiples of 8
  const float a2 = on ? static_cast<const float*>(a.A.ptr)[d * a.A.s0 + n * a.A.s1] * kLog2e : 0.f;
  const float bias = a.delta_bias.ptr ? static_cast<const float*>(a.delta_bias.ptr)[d * a.delta_bias.s0] : 0.f;
  // the step of A_bar: delta' (or deltaA)
  const IT* pd = kDA ? static_cast<const IT*>(a.deltaA.ptr) + b * a.deltaA.s0 + d * a.deltaA.s1
                     : static_cast<const IT*>(a.delta.ptr) + b * a.delta.s0 + d * a.delta.s1;
  const IT* pdo = static_cast<const IT*>(a.dout.ptr) + b * a.dout.s0 + d * a.dout.s1;
  const IT* pz = kZ ? static_cast<const IT*>(a.z.ptr) + b * a.z.s0 + d * a.z.s1 : nullptr;
  const IT* pc = static_cast<const IT*>(a.C.ptr) + b * a.C.s0 + grp * a.C.s1 + (on ? n : 0) * a.C.s2;
  float g = 0.f, ssum = 0.f;
  for (int64_t tb = t1 - 8; tb >= t0; tb -= 8) {
    float vd[8], vdo[8], vz[8], vc[8];
    ld8_f32<IT>(pd + tb, vd);
    ld8_f32<IT>(pdo + tb, vdo);
    if constexpr (kZ) ld8_f32<IT>(pz + tb, vz);
    ld8_f32<IT>(pc + tb, vc);
#pragma unroll
    for (int j = 7; j >= 0; --j) {
      float dl = kDA ? vd[j] : vd[j] + bias;
      if constexpr (kSP && !kDA) dl = ssf::softplus20_fast(dl);
      float dy = vdo[j];
      if constexpr (kZ) dy *= vz[j] * ssf::sigmoidf_fast(vz[j]);
      ssum += dl;
      g = __builtin_amdgcn_exp2f(dl * a2) * fmaf(dy, vc[j], g);
    }
  }
  if (on) ws[wo.g_loc + ((s * B + b) * N + n) * D + d] = g;
  if (n == 0) ws[wo.dsum + (s * B + b) * D + d] = ssum;
}

// Split of L, adjoint chain (right to left) per (b, n, d): the adjoint entering
// segment S-1 is 0; entering segment s it is
// exp(A sum delta'(s + 1)) g_in(s + 1) + g_loc(s + 1).
template <typename IT>  // one instantiation per unit that launches it
__global__ void __launch_bounds__(256)
ssf_bwd_adj_chain_kernel(const lrnnx_selective_scan_args a, const int n_seg, float* ws, const SSBwdWs wo) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (b, n, d)
  const int64_t B = a.batch, D = a.dim, N = a.dstate;
  if (i >= B * N * D) return;
  const int64_t d = i % D, n = (i / D) % N, b = i / (D * N);
  const float a2 = static_cast<const float*>(a.A.ptr)[d * a.A.s0 + n * a.A.s1] * kLog2e;
  float gi = 0.f;
  ws[wo.g_init + (((int64_t)(n_seg - 1) * B + b) * N + n) * D + d] = 0.f;
  for (int s = n_seg - 2; s >= 0; --s) {
    const int64_t r = (int64_t)(s + 1) * B + b;
    gi = fmaf(__builtin_amdgcn_exp2f(a2 * ws[wo.dsum + r * D + d]), gi, ws[wo.g_loc + (r * N + n) * D + d]);
    ws[wo.g_init + (((int64_t)s * B + b) * N + n) * D + d] = gi;
  }
}

// Shape / option coverage of the fast backward: the forward's.
template <typename IT>
inline bool ssf_bwd_shape_ok(const lrnnx_selective_scan_args& a) {
  return ssf::shape_ok<IT>(a, ssf::kCk, false, true);
}

// Whether the fast backward covers this call.
template <typename IT>
inline bool ssf_bwd_eligible(const lrnnx_selective_scan_args& a) {
  using ssf::rows_aligned;
  if (!ssf_bwd_shape_ok<IT>(a)) return false;
  if (a.deltaA.ptr && (!a.ddeltaA.ptr || !rows_aligned<IT>(a.ddeltaA, false))) return false;
  if (a.z.ptr && (!a.out_saved.ptr || !a.dz.ptr)) return false;
  return rows_aligned<IT>(a.dout, false) && rows_aligned<IT>(a.out_saved, false) && rows_aligned<IT>(a.du, false) &&
         rows_aligned<IT>(a.ddelta, false) && rows_aligned<IT>(a.dz, false);
}

// Segments of the backward's split of L (1: no split): the forward's rule,
// from shapes and options only, so that the workspace size and the launch agree.
template <typename IT>
inline int64_t ssf_bwd_segs(const lrnnx_selective_scan_args& a) {
  // (zoh / bilinear run unsplit: their 32-channel grid is twice the 64-channel one)
  if (!ssf_bwd_shape_ok<IT>(a) || a.method == LRNNX_ZOH || a.method == LRNNX_BILINEAR) return 1;
  const int64_t steps = ssf::seg_steps(a);
  return steps ? ssf::n_segs(a, steps) : 1;
}

// Channels per workgroup of the fast backward (64 or 32), from shapes and
// options only, so that the workspace layout and the launch agree: 32 for an
// unsplit grid of at most 256 64-channel workgroups (with 16-bit I/O only
// together with two-tile fetches, L a multiple of 32), else 64.
// LRNNX_SCAN_CHANNELS forces either where 32 is possible.
template <typename IT>
inline int ssf_bwd_chans(const lrnnx_selective_scan_args& a) {
  if (!ssf_bwd_shape_ok<IT>(a)) return kWave;
  if (a.method == LRNNX_ZOH || a.method == LRNNX_BILINEAR) return kWave / 2;   // (fp32: kRT = 16)
  if (ssf_bwd_segs<IT>(a) > 1) return kWave;
  if (sizeof(IT) == 2 && a.seqlen % (2 * ssf::kCk) != 0) return kWave;
  const int o = scan_channels_override();
  if (o) return o;
  return (a.dim / kWave) * a.batch <= 256 ? kWave / 2 : kWave;
}

// The backward's geometry: channel blocks of the fast kernel's width (the
// dB / dC partials are per channel block).
template <typename IT>
inline SSGeom ssf_bwd_geom(const lrnnx_selective_scan_args& a) {
  SSGeom g = ss_geom(a);
  if (ssf_bwd_chans<IT>(a) == kWave / 2) {
    g.CB = kWave / 2;
    g.n_cb = (int)(a.dim / g.CB);
  }
  return g;
}

template <typename IT, bool kSP, bool kZ, int kM, bool kDA = false>
inline void ssf_bwd_launch_t(const lrnnx_selective_scan_args& a, const SSGeom& g, float* ws, const SSBwdWs& wo,
                             const float* ckp, int64_t seg_steps, hipStream_t st) {
  // Two-tile raw fetches for 16-bit I/O when every segment holds an even
  // number of tiles: L a multiple of 32 (the split's segments are powers of
  // two >= 128 steps).
  constexpr bool kTwo = sizeof(IT) == 2;
  const bool c32 = g.CB == kWave / 2;
  const int64_t S = wo.S, B = a.batch, D = a.dim, N = a.dstate;
  const int64_t seg_tiles = S > 1 ? seg_steps / ssf::kCk : a.seqlen / ssf::kCk;
  if (S > 1) {
    const int64_t nsum = (S - 1) * B * D * 16, nch = B * N * D;
    hipLaunchKernelGGL((ssf_bwd_adj_summary_kernel<IT, kSP, kZ, kDA>), dim3((unsigned)((nsum + 255) / 256)), dim3(256), 0,
                       st, a, seg_steps, (int)S, ws, wo);
    hipLaunchKernelGGL(ssf_bwd_adj_chain_kernel<IT>, dim3((unsigned)((nch + 255) / 256)), dim3(256), 0, st, a, (int)S,
                       ws, wo);
  }
  const dim3 grid((unsigned)(a.dim / g.CB), (unsigned)a.batch, (unsigned)S);
  const dim3 blk(ssf::kNT);
  if constexpr (kTwo) {
    if (a.seqlen % (2 * ssf::kCk) == 0) {
      if (c32)
        hipLaunchKernelGGL((ssf_bwd_kernel<IT, kSP, kZ, 2 * ssf::kCk, kWave / 2, kM, kDA>), grid, blk, 0, st, a, g.n_ck, ws,
                           wo, ckp, seg_tiles);
      else
        hipLaunchKernelGGL((ssf_bwd_kernel<IT, kSP, kZ, 2 * ssf::kCk, kWave, kM, kDA>), grid, blk, 0, st, a, g.n_ck, ws, wo,
                           ckp, seg_tiles);
      return;
    }
    // (the 32-channel form comes with two-tile fetches only: ssf_bwd_chans)
    hipLaunchKernelGGL((ssf_bwd_kernel<IT, kSP, kZ, ssf::kCk, kWave, kM, kDA>), grid, blk, 0, st, a, g.n_ck, ws, wo, ckp,
                       seg_tiles);
  } else if constexpr (kM == LRNNX_ZOH || kM == LRNNX_BILINEAR) {   // 32 channels only (ssf_bwd_chans)
    hipLaunchKernelGGL((ssf_bwd_kernel<IT, kSP, kZ, ssf::kCk, kWave / 2, kM, kDA>), grid, blk, 0, st, a, g.n_ck, ws, wo,
                       ckp, seg_tiles);
  } else {
    if (c32)
      hipLaunchKernelGGL((ssf_bwd_kernel<IT, kSP, kZ, ssf::kCk, kWave / 2, kM, kDA>), grid, blk, 0, st, a, g.n_ck, ws, wo, ckp,
                         seg_tiles);
    else
      hipLaunchKernelGGL((ssf_bwd_kernel<IT, kSP, kZ, ssf::kCk, kWave, kM, kDA>), grid, blk, 0, st, a, g.n_ck, ws, wo, ckp,
                         seg_tiles);
  }
}

template <typename IT>
inline hipError_t ssf_bwd_launch(const lrnnx_selective_scan_args& a, float* ws, const float* ckp, hipStream_t st) {
  const SSGeom g = ssf_bwd_geom<IT>(a);
  const int64_t S = ssf_bwd_segs<IT>(a);
  const SSBwdWs wo = ss_bwd_ws(a, g, a.ckpt == nullptr, S);
  const int64_t steps = S > 1 ? ssf::seg_steps(a) : 0;
  const bool z = a.z.ptr != nullptr;
  auto by_opts = [&](auto m) __attribute__((always_inline)) {
    constexpr int kM = decltype(m)::value;
    if (a.delta_softplus) {
      if (z) ssf_bwd_launch_t<IT, true, true, kM>(a, g, ws, wo, ckp, steps, st);
      else ssf_bwd_launch_t<IT, true, false, kM>(a, g, ws, wo, ckp, steps, st);
    } else {
      if (z) ssf_bwd_launch_t<IT, false, true, kM>(a, g, ws, wo, ckp, steps, st);
      else ssf_bwd_launch_t<IT, false, false, kM>(a, g, ws, wo, ckp, steps, st);
    }
  };
  bool done = false;
  if (a.deltaA.ptr) {   // mamba only (ssf_bwd_shape_ok)
    if (a.delta_softplus) {
      if (z) ssf_bwd_launch_t<IT, true, true, LRNNX_MAMBA, true>(a, g, ws, wo, ckp, steps, st);
      else ssf_bwd_launch_t<IT, true, false, LRNNX_MAMBA, true>(a, g, ws, wo, ckp, steps, st);
    } else {
      if (z) ssf_bwd_launch_t<IT, false, true, LRNNX_MAMBA, true>(a, g, ws, wo, ckp, steps, st);
      else ssf_bwd_launch_t<IT, false, false, LRNNX_MAMBA, true>(a, g, ws, wo, ckp, steps, st);
    }
    done = true;
  } else if constexpr (sizeof(IT) == 4) {   // the other methods: fp32 input only (shape_ok)
    done = true;
    switch (a.method) {
      case LRNNX_DIRAC: by_opts(std::integral_constant<int, LRNNX_DIRAC>{}); break;
      case LRNNX_ZOH: by_opts(std::integral_constant<int, LRNNX_ZOH>{}); break;
      case LRNNX_BILINEAR: by_opts(std::integral_constant<int, LRNNX_BILINEAR>{}); break;
      default: done = false;
    }
  }
  if (!done) by_opts(std::integral_constant<int, LRNNX_MAMBA>{});
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return ss_bwd_reductions<IT, true, true>(a, g, ws, wo, st);
}

}  // namespace lrnnx
