// Selective scan forward, fast path of the headline case (gfx950).
//
// Covers: method "mamba" (f32 / bf16 / f16 I/O; with or without deltaA, the
// step of A_bar in Mamba's event mode), and at f32 I/O "dirac" (input term
// B u), "zoh" (A_bar = exp(delta' A), input factor expm1(delta' A) / A) and
// "bilinear" (A_bar = (1 + delta' A / 2) / (1 - delta' A / 2), input factor
// delta' / (1 - delta' A / 2)), variable B and C of any group count,
// d_state <= 16, real fp32 A, d_model a multiple
// of 64 per group, L a multiple of the tile length, 16-byte aligned rows
// (ssf_fwd_eligible).  Everything else runs the generic kernel of
// ss_fwd_impl.h.  Semantics are those of the reference kernel
// csrc/selective_scan/selective_scan.cuh:73-382 (delta' = softplus(delta +
// bias) with threshold 20, h_t = exp(delta' A) h_{t-1} + delta' B_t u_t,
// y = sum_n C_t h_t + D u, out_z = y silu(z), chunk carries every 2048 steps).
//
// Decomposition: one workgroup = one batch row and 64 channels; 4 waves, wave
// w owns states 4w..4w+3 of every channel (lane = channel) with their fp32 h
// in VGPRs.  L is walked in tiles of kT steps (64 bytes of every input row).
// Per tile k:
//   compute(k)  issue the LDS-DMA fetch of raw tile k+1 (u, delta, z, B, C),
//               then run the kT steps of the recurrence for the wave's states
//               and write the wave's partial y (sum over its states of C h).
//   finish(k)   wait + barrier; epilogue of tile k: y = partials of the 4
//               waves + D u (a fifth partial written by the conversion),
//               out / out_z as 16-byte stores; conversion of raw tile k+1 into
//               the fp32 operands delta', delta' u, D u and B, C rows.
// The per-element work of both phases is done by a fixed thread -> (channel,
// 16-byte block) map, so a thread rewrites its own D u slot right after the
// epilogue has read it.  The chunk carries x hold, at each 2048-step chunk
// end, the product of A_bar since the sequence start (the reference's running
// prefix, selective_scan.cuh:316-333), exp(A sum delta'); each thread
// accumulates the sum of its own block over the tiles and the block sums of a
// channel are added when a chunk ends.
#pragma once
#include <type_traits>

#include "ss_common.h"
#include "tile_io.h"

namespace lrnnx {

namespace ssf {

constexpr int kNW = 4;             // waves per workgroup
constexpr int kS = 4;              // states per wave
constexpr int kNT = kNW * kWave;   // threads per workgroup
constexpr int kCk = 16;            // checkpoint interval (same layout as ss_fwd_kernel with kS = 4)

template <typename IT>
__host__ __device__ constexpr int tile_steps() { return (int)(64 / sizeof(IT)); }  // 64-byte rows

// softplus with the reference's threshold 20; log1p by a 4-term series below 1/32
__device__ __forceinline__ float softplus20_fast(float x) {
  const float e = __builtin_amdgcn_exp2f(x * kLog2e);
  const float small = e * fmaf(e, fmaf(e, fmaf(e, -0.25f, 0.33333334f), -0.5f), 1.f);
  const float big = __builtin_amdgcn_logf(1.f + e) * kLn2;
  const float r = e < 0.03125f ? small : big;
  return x > 20.f ? x : r;
}

// Float offset of (4-step group g, channel row r) in a [g][64][4] fp32 operand
// tile.  Rows are XOR-swizzled by 2 * (g >> kSh) so that both access patterns
// are free of LDS bank conflicts: a wave reading one group for its 64 lanes
// (a permutation of 64 consecutive 16-byte slots), and the per-element phases,
// where lane 4 r + q handles groups of one row r (consecutive lanes then hit
// different 16-byte bank groups).  kSh = log2(4-step groups per thread).
template <int kSh, int kRows = kWave>
__device__ __forceinline__ int op_off(int g, int r) {
  return (g * kRows + (r ^ ((g >> kSh) << 1))) * 4;
}

__device__ __forceinline__ float sigmoidf_fast(float z) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-z * kLog2e));
}

// Split of L into segments for grids too small to fill the chip (blockIdx.z =
// segment).  Segment s covers tiles [s * tiles, min((s + 1) * tiles, n_tiles)).
// Summary pass: h_end != nullptr; the segment runs from h = 0 and writes its
// final state and its sum of delta' (no other outputs).  Main pass: h_init !=
// nullptr; the segment starts from h_init and from dsum_pre, the sum of delta'
// from the sequence start to the segment start (for the x carries).
// Buffers: states [seg][b][n][d], sums [seg][b][d].  Checkpoint rebuild
// (kOut = false, below): x_seed != nullptr; segments are the 2048-step chunks
// of the x carries and segment s > 0 starts from the state x holds at the end
// of chunk s - 1.
struct SsfSeg {
  int64_t tiles;
  const float* h_init;
  const float* dsum_pre;
  float* h_end;
  float* dsum_seg;
  const float* x_seed;
};

}  // namespace ssf

// kOut = false: checkpoint rebuild for a backward that was given no
// checkpoints.  Only the states run (no C, no y, no z, no out / x writes):
// the per-step work drops to exp, two multiplies and the state FMA, and the
// per-element work to softplus and delta' u.
// kCh: channels per workgroup.  64: lane = channel, 4 states per lane (wave
// w: states 4w..4w+3).  32: lane = channel + 32 half, 2 states per lane (the
// lower half of wave w holds states 4w, 4w+1, the upper half 4w+2, 4w+3), so
// that a grid too small to give every CU two 64-channel workgroups (at most
// 256 of them) runs twice as many workgroups, two per CU.  The 32-channel
// form walks 32-step tiles whatever the element size.
// kDA: deltaA given (mamba): A_bar = exp(deltaA A), the chunk carries' sums
// run over deltaA, and delta' enters the input term only.  Its raw tile takes
// the LDS of the D u partial, which stays in registers (no faster, no slower).
// kM: the method (LRNNX_MAMBA, DIRAC, ZOH or BILINEAR), compile-time.
template <typename IT, bool kSP, bool kZ, bool kOut = true, int kCh = kWave, int kM = LRNNX_MAMBA, bool kDA = false>
__global__ void __launch_bounds__(ssf::kNT)
ssf_fwd_kernel(const lrnnx_selective_scan_args a, const int64_t n_ck, const ssf::SsfSeg sg) {
  using namespace ssf;
  static_assert(kOut || !kZ, "the checkpoint rebuild reads no z");
  static_assert(kCh == kWave || kCh == kWave / 2, "64 or 32 channels per workgroup");
  static_assert(kM == LRNNX_MAMBA || kM == LRNNX_DIRAC || kM == LRNNX_ZOH || kM == LRNNX_BILINEAR, "method");
  static_assert(kM == LRNNX_MAMBA || sizeof(IT) == 4, "methods other than mamba take fp32 input only");
  static_assert(kM == LRNNX_MAMBA || !kDA, "deltaA on the fast path: mamba only");
  constexpr bool kUx = kM != LRNNX_MAMBA;        // the operand x is u (the input factor is per state)
  constexpr bool kProd = kM == LRNNX_BILINEAR;   // chunk carries from a running product of A_bar
  constexpr int kH = kWave / kCh;                                 // lane halves per wave
  constexpr int kS = 16 / kNW / kH;                               // states per lane
  constexpr int kT = kCh == kWave ? tile_steps<IT>() : 32;        // steps per tile
  constexpr int kE = 16 / sizeof(IT);                             // elements per 16-byte block
  constexpr int kQ = kT / kE;                                     // blocks per raw row
  constexpr int kEt = kCh * kT / kNT;                             // elements per thread (per-element phases)
  constexpr int kP = kT / kEt;                                    // threads per row
  constexpr int kG = kT / 4;                                      // groups of 4 steps
  constexpr int kSh = kEt == 8 ? 1 : 0;                           // log2(4-step groups per thread)
  constexpr int kNP = kNW * kH;                                   // y partials per element
  constexpr int kOp = kG * kCh * 4;                               // floats of a [g][ch][4] operand tile
  constexpr int kRaw = kCh * kT * (int)sizeof(IT);                // [kCh][kT] raw tile, bytes
  constexpr int kRawS = 16 * kT * (int)sizeof(IT);                // [16][kT] raw B or C tile
  constexpr int kInR = kCh * kQ / kWave;                          // fetch instructions per channel tile
  constexpr int kInS = (16 * kQ + kWave - 1) / kWave;             // fetch instructions per B / C tile
  static_assert(kEt == 4 || kEt == 8, "a thread converts one or two 4-step groups");
  static_assert(kEt == kE || (kEt == 4 && sizeof(IT) == 2), "a thread reads one block or half of one");
  static_assert(kInR <= kNW && 2 * kInS <= kNW, "one fetch instruction per wave and tensor");
  static_assert(kCk % kT == 0 || kT % kCk == 0, "checkpoint interval vs tile");

  __shared__ __attribute__((aligned(16))) char s_raw_u[kRaw];
  __shared__ __attribute__((aligned(16))) char s_raw_d[kRaw];
  __shared__ __attribute__((aligned(16))) char s_raw_z[kZ ? 2 * kRaw : 16];
  __shared__ __attribute__((aligned(16))) char s_raw_b[kRawS];
  __shared__ __attribute__((aligned(16))) char s_raw_c[kOut ? kRawS : 16];
  __shared__ __attribute__((aligned(16))) char s_raw_a[kDA ? kRaw : 16];       // deltaA
  __shared__ __attribute__((aligned(16))) float s_dl[kOp];                  // [g][ch][4] delta' (deltaA: deltaA)
  __shared__ __attribute__((aligned(16))) float s_x[kOp];                   // [g][ch][4] delta' u (other methods: u)
  __shared__ __attribute__((aligned(16))) float s_B[16 * kT];               // [n][t]
  __shared__ __attribute__((aligned(16))) float s_C[kOut ? 16 * kT : 4];
  constexpr int kYSlots = kNP + (kDA ? 0 : 1);   // wave partials (+ D u)
  __shared__ __attribute__((aligned(16))) float s_Y[kOut ? kYSlots * kOp : 4];  // [partial][g][ch][4]; kNP: D u
  __shared__ __attribute__((aligned(16))) float s_dsum[kNT];                // [ch][kP] chunk sums of delta'

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ch = lane & (kCh - 1), hf = lane / kCh;   // the lane's channel and lane half
  const int64_t b = blockIdx.y;
  const int64_t D = a.dim, L = a.seqlen;
  const int N = (int)a.dstate;
  const int64_t d0 = (int64_t)blockIdx.x * kCh;
  const int64_t grp = d0 / (D / a.n_groups);
  const int n0 = w * (16 / kNW) + hf * kS;            // the lane's first state

  // thread -> (row er, piece eq of kEt elements) of the per-element phases
  const int er = tid / kP, eq = tid % kP;

  const IT* gu = static_cast<const IT*>(a.u.ptr) + b * a.u.s0 + d0 * a.u.s1;
  const IT* gd = static_cast<const IT*>(a.delta.ptr) + b * a.delta.s0 + d0 * a.delta.s1;
  const IT* gz = kZ ? static_cast<const IT*>(a.z.ptr) + b * a.z.s0 + d0 * a.z.s1 : nullptr;
  const IT* gB = static_cast<const IT*>(a.B.ptr) + b * a.B.s0 + grp * a.B.s1;
  const IT* gC = static_cast<const IT*>(a.C.ptr) + b * a.C.s0 + grp * a.C.s1;
  IT* go = a.out.ptr ? static_cast<IT*>(a.out.ptr) + b * a.out.s0 + (d0 + er) * a.out.s1 + eq * kEt : nullptr;
  IT* goz = kZ ? static_cast<IT*>(a.out_z.ptr) + b * a.out_z.s0 + (d0 + er) * a.out_z.s1 + eq * kEt : nullptr;
  const IT* gA = kDA ? static_cast<const IT*>(a.deltaA.ptr) + b * a.deltaA.s0 + d0 * a.deltaA.s1 : nullptr;
  const uint32_t su = (uint32_t)a.u.s1, sd = (uint32_t)a.delta.s1, sz = (uint32_t)a.z.s1;
  const uint32_t sBn = (uint32_t)a.B.s2, sCn = (uint32_t)a.C.s2;
  float* ckp = static_cast<float*>(a.ckpt);
  float* xp = kOut ? static_cast<float*>(a.x) : nullptr;

  // per-lane constants of the recurrence (channel d0 + ch, states n0 .. n0 + kS - 1)
  float a2[kS], h[kS];
  float Ar[kM == LRNNX_ZOH || kProd ? kS : 1], iA[kM == LRNNX_ZOH ? kS : 1], pA[kProd ? kS : 1];
#pragma unroll
  for (int k = 0; k < kS; ++k) {
    const int n = n0 + k;
    const float Av = n < N ? static_cast<const float*>(a.A.ptr)[(d0 + ch) * a.A.s0 + n * a.A.s1] : -1.f;
    a2[k] = Av * kLog2e;
    if constexpr (kM == LRNNX_ZOH || kProd) Ar[k] = Av;
    if constexpr (kM == LRNNX_ZOH) iA[k] = 1.f / Av;
    if constexpr (kProd) pA[k] = 1.f;   // product of A_bar since the sequence start
    h[k] = (sg.h_init && n < N) ? sg.h_init[((blockIdx.z * a.batch + b) * N + n) * D + d0 + ch] : 0.f;
    if (!kOut && sg.x_seed && blockIdx.z > 0 && n < N)   // the state at the end of chunk z - 1
      h[k] = sg.x_seed[((b * D + d0 + ch) * ((L + kXChunk - 1) / kXChunk) + blockIdx.z - 1) * 2 * N + 2 * n + 1];
  }
  // per-thread constants of the per-element phases (channel d0 + er)
  const float e_bias = a.delta_bias.ptr ? static_cast<const float*>(a.delta_bias.ptr)[(d0 + er) * a.delta_bias.s0] : 0.f;
  const float e_D = a.D.ptr ? static_cast<const float*>(a.D.ptr)[(d0 + er) * a.D.s0] : 0.f;
  // sum of this thread's delta' since the sequence start (a segment takes the
  // sum before its start on one thread of each channel)
  float e_dsum = (sg.dsum_pre && eq == 0) ? sg.dsum_pre[(blockIdx.z * a.batch + b) * D + d0 + er] : 0.f;
  float e_seg = 0.f;  // sum of this thread's delta' over the segment (summary pass)
  float e_du[kDA ? kEt : 1];  // deltaA: this thread's D u of the converted tile

  const int64_t n_tiles = L / kT;
  const int64_t tb = (int64_t)blockIdx.z * sg.tiles;                     // this segment's tiles
  const int64_t te = tb + sg.tiles < n_tiles ? tb + sg.tiles : n_tiles;
  const int64_t n_xc = (L + kXChunk - 1) / kXChunk;

  // Tile fetches: at most one LDS-DMA instruction per wave and tensor (kCh
  // rows x kQ blocks: waves 0 .. kInR - 1), with per-lane byte offsets fixed
  // along L; per tile only the scalar base moves.  B on waves [0, kInS), C on
  // waves [kInS, 2 kInS) (N * kQ blocks each).
  const bool bc_b = w < kInS;
  const int bc_i = bc_b ? w : w - kInS;
  const uint32_t off_u = dma_lane_offset<IT, kQ>(su, w, lane);
  const uint32_t off_d = dma_lane_offset<IT, kQ>(sd, w, lane);
  const uint32_t off_z = kZ ? dma_lane_offset<IT, kQ>(sz, w, lane) : 0u;
  const uint32_t off_a = kDA ? dma_lane_offset<IT, kQ>((uint32_t)a.deltaA.s1, w, lane) : 0u;
  const uint32_t off_bc = dma_lane_offset<IT, kQ>(bc_b ? sBn : sCn, bc_i, lane);
  auto fetch = [&](int64_t tile) __attribute__((always_inline)) {
    const int64_t t0 = tile * kT;
    tile_fetch_async_s<kQ>(gu + t0, off_u, kCh, s_raw_u, w, lane);
    tile_fetch_async_s<kQ>(gd + t0, off_d, kCh, s_raw_d, w, lane);
    if constexpr (kZ) tile_fetch_async_s<kQ>(gz + t0, off_z, kCh, s_raw_z + (tile & 1) * kRaw, w, lane);
    if constexpr (kDA) tile_fetch_async_s<kQ>(gA + t0, off_a, kCh, s_raw_a, w, lane);
    if (bc_b) tile_fetch_async_s<kQ>(gB + t0, off_bc, N, s_raw_b, bc_i, lane);
    else if (kOut && w < 2 * kInS) tile_fetch_async_s<kQ>(gC + t0, off_bc, N, s_raw_c, bc_i, lane);
  };

  // kEt raw elements of this thread (byte offset kEt * sizeof(IT) * tid of a raw tile) -> floats
  auto load_el = [&](const char* raw, float* v) __attribute__((always_inline)) {
    if constexpr (kEt == kE) raw_to_f32<IT>(*reinterpret_cast<const uint4*>(raw + 16 * tid), v);
    else raw4_to_f32<IT>(raw + kEt * (int)sizeof(IT) * tid, v);
  };
  auto store_el = [&](IT* p, const float* v) __attribute__((always_inline)) {
    if constexpr (kEt == kE) *reinterpret_cast<uint4*>(p) = f32_to_raw<IT>(v);
    else store4<IT>(p, v);
  };

  // raw tile -> fp32 operands; thread tid owns row er, steps eq*kEt .. +kEt
  auto convert = [&]() __attribute__((always_inline)) {
    float vu[kEt], vd[kEt], va[kEt];
    load_el(s_raw_u, vu);
    load_el(s_raw_d, vd);
    if constexpr (kDA) load_el(s_raw_a, va);
    float dsum = 0.f;
#pragma unroll
    for (int i = 0; i < kEt; ++i) {
      const float x = vd[i] + e_bias;
      const float dl = kSP ? softplus20_fast(x) : x;
      dsum += kDA ? va[i] : dl;
      vd[i] = dl;
    }
    e_dsum += dsum;
    e_seg += dsum;
#pragma unroll
    for (int i = 0; i < kEt; i += 4) {
      const int o = op_off<kSh, kCh>((eq * kEt + i) >> 2, er);
      if constexpr (kDA)
        *reinterpret_cast<float4*>(s_dl + o) = make_float4(va[i], va[i + 1], va[i + 2], va[i + 3]);
      else
        *reinterpret_cast<float4*>(s_dl + o) = make_float4(vd[i], vd[i + 1], vd[i + 2], vd[i + 3]);
      if constexpr (kUx)
        *reinterpret_cast<float4*>(s_x + o) = make_float4(vu[i], vu[i + 1], vu[i + 2], vu[i + 3]);
      else
        *reinterpret_cast<float4*>(s_x + o) =
            make_float4(vd[i] * vu[i], vd[i + 1] * vu[i + 1], vd[i + 2] * vu[i + 2], vd[i + 3] * vu[i + 3]);
      if constexpr (kOut && kDA) {
#pragma unroll
        for (int m = 0; m < 4; ++m) e_du[i + m] = e_D * vu[i + m];
      } else if constexpr (kOut) {
        *reinterpret_cast<float4*>(s_Y + kNP * kOp + o) =
            make_float4(e_D * vu[i], e_D * vu[i + 1], e_D * vu[i + 2], e_D * vu[i + 3]);
      }
    }
    // B / C rows: threads [0, 16 kQ) convert B, [16 kQ, 32 kQ) C, one 16-byte
    // block each; rows >= N are zero
    if (tid < (kOut ? 2 : 1) * 16 * kQ) {
      const bool isC = tid >= 16 * kQ;
      const int j = isC ? tid - 16 * kQ : tid;
      const int n = j / kQ;
      float v[kE];
      raw_to_f32<IT>(*reinterpret_cast<const uint4*>((isC ? s_raw_c : s_raw_b) + 16 * j), v);
      float* dst = (isC ? s_C : s_B) + j * kE;
#pragma unroll
      for (int i = 0; i < kE; i += 4)
        *reinterpret_cast<float4*>(dst + i) = n < N ? make_float4(v[i], v[i + 1], v[i + 2], v[i + 3])
                                                    : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };

  auto epilogue = [&](int64_t tile) __attribute__((always_inline)) {
    float y[kEt];
#pragma unroll
    for (int i = 0; i < kEt; i += 4) {
      const int o = op_off<kSh, kCh>((eq * kEt + i) >> 2, er);
      float4 acc;
      if constexpr (kDA) acc = make_float4(e_du[i], e_du[i + 1], e_du[i + 2], e_du[i + 3]);
      else acc = *reinterpret_cast<const float4*>(s_Y + kNP * kOp + o);
#pragma unroll
      for (int p = 0; p < kNP; ++p) {
        const float4 q = *reinterpret_cast<const float4*>(s_Y + p * kOp + o);
        acc.x += q.x; acc.y += q.y; acc.z += q.z; acc.w += q.w;
      }
      y[i] = acc.x; y[i + 1] = acc.y; y[i + 2] = acc.z; y[i + 3] = acc.w;
    }
    const int64_t t0 = tile * kT;
    if (go) store_el(go + t0, y);
    if constexpr (kZ) {
      float vz[kEt];
      load_el(s_raw_z + (tile & 1) * kRaw, vz);
#pragma unroll
      for (int i = 0; i < kEt; ++i) y[i] *= vz[i] * sigmoidf_fast(vz[i]);
      store_el(goz + t0, y);
    }
  };

  // chunk carry after the last step of `tile`: (exp(A sum delta'), h) per
  // state; bilinear: (the running product of A_bar, h)
  auto store_x = [&](int64_t tile) __attribute__((always_inline)) {
    float S = 0.f;
#pragma unroll
    for (int q = 0; q < kP; q += 4) {
      const float4 s4 = *reinterpret_cast<const float4*>(s_dsum + ch * kP + q);
      S += (s4.x + s4.y) + (s4.z + s4.w);
    }
    const int64_t c = (tile * kT) / kXChunk;
    float* xr = xp + ((b * D + d0 + ch) * n_xc + c) * 2 * N;
#pragma unroll
    for (int k = 0; k < kS; ++k) {
      if (n0 + k < N) {
        if constexpr (kProd) xr[2 * (n0 + k)] = pA[k];
        else xr[2 * (n0 + k)] = __builtin_amdgcn_exp2f(a2[k] * S);
        xr[2 * (n0 + k) + 1] = h[k];
      }
    }
  };
  // fp32 state hv after step t_end - 1 (t_end a multiple of kCk): checkpoint t_end / kCk - 1
  auto store_ckpt = [&](int64_t t_end, const float* hv) __attribute__((always_inline)) {
    float* cp = ckp + ((b * n_ck + t_end / kCk - 1) * N + n0) * D + d0 + ch;
#pragma unroll
    for (int k = 0; k < kS; ++k)
      if (n0 + k < N) cp[(int64_t)k * D] = hv[k];
  };
  auto chunk_end = [&](int64_t tile) __attribute__((always_inline)) {
    return ((tile + 1) * kT) % kXChunk == 0 || tile + 1 == n_tiles;
  };

  // ---- prologue: the segment's first tile
  fetch(tb);
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  __syncthreads();
  convert();
  __syncthreads();

  float* sYw = s_Y + (w * kH + hf) * kOp;   // this lane's y partial slot
  for (int64_t tile = tb; tile < te; ++tile) {
    if (tile + 1 < te) fetch(tile + 1);
    if (tile > tb && xp && chunk_end(tile - 1)) store_x(tile - 1);

    // ---- compute(tile)
    const int64_t t0 = tile * kT;
    constexpr int kMid = kT > kCk ? kT / kCk - 1 : 0;   // checkpoints inside a tile
    float hmid[kMid > 0 ? kMid : 1][kS];
#pragma unroll
    for (int g = 0; g < kG; ++g) {
      const int og = op_off<kSh, kCh>(g, ch);
      const float4 dl4 = *reinterpret_cast<const float4*>(s_dl + og);
      const float4 x4 = *reinterpret_cast<const float4*>(s_x + og);
      float4 b4[kS], c4[kS];
#pragma unroll
      for (int k = 0; k < kS; ++k) {
        b4[k] = *reinterpret_cast<const float4*>(s_B + (n0 + k) * kT + 4 * g);
        if constexpr (kOut) c4[k] = *reinterpret_cast<const float4*>(s_C + (n0 + k) * kT + 4 * g);
      }
      const float dlv[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
      const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < kS; ++k) {
          float ab, xk = xv[i];   // A_bar and the input factor times u
          if constexpr (kM == LRNNX_BILINEAR) {
            const float v = 0.5f * dlv[i] * Ar[k];
            const float r = __builtin_amdgcn_rcpf(1.f - v);
            ab = (1.f + v) * r;
            xk = dlv[i] * r * xv[i];
            pA[k] *= ab;
          } else {
            ab = __builtin_amdgcn_exp2f(dlv[i] * a2[k]);
            if constexpr (kM == LRNNX_ZOH) xk = expm1_from(dlv[i] * Ar[k], ab) * iA[k] * xv[i];
          }
          h[k] = fmaf(ab, h[k], xk * (&b4[k].x)[i]);
          if constexpr (kOut) acc = fmaf((&c4[k].x)[i], h[k], acc);
        }
        y[i] = acc;
      }
      if constexpr (kOut) *reinterpret_cast<float4*>(sYw + og) = make_float4(y[0], y[1], y[2], y[3]);
      // checkpoints inside the tile: kept in registers and stored after the
      // barrier below with the one at the tile end, so that the wait before
      // the barrier (for the next tile's fetch) does not wait for them
      if (ckp != nullptr && ((4 * g + 4) % kCk) == 0 && 4 * g + 4 < kT) {
#pragma unroll
        for (int k = 0; k < kS; ++k) hmid[(4 * g + 4) / kCk - 1][k] = h[k];
      }
    }

    // ---- finish(tile).  The wait covers the fetch of tile + 1 and the stores
    // of the previous finish phase.
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    if (ckp != nullptr) {
#pragma unroll
      for (int m = 0; m < kMid; ++m) store_ckpt(t0 + (m + 1) * kCk, hmid[m]);
      store_ckpt(t0 + kT, h);
    }
    if constexpr (kOut) epilogue(tile);
    if (chunk_end(tile)) {
      s_dsum[tid] = e_dsum;
    }
    if (tile + 1 < te) convert();
    __syncthreads();
  }
  if (xp && chunk_end(te - 1)) store_x(te - 1);
  if (sg.h_end) {  // summary pass: the segment's final state and sum of delta'
#pragma unroll
    for (int k = 0; k < kS; ++k)
      if (n0 + k < N) sg.h_end[((blockIdx.z * a.batch + b) * N + n0 + k) * D + d0 + ch] = h[k];
    // the kP threads of a channel are consecutive lanes
    e_seg += dpp_mov<kDppQuadXor1>(e_seg);
    e_seg += dpp_mov<kDppQuadXor2>(e_seg);
    if constexpr (kP == 8) e_seg += __shfl_xor(e_seg, 4);
    if (eq == 0) sg.dsum_seg[(blockIdx.z * a.batch + b) * D + d0 + er] = e_seg;
  }
}

// Chains the segments' carries, in segment order, per (b, n, d):
// h_init[0] = 0, h_init[s + 1] = exp(A dsum_seg[s]) h_init[s] + h_end[s];
// and per (b, d) the sum of delta' before each segment's start.
template <typename IT>  // one instantiation per unit that launches it
__global__ void __launch_bounds__(256)
ssf_seg_chain_kernel(const lrnnx_selective_scan_args a, const ssf::SsfSeg sg, const int n_seg,
                     float* __restrict__ h_init, float* __restrict__ dsum_pre) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (b, n, d)
  const int64_t B = a.batch, D = a.dim, N = a.dstate;
  if (i >= B * N * D) return;
  const int64_t d = i % D, n = (i / D) % N, b = i / (D * N);
  const float a2 = static_cast<const float*>(a.A.ptr)[d * a.A.s0 + n * a.A.s1] * kLog2e;
  float carry = 0.f, pre = 0.f;
  for (int s = 0; s < n_seg; ++s) {
    const int64_t o = ((s * B + b) * N + n) * D + d;
    h_init[o] = carry;
    if (n == 0) dsum_pre[(s * B + b) * D + d] = pre;
    if (s + 1 < n_seg) {
      const float ds = sg.dsum_seg[(s * B + b) * D + d];
      carry = fmaf(__builtin_amdgcn_exp2f(a2 * ds), carry, sg.h_end[o]);
      pre += ds;
    }
  }
}

namespace ssf {
// A sequence view whose rows (and, for 4-D B / C, state rows) all start on
// 16-byte boundaries, as the LDS-DMA tile fetch and the vector stores need.
template <typename IT>
inline bool rows_aligned(const lrnnx_view& v, bool four_d) {
  if (v.ptr == nullptr) return true;
  const int64_t s = sizeof(IT);
  return (reinterpret_cast<uintptr_t>(v.ptr) & 15u) == 0 && (v.s0 * s) % 16 == 0 && (v.s1 * s) % 16 == 0 &&
         (!four_d || (v.s2 * s) % 16 == 0);
}

// The tile fetches' 32-bit lane offsets reach a tile of this view: 64 channel
// rows (s1 apart; 16 state rows s2 apart for B / C) of `row_bytes` bytes.
template <typename IT>
inline bool fetch_fits(const lrnnx_view& v, bool states, int64_t row_bytes) {
  if (v.ptr == nullptr) return true;
  return dma_offsets_fit(states ? v.s2 : v.s1, states ? 16 : kWave, row_bytes, sizeof(IT));
}

// Shape / option part of the fast-path coverage (both directions).
// fwd: the coverage of the forward (deltaA with mamba), else of the backward
// (ssf_bwd_shape_ok adds deltaA without softplus).
template <typename IT>
inline bool shape_ok(const lrnnx_selective_scan_args& a, int64_t tile, bool fwd = false, bool bwd_dA = false) {
  // "mamba" at every input type; "dirac", "zoh" and "bilinear" at fp32 input
  const bool f32 = sizeof(IT) == 4;
  const bool m_ok = a.method == LRNNX_MAMBA ||
                    (f32 && (a.method == LRNNX_DIRAC || a.method == LRNNX_ZOH || a.method == LRNNX_BILINEAR));
  if (!m_ok || a.wtype != LRNNX_F32 || !a.var_B || !a.var_C) return false;
  if (a.deltaA.ptr && (!(fwd || bwd_dA) || a.method != LRNNX_MAMBA)) return false;
  if (a.deltaA.ptr && (!fetch_fits<IT>(a.deltaA, false, 64) || !rows_aligned<IT>(a.deltaA, false))) return false;
  if (a.dstate < 1 || a.dstate > 16 || a.seqlen <= 0 || a.seqlen % tile != 0) return false;
  if (a.n_groups <= 0 || a.dim % a.n_groups != 0 || (a.dim / a.n_groups) % kWave != 0) return false;
  // the checkpoint rows (d_state rows of 64 fp32, D apart) of the backward's fetch
  if (!dma_offsets_fit(a.dim, a.dstate, kWave * 4, 4)) return false;
  const int64_t rb = 64;  // bytes of one row of the largest tile (64-byte rows)
  if (!fetch_fits<IT>(a.u, false, rb) || !fetch_fits<IT>(a.delta, false, rb) || !fetch_fits<IT>(a.z, false, rb) ||
      !fetch_fits<IT>(a.dout, false, rb) || !fetch_fits<IT>(a.out_saved, false, rb) ||
      !fetch_fits<IT>(a.B, true, rb) || !fetch_fits<IT>(a.C, true, rb))
    return false;
  return rows_aligned<IT>(a.u, false) && rows_aligned<IT>(a.delta, false) && rows_aligned<IT>(a.z, false) &&
         rows_aligned<IT>(a.B, true) && rows_aligned<IT>(a.C, true);
}
}  // namespace ssf

// Whether the fast forward covers this call (see the header comment).
template <typename IT>
inline bool ssf_fwd_eligible(const lrnnx_selective_scan_args& a) {
  if (!ssf::shape_ok<IT>(a, ssf::tile_steps<IT>(), true)) return false;   // (forward coverage)
  if ((a.z.ptr != nullptr) != (a.out_z.ptr != nullptr)) return false;
  return ssf::rows_aligned<IT>(a.out, false) && ssf::rows_aligned<IT>(a.out_z, false);
}

bool l_split_enabled();         // capi.hip: LRNNX_SCAN_NO_SPLIT
int scan_channels_override();   // capi.hip: LRNNX_SCAN_CHANNELS

namespace ssf {
// Steps per segment of the L split: 0 (no split) when the split is switched
// off (l_split_enabled) or for grids of more than 64 workgroups (B * D / 64),
// which run unsplit in 32-channel workgroups (chans_for) on at least half the
// CUs; there the split's summary pass costs more than its parallelism gains
// (measured at 96 and 128 workgroups, L = 2048: unsplit fwd 0.145-0.151 ms /
// bwd 0.37-0.39 ms against split 0.155-0.167 / 0.41-0.47 ms).  Otherwise the
// shortest power of two >= 128 steps that keeps the grid at most 512
// workgroups.  Powers of two keep every 2048-step chunk boundary on a
// segment boundary and are multiples of every tile length.
inline int64_t seg_steps(const lrnnx_selective_scan_args& a) {
  const int64_t wgs = (a.dim / kWave) * a.batch;
  // (the carry chain is exp(A sum delta') h: not bilinear's A_bar)
  if (wgs > 64 || !l_split_enabled() || a.method == LRNNX_BILINEAR) return 0;
  int64_t steps = 128;
  while (steps < a.seqlen && wgs * ((a.seqlen + steps - 1) / steps) > 512) steps *= 2;
  return steps < a.seqlen ? steps : 0;
}
inline int64_t n_segs(const lrnnx_selective_scan_args& a, int64_t steps) { return (a.seqlen + steps - 1) / steps; }
// Channels per workgroup of an unsplit output launch: 32 when 64-channel
// workgroups would number at most 256 (one per CU, one wave per SIMD), so
// that the doubled grid puts two independent workgroups on a CU; 64
// otherwise.  The 32-channel form needs L a multiple of its 32-step tile.
inline int chans_for(const lrnnx_selective_scan_args& a) {
  const int o = scan_channels_override();
  const bool can32 = a.seqlen % 32 == 0;
  if (o == 32 && can32) return 32;
  if (o) return kWave;
  return (can32 && (a.dim / kWave) * a.batch <= 256) ? 32 : kWave;
}
// workspace of the split: h_end and h_init [seg][b][n][d], dsum_seg and dsum_pre [seg][b][d]
inline int64_t split_ws_floats(const lrnnx_selective_scan_args& a, int64_t S) {
  return 2 * S * a.batch * a.dstate * a.dim + 2 * S * a.batch * a.dim;
}
}  // namespace ssf

// Bytes of forward workspace the fast path uses for this call (0: no split).
// Depends on shapes and options only (the output pointers need not be set).
template <typename IT>
inline int64_t ssf_fwd_ws_bytes(const lrnnx_selective_scan_args& a) {
  if (!ssf::shape_ok<IT>(a, ssf::tile_steps<IT>(), true)) return 0;
  const int64_t steps = ssf::seg_steps(a);
  return steps ? ssf::split_ws_floats(a, ssf::n_segs(a, steps)) * (int64_t)sizeof(float) : 0;
}

namespace ssf {
enum class FwdKind { kOutZ, kOut, kStates };  // with z gate / without / states and checkpoints only
}

// chans: 64 or 32 for the output kinds (ssf::chans_for); the states-only
// kind (split summaries, checkpoint rebuild) always runs 64.
template <typename IT, bool kSP, int kM, bool kDA = false>
inline void ssf_fwd_launch_t(const lrnnx_selective_scan_args& a, int64_t n_ck, const ssf::SsfSeg& sg, unsigned nz,
                             ssf::FwdKind kind, int chans, hipStream_t st) {
  const dim3 grid64((unsigned)(a.dim / kWave), (unsigned)a.batch, nz);
  const dim3 grid32((unsigned)(a.dim / (kWave / 2)), (unsigned)a.batch, nz);
  const dim3 blk(ssf::kNT);
  switch (kind) {
    case ssf::FwdKind::kOutZ:
      if (chans == 32) hipLaunchKernelGGL((ssf_fwd_kernel<IT, kSP, true, true, 32, kM, kDA>), grid32, blk, 0, st, a, n_ck, sg);
      else hipLaunchKernelGGL((ssf_fwd_kernel<IT, kSP, true, true, 64, kM, kDA>), grid64, blk, 0, st, a, n_ck, sg);
      break;
    case ssf::FwdKind::kOut:
      if (chans == 32) hipLaunchKernelGGL((ssf_fwd_kernel<IT, kSP, false, true, 32, kM, kDA>), grid32, blk, 0, st, a, n_ck, sg);
      else hipLaunchKernelGGL((ssf_fwd_kernel<IT, kSP, false, true, 64, kM, kDA>), grid64, blk, 0, st, a, n_ck, sg);
      break;
    case ssf::FwdKind::kStates:
      hipLaunchKernelGGL((ssf_fwd_kernel<IT, kSP, false, false, 64, kM, kDA>), grid64, blk, 0, st, a, n_ck, sg);
      break;
  }
}

// One launch over the whole of L, or, for small grids and with a workspace of
// ssf_fwd_ws_bytes, the three-pass split: segment summaries (every segment
// but the last; states only), the carry chain, then every segment from its
// initial state.  states_only: the checkpoint rebuild of a backward (writes
// a.ckpt and nothing else); then, when the grid does not split, the x carries
// `x_seed` (if given) let the 2048-step chunks run in parallel.
template <typename IT>
inline hipError_t ssf_fwd_launch(const lrnnx_selective_scan_args& a, int64_t n_ck, hipStream_t st,
                                 bool states_only = false, const float* x_seed = nullptr) {
  constexpr int kT = ssf::tile_steps<IT>();
  const int64_t n_tiles = a.seqlen / kT;
  const ssf::FwdKind kind = states_only             ? ssf::FwdKind::kStates
                            : a.z.ptr != nullptr    ? ssf::FwdKind::kOutZ
                                                    : ssf::FwdKind::kOut;
  auto launch = [&](const lrnnx_selective_scan_args& x, const ssf::SsfSeg& sg, unsigned nz, ssf::FwdKind k,
                    int chans) {
    if (x.deltaA.ptr) {   // mamba only (shape_ok)
      if (x.delta_softplus) ssf_fwd_launch_t<IT, true, LRNNX_MAMBA, true>(x, n_ck, sg, nz, k, chans, st);
      else ssf_fwd_launch_t<IT, false, LRNNX_MAMBA, true>(x, n_ck, sg, nz, k, chans, st);
      return;
    }
    auto by_sp = [&](auto m) __attribute__((always_inline)) {
      constexpr int kM = decltype(m)::value;
      if (x.delta_softplus) ssf_fwd_launch_t<IT, true, kM>(x, n_ck, sg, nz, k, chans, st);
      else ssf_fwd_launch_t<IT, false, kM>(x, n_ck, sg, nz, k, chans, st);
    };
    if constexpr (sizeof(IT) == 4) {   // the other methods: fp32 input only (shape_ok)
      switch (x.method) {
        case LRNNX_DIRAC: by_sp(std::integral_constant<int, LRNNX_DIRAC>{}); return;
        case LRNNX_ZOH: by_sp(std::integral_constant<int, LRNNX_ZOH>{}); return;
        case LRNNX_BILINEAR: by_sp(std::integral_constant<int, LRNNX_BILINEAR>{}); return;
        default: break;
      }
    }
    by_sp(std::integral_constant<int, LRNNX_MAMBA>{});
  };
  const int64_t steps = ssf::seg_steps(a);
  const int64_t need = ssf_fwd_ws_bytes<IT>(a);
  if (steps == 0 || need == 0 || a.workspace == nullptr || a.workspace_bytes < need ||
      (reinterpret_cast<uintptr_t>(a.workspace) & 15u) != 0) {
    const int64_t n_xc = (a.seqlen + kXChunk - 1) / kXChunk;
    if (states_only && x_seed != nullptr && n_xc > 1) {
      launch(a, ssf::SsfSeg{kXChunk / kT, nullptr, nullptr, nullptr, nullptr, x_seed}, (unsigned)n_xc, kind, kWave);
    } else {
      const int chans = states_only ? kWave : ssf::chans_for(a);
      // the 32-channel form walks 32-step tiles
      launch(a, ssf::SsfSeg{chans == 32 ? a.seqlen / 32 : n_tiles, nullptr, nullptr, nullptr, nullptr, nullptr}, 1,
             kind, chans);
    }
    return hipGetLastError();
  }
  const int64_t S = ssf::n_segs(a, steps), tiles = steps / kT;
  float* ws = static_cast<float*>(a.workspace);
  const int64_t ns = S * a.batch * a.dstate * a.dim, nd = S * a.batch * a.dim;
  float* h_end = ws;
  float* h_init = ws + ns;
  float* dsum_seg = ws + 2 * ns;
  float* dsum_pre = ws + 2 * ns + nd;
  // summaries: the states only
  lrnnx_selective_scan_args s = a;
  s.out.ptr = nullptr;
  s.out_z.ptr = nullptr;
  s.z.ptr = nullptr;
  s.x = nullptr;
  s.ckpt = nullptr;
  launch(s, ssf::SsfSeg{tiles, nullptr, nullptr, h_end, dsum_seg, nullptr}, (unsigned)(S - 1), ssf::FwdKind::kStates,
         kWave);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const ssf::SsfSeg chain{tiles, nullptr, nullptr, h_end, dsum_seg, nullptr};
  const int64_t nt = a.batch * a.dstate * a.dim;
  hipLaunchKernelGGL(ssf_seg_chain_kernel<IT>, dim3((unsigned)((nt + 255) / 256)), dim3(256), 0, st, a, chain, (int)S,
                     h_init, dsum_pre);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  launch(a, ssf::SsfSeg{tiles, h_init, dsum_pre, nullptr, nullptr, nullptr}, (unsigned)S, kind, kWave);
  return hipGetLastError();
}

}  // namespace lrnnx
