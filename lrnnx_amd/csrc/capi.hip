// extern "C" entry points of liblrnnx_scan.so: argument checks, workspace
// sizing and dispatch to the gfx950 kernels.
//
// The checks mirror the reference host code (TORCH_CHECKs of
// csrc/selective_scan/selective_scan_cpu.cpp:263-632 and
// csrc/simplified_scan/simplified_scan_cpu.cpp:160-331); a failed check
// returns 1 and leaves the message in lrnnx_last_error().
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>

#include "ss_common.h"

namespace lrnnx {
// LRNNX_SCAN_GENERIC=1 in the environment routes every call to the generic
// kernels (for A/B timing and cross-checks of the fast paths).
bool fast_paths_enabled() {
  const char* v = getenv("LRNNX_SCAN_GENERIC");
  return !(v && v[0] && v[0] != '0');
}
// LRNNX_SCAN_NO_SPLIT=1 keeps the fast paths from splitting L on small grids,
// so that tests can run the unsplit schedule at shapes the oracle finishes
// quickly.
bool l_split_enabled() {
  const char* v = getenv("LRNNX_SCAN_NO_SPLIT");
  return !(v && v[0] && v[0] != '0');
}

// LRNNX_SCAN_CHANNELS=64 or 32 forces the fast forward's channels per
// workgroup (cross-checks); 0 otherwise (the launch picks).
int scan_channels_override() {
  const char* v = getenv("LRNNX_SCAN_CHANNELS");
  if (!v) return 0;
  const int c = atoi(v);
  return (c == 64 || c == 32) ? c : 0;
}

hipError_t ss_fwd_mamba_f32(const lrnnx_selective_scan_args&, hipStream_t);
hipError_t ss_fwd_mamba_bf16(const lrnnx_selective_scan_args&, hipStream_t);
hipError_t ss_fwd_mamba_f16(const lrnnx_selective_scan_args&, hipStream_t);
bool ssf_fwd_f32(const lrnnx_selective_scan_args&, hipStream_t, hipError_t*);
bool ssf_fwd_bf16(const lrnnx_selective_scan_args&, hipStream_t, hipError_t*);
bool ssf_fwd_f16(const lrnnx_selective_scan_args&, hipStream_t, hipError_t*);
bool ssf_bwd_f32(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t, hipError_t*);
bool ssf_bwd_bf16(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t, hipError_t*);
bool ssf_bwd_f16(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t, hipError_t*);
bool ssf_ckpt_rebuild_f32(const lrnnx_selective_scan_args&, float*, float*, int64_t, const float*, hipStream_t,
                          hipError_t*);
bool ssf_ckpt_rebuild_bf16(const lrnnx_selective_scan_args&, float*, float*, int64_t, const float*, hipStream_t,
                           hipError_t*);
bool ssf_ckpt_rebuild_f16(const lrnnx_selective_scan_args&, float*, float*, int64_t, const float*, hipStream_t,
                          hipError_t*);
hipError_t ss_fwd_other_f32(const lrnnx_selective_scan_args&, hipStream_t);
int64_t ssf_fwd_workspace_bytes(const lrnnx_selective_scan_args&);
hipError_t ss_bwd_mamba_f32(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t);
hipError_t ss_bwd_mamba_bf16(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t);
hipError_t ss_bwd_mamba_f16(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t);
hipError_t ss_bwd_other_f32(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t);
hipError_t ssc_fwd_launch(const lrnnx_selective_scan_args&, hipStream_t);
hipError_t ssc_bwd_launch(const lrnnx_selective_scan_args&, float*, const float*, hipStream_t);
int64_t ssc_ckpt_bytes(const lrnnx_selective_scan_args&);
int64_t ssc_bwd_ws_bytes(const lrnnx_selective_scan_args&);
hipError_t simp_fwd_launch(const lrnnx_simplified_scan_args&, hipStream_t);
hipError_t simp_bwd_launch(const lrnnx_simplified_scan_args&, hipStream_t);
int64_t simp_ckpt_bytes(const lrnnx_simplified_scan_args&);
int64_t simp_ws_bytes(const lrnnx_simplified_scan_args&, int);
hipError_t state_update_launch(const lrnnx_state_update_args&, hipStream_t);
hipError_t simp_state_update_launch(const lrnnx_simplified_state_update_args&, hipStream_t);
hipError_t cconv_launch(const lrnnx_causal_conv1d_args&, int, float*, hipStream_t);
hipError_t ln_launch(const lrnnx_layer_norm_args&, bool, float*, hipStream_t);
int64_t ln_workspace_bytes(const lrnnx_layer_norm_args&);

// defined in ss_bwd_layout.hip (shares ss_bwd_ws with the backward units)
int64_t ss_bwd_ws_bytes(const lrnnx_selective_scan_args&);
int64_t ss_bwd_ckpt_offset_bytes(const lrnnx_selective_scan_args&);
int64_t ss_bwd_fws_offset_bytes(const lrnnx_selective_scan_args&, int64_t*);
}  // namespace lrnnx

using namespace lrnnx;

namespace {
thread_local std::string g_err;

int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return 1;
}

int from_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return 0;
  return fail("%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

const char* method_name(int m) {
  switch (m) {
    case LRNNX_ZOH: return "zoh";
    case LRNNX_BILINEAR: return "bilinear";
    case LRNNX_DIRAC: return "dirac";
    case LRNNX_MAMBA: return "mamba";
    case LRNNX_S7: return "s7";
    case LRNNX_RGLRU: return "rglru";
  }
  return "?";
}


// Methods with a fast path (forward and backward): "mamba" at every input
// type; "dirac", "zoh" and "bilinear", whose input is fp32.
bool has_fast_path(int method) {
  return method == LRNNX_MAMBA || method == LRNNX_DIRAC || method == LRNNX_ZOH || method == LRNNX_BILINEAR;
}

// Forward workspace of the fast path's split of L (0: the call does not split).
int64_t fwd_split_ws_bytes(const lrnnx_selective_scan_args& a) {
  if (!has_fast_path(a.method) || !fast_paths_enabled()) return 0;
  return ssf_fwd_workspace_bytes(a);
}

// Forward of the "mamba" method: fast path when it covers the call, else the
// generic kernel.
hipError_t fwd_mamba(const lrnnx_selective_scan_args& a, hipStream_t st) {
  hipError_t e = hipSuccess;
  if (fast_paths_enabled()) {
    const bool done = a.itype == LRNNX_F32    ? ssf_fwd_f32(a, st, &e)
                      : a.itype == LRNNX_BF16 ? ssf_fwd_bf16(a, st, &e)
                                              : ssf_fwd_f16(a, st, &e);
    if (done) return e;
  }
  switch (a.itype) {
    case LRNNX_F32: return ss_fwd_mamba_f32(a, st);
    case LRNNX_BF16: return ss_fwd_mamba_bf16(a, st);
    default: return ss_fwd_mamba_f16(a, st);
  }
}

// Backward of the "mamba" method: fast path when it covers the call, else the
// generic kernel.
hipError_t bwd_mamba(const lrnnx_selective_scan_args& a, float* ws, const float* ckp, hipStream_t st) {
  hipError_t e = hipSuccess;
  if (fast_paths_enabled()) {
    const bool done = a.itype == LRNNX_F32    ? ssf_bwd_f32(a, ws, ckp, st, &e)
                      : a.itype == LRNNX_BF16 ? ssf_bwd_bf16(a, ws, ckp, st, &e)
                                              : ssf_bwd_f16(a, ws, ckp, st, &e);
    if (done) return e;
  }
  switch (a.itype) {
    case LRNNX_F32: return ss_bwd_mamba_f32(a, ws, ckp, st);
    case LRNNX_BF16: return ss_bwd_mamba_bf16(a, ws, ckp, st);
    default: return ss_bwd_mamba_f16(a, ws, ckp, st);
  }
}

// Forward / backward of the other real methods (fp32 input): the fast path
// for "dirac", "zoh" and "bilinear" when it covers the call; else the
// generic kernels.
hipError_t fwd_other(const lrnnx_selective_scan_args& a, hipStream_t st) {
  hipError_t e = hipSuccess;
  if (has_fast_path(a.method) && fast_paths_enabled() && ssf_fwd_f32(a, st, &e)) return e;
  return ss_fwd_other_f32(a, st);
}
hipError_t bwd_other(const lrnnx_selective_scan_args& a, float* ws, const float* ckp, hipStream_t st) {
  hipError_t e = hipSuccess;
  if (has_fast_path(a.method) && fast_paths_enabled() && ssf_bwd_f32(a, ws, ckp, st, &e)) return e;
  return ss_bwd_other_f32(a, ws, ckp, st);
}

int check_ss(const lrnnx_selective_scan_args* a, bool bwd) {
  if (!a) return fail("null argument struct");
  if (a->itype != LRNNX_F32 && a->itype != LRNNX_F16 && a->itype != LRNNX_BF16)
    return fail("input dtype must be float32, float16 or bfloat16");
  if (a->wtype != LRNNX_F32 && a->wtype != LRNNX_C64) return fail("weight dtype must be float32 or complex64");
  if (a->method < LRNNX_ZOH || a->method > LRNNX_RGLRU) return fail("Discretization method not supported");
  if (a->method == LRNNX_S7 && a->wtype != LRNNX_F32)
    return fail("S7 discretization only supports real (float) weights, not complex");
  if (a->method == LRNNX_RGLRU && a->wtype != LRNNX_F32)
    return fail("RGLRU discretization only supports real (float) weights, not complex");
  if (a->method != LRNNX_MAMBA && a->itype != LRNNX_F32)
    return fail("discretization '%s' supports float32 input only (as the reference kernels)", method_name(a->method));
  if (a->wtype == LRNNX_C64 && a->itype != LRNNX_F32)
    return fail("complex weights support float32 input only (as the reference kernels)");
  if (a->batch <= 0 || a->dim <= 0 || a->seqlen <= 0 || a->dstate <= 0)
    return fail("empty or negative shape (batch=%lld dim=%lld seqlen=%lld dstate=%lld)", (long long)a->batch,
                (long long)a->dim, (long long)a->seqlen, (long long)a->dstate);
  if (a->dstate > 256) return fail("selective_scan only supports state dimension <= 256");
  if ((a->var_B || a->var_C) && (a->n_groups <= 0 || a->dim % a->n_groups != 0))
    return fail("dim (%lld) must be a multiple of the number of B/C groups (%lld)", (long long)a->dim,
                (long long)a->n_groups);
  if (!a->u.ptr || !a->delta.ptr || !a->A.ptr || !a->B.ptr || !a->C.ptr) return fail("u, delta, A, B, C are required");
  if (a->z.ptr && !bwd && !a->out_z.ptr) return fail("out_z is required when z is given");
  if (!bwd && !a->z.ptr && !a->out.ptr && !a->ckpt && !a->x) return fail("nothing to compute: no outputs given");
  if (bwd) {
    if (!a->dout.ptr) return fail("dout is required");
    if (a->z.ptr && !a->out_saved.ptr) return fail("out is required by the backward when z is given");
    if (a->z.ptr && !a->dz.ptr) return fail("dz is required when z is given");
    if (!a->du.ptr || !a->ddelta.ptr || !a->dA.ptr || !a->dB.ptr || !a->dC.ptr) return fail("du, ddelta, dA, dB, dC are required");
    if (a->deltaA.ptr && !a->ddeltaA.ptr) return fail("ddeltaA is required when deltaA is given");
  }
  return 0;
}
}  // namespace

// Device scratch of lrnnx_selective_scan_fwd_noalloc: the segment summaries
// and carries of the forward's split of L (h_end, h_init [seg][b][n][d],
// dsum_seg, dsum_pre [seg][b][d], fp32).  The split keeps segments x
// batch x dim / 64 <= 512 and the fast path has d_state <= 16, so any call
// needs at most 2 * 32768 * 16 + 2 * 32768 floats = 4 456 448 bytes.  Each GPU
// holds its own copy from the library's load until the process ends.
constexpr int64_t kFwdScratchBytes = LRNNX_FWD_NOALLOC_SCRATCH_BYTES;
static_assert(kFwdScratchBytes == 2 * 32768 * 16 * 4 + 2 * 32768 * 4, "bound of the split's summaries");
static __device__ __align__(256) char scratch[kFwdScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of this device's `scratch`, looked up once per device with
// that device current (the array's host-side name is not a device address).
int scratch_of_current_device(void** out) {
  int dev = -1;
  if (from_hip(hipGetDevice(&dev), "hipGetDevice")) return 1;
  if (dev < 0 || dev >= kMaxDevices) return fail("device index %d out of range (at most %d devices)", dev, kMaxDevices);
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      if (from_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return 1;
      if (!p) return fail("hipGetSymbolAddress(scratch) returned a null address");
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return 0;
}
}  // namespace

extern "C" {

const char* lrnnx_last_error(void) { return g_err.c_str(); }

int lrnnx_abi_version(void) { return LRNNX_ABI_VERSION; }

int64_t lrnnx_selective_scan_ckpt_size(const lrnnx_selective_scan_args* a) {
  if (!a) return -1;
  if (a->wtype == LRNNX_C64) return ssc_ckpt_bytes(*a);
  const SSGeom g = ss_geom(*a);
  return a->batch * g.n_ck * a->dstate * a->dim * (int64_t)sizeof(float);
}

int64_t lrnnx_selective_scan_workspace_size(const lrnnx_selective_scan_args* a, int bwd) {
  if (!a) return -1;
  if (!bwd) {  // optional: the state blocks' partial y (d_state > 64), or the fast path's split of L
    if (a->wtype == LRNNX_C64) return 0;
    const int64_t blk = ss_fwd_blocks_ws_bytes(*a);
    return blk > 0 ? blk : fwd_split_ws_bytes(*a);
  }
  if (a->wtype == LRNNX_C64) return ssc_bwd_ws_bytes(*a);
  return ss_bwd_ws_bytes(*a);
}

int lrnnx_selective_scan_fwd(const lrnnx_selective_scan_args* a, void* stream) {
  if (check_ss(a, false)) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->wtype == LRNNX_C64) return from_hip(ssc_fwd_launch(*a, st), "selective_scan_fwd (complex)");
  hipError_t e;
  if (a->method == LRNNX_MAMBA) {
    e = fwd_mamba(*a, st);
  } else {
    e = fwd_other(*a, st);
  }
  return from_hip(e, "selective_scan_fwd");
}

int lrnnx_selective_scan_fwd_noalloc(const lrnnx_selective_scan_args* a, void* stream) {
  if (check_ss(a, false)) return 1;
  lrnnx_selective_scan_args f = *a;  // the caller's workspace fields are ignored
  f.workspace = nullptr;
  f.workspace_bytes = 0;
  // the split's summaries (d_state > 64 runs without a workspace: one state
  // block, no partial sums)
  const int64_t need = a->wtype == LRNNX_C64 ? 0 : fwd_split_ws_bytes(f);
  if (need > kFwdScratchBytes)
    return fail("selective_scan_fwd_noalloc: the call needs %lld bytes of scratch, more than the %lld it holds",
                (long long)need, (long long)kFwdScratchBytes);
  if (need > 0) {
    void* p = nullptr;
    if (scratch_of_current_device(&p)) return 1;
    f.workspace = p;
    f.workspace_bytes = kFwdScratchBytes;
  }
  return lrnnx_selective_scan_fwd(&f, stream);
}

int lrnnx_selective_scan_bwd(const lrnnx_selective_scan_args* a, void* stream) {
  if (check_ss(a, true)) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t need = lrnnx_selective_scan_workspace_size(a, 1);
  if (need > 0 && (!a->workspace || a->workspace_bytes < need))
    return fail("workspace too small: %lld bytes given, %lld needed", (long long)a->workspace_bytes, (long long)need);
  if ((reinterpret_cast<uintptr_t>(a->workspace) & 255u) != 0) return fail("workspace must be 256-byte aligned");
  float* ws = static_cast<float*>(a->workspace);
  if (a->wtype == LRNNX_C64) return from_hip(ssc_bwd_launch(*a, ws, static_cast<const float*>(a->ckpt), st),
                                             "selective_scan_bwd (complex)");
  const float* ckp = static_cast<const float*>(a->ckpt);
  if (!ckp) {
    // rebuild the fine checkpoints into the workspace.  The fast forward
    // (has_fast_path) has a states-only form: split like the forward on small grids, or
    // with the caller's x carries (the reference's seeds,
    // selective_scan_backward.cuh:330) one 2048-step chunk per grid slice.
    char* wsb = reinterpret_cast<char*>(a->workspace);
    float* ck = reinterpret_cast<float*>(wsb + ss_bwd_ckpt_offset_bytes(*a));
    hipError_t e = hipSuccess;
    bool done = false;
    if (has_fast_path(a->method) && fast_paths_enabled()) {
      int64_t fws_bytes = 0;
      float* fws = reinterpret_cast<float*>(wsb + ss_bwd_fws_offset_bytes(*a, &fws_bytes));
      if (fws_bytes == 0) fws = nullptr;
      const float* xs = static_cast<const float*>(a->x);
      done = a->itype == LRNNX_F32    ? ssf_ckpt_rebuild_f32(*a, ck, fws, fws_bytes, xs, st, &e)
             : a->itype == LRNNX_BF16 ? ssf_ckpt_rebuild_bf16(*a, ck, fws, fws_bytes, xs, st, &e)
                                      : ssf_ckpt_rebuild_f16(*a, ck, fws, fws_bytes, xs, st, &e);
    }
    if (!done) {  // a forward pass that writes nothing else
      lrnnx_selective_scan_args f = *a;
      f.out.ptr = nullptr;
      f.out_z.ptr = nullptr;
      f.z.ptr = nullptr;
      f.x = nullptr;
      f.ckpt = ck;
      f.workspace = nullptr;  // unsplit
      f.workspace_bytes = 0;
      e = a->method == LRNNX_MAMBA ? fwd_mamba(f, st) : fwd_other(f, st);
    }
    if (from_hip(e, "selective_scan_bwd (checkpoint rebuild)")) return 1;
    ckp = ck;
  }
  hipError_t e;
  if (a->method == LRNNX_MAMBA) {
    e = bwd_mamba(*a, ws, ckp, st);
  } else {
    e = bwd_other(*a, ws, ckp, st);
  }
  return from_hip(e, "selective_scan_bwd");
}

int64_t lrnnx_simplified_scan_ckpt_size(const lrnnx_simplified_scan_args* a) {
  return a ? simp_ckpt_bytes(*a) : -1;
}

int64_t lrnnx_simplified_scan_workspace_size(const lrnnx_simplified_scan_args* a, int bwd) {
  return a ? simp_ws_bytes(*a, bwd) : -1;
}

static int check_simp(const lrnnx_simplified_scan_args* a, bool bwd) {
  if (!a) return fail("null argument struct");
  if (a->method != LRNNX_ZOH && a->method != LRNNX_BILINEAR && a->method != LRNNX_DIRAC)
    return fail("Discretization method not supported (simplified scan: zoh, bilinear, dirac)");
  if (a->batch <= 0 || a->dim <= 0 || a->seqlen <= 0 || a->dstate <= 0) return fail("empty or negative shape");
  if (a->dstate > 256) return fail("simplified_scan only supports state dimension <= 256");
  if (!a->u.ptr || !a->delta.ptr || !a->A.ptr || !a->B.ptr || !a->C.ptr) return fail("u, delta, A, B, C are required");
  if (!a->workspace && simp_ws_bytes(*a, bwd) > 0) return fail("workspace is required");
  if (a->workspace_bytes < simp_ws_bytes(*a, bwd))
    return fail("workspace too small: %lld bytes given, %lld needed", (long long)a->workspace_bytes,
                (long long)simp_ws_bytes(*a, bwd));
  if (bwd) {
    if (!a->dout.ptr || !a->du.ptr || !a->dA.ptr || !a->dB.ptr || !a->dC.ptr) return fail("dout, du, dA, dB, dC are required");
    if (a->need_ddelta && !a->ddelta.ptr) return fail("ddelta is required");
    if (a->need_ddelta && a->deltaA.ptr && !a->ddeltaA.ptr) return fail("ddeltaA is required when deltaA is given");
  }
  return 0;
}

int lrnnx_simplified_scan_fwd(const lrnnx_simplified_scan_args* a, void* stream) {
  if (check_simp(a, false)) return 1;
  return from_hip(simp_fwd_launch(*a, static_cast<hipStream_t>(stream)), "simplified_scan_fwd");
}

int lrnnx_simplified_scan_bwd(const lrnnx_simplified_scan_args* a, void* stream) {
  if (check_simp(a, true)) return 1;
  return from_hip(simp_bwd_launch(*a, static_cast<hipStream_t>(stream)), "simplified_scan_bwd");
}

int lrnnx_selective_state_update(const lrnnx_state_update_args* a, void* stream) {
  if (!a) return fail("null argument struct");
  if (a->method < LRNNX_ZOH || a->method > LRNNX_RGLRU) return fail("Discretization method not supported");
  if (a->batch <= 0 || a->nheads <= 0 || a->dim <= 0 || a->dstate <= 0) return fail("empty or negative shape");
  if (a->ngroups <= 0 || a->nheads % a->ngroups != 0) return fail("nheads must be divisible by ngroups");
  if (!a->state || !a->x || !a->dt || !a->A || !a->B || !a->C || !a->out) return fail("state, x, dt, A, B, C, out are required");
  for (int t : {a->state_type, a->x_type, a->bc_type})
    if (t != LRNNX_F32 && t != LRNNX_F16 && t != LRNNX_BF16) return fail("unsupported dtype code %d", t);
  return from_hip(state_update_launch(*a, static_cast<hipStream_t>(stream)), "selective_state_update");
}

static int check_cconv(const lrnnx_causal_conv1d_args* a, int which) {
  if (!a) return fail("null argument struct");
  if (a->itype != LRNNX_F32 && a->itype != LRNNX_F16 && a->itype != LRNNX_BF16)
    return fail("x must be float32, float16 or bfloat16");
  if (a->width < 1 || a->width > 8) return fail("causal_conv1d: width must be between 1 and 8 (got %lld)",
                                                (long long)a->width);
  if (a->batch <= 0 || a->dim <= 0 || a->seqlen <= 0) return fail("empty or negative shape");
  if (!a->x.ptr || !a->weight.ptr || !a->out.ptr) return fail("x, weight, out are required");
  if (which != 2 && a->x.s2 != 1) return fail("causal_conv1d: x must have unit stride along the sequence");
  if (which == 1) {
    if (!a->dout.ptr || !a->dx.ptr || !a->dweight.ptr) return fail("dout, dx, dweight are required");
    if (a->dout.s2 != 1 || a->dx.s2 != 1) return fail("causal_conv1d: dout / dx must have unit stride along the sequence");
    if (a->bias.ptr && !a->dbias.ptr) return fail("dbias is required when bias is given");
    if (!a->workspace || a->workspace_bytes < lrnnx_causal_conv1d_workspace_size(a))
      return fail("workspace too small");
  }
  if (which == 2) {
    if (!a->conv_state.ptr) return fail("conv_state is required");
    if (a->state_len < a->width - 1) return fail("conv_state must hold at least width - 1 steps");
  }
  return 0;
}

int64_t lrnnx_causal_conv1d_workspace_size(const lrnnx_causal_conv1d_args* a) {
  return a ? a->batch * a->dim * (a->width + 1) * (int64_t)sizeof(float) : -1;
}

int lrnnx_causal_conv1d_fwd(const lrnnx_causal_conv1d_args* a, void* stream) {
  if (check_cconv(a, 0)) return 1;
  return from_hip(cconv_launch(*a, 0, nullptr, static_cast<hipStream_t>(stream)), "causal_conv1d_fwd");
}

int lrnnx_causal_conv1d_bwd(const lrnnx_causal_conv1d_args* a, void* stream) {
  if (check_cconv(a, 1)) return 1;
  return from_hip(cconv_launch(*a, 1, static_cast<float*>(a->workspace), static_cast<hipStream_t>(stream)),
                  "causal_conv1d_bwd");
}

int lrnnx_causal_conv1d_update(const lrnnx_causal_conv1d_args* a, void* stream) {
  if (check_cconv(a, 2)) return 1;
  return from_hip(cconv_launch(*a, 2, nullptr, static_cast<hipStream_t>(stream)), "causal_conv1d_update");
}

int lrnnx_simplified_state_update(const lrnnx_simplified_state_update_args* a, void* stream) {
  if (!a) return fail("null argument struct");
  if (a->method != LRNNX_ZOH && a->method != LRNNX_BILINEAR && a->method != LRNNX_DIRAC)
    return fail("discretization must be one of ['bilinear', 'zoh', 'dirac']");
  if (a->batch <= 0 || a->H <= 0 || a->P <= 0) return fail("empty or negative shape");
  if (!a->state || !a->x || !a->dt || !a->A || !a->B || !a->C || !a->out)
    return fail("state, x, dt, A, B, C, out are required");
  // x staged in LDS together with the updated state
  if ((a->H + 2 * a->P) * 4 > 64 * 1024) return fail("H + 2 P must fit 64 KiB of LDS (H=%lld, P=%lld)",
                                                     (long long)a->H, (long long)a->P);
  return from_hip(simp_state_update_launch(*a, static_cast<hipStream_t>(stream)), "simplified_state_update");
}

static int check_ln(const lrnnx_layer_norm_args* a, bool bwd) {
  if (!a) return fail("null argument struct");
  for (int t : {a->xtype, a->rtype, a->wtype})
    if (t != LRNNX_F32 && t != LRNNX_F16 && t != LRNNX_BF16) return fail("unsupported dtype code %d", t);
  if (a->rows <= 0 || a->cols <= 0) return fail("empty or negative shape");
  // the reference's one-pass kernel holds a row of x in 64 KiB (layer_norm.py:405-411)
  if (a->cols * (a->xtype == LRNNX_F32 ? 4 : 2) > 65536)
    return fail("This layer norm doesn't support feature dim >= 64KB.");
  if (!a->weight.ptr || !a->rstd || (!a->is_rms_norm && !a->mean)) return fail("weight, rstd and mean are required");
  if (!bwd) {
    if (!a->x.ptr || !a->y.ptr) return fail("x and y are required");
    return 0;
  }
  if (!a->x_saved.ptr || !a->dy.ptr || !a->dx.ptr || !a->dweight.ptr) return fail("x, dy, dx, dweight are required");
  if (a->bias.ptr && !a->dbias.ptr) return fail("dbias is required when bias is given");
  if (!a->workspace || a->workspace_bytes < ln_workspace_bytes(*a)) return fail("workspace too small");
  return 0;
}

int64_t lrnnx_layer_norm_workspace_size(const lrnnx_layer_norm_args* a) {
  return a ? ln_workspace_bytes(*a) : -1;
}

int lrnnx_layer_norm_fwd(const lrnnx_layer_norm_args* a, void* stream) {
  if (check_ln(a, false)) return 1;
  return from_hip(ln_launch(*a, false, nullptr, static_cast<hipStream_t>(stream)), "layer_norm_fwd");
}

int lrnnx_layer_norm_bwd(const lrnnx_layer_norm_args* a, void* stream) {
  if (check_ln(a, true)) return 1;
  return from_hip(ln_launch(*a, true, static_cast<float*>(a->workspace), static_cast<hipStream_t>(stream)),
                  "layer_norm_bwd");
}

}  // extern "C"
