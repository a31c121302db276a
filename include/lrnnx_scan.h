/*
 * lrnnx_scan.h -- C ABI of the MI355X (gfx950) scan hot path of lrnnx.
 *
 * The library (lrnnx_amd/liblrnnx_scan.so) replaces the two pybind11 torch
 * extensions of the reference, `selective_scan_cuda` and
 * `simplified_scan_cuda` (reference csrc/selective_scan/bindings.cpp:5-8,
 * csrc/simplified_scan/bindings.cpp:5-8), and the Triton decode kernels
 * `_selective_scan_update_kernel` and `_simplified_state_update_kernel`
 * (lrnnx/ops/triton/selective_state_update.py:17-297,
 * lrnnx/ops/triton/simplified_state_update.py:13-251).
 *
 * Conventions
 *  - Plain pointers and sizes only.  Every buffer (inputs, outputs and the
 *    workspace) is allocated by the caller; the library never allocates, so
 *    every entry point may be captured in a HIP graph.
 *  - Sequence tensors have unit stride along L; their batch / channel
 *    strides are given in ELEMENTS (int64).  Complex tensors are interleaved
 *    (re, im) float pairs and their strides count complex elements.
 *  - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream of
 *    the current device).  No host synchronisation happens inside.
 *  - Return 0 on success.  Non-zero means the arguments were rejected or a
 *    launch failed; `lrnnx_last_error()` then returns the message
 *    (thread-local).  This mirrors the reference's TORCH_CHECK failures
 *    (selective_scan_cpu.cpp:271-367) and C10_CUDA_KERNEL_LAUNCH_CHECK.
 */
#ifndef LRNNX_SCAN_H
#define LRNNX_SCAN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (reference accepts u in {f32, f16, bf16}, weights in {f32, c64};
 * selective_scan_cpu.cpp:268-270). */
enum lrnnx_dtype { LRNNX_F32 = 0, LRNNX_F16 = 1, LRNNX_BF16 = 2, LRNNX_C64 = 3 };

/* Discretisation methods, same numbering as the reference enum
 * DiscretizationMethod (csrc/selective_scan/selective_scan.h:14-21). */
enum lrnnx_method {
  LRNNX_ZOH = 0, LRNNX_BILINEAR = 1, LRNNX_DIRAC = 2,
  LRNNX_MAMBA = 3, LRNNX_S7 = 4, LRNNX_RGLRU = 5
};

/* A 1-to-4-D tensor view: pointer + element strides of the leading dims.
 * For (b, d, l) sequences: s0 = batch stride, s1 = channel stride.
 * For variable B/C (b, g, n, l): s0 = batch, s1 = group, s2 = state.
 * For (d, n) weights: s0 = channel stride, s1 = state stride.
 * For (d) vectors: s0 = channel stride. */
typedef struct lrnnx_view {
  void *ptr;
  int64_t s0, s1, s2;
} lrnnx_view;

/*
 * Selective scan (S6 / Mamba and the other discretisations).
 * One struct serves forward and backward; fields unused by a call are ignored.
 *
 * Replaces selective_scan_cuda.fwd / .bwd
 *   (reference csrc/selective_scan/selective_scan.h:114-136,
 *    host code csrc/selective_scan/selective_scan_cpu.cpp:263-632).
 */
typedef struct lrnnx_selective_scan_args {
  int64_t batch, dim, seqlen, dstate, n_groups;
  int32_t itype;          /* dtype of u, delta, deltaA, z, out, out_z, dout, du, ddelta, ddeltaA, dz, variable B/C */
  int32_t wtype;          /* LRNNX_F32 or LRNNX_C64: A and constant B/C */
  int32_t method;         /* enum lrnnx_method */
  int32_t var_B, var_C;   /* 1: (b, g, n, l) sequences (complex: real (.., 2l) interleaved); 0: (d, n) weights */
  int32_t delta_softplus;
  /* inputs (ptr == NULL means absent for D, z, delta_bias, deltaA) */
  lrnnx_view u, delta, A, B, C, D, z, delta_bias, deltaA;
  /* forward outputs */
  lrnnx_view out;         /* y + D u before gating; may be NULL when z is given (then only out_z is written) */
  lrnnx_view out_z;       /* out * silu(z); required iff z is given */
  void *x;                /* chunk carries (b, d, ceil(l/2048), 2n) contiguous, weight dtype; may be NULL */
  void *ckpt;             /* fine state checkpoints (fp32) for the backward; may be NULL in forward */
  /* backward inputs/outputs */
  lrnnx_view dout;        /* gradient of out_z (or of out when z is absent) */
  lrnnx_view out_saved;   /* forward `out` (pre-gating); required by backward when z is given */
  lrnnx_view du, ddelta, dA, dB, dC, dD, ddelta_bias, ddeltaA, dz;
  /* scratch: at least lrnnx_selective_scan_workspace_size() bytes, 256-byte aligned */
  void *workspace;
  int64_t workspace_bytes;
} lrnnx_selective_scan_args;

/* Bytes of fp32 state checkpoints `ckpt` written by the forward for a later
 * backward (0 if the shape needs none). */
int64_t lrnnx_selective_scan_ckpt_size(const lrnnx_selective_scan_args *a);

/* Bytes of workspace the call needs (bwd = 0: forward, 1: backward).  The
 * forward's is optional.  Given at least this many bytes (16-byte aligned):
 * for d_state > 64 (real weights) the states run in blocks of at most 64,
 * whose partial sums of y go there (batch * dim * L floats per block); the
 * fast path (methods mamba and dirac) splits L into segments when
 * batch * dim / 64 workgroups are too few to fill the GPU (a segment summary
 * pass, a carry chain, then every segment from its initial state).  Without
 * it the forward runs unsplit, and d_state > 64 in one slower block.  It is
 * 0 when neither applies.  No reference counterpart (the reference's forward
 * allocates nothing beyond its outputs). */
int64_t lrnnx_selective_scan_workspace_size(const lrnnx_selective_scan_args *a, int bwd);

/* Forward.  Writes out / out_z / x and, if ckpt != NULL, the checkpoints.
 * Replaces selective_scan_fwd (selective_scan_cpu.cpp:263-421). */
int lrnnx_selective_scan_fwd(const lrnnx_selective_scan_args *a, void *stream);

/* Forward that allocates nothing and takes no workspace.  No counterpart in
 * the reference: it is for callers that cannot allocate (code under HIP graph
 * capture, serving loops, harnesses that forbid allocation) and still want the
 * small-grid split of L.  Same arguments and results as
 * lrnnx_selective_scan_fwd; `workspace` / `workspace_bytes` are ignored and
 * the split's segment summaries go to a scratch array in device memory that
 * the library holds per GPU (LRNNX_FWD_NOALLOC_SCRATCH_BYTES: enough for
 * every call the split covers; a larger need is rejected; d_state > 64 runs
 * in one block, as lrnnx_selective_scan_fwd without a workspace).  Calls on
 * one GPU share that array, so calls that overlap on one GPU (concurrent
 * streams) race; nothing in it needs to start at zero. */
int lrnnx_selective_scan_fwd_noalloc(const lrnnx_selective_scan_args *a, void *stream);
#define LRNNX_FWD_NOALLOC_SCRATCH_BYTES 4456448

/* Backward.  Needs `ckpt` from a forward over the same inputs; when
 * ckpt == NULL the checkpoints are rebuilt into the workspace first (the
 * reference re-runs its chunk scan from `x`, selective_scan_backward.cuh:330).
 * `x` is optional here; when given (the forward's chunk carries of the same
 * inputs) the rebuild starts every 2048-step chunk from them, in parallel.
 * Writes du, ddelta, dA, dB, dC, dD, ddelta_bias, ddeltaA (if deltaA), dz
 * (if z).  Variable dB/dC are written in the input dtype (the reference
 * accumulates them in fp32 and casts, selective_scan_cpu.cpp:627); constant
 * dB/dC and dA in the weight dtype; dD, ddelta_bias in f32.
 * Replaces selective_scan_bwd (selective_scan_cpu.cpp:423-632). */
int lrnnx_selective_scan_bwd(const lrnnx_selective_scan_args *a, void *stream);

/*
 * Simplified complex diagonal scan (S5 / LRU), complex64 only.
 * u, out, du, dout: (b, p, l) complex; delta, deltaA, ddelta, ddeltaA:
 * (b, p, l) real f32.  For delta / deltaA the view's s2 is the L stride and
 * may be 0 (value constant along L; then A_bar is computed once per channel).
 * A, B, C, dA, dB, dC: (p, ds) complex.  The forward writes `ckpt` (chunk
 * start states) that the backward reuses; without it the backward rebuilds
 * them in the workspace.
 * Replaces simplified_scan_cuda.fwd / .bwd
 *   (reference csrc/simplified_scan/simplified_scan.h:98-109,
 *    host code csrc/simplified_scan/simplified_scan_cpu.cpp:160-331).
 */
typedef struct lrnnx_simplified_scan_args {
  int64_t batch, dim, seqlen, dstate;
  int32_t method;          /* LRNNX_ZOH, LRNNX_BILINEAR or LRNNX_DIRAC */
  int32_t need_ddelta;     /* backward: 0 skips ddelta/ddeltaA (they are not written) */
  lrnnx_view u, delta, A, B, C, deltaA;
  lrnnx_view out;
  void *x;                 /* (b, p, ceil(l/2048), 2 ds) complex, may be NULL */
  void *ckpt;              /* per-chunk start states written by the forward (complex); may be NULL */
  lrnnx_view dout;
  lrnnx_view du, ddelta, dA, dB, dC, ddeltaA;
  void *workspace;
  int64_t workspace_bytes;
} lrnnx_simplified_scan_args;

/* Bytes of the forward's chunk-start states `ckpt` (complex64). */
int64_t lrnnx_simplified_scan_ckpt_size(const lrnnx_simplified_scan_args *a);
int64_t lrnnx_simplified_scan_workspace_size(const lrnnx_simplified_scan_args *a, int bwd);
int lrnnx_simplified_scan_fwd(const lrnnx_simplified_scan_args *a, void *stream);
int lrnnx_simplified_scan_bwd(const lrnnx_simplified_scan_args *a, void *stream);

/*
 * One-token decode update, in place on `state`.
 * state (b, h, d, n) in f32/f16/bf16 (math in fp32); x, dt, z, deltaA, out
 * (b, h, d); A (h, d, n) f32; B, C (b, g, n); D, dt_bias (h, d) f32.
 * state_batch_indices (b) int32 or NULL.
 * Replaces selective_state_update
 *   (reference lrnnx/ops/triton/selective_state_update.py:300-476).
 */
typedef struct lrnnx_state_update_args {
  int64_t batch, nheads, dim, dstate, ngroups;
  int32_t state_type, x_type, bc_type;   /* enum lrnnx_dtype (not C64) */
  int32_t method;
  int32_t dt_softplus;
  void *state; int64_t state_s0, state_s1, state_s2, state_s3;
  const void *x; int64_t x_s0, x_s1, x_s2;
  const void *dt; int64_t dt_s0, dt_s1, dt_s2;
  const void *A; int64_t A_s0, A_s1, A_s2;
  const void *B; int64_t B_s0, B_s1, B_s2;
  const void *C; int64_t C_s0, C_s1, C_s2;
  const void *D; int64_t D_s0, D_s1;
  const void *z; int64_t z_s0, z_s1, z_s2;
  const void *dt_bias; int64_t dtb_s0, dtb_s1;
  const void *deltaA; int64_t dA_s0, dA_s1, dA_s2;
  const int32_t *state_batch_indices;
  void *out; int64_t out_s0, out_s1, out_s2;
} lrnnx_state_update_args;

int lrnnx_selective_state_update(const lrnnx_state_update_args *a, void *stream);

/*
 * One-token S5 decode update, in place on the complex state.
 * state (b, P) complex64; x (b, H) f32; dt, deltaA (b, P) f32 (s0 = 0 for a
 * (P,) vector shared by the batch); A (P) complex64; B (P, H) and C (H, P)
 * complex64; D (H, H) f32 or NULL; out (b, H) f32.
 *   A_bar = bilinear | exp(dtA A),  gamma = dt / (1 - dt A / 2) | (exp(dt A) - 1) / A | 1,
 *   state = A_bar state + gamma (B @ x),
 *   out   = (conj_sym ? 2 : 1) Re(C @ state) + x @ D^T.
 * Strides in elements (complex elements for complex tensors).
 * Replaces simplified_state_update
 *   (reference lrnnx/ops/triton/simplified_state_update.py:254-401).
 */
typedef struct lrnnx_simplified_state_update_args {
  int64_t batch, H, P;
  int32_t method;          /* LRNNX_ZOH, LRNNX_BILINEAR or LRNNX_DIRAC */
  int32_t conj_sym;
  void *state; int64_t state_s0, state_s1;
  const void *x; int64_t x_s0, x_s1;
  const void *dt; int64_t dt_s0, dt_s1;
  const void *A; int64_t A_s0;
  const void *B; int64_t B_s0, B_s1;
  const void *C; int64_t C_s0, C_s1;
  const void *D; int64_t D_s0, D_s1;
  const void *deltaA; int64_t dA_s0, dA_s1;
  void *out; int64_t out_s0, out_s1;
} lrnnx_simplified_state_update_args;

int lrnnx_simplified_state_update(const lrnnx_simplified_state_update_args *a, void *stream);

/*
 * Depthwise causal conv1d (the short convolution of the Mamba block), the
 * operator of the causal-conv1d package that lrnnx calls (pyproject.toml:33,
 * optional dependency; lrnnx/models/ltv/mamba.py:274, :411 and
 * lrnnx/ops/selective_scan.py:448, :640).  Semantics are the reference's own
 * fallback (mamba.py:271, :398-410):
 *   out[b,d,t] = act(bias[d] + sum_{k<W} weight[d,k] x[b,d,t-W+1+k]),  x[t<0] = 0,
 *   act = silu if `silu` else identity.
 * x, out, dout, dx, conv_state in `itype` (f32 / f16 / bf16); weight (dim,
 * width), bias (dim), dweight, dbias in f32.  width 1..8.  x / out / dout / dx
 * views: s0 batch, s1 channel, s2 step (must be 1 for fwd / bwd).
 * Update: conv_state (batch, dim, state_len >= width - 1) holds the last
 * state_len inputs and is shifted in place; x (batch, dim, seqlen) are the
 * new inputs (seqlen usually 1).
 */
typedef struct lrnnx_causal_conv1d_args {
  int64_t batch, dim, seqlen, width, state_len;
  int32_t itype;
  int32_t silu;
  lrnnx_view x, weight, bias, out;
  lrnnx_view dout, dx, dweight, dbias;
  lrnnx_view conv_state;
  void *workspace;                 /* backward: >= lrnnx_causal_conv1d_workspace_size() bytes */
  int64_t workspace_bytes;
} lrnnx_causal_conv1d_args;

/* Replaces causal_conv1d_fwd_function (x, weight, bias, None, None, None, silu). */
int lrnnx_causal_conv1d_fwd(const lrnnx_causal_conv1d_args *a, void *stream);
int64_t lrnnx_causal_conv1d_workspace_size(const lrnnx_causal_conv1d_args *a);
/* Replaces causal_conv1d_bwd_function (x, weight, bias, dout, None, None, None, dx, False, silu):
 * writes dx, dweight, dbias (if bias given). */
int lrnnx_causal_conv1d_bwd(const lrnnx_causal_conv1d_args *a, void *stream);
/* Replaces causal_conv1d_update (x, conv_state, weight, bias, activation). */
int lrnnx_causal_conv1d_update(const lrnnx_causal_conv1d_args *a, void *stream);

/* Fused residual-add + LayerNorm / RMSNorm over the last dimension of a
 * (rows, cols) matrix (reference lrnnx/ops/triton/layer_norm.py: _layer_norm_fwd
 * :323-470, _layer_norm_bwd :650-805, for the options lrnnx's blocks use:
 * no dropout, rowscale or second (x1 / weight1) branch).  Views use s0 = row
 * stride in elements; the columns are contiguous.
 *   xtype: x, y, dy, dx.   rtype: residual, residual_out, x_saved, dresidual,
 *   dresidual_in.          wtype: weight, bias, dweight, dbias.
 * mean (LayerNorm only) and rstd are fp32 per row. */
typedef struct lrnnx_layer_norm_args {
  int64_t rows, cols;
  int32_t xtype, rtype, wtype;
  int32_t is_rms_norm;
  float eps;
  int32_t reserved;
  lrnnx_view x, residual, weight, bias;  /* forward inputs (residual, bias optional) */
  lrnnx_view y, residual_out;            /* forward outputs (residual_out optional) */
  float *mean, *rstd;                    /* written by the forward, read by the backward */
  lrnnx_view x_saved, dy, dresidual;     /* backward inputs (dresidual optional) */
  lrnnx_view dx, dresidual_in, dweight, dbias;  /* backward outputs (dresidual_in, dbias optional) */
  void *workspace;                       /* backward: >= lrnnx_layer_norm_workspace_size() bytes */
  int64_t workspace_bytes;
} lrnnx_layer_norm_args;

/* Replaces _layer_norm_fwd (layer_norm.py:323-470): writes y, residual_out (if
 * given), mean (LayerNorm), rstd. */
int lrnnx_layer_norm_fwd(const lrnnx_layer_norm_args *a, void *stream);
int64_t lrnnx_layer_norm_workspace_size(const lrnnx_layer_norm_args *a);
/* Replaces _layer_norm_bwd (layer_norm.py:650-805): writes dx, dresidual_in (if
 * given: dx in the residual dtype), dweight, dbias (if given). */
int lrnnx_layer_norm_bwd(const lrnnx_layer_norm_args *a, void *stream);

/* Last error message of this thread ("" if none). */
const char *lrnnx_last_error(void);

/* ABI version of this header (bumped on any struct change). */
int lrnnx_abi_version(void);

#define LRNNX_ABI_VERSION 4

#ifdef __cplusplus
}
#endif

#endif /* LRNNX_SCAN_H */
