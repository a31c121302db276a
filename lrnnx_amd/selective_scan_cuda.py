"""Drop-in replacement of the reference's pybind11 module ``selective_scan_cuda``.

``fwd`` and ``bwd`` take the same positional arguments and return the same
lists as the reference binding (csrc/selective_scan/bindings.cpp:5-8,
signatures csrc/selective_scan/selective_scan.h:114-136, host code
csrc/selective_scan/selective_scan_cpu.cpp:263-632), so
``lrnnx/ops/{selective_scan,s7_scan,rglru_scan}.py`` can import this module
under that name unchanged.  Every output is allocated here with torch; the
gfx950 kernels are reached through the C ABI of liblrnnx_scan.so.

Differences from the reference, all supersets:
* bf16 / fp16 input is accepted for the "mamba" method (the reference
  kernels are fp32-only, selective_scan_cpu.cpp:404, :612);
* inputs need unit stride along L only (the reference additionally copies
  non-contiguous tensors in its Python wrapper);
* ``bwd`` does not need ``x``: it rebuilds its fine checkpoints itself
  (from the x carries when given, chunk-parallel).

What the backward keeps from the forward (``set_save_mode``, or
``LRNNX_SCAN_SAVE`` in the environment):
* "checkpoints" (default): the forward also writes fp32 states every 16
  steps (B x L/16 x N x D x 4 bytes) and the backward reuses them.  ``fwd``
  attaches them to the returned ``x`` (attribute ``_lrnnx_ckpt``), so that a
  caller that saves ``x`` and hands it to ``bwd``, as the reference's
  wrappers do, gets the fast backward without a rebuild; they live as long
  as ``x`` does.
* "x": only the reference's chunk carries ``x`` (B x D x L/2048 x 2N x 4
  bytes) are kept, as in the reference; the backward first rebuilds the
  checkpoints in its workspace (a states-only forward pass).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib

import os

CHUNK = 2048

_SAVE_MODES = ("checkpoints", "x")
_save_mode = os.environ.get("LRNNX_SCAN_SAVE", "checkpoints")
if _save_mode not in _SAVE_MODES:
    raise RuntimeError(f"LRNNX_SCAN_SAVE must be one of {_SAVE_MODES}, got {_save_mode!r}")


def set_save_mode(mode: str) -> None:
    """"checkpoints" (fast backward, B L N D / 16 fp32 values kept per call) or
    "x" (the reference's chunk carries only; the backward rebuilds)."""
    global _save_mode
    if mode not in _SAVE_MODES:
        raise ValueError(f"save mode must be one of {_SAVE_MODES}, got {mode!r}")
    _save_mode = mode


def save_mode() -> str:
    return _save_mode


def keeps_checkpoints() -> bool:
    return _save_mode == "checkpoints"


def for_backward(x, ckpt):
    """The tensor a wrapper saves for ``run_bwd``: the checkpoints, or x in
    the "x" mode."""
    return ckpt if (ckpt is not None and keeps_checkpoints()) else x


def _n_chunks(L: int) -> int:
    return (L + CHUNK - 1) // CHUNK


def _method(name) -> int:
    if name is None:
        name = "mamba"
    try:
        return _lib.METHODS[name]
    except KeyError:
        raise RuntimeError("Discretization method not supported") from None


def _check_last_stride(t, name):
    if t is not None and not (t.stride(-1) == 1 or t.size(-1) == 1):
        raise RuntimeError(f"{name} must have unit stride in its last dimension")


def _shape(t, *shape, name="tensor"):
    if tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


def build_args(u, delta, A, B, C, D, z, delta_bias, deltaA, delta_softplus, discretization):
    """Validate like the reference host code and fill the C argument struct."""
    _lib.require_gpu(u, delta, A, B, C, D, z, delta_bias, deltaA)
    itype, wtype = u.dtype, A.dtype
    if itype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError("u must be float32, float16 or bfloat16")
    if wtype not in (torch.float32, torch.complex64):
        raise RuntimeError("A must be float32 or complex64")
    is_complex = wtype == torch.complex64
    var_B, var_C = B.dim() >= 3, C.dim() >= 3
    if delta.dtype != itype:
        raise RuntimeError("delta must have the dtype of u")
    if B.dtype != (itype if var_B else wtype) or C.dtype != (itype if var_C else wtype):
        raise RuntimeError("variable B/C must have the dtype of u, constant B/C the dtype of A")
    batch, dim, L = u.shape
    N = A.shape[1]
    G = B.shape[1] if var_B else (C.shape[1] if var_C else 1)
    if N > 256:
        raise RuntimeError("selective_scan only supports state dimension <= 256")
    _shape(delta, batch, dim, L, name="delta")
    _shape(A, dim, N, name="A")
    Lb = 2 * L if is_complex else L
    for X, nm, var in ((B, "B", var_B), (C, "C", var_C)):
        if var:
            _shape(X, batch, G, N, Lb, name=nm)
            _check_last_stride(X, nm)
        else:
            _shape(X, dim, N, name=nm)
    if var_B and var_C and B.shape[1] != C.shape[1]:
        raise RuntimeError("B and C must have the same number of groups")
    for t, nm in ((u, "u"), (delta, "delta"), (z, "z"), (deltaA, "deltaA")):
        _check_last_stride(t, nm)
        if t is not None:
            _shape(t, batch, dim, L, name=nm)
            if t.dtype != itype:
                raise RuntimeError(f"{nm} must have the dtype of u")
    for t, nm in ((D, "D"), (delta_bias, "delta_bias")):
        if t is not None:
            if t.dtype != torch.float32:
                raise RuntimeError(f"{nm} must be float32")
            _shape(t, dim, name=nm)
    a = _lib.SelectiveScanArgs()
    a.batch, a.dim, a.seqlen, a.dstate, a.n_groups = batch, dim, L, N, G
    a.itype, a.wtype = _lib.dtype_code(itype), _lib.dtype_code(wtype)
    a.method = _method(discretization)
    a.var_B, a.var_C, a.delta_softplus = int(var_B), int(var_C), int(bool(delta_softplus))
    a.u, a.delta, a.z, a.deltaA = (_lib.view(t, 2) for t in (u, delta, z, deltaA))
    a.A = _lib.view(A, 2) if A.dim() == 2 else _lib.view(A)
    a.B = _lib.view(B, 3) if var_B else _lib.view(B, 2)
    a.C = _lib.view(C, 3) if var_C else _lib.view(C, 2)
    a.D, a.delta_bias = _lib.view(D, 1), _lib.view(delta_bias, 1)
    if a.D.ptr:
        a.D.s0 = D.stride(0)
    if a.delta_bias.ptr:
        a.delta_bias.s0 = delta_bias.stride(0)
    return a


def run_fwd(a, u, delta, A, z, want_out=True, want_ckpt=False):
    """Allocate out / out_z / x (/ ckpt) and launch the forward."""
    batch, dim, L = u.shape
    N = A.shape[1]
    out = torch.empty_like(delta) if want_out else None
    out_z = torch.empty_like(z) if z is not None else None
    x = torch.empty((batch, dim, _n_chunks(L), 2 * N), dtype=A.dtype, device=u.device)
    ckpt = None
    a.out = _lib.view(out, 2)
    a.out_z = _lib.view(out_z, 2)
    a.x = x.data_ptr()
    if want_ckpt:
        n = _lib.lib().lrnnx_selective_scan_ckpt_size(a)
        ckpt = torch.empty(max(n, 4) // 4, dtype=torch.float32, device=u.device)
        a.ckpt = ckpt.data_ptr()
    nws = _lib.lib().lrnnx_selective_scan_workspace_size(a, 0)
    ws = None
    if nws > 0:  # small grids: the forward splits L into segments
        ws = torch.empty(nws, dtype=torch.uint8, device=u.device)
        a.workspace, a.workspace_bytes = ws.data_ptr(), nws
    with _lib.on_device(u):
        _lib.check(_lib.lib().lrnnx_selective_scan_fwd(a, _lib.stream_of(u)), "selective_scan_fwd")
    return out, x, out_z, ckpt


def run_bwd(a, u, delta, A, B, C, D, z, delta_bias, deltaA, dout, out, saved, dz=None):
    """Allocate the gradients and launch the backward.  ``saved`` is what
    ``for_backward`` chose: the forward's checkpoints (flat fp32), its x
    carries (4-D; the backward rebuilds the checkpoints from them) or None.
    Returns the reference's list [du, ddelta, dA, dB, dC, dD, ddelta_bias,
    (ddeltaA), (dz)]."""
    ckpt = saved if (saved is not None and saved.dim() == 1) else None
    x = saved if (saved is not None and saved.dim() == 4) else None
    _lib.require_gpu(dout)
    _check_last_stride(dout, "dout")
    if dout.dtype != u.dtype:
        raise RuntimeError("dout must have the dtype of u")
    _shape(dout, *u.shape, name="dout")
    if z is not None:
        if out is None:
            raise RuntimeError("out is required by the backward when z is given")
        _check_last_stride(out, "out")
    var_B, var_C = bool(a.var_B), bool(a.var_C)
    du = torch.empty_like(u)
    ddelta = torch.empty_like(delta)
    dA = torch.empty_like(A)
    dB = torch.empty_like(B)
    dC = torch.empty_like(C)
    dD = torch.empty_like(D) if D is not None else None
    ddb = torch.empty_like(delta_bias) if delta_bias is not None else None
    ddA = torch.empty_like(deltaA) if deltaA is not None else None
    if z is not None and dz is None:
        dz = torch.empty_like(z)
    a.dout = _lib.view(dout, 2)
    a.out_saved = _lib.view(out, 2)
    a.du, a.ddelta, a.ddeltaA, a.dz = (_lib.view(t, 2) for t in (du, ddelta, ddA, dz))
    a.dA = _lib.view(dA, 2)
    a.dB = _lib.view(dB, 3) if var_B else _lib.view(dB, 2)
    a.dC = _lib.view(dC, 3) if var_C else _lib.view(dC, 2)
    a.dD, a.ddelta_bias = _lib.view(dD, 1), _lib.view(ddb, 1)
    a.ckpt = ckpt.data_ptr() if ckpt is not None else None
    if ckpt is None and x is not None and x.dtype == torch.float32:
        _shape(x, u.shape[0], u.shape[1], _n_chunks(u.shape[2]), 2 * A.shape[1], name="x")
        if not x.is_contiguous():
            raise RuntimeError("x must be contiguous")
        a.x = x.data_ptr()   # seeds of the checkpoint rebuild
    L = _lib.lib()
    nws = L.lrnnx_selective_scan_workspace_size(a, 1)
    ws = torch.empty(max(nws, 256), dtype=torch.uint8, device=u.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    with _lib.on_device(u):
        _lib.check(L.lrnnx_selective_scan_bwd(a, _lib.stream_of(u)), "selective_scan_bwd")
    res = [du, ddelta, dA, dB, dC, dD, ddb]
    if deltaA is not None:
        res.append(ddA)
    if z is not None:
        res.append(dz)
    return res


def fwd(u, delta, A, B, C, D, z, delta_bias, deltaA, delta_softplus, discretization):
    """selective_scan_cuda.fwd: returns [out, x] (+ [out_z] if z is given)."""
    a = build_args(u, delta, A, B, C, D, z, delta_bias, deltaA, delta_softplus, discretization)
    out, x, out_z, ckpt = run_fwd(a, u, delta, A, z, want_ckpt=keeps_checkpoints())
    if ckpt is not None:
        x._lrnnx_ckpt = ckpt   # picked up by bwd when it is handed this x
    res = [out, x]
    if z is not None:
        res.append(out_z)
    return res


def bwd(u, delta, A, B, C, D, z, delta_bias, deltaA, dout, x, out, dz, delta_softplus, recompute_out_z,
        discretization):
    """selective_scan_cuda.bwd: returns [du, ddelta, dA, dB, dC, dD, ddelta_bias]
    (+ [ddeltaA] if deltaA, + [dz] if z, + [out_z] if recompute_out_z)."""
    a = build_args(u, delta, A, B, C, D, z, delta_bias, deltaA, delta_softplus, discretization)
    saved = x
    ck = getattr(x, "_lrnnx_ckpt", None) if x is not None else None
    if ck is not None and ck.device == u.device and ck.numel() * 4 == _lib.lib().lrnnx_selective_scan_ckpt_size(a):
        saved = ck   # the checkpoints fwd wrote with this x
    res = run_bwd(a, u, delta, A, B, C, D, z, delta_bias, deltaA, dout, out, saved, dz)
    if recompute_out_z and z is not None:
        res.append((out.float() * F.silu(z.float())).to(out.dtype))
    return res
