"""Drop-in replacement of the reference's pybind11 module ``simplified_scan_cuda``.

``fwd(u, delta, A, B, C, deltaA, discretization) -> [out, x]`` and
``bwd(u, delta, A, B, C, deltaA, dout, x, discretization) -> [du, ddelta, dA, dB, dC, (ddeltaA)]``
keep the reference binding's positional signatures and return lists
(csrc/simplified_scan/bindings.cpp:5-8, simplified_scan.h:98-109, host code
csrc/simplified_scan/simplified_scan_cpu.cpp:160-331).  Superset: delta /
deltaA may have a zero stride along L (a broadcast time step).
"""

from __future__ import annotations

import torch

from . import _lib

CHUNK = 2048
_VALID = {"zoh": 0, "bilinear": 1, "dirac": 2}


def build_args(u, delta, A, B, C, deltaA, discretization):
    _lib.require_gpu(u, delta, A, B, C, deltaA)
    if u.dtype != torch.complex64 or A.dtype != torch.complex64:
        raise RuntimeError("simplified scan: u and A must be complex64")
    if discretization not in _VALID:
        raise RuntimeError("Discretization method not supported")
    batch, P, L = u.shape
    ds = A.shape[1]
    if ds > 256:
        raise RuntimeError("simplified_scan only supports state dimension <= 256")
    if u.stride(-1) != 1 and L != 1:
        raise RuntimeError("u must have unit stride along L")
    for t, nm in ((delta, "delta"), (deltaA, "deltaA")):
        if t is None:
            continue
        if t.dtype != torch.float32:
            raise RuntimeError(f"{nm} must be float32")
        if tuple(t.shape) != (batch, P, L):
            raise RuntimeError(f"{nm} must have shape {(batch, P, L)}")
        if t.stride(-1) not in (0, 1) and L != 1:
            raise RuntimeError(f"{nm} must have stride 1 (or 0) along L")
    for t, nm in ((A, "A"), (B, "B"), (C, "C")):
        if tuple(t.shape) != (P, ds) or t.dtype != torch.complex64:
            raise RuntimeError(f"{nm} must be complex64 of shape {(P, ds)}")
    a = _lib.SimplifiedScanArgs()
    a.batch, a.dim, a.seqlen, a.dstate = batch, P, L, ds
    a.method = _VALID[discretization]
    a.u = _lib.view(u, 2)
    a.delta = _lib.view_full(delta)
    a.deltaA = _lib.view_full(deltaA)
    a.A, a.B, a.C = _lib.view(A, 2), _lib.view(B, 2), _lib.view(C, 2)
    return a


def _workspace(a, bwd, device):
    n = _lib.lib().lrnnx_simplified_scan_workspace_size(a, int(bwd))
    ws = torch.empty(max(n, 256), dtype=torch.uint8, device=device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    return ws


def run_fwd(a, u, want_ckpt=False):
    batch, P, L = u.shape
    out = torch.empty_like(u)
    x = torch.empty((batch, P, (L + CHUNK - 1) // CHUNK, 2 * a.dstate), dtype=torch.complex64, device=u.device)
    a.out = _lib.view(out, 2)
    a.x = x.data_ptr()
    ckpt = None
    if want_ckpt:
        n = _lib.lib().lrnnx_simplified_scan_ckpt_size(a)
        ckpt = torch.empty(max(n, 8) // 8, dtype=torch.complex64, device=u.device)
        a.ckpt = ckpt.data_ptr()
    ws = _workspace(a, False, u.device)
    with _lib.on_device(u):
        _lib.check(_lib.lib().lrnnx_simplified_scan_fwd(a, _lib.stream_of(u)), "simplified_scan_fwd")
    del ws
    return out, x, ckpt


def run_bwd(a, u, delta, A, B, C, deltaA, dout, ckpt=None, need_ddelta=True):
    _lib.require_gpu(dout)
    if dout.dtype != torch.complex64 or tuple(dout.shape) != tuple(u.shape):
        raise RuntimeError("dout must be complex64 with the shape of u")
    if dout.stride(-1) != 1:
        dout = dout.contiguous()
    du = torch.empty_like(u)
    ddelta = torch.empty(u.shape, dtype=torch.float32, device=u.device) if need_ddelta else None
    ddA = torch.empty(u.shape, dtype=torch.float32, device=u.device) if (need_ddelta and deltaA is not None) else None
    dA, dB, dC = torch.empty_like(A), torch.empty_like(B), torch.empty_like(C)
    a.need_ddelta = int(need_ddelta)
    a.dout = _lib.view(dout, 2)
    a.du = _lib.view(du, 2)
    a.ddelta, a.ddeltaA = _lib.view_full(ddelta), _lib.view_full(ddA)
    a.dA, a.dB, a.dC = _lib.view(dA, 2), _lib.view(dB, 2), _lib.view(dC, 2)
    a.ckpt = ckpt.data_ptr() if ckpt is not None else None
    ws = _workspace(a, True, u.device)
    with _lib.on_device(u):
        _lib.check(_lib.lib().lrnnx_simplified_scan_bwd(a, _lib.stream_of(u)), "simplified_scan_bwd")
    del ws
    res = [du, ddelta, dA, dB, dC]
    if deltaA is not None:
        res.append(ddA)
    return res


def fwd(u, delta, A, B, C, deltaA, discretization):
    a = build_args(u, delta, A, B, C, deltaA, discretization)
    out, x, _ = run_fwd(a, u)
    return [out, x]


def bwd(u, delta, A, B, C, deltaA, dout, x, discretization):
    a = build_args(u, delta, A, B, C, deltaA, discretization)
    return run_bwd(a, u, delta, A, B, C, deltaA, dout)
