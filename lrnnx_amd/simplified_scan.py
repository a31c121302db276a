"""Simplified (S5) scan with the reference's Python API.

Mirrors ``SimplifiedScanFn`` / ``simplified_scan_fn`` and ``S5InnerFn`` /
``s5_inner_fn`` (reference lrnnx/ops/simplified_scan.py:14-230, :343-583):
Bu = B @ u and y = C @ states are torch complex GEMMs around the gfx950 scan
kernel, exactly as in the reference.

Differences (same values):
* ``return_last_state`` returns h_L of shape (batch, P), the value the
  reference's own ``simplified_scan_ref`` returns (simplified_scan.py:329);
  the reference's CUDA-path wrapper slices ``out[:, -1, 1::2] + 1j*out[:, -1, 0::2]``
  (simplified_scan.py:106-108), which is not the last state;
* a delta broadcast along L (stride 0) is not materialised;
* ddelta is not computed when delta does not require grad.
"""

from __future__ import annotations

import torch

from . import simplified_scan_cuda as _sc


def _kernel_A(A):
    return A.unsqueeze(-1) if A.dim() == 1 else A


def _lastdim_ok(t):
    if t is None:
        return None
    return t if t.stride(-1) in (0, 1) else t.contiguous()


class SimplifiedScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, u, delta, A, B, C, deltaA, discretization, return_last_state=False):
        if u.stride(-1) != 1:
            u = u.contiguous()
        delta, deltaA = _lastdim_ok(delta), _lastdim_ok(deltaA)
        A_k = _kernel_A(A)
        P, ds = A_k.shape
        Bu = torch.einsum("ph,bhl->bpl", B, u).contiguous()
        Bi = torch.ones(P, ds, dtype=A.dtype, device=A.device)
        Ci = torch.ones(P, ds, dtype=A.dtype, device=A.device)
        a = _sc.build_args(Bu, delta, A_k, Bi, Ci, deltaA, discretization)
        out, x, ckpt = _sc.run_fwd(a, Bu, want_ckpt=True)
        y = torch.einsum("hp,bpl->bhl", C, out)
        ctx.discretization = discretization
        ctx.has_deltaA = deltaA is not None
        ctx.A_was_1d = A.dim() == 1
        ctx.save_for_backward(u, delta, A_k, B, C, Bu, out, ckpt, Bi, Ci, deltaA)
        if return_last_state:
            return y, x[:, :, -1, 1]
        return y

    @staticmethod
    def backward(ctx, dout, *args):
        u, delta, A, B, C, Bu, out, ckpt, Bi, Ci, deltaA = ctx.saved_tensors
        dx_out = torch.einsum("hp,bhl->bpl", C.conj(), dout).contiguous()
        dC = torch.einsum("bhl,bpl->hp", dout, out.conj())
        need_dd = bool(ctx.needs_input_grad[1] or ctx.needs_input_grad[5])
        a = _sc.build_args(Bu, delta, A, Bi, Ci, deltaA, ctx.discretization)
        res = _sc.run_bwd(a, Bu, delta, A, Bi, Ci, deltaA, dx_out, ckpt, need_ddelta=need_dd)
        dBu, ddelta, dA = res[0], res[1], res[2]
        ddeltaA = res[5] if ctx.has_deltaA else None
        du = torch.einsum("ph,bpl->bhl", B.conj(), dBu)
        dB = torch.einsum("bpl,bhl->ph", dBu, u.conj())
        if dA.dim() == 2 and dA.shape[1] == 1 and ctx.A_was_1d:
            dA = dA.squeeze(-1)
        return du, ddelta, dA, dB, dC, ddeltaA, None, None


def simplified_scan_fn(u, delta, A, B, C, deltaA=None, return_last_state=False, discretization="bilinear"):
    """u (b, H, l) complex64; delta (b, P, l) float32; A (P,) or (P, 1) complex64;
    B (P, H), C (H, P) complex64.  Returns y (b, H, l) (and h_L (b, P))."""
    valid = ("bilinear", "zoh", "dirac")
    if discretization not in valid:
        raise ValueError(f"discretization must be one of {valid}, got '{discretization}'")
    return SimplifiedScanFn.apply(u, delta, A, B, C, deltaA, discretization, return_last_state)


class S5InnerFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, u, delta, A, B, C, D, deltaA, discretization, conj_sym):
        if u.stride(-1) != 1:
            u = u.contiguous()
        delta, deltaA = _lastdim_ok(delta), _lastdim_ok(deltaA)
        A_k = _kernel_A(A)
        P, ds = A_k.shape
        Bu = torch.einsum("ph,bhl->bpl", B, u).contiguous()
        Bi = torch.ones(P, ds, dtype=A.dtype, device=A.device)
        Ci = torch.ones(P, ds, dtype=A.dtype, device=A.device)
        a = _sc.build_args(Bu, delta, A_k, Bi, Ci, deltaA, discretization)
        scan_out, x, ckpt = _sc.run_fwd(a, Bu, want_ckpt=True)
        y_c = torch.einsum("hp,bpl->bhl", C, scan_out)
        y_real = 2 * y_c.real if conj_sym else y_c.real
        u_real = u.real if u.is_complex() else u
        y = y_real + D.unsqueeze(0).unsqueeze(-1) * u_real
        ctx.discretization, ctx.conj_sym = discretization, conj_sym
        ctx.has_deltaA = deltaA is not None
        ctx.A_was_1d = A.dim() == 1
        ctx.save_for_backward(u, delta, A_k, B, C, D, Bu, scan_out, ckpt, Bi, Ci, deltaA)
        return y

    @staticmethod
    def backward(ctx, dout):
        u, delta, A, B, C, D, Bu, scan_out, ckpt, Bi, Ci, deltaA = ctx.saved_tensors
        u_real = u.real if u.is_complex() else u
        dD = torch.einsum("bhl,bhl->h", dout, u_real)
        du_skip = D.unsqueeze(0).unsqueeze(-1) * dout
        scale = 2.0 if ctx.conj_sym else 1.0
        dy_c = torch.complex(scale * dout, torch.zeros_like(dout))
        dscan = torch.einsum("hp,bhl->bpl", C.conj(), dy_c).contiguous()
        dC = torch.einsum("bhl,bpl->hp", dy_c, scan_out.conj())
        need_dd = bool(ctx.needs_input_grad[1] or ctx.needs_input_grad[6])
        a = _sc.build_args(Bu, delta, A, Bi, Ci, deltaA, ctx.discretization)
        res = _sc.run_bwd(a, Bu, delta, A, Bi, Ci, deltaA, dscan, ckpt, need_ddelta=need_dd)
        dBu, ddelta, dA = res[0], res[1], res[2]
        ddeltaA = res[5] if ctx.has_deltaA else None
        du_scan = torch.einsum("ph,bpl->bhl", B.conj(), dBu)
        dB = torch.einsum("bpl,bhl->ph", dBu, u.conj())
        du = du_scan + torch.complex(du_skip, torch.zeros_like(du_skip)) if u.is_complex() else du_scan.real + du_skip
        if dA.dim() == 2 and dA.shape[1] == 1 and ctx.A_was_1d:
            dA = dA.squeeze(-1)
        return du, ddelta, dA, dB, dC, dD, ddeltaA, None, None


def s5_inner_fn(u, delta, A, B, C, D, deltaA=None, discretization="bilinear", conj_sym=True):
    """out = (2 if conj_sym else 1) * Re(C @ scan(B @ u)) + D * Re(u), real (b, H, l)."""
    return S5InnerFn.apply(u, delta, A, B, C, D, deltaA, discretization, conj_sym)
