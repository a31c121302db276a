"""Selective scan (S6 / Mamba) with the reference's Python API.

Mirrors ``SelectiveScanFn`` / ``selective_scan_fn`` of the reference
(lrnnx/ops/selective_scan.py:30-197): same argument order and defaults, same
return conventions (``out`` or ``(out, last_state)``, last_state multiplied by
a constant B, the z-gated output when z is given), same gradient order.

Implementation differences (same results):
* by default the forward also writes fp32 state checkpoints every 16 steps,
  which the backward reuses instead of re-scanning 2048-step chunks from
  ``x``; ``selective_scan_cuda.set_save_mode("x")`` (or LRNNX_SCAN_SAVE=x)
  keeps only ``x``, as the reference does, and the backward rebuilds them;
* tensors are copied only when their last stride is not 1 (the kernels take
  batch / channel strides), so Mamba's strided x / z halves of ``xz`` are
  not copied;
* bf16 / fp16 input works (fp32 state and arithmetic).
"""

from __future__ import annotations

import torch

from . import _lib
from . import selective_scan_cuda as _ss


def _lastdim_contig(t):
    if t is None:
        return None
    return t if (t.stride(-1) == 1 or t.size(-1) == 1) else t.contiguous()


class SelectiveScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, u, delta, A, B, C, D=None, z=None, delta_bias=None, deltaA=None, delta_softplus=False,
                return_last_state=False, discretization=None):
        u, delta, z, deltaA = (_lastdim_contig(t) for t in (u, delta, z, deltaA))
        B, C = _lastdim_contig(B), _lastdim_contig(C)
        if D is not None:
            D = D.contiguous()
        ctx.squeeze_B = B.dim() == 3
        ctx.squeeze_C = C.dim() == 3
        if B.dim() == 3:
            B = B.unsqueeze(1)
        if C.dim() == 3:
            C = C.unsqueeze(1)
        a = _ss.build_args(u, delta, A, B, C, D, z, delta_bias, deltaA, delta_softplus, discretization)
        # no backward will run (inference, no_grad): no checkpoints
        need_bwd = any(ctx.needs_input_grad[:9])
        out, x, out_z, ckpt = _ss.run_fwd(a, u, delta, A, z, want_out=True,
                                          want_ckpt=need_bwd and _ss.keeps_checkpoints())
        ctx.delta_softplus = delta_softplus
        ctx.discretization = discretization
        ctx.has_z = z is not None
        ctx.has_deltaA = deltaA is not None
        last_state = x[:, :, -1, 1::2]
        if B.dim() < 3 and return_last_state:
            last_state = last_state * B
        ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias, deltaA, _ss.for_backward(x, ckpt),
                              out if z is not None else None)
        res = out_z if z is not None else out
        return (res, last_state) if return_last_state else res

    @staticmethod
    def backward(ctx, dout, *args):
        u, delta, A, B, C, D, z, delta_bias, deltaA, saved, out = ctx.saved_tensors
        dout = _lastdim_contig(dout)
        a = _ss.build_args(u, delta, A, B, C, D, z, delta_bias, deltaA, ctx.delta_softplus, ctx.discretization)
        res = _ss.run_bwd(a, u, delta, A, B, C, D, z, delta_bias, deltaA, dout, out, saved)
        du, ddelta, dA, dB, dC, dD, ddelta_bias = res[:7]
        rest = res[7:]
        ddeltaA = rest.pop(0) if ctx.has_deltaA else None
        dz = rest.pop(0) if ctx.has_z else None
        if ctx.squeeze_B:
            dB = dB.squeeze(1)
        if ctx.squeeze_C:
            dC = dC.squeeze(1)
        return (du, ddelta, dA, dB, dC, dD if D is not None else None, dz,
                ddelta_bias if delta_bias is not None else None, ddeltaA, None, None, None)


def selective_scan_fn(u, delta, A, B, C, D=None, z=None, delta_bias=None, deltaA=None, delta_softplus=False,
                      return_last_state=False, discretization="mamba"):
    """If return_last_state is True, returns (out, last_state); last_state has
    shape (batch, dim, dstate).  The gradient of last_state is not propagated
    (as in the reference, lrnnx/ops/selective_scan.py:166-197)."""
    return SelectiveScanFn.apply(u, delta, A, B, C, D, z, delta_bias, deltaA, delta_softplus, return_last_state,
                                 discretization)
