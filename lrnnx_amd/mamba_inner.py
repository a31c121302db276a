"""Fused Mamba inner block with the reference's API: ``mamba_inner_fn`` /
``MambaInnerFn`` (reference lrnnx/ops/selective_scan.py:389-786).

in_proj output xz -> causal conv1d (silu) -> x_proj -> delta_proj -> selective
scan (variable B / C taken from x_proj's output) -> out_proj, with the
backward recomputing the conv output and delta (checkpoint_lvl 1), as the
reference does.  The conv and the scan run in this package's HIP kernels
(``causal_conv1d_*_function``, the selective-scan C ABI); the projections
are torch GEMMs, as in the reference.

Differences from the reference, each where the reference cannot run or is wrong:
* the scan is called with the binding's full arity (the reference passes 9 of
  the 11 forward and 14 of the 16 backward arguments,
  selective_scan.py:520-522, :637-654, so its fused path fails at call time);
* the scan's forward checkpoints are kept for the backward (no re-scan);
* ``out_proj_bias``'s gradient is the sum over batch and length per output
  channel (the reference sums ``dout`` after reshaping it to (e, b l) over both
  dimensions, which gives a scalar);
* the B / C / dt RMSNorm options (selective_scan.py:501-518: RMSNorm over
  d_state of variable B / C after their projection bias, over the channels of
  delta) run in this package's fused norm kernels with their full backward:
  the gradients of B / C / delta pass through the norm, and the norm weights
  get gradients.  The reference's backward re-normalises the already
  normalised B / C (:608-630), passes dB / dC / ddelta through without the
  norm's Jacobian and returns no gradient for the weights (:731).  They are
  supported for real A and variable B / C (the reference's rearrange cannot
  take the complex layout).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import selective_scan_cuda as _ss
from .causal_conv1d import causal_conv1d_bwd_function, causal_conv1d_fwd_function
from .layer_norm import _layer_norm_bwd, _layer_norm_fwd


def _rms_rows(X, w, eps):
    """RMSNorm over the last dim of a (rows, n) matrix -> (normalised, rstd)."""
    y, _, _, rstd, _, _, _, _ = _layer_norm_fwd(X, w.contiguous(), None, eps, is_rms_norm=True)
    return y, rstd


def _rms_rows_bwd(dY, X, w, rstd, eps):
    """Gradients of _rms_rows: (dX, dw)."""
    dX, dw, _, _, _, _, _ = _layer_norm_bwd(dY.contiguous(), X, w.contiguous(), None, eps, None, rstd,
                                            is_rms_norm=True)
    return dX, dw


def _delta_rows(delta):
    # b d l -> (b l) d
    b, d, L = delta.shape
    return delta.transpose(1, 2).reshape(b * L, d).contiguous()


def _delta_from_rows(rows, b):
    # (b l) d -> b d l (unit stride along l)
    bl, d = rows.shape
    return rows.reshape(b, bl // b, d).transpose(1, 2).contiguous()


def _bc_from_xdbl(X, L, complex_A):
    # (b l) n -> b 1 n l   (complex A: (b l) (n two) -> b 1 n (l two))
    bl, n2 = X.shape
    b = bl // L
    if not complex_A:
        return X.reshape(b, L, n2).permute(0, 2, 1).unsqueeze(1).contiguous()
    return X.reshape(b, L, n2 // 2, 2).permute(0, 2, 1, 3).reshape(b, 1, n2 // 2, 2 * L).contiguous()


def _bc_to_xdbl(dX, complex_A):
    # inverse of _bc_from_xdbl for the gradients
    b, _, n, Lx = dX.shape
    if not complex_A:
        return dX[:, 0].permute(0, 2, 1).reshape(b * Lx, n)
    L = Lx // 2
    return dX[:, 0].reshape(b, n, L, 2).permute(0, 2, 1, 3).reshape(b * L, 2 * n)


class MambaInnerFn(torch.autograd.Function):
    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
                out_proj_bias, A, B=None, C=None, D=None, delta_bias=None, B_proj_bias=None, C_proj_bias=None,
                delta_softplus=True, checkpoint_lvl=1, b_rms_weight=None, c_rms_weight=None, dt_rms_weight=None,
                b_c_dt_rms_eps=1e-6):
        """xz: (batch, 2 * dim, seqlen)"""
        assert checkpoint_lvl in [0, 1]
        L = xz.shape[-1]
        delta_rank = delta_proj_weight.shape[1]
        complex_A = A.is_complex()
        d_state = A.shape[-1] * (2 if complex_A else 1)
        if complex_A and (b_rms_weight is not None or c_rms_weight is not None or dt_rms_weight is not None):
            raise NotImplementedError("mamba_inner_fn: the B / C / dt RMSNorm options need a real A")
        if (b_rms_weight is not None and B is not None) or (c_rms_weight is not None and C is not None):
            raise NotImplementedError("mamba_inner_fn: the B / C RMSNorm options apply to variable B / C")
        if torch.is_autocast_enabled():
            dt_ = torch.get_autocast_gpu_dtype()
            x_proj_weight = x_proj_weight.to(dtype=dt_)
            delta_proj_weight = delta_proj_weight.to(dtype=dt_)
            out_proj_weight = out_proj_weight.to(dtype=dt_)
            out_proj_bias = out_proj_bias.to(dtype=dt_) if out_proj_bias is not None else None
        if xz.stride(-1) != 1:
            xz = xz.contiguous()
        conv1d_weight = conv1d_weight[:, 0, :] if conv1d_weight.dim() == 3 else conv1d_weight
        x, z = xz.chunk(2, dim=1)
        conv1d_bias = conv1d_bias.contiguous() if conv1d_bias is not None else None
        conv1d_out = causal_conv1d_fwd_function(x, conv1d_weight, conv1d_bias, None, None, None, True)
        b = xz.shape[0]
        x_dbl = F.linear(conv1d_out.transpose(1, 2).reshape(b * L, -1), x_proj_weight)   # (b l) (r + 2n)
        delta = (delta_proj_weight @ x_dbl[:, :delta_rank].t()).reshape(-1, b, L).transpose(0, 1)   # b d l
        eps = b_c_dt_rms_eps
        rms_saved = [None] * 6   # B rows, B rstd, C rows, C rstd, delta rows, delta rstd
        if dt_rms_weight is not None:
            rows = _delta_rows(delta)
            normed, rstd = _rms_rows(rows, dt_rms_weight, eps)
            delta = _delta_from_rows(normed, b)
            rms_saved[4], rms_saved[5] = (rows if checkpoint_lvl == 0 else None), rstd
        ctx.is_variable_B, ctx.is_variable_C = B is None, C is None
        ctx.B_proj_bias_is_None, ctx.C_proj_bias_is_None = B_proj_bias is None, C_proj_bias is None
        if B is None:
            Bx = x_dbl[:, delta_rank:delta_rank + d_state]
            if B_proj_bias is not None:
                Bx = Bx + B_proj_bias.to(dtype=Bx.dtype)
            if b_rms_weight is not None:
                Bx = Bx.contiguous()
                rms_saved[0] = Bx
                Bx, rms_saved[1] = _rms_rows(Bx, b_rms_weight, eps)
            B = _bc_from_xdbl(Bx, L, complex_A)
        elif B.stride(-1) != 1:
            B = B.contiguous()
        if C is None:
            Cx = x_dbl[:, -d_state:]
            if C_proj_bias is not None:
                Cx = Cx + C_proj_bias.to(dtype=Cx.dtype)
            if c_rms_weight is not None:
                Cx = Cx.contiguous()
                rms_saved[2] = Cx
                Cx, rms_saved[3] = _rms_rows(Cx, c_rms_weight, eps)
            C = _bc_from_xdbl(Cx, L, complex_A)
        elif C.stride(-1) != 1:
            C = C.contiguous()
        if D is not None:
            D = D.contiguous()
        a = _ss.build_args(conv1d_out, delta, A, B, C, D, z, delta_bias, None, delta_softplus, "mamba")
        out, x, out_z, ckpt = _ss.run_fwd(a, conv1d_out, delta, A, z, want_out=True,
                                          want_ckpt=_ss.keeps_checkpoints())
        ckpt = _ss.for_backward(x, ckpt)
        ctx.delta_softplus = delta_softplus
        ctx.out_proj_bias_is_None = out_proj_bias is None
        ctx.checkpoint_lvl = checkpoint_lvl
        if checkpoint_lvl >= 1:   # recomputed in the backward
            conv1d_out, delta = None, None
        ctx.eps = eps
        ctx.save_for_backward(xz, conv1d_weight, conv1d_bias, x_dbl, x_proj_weight, delta_proj_weight,
                              out_proj_weight, conv1d_out, delta, A, B, C, D, delta_bias, ckpt, out,
                              b_rms_weight, c_rms_weight, dt_rms_weight, *rms_saved)
        return F.linear(out_z.transpose(1, 2), out_proj_weight, out_proj_bias)

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        # dout: (batch, seqlen, dim_model)
        (xz, conv1d_weight, conv1d_bias, x_dbl, x_proj_weight, delta_proj_weight, out_proj_weight, conv1d_out,
         delta, A, B, C, D, delta_bias, ckpt, out, b_rms_weight, c_rms_weight, dt_rms_weight,
         B_rows, B_rstd, C_rows, C_rstd, dt_rows, dt_rstd) = ctx.saved_tensors
        L = xz.shape[-1]
        b = xz.shape[0]
        delta_rank = delta_proj_weight.shape[1]
        complex_A = A.is_complex()
        d_state = A.shape[-1] * (2 if complex_A else 1)
        x, z = xz.chunk(2, dim=1)
        if dout.stride(-1) != 1:
            dout = dout.contiguous()
        if ctx.checkpoint_lvl == 1:
            conv1d_out = causal_conv1d_fwd_function(x, conv1d_weight, conv1d_bias, None, None, None, True)
            delta = (delta_proj_weight @ x_dbl[:, :delta_rank].t()).reshape(-1, b, L).transpose(0, 1)
            if dt_rms_weight is not None:   # the forward's normalisation, with its saved rstd
                dt_rows = _delta_rows(delta)
                delta = _delta_from_rows(_rms_rows(dt_rows, dt_rms_weight, ctx.eps)[0], b)
        dxz = torch.empty_like(xz)
        dx, dz = dxz.chunk(2, dim=1)
        dout2 = dout.reshape(b * L, -1).t()                                   # e (b l)
        dout_y = (out_proj_weight.t() @ dout2).reshape(-1, b, L).transpose(0, 1)   # b d l
        if dout_y.stride(-1) != 1:
            dout_y = dout_y.contiguous()
        a = _ss.build_args(conv1d_out, delta, A, B, C, D, z, delta_bias, None, ctx.delta_softplus, "mamba")
        res = _ss.run_bwd(a, conv1d_out, delta, A, B, C, D, z, delta_bias, None, dout_y, out, ckpt, dz=dz)
        dconv1d_out, ddelta, dA, dB, dC, dD, ddelta_bias = res[:7]
        out_z = (out.float() * F.silu(z.float())).to(out.dtype)
        dout_proj_weight = dout2 @ out_z.transpose(1, 2).reshape(b * L, -1)   # e d
        dout_proj_bias = dout2.sum(dim=1) if not ctx.out_proj_bias_is_None else None
        dD = dD if D is not None else None
        dx_dbl = torch.empty_like(x_dbl)
        dB_proj_bias = dC_proj_bias = None
        db_rms = dc_rms = ddt_rms = None
        if ctx.is_variable_B:
            dBx = _bc_to_xdbl(dB, complex_A).to(x_dbl.dtype)
            if b_rms_weight is not None:
                dBx, db_rms = _rms_rows_bwd(dBx, B_rows, b_rms_weight, B_rstd, ctx.eps)
                dBx = dBx.to(x_dbl.dtype)
            dB_proj_bias = dBx.sum(0) if not ctx.B_proj_bias_is_None else None
            dx_dbl[:, delta_rank:delta_rank + d_state] = dBx
            dB = None
        if ctx.is_variable_C:
            dCx = _bc_to_xdbl(dC, complex_A).to(x_dbl.dtype)
            if c_rms_weight is not None:
                dCx, dc_rms = _rms_rows_bwd(dCx, C_rows, c_rms_weight, C_rstd, ctx.eps)
                dCx = dCx.to(x_dbl.dtype)
            dC_proj_bias = dCx.sum(0) if not ctx.C_proj_bias_is_None else None
            dx_dbl[:, -d_state:] = dCx
            dC = None
        if dt_rms_weight is not None:
            drows, ddt_rms = _rms_rows_bwd(_delta_rows(ddelta), dt_rows, dt_rms_weight, dt_rstd, ctx.eps)
            ddelta = _delta_from_rows(drows.to(ddelta.dtype), b)
        ddelta2 = ddelta.transpose(0, 1).reshape(ddelta.shape[1], -1)        # d (b l)
        ddelta_proj_weight = ddelta2 @ x_dbl[:, :delta_rank]                  # d r
        dx_dbl[:, :delta_rank] = ddelta2.t() @ delta_proj_weight              # (b l) r
        conv_flat = conv1d_out.transpose(1, 2).reshape(b * L, -1)             # (b l) d
        dx_proj_weight = dx_dbl.t() @ conv_flat                                # (r + 2n) d
        dconv1d_out = dconv1d_out + (dx_dbl @ x_proj_weight).reshape(b, L, -1).transpose(1, 2)
        dxr, dconv1d_weight, dconv1d_bias, _ = causal_conv1d_bwd_function(
            x, conv1d_weight, conv1d_bias, dconv1d_out.contiguous(), None, None, None, dx, False, True)
        dconv1d_weight = dconv1d_weight.to(conv1d_weight.dtype).unsqueeze(1)
        dconv1d_bias = dconv1d_bias.to(conv1d_bias.dtype) if conv1d_bias is not None else None
        return (dxz, dconv1d_weight, dconv1d_bias, dx_proj_weight, ddelta_proj_weight, dout_proj_weight,
                dout_proj_bias, dA, dB, dC, dD, ddelta_bias if delta_bias is not None else None, dB_proj_bias,
                dC_proj_bias, None, None,
                db_rms.to(b_rms_weight.dtype) if db_rms is not None else None,
                dc_rms.to(c_rms_weight.dtype) if dc_rms is not None else None,
                ddt_rms.to(dt_rms_weight.dtype) if ddt_rms is not None else None, None)


def mamba_inner_fn(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight, out_proj_bias,
                   A, B=None, C=None, D=None, delta_bias=None, B_proj_bias=None, C_proj_bias=None,
                   delta_softplus=True, checkpoint_lvl=1, b_rms_weight=None, c_rms_weight=None, dt_rms_weight=None,
                   b_c_dt_rms_eps=1e-6):
    """Returns out_proj(scan(...)) of shape (batch, seqlen, dim_model)."""
    return MambaInnerFn.apply(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
                              out_proj_bias, A, B, C, D, delta_bias, B_proj_bias, C_proj_bias, delta_softplus,
                              checkpoint_lvl, b_rms_weight, c_rms_weight, dt_rms_weight, b_c_dt_rms_eps)
