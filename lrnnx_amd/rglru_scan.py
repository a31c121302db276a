"""RG-LRU scan with the reference's API (reference lrnnx/ops/rglru_scan.py):
``RGLRUScanFn`` / ``rglru_scan_fn`` (:28-145) and the fused block
``rglru_inner_fn`` (:206-574).

The scan runs through this package's ``selective_scan_cuda`` binding with the
``"rglru"`` discretisation (A_bar = a ** delta, B_bar = sqrt(1 - A_bar^2),
identity B / C), exactly as the reference's wrapper drives its own binding;
the forward keeps the binding's fine state checkpoints for the backward, so
the backward does not re-run the forward to rebuild them.

``rglru_inner_fn`` computes the reference's ``RGLRUInnerFn`` forward (causal
conv1d, the recurrence and input gates, the scan, the stream-1 gate and the
output projection) as a composition of torch ops, this package's
``causal_conv1d_fn`` and ``RGLRUScanFn``; its gradient is autograd's.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import selective_scan_cuda as _ss
from .causal_conv1d import causal_conv1d_fn


class RGLRUScanFn(torch.autograd.Function):
    """Reference ``RGLRUScanFn`` (rglru_scan.py:28-121): u, delta (batch, dim, L)
    float32, A (dim, dstate) in (0, 1)."""

    @staticmethod
    def forward(ctx, u, delta, A, return_last_state=False):
        if not u.is_contiguous():
            u = u.contiguous()
        if not delta.is_contiguous():
            delta = delta.contiguous()
        if not A.is_contiguous():
            A = A.contiguous()
        dim, dstate = A.shape
        B = torch.ones(dim, dstate, dtype=u.dtype, device=u.device)
        C = torch.ones(dim, dstate, dtype=u.dtype, device=u.device)
        # the binding's fwd, keeping the fine state checkpoints for the backward
        # (the reference's wrapper saves x, from which its backward restarts;
        # so does the "x" save mode)
        a = _ss.build_args(u, delta, A, B, C, None, None, None, None, False, "rglru")
        out, x, _, ckpt = _ss.run_fwd(a, u, delta, A, None, want_out=True, want_ckpt=_ss.keeps_checkpoints())
        last_state = x[:, :, -1, 1::2]
        ctx.save_for_backward(u, delta, A, B, C, _ss.for_backward(x, ckpt))
        if return_last_state:
            return out, last_state
        return out

    @staticmethod
    def backward(ctx, dout, *args):
        u, delta, A, B, C, ckpt = ctx.saved_tensors
        if not dout.is_contiguous():
            dout = dout.contiguous()
        a = _ss.build_args(u, delta, A, B, C, None, None, None, None, False, "rglru")
        du, ddelta, dA = _ss.run_bwd(a, u, delta, A, B, C, None, None, None, None, dout, None, ckpt)[:3]
        return du, ddelta, dA, None


def rglru_scan_fn(u, delta, A, return_last_state=False):
    """Reference ``rglru_scan_fn`` (rglru_scan.py:124-145)."""
    return RGLRUScanFn.apply(u, delta, A, return_last_state)


def rglru_inner_fn(x, conv1d_weight, conv1d_bias, a, recurrent_gate_weight, recurrent_gate_bias, input_gate_weight,
                   input_gate_bias, out_proj_weight, out_proj_bias, gate, c=8.0):
    """Reference ``rglru_inner_fn`` (rglru_scan.py:516-574; forward of
    RGLRUInnerFn :224-364): x (batch, dim, L) before the conv, gate (batch, L,
    dim) -> (batch, L, d_model)."""
    dtype_in = x.dtype
    batch = x.shape[0]
    if a.dim() == 1:
        a = a.unsqueeze(-1)
    if x.stride(-1) != 1:
        x = x.contiguous()
    w = conv1d_weight[:, 0, :] if conv1d_weight.dim() == 3 else conv1d_weight
    x_f = causal_conv1d_fn(x, w, conv1d_bias, activation=None).float()
    x_flat = x_f.permute(0, 2, 1).reshape(-1, x_f.shape[1])                              # (b l) d
    rg = torch.sigmoid(F.linear(x_flat, recurrent_gate_weight.float(), recurrent_gate_bias.float()))
    ig = torch.sigmoid(F.linear(x_flat, input_gate_weight.float(), input_gate_bias.float()))
    rg = rg.reshape(batch, -1, x_f.shape[1]).permute(0, 2, 1)                             # b d l
    ig = ig.reshape(batch, -1, x_f.shape[1]).permute(0, 2, 1)
    delta = c * rg
    u_gated = ig * x_f
    y = rglru_scan_fn(u_gated, delta, a.float().contiguous()).permute(0, 2, 1)           # b l d
    out = F.linear(gate.float() * y, out_proj_weight.float(),
                   out_proj_bias.float() if out_proj_bias is not None else None)
    return out.to(dtype_in)
