"""S7 scan with the reference's API (reference lrnnx/ops/s7_scan.py):
``S7ScanFn`` / ``s7_scan_fn`` (:16-176) and the fused block ``s7_inner_fn``
(:236-509).

The scan runs through this package's ``selective_scan_cuda`` binding with the
``"s7"`` discretisation (the forward keeping the fine state checkpoints for
the backward), exactly as the reference's wrapper drives its own
binding: the time-varying A goes in as delta, the kernel's A is zero and its
B / C are ones, one state per "channel" (the S7 state index), and the input
and output projections B u and C h are einsums around the kernel.

``s7_inner_fn`` computes the reference's ``S7InnerFn`` forward (in_proj,
x_proj split into A, B, C, D, bias, the scan, the D skip, the GELU / sigmoid
gate and the residual) as a composition of torch ops and ``S7ScanFn``; its
gradient is autograd's.  The reference's hand-written backward differs from
its own forward there: the forward applies the exact (erf) GELU while the
backward uses the derivative of the tanh approximation (s7_scan.py:326 vs
:388-396), so gradients through the gate are exact here and approximate in the
reference.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import selective_scan_cuda as _ss

_fwd = torch.amp.custom_fwd(device_type="cuda")
_bwd = torch.amp.custom_bwd(device_type="cuda")


class S7ScanFn(torch.autograd.Function):
    """Reference ``S7ScanFn`` (s7_scan.py:16-143): u (batch, dim, L), A (batch,
    dstate, L), B (batch, dstate, dim, L), C (batch, dim, dstate, L), bias
    (batch, dstate, L) or None."""

    @staticmethod
    @_fwd
    def forward(ctx, u, A, B, C, bias=None, return_last_state=False):
        dstate = A.shape[1]
        if not u.is_contiguous():
            u = u.contiguous()
        Bu = torch.einsum("bnhl,bhl->bnl", B.float(), u.float())
        if bias is not None:
            Bu = Bu + bias.float()
        Bu = Bu.contiguous()
        delta = A.contiguous()
        A_k = torch.zeros(dstate, 1, dtype=Bu.dtype, device=Bu.device)
        B_k = torch.ones(dstate, 1, dtype=Bu.dtype, device=Bu.device)
        C_k = torch.ones(dstate, 1, dtype=Bu.dtype, device=Bu.device)
        # the binding's fwd, keeping the fine state checkpoints for the backward
        a = _ss.build_args(Bu, delta, A_k, B_k, C_k, None, None, None, None, False, "s7")
        out_k, x_k, _, ckpt = _ss.run_fwd(a, Bu, delta, A_k, None, want_out=True,
                                          want_ckpt=_ss.keeps_checkpoints())
        y = torch.einsum("bhnl,bnl->bhl", C.float(), out_k.float())
        last_state = out_k[:, :, -1]
        ctx.save_for_backward(u, B, C, bias, Bu, out_k, _ss.for_backward(x_k, ckpt), delta, A_k, B_k, C_k)
        if return_last_state:
            return y.to(u.dtype), last_state
        return y.to(u.dtype)

    @staticmethod
    @_bwd
    def backward(ctx, dout, *args):
        u, B, C, bias, Bu, out_k, ckpt, delta, A_k, B_k, C_k = ctx.saved_tensors
        dout = dout.float()
        if dout.stride(-1) != 1:
            dout = dout.contiguous()
        dC = torch.einsum("bhl,bnl->bhnl", dout, out_k.float())
        dout_k = torch.einsum("bhnl,bhl->bnl", C.float(), dout).contiguous()
        a = _ss.build_args(Bu, delta, A_k, B_k, C_k, None, None, None, None, False, "s7")
        dBu, ddelta = _ss.run_bwd(a, Bu, delta, A_k, B_k, C_k, None, None, None, None, dout_k, None, ckpt)[:2]
        dB = torch.einsum("bnl,bhl->bnhl", dBu, u.float())
        du = torch.einsum("bnhl,bnl->bhl", B.float(), dBu)
        return du.to(u.dtype), ddelta, dB, dC, (dBu if bias is not None else None), None


def s7_scan_fn(u, A, B, C, bias=None, return_last_state=False):
    """Reference ``s7_scan_fn`` (s7_scan.py:146-176)."""
    return S7ScanFn.apply(u, A, B, C, bias, return_last_state)


def s7_inner_fn(hidden_states, in_proj_weight, x_proj_weight, gate_proj_weight, d_state, base_params):
    """Reference ``s7_inner_fn`` (s7_scan.py:493-509; forward of S7InnerFn
    :241-350): hidden_states (batch, L, d_model) -> (batch, L, d_model)."""
    batch, seqlen, d_model = hidden_states.shape
    if hidden_states.stride(-1) != 1:
        hidden_states = hidden_states.contiguous()
    x = F.linear(hidden_states, in_proj_weight)
    x_dbl = F.linear(x.reshape(batch * seqlen, d_model), x_proj_weight)
    A, B, C, D, bias = torch.split(x_dbl, [d_state, d_model * d_state, d_model * d_state, d_model, d_state], dim=-1)
    A = A.reshape(batch, seqlen, d_state).permute(0, 2, 1) + base_params.unsqueeze(0).unsqueeze(-1)
    B = B.reshape(batch, seqlen, d_model, d_state).permute(0, 3, 2, 1)            # b n h l
    C = C.reshape(batch, seqlen, d_model, d_state).permute(0, 2, 3, 1)            # b h n l
    D_tv = D.reshape(batch, seqlen, d_model).permute(0, 2, 1)                     # b h l
    bias = bias.reshape(batch, seqlen, d_state).permute(0, 2, 1)                  # b n l
    u = x.permute(0, 2, 1)                                                         # b h l
    # the scan's output in fp32, as the reference computes y before the D skip
    y = s7_scan_fn(u.float(), A, B, C, bias=bias)
    y = y + D_tv.float() * u.float()
    y_t = y.permute(0, 2, 1)
    gate = torch.sigmoid(F.linear(F.gelu(y_t), gate_proj_weight))
    out = gate * y_t + hidden_states
    return out.to(hidden_states.dtype)
