"""Depthwise causal conv1d with the API of the causal-conv1d package.

lrnnx calls the package (an optional dependency, reference pyproject.toml:33)
at lrnnx/models/ltv/mamba.py:274 (``causal_conv1d_fn``), :411
(``causal_conv1d_update``) and lrnnx/ops/selective_scan.py:448, :640
(``causal_conv1d_fwd_function`` / ``causal_conv1d_bwd_function``).  This module
provides those four names with the same arguments; the compute runs in the
gfx950 kernels of liblrnnx_scan.so (``lrnnx_causal_conv1d_*``).  Semantics
are the Mamba layer's own fallbacks (mamba.py:271, :398-410):
``out = act(conv1d(x, weight, bias, padding=w-1, groups=d)[..., :seqlen])``.

Supported: activation None / "silu" / "swish", width 1..8, x in f32 / f16 /
bf16.  The package's ``seq_idx``, ``initial_states`` / final states,
``cache_seqlens`` and ``conv_state_indices`` options are not used by lrnnx
and raise NotImplementedError here.
"""

from __future__ import annotations

import torch

from . import _lib


def _silu_flag(activation):
    if activation in (None, False):
        return 0
    if activation in ("silu", "swish", True):
        return 1
    raise NotImplementedError("activation must be None, 'silu' or 'swish'")


def _args(x, weight, bias, silu):
    _lib.require_gpu(x, weight, bias)
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError("x must be float32, float16 or bfloat16")
    if weight.dim() == 3:
        weight = weight[:, 0, :]
    batch, dim, seqlen = x.shape
    if weight.shape[0] != dim:
        raise RuntimeError(f"weight must have shape ({dim}, width), got {tuple(weight.shape)}")
    a = _lib.CausalConv1dArgs()
    a.batch, a.dim, a.seqlen, a.width = batch, dim, seqlen, weight.shape[1]
    a.itype = _lib.dtype_code(x.dtype)
    a.silu = int(silu)
    w32 = weight.float()
    b32 = bias.float() if bias is not None else None
    a.x = _lib.view_full(x)
    a.weight = _lib.view_full(w32)
    a.bias = _lib.view_full(b32)
    return a, (w32, b32)


def causal_conv1d_fwd_function(x, weight, bias, seq_idx, initial_states, final_states_out, silu_activation):
    """out = act(causal conv of x); x (b, d, l)."""
    if seq_idx is not None or initial_states is not None or final_states_out is not None:
        raise NotImplementedError("seq_idx / initial_states / final_states_out are not supported")
    if x.stride(-1) != 1:
        x = x.contiguous()
    a, keep = _args(x, weight, bias, bool(silu_activation))
    out = torch.empty_like(x, memory_format=torch.contiguous_format)
    a.out = _lib.view_full(out)
    with _lib.on_device(x):
        _lib.check(_lib.lib().lrnnx_causal_conv1d_fwd(a, _lib.stream_of(x)), "causal_conv1d_fwd")
    return out


def causal_conv1d_bwd_function(x, weight, bias, dout, seq_idx, initial_states, dfinal_states, dx,
                               return_dinitial_states, silu_activation):
    """Returns (dx, dweight, dbias, None); dweight (d, w) and dbias in fp32."""
    if seq_idx is not None or initial_states is not None or dfinal_states is not None or return_dinitial_states:
        raise NotImplementedError("seq_idx / initial states are not supported")
    if x.stride(-1) != 1:
        x = x.contiguous()
    if dout.stride(-1) != 1:
        dout = dout.contiguous()
    a, keep = _args(x, weight, bias, bool(silu_activation))
    if dx is None:
        dx = torch.empty_like(x, memory_format=torch.contiguous_format)
    dweight = torch.empty(a.dim, a.width, dtype=torch.float32, device=x.device)
    dbias = torch.empty(a.dim, dtype=torch.float32, device=x.device) if bias is not None else None
    a.out = _lib.view_full(dout)   # unused by the backward; must be non-null
    a.dout, a.dx = _lib.view_full(dout), _lib.view_full(dx)
    a.dweight, a.dbias = _lib.view_full(dweight), _lib.view_full(dbias)
    n = _lib.lib().lrnnx_causal_conv1d_workspace_size(a)
    ws = torch.empty(max(n, 256), dtype=torch.uint8, device=x.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    with _lib.on_device(x):
        _lib.check(_lib.lib().lrnnx_causal_conv1d_bwd(a, _lib.stream_of(x)), "causal_conv1d_bwd")
    return dx, dweight, dbias, None


class CausalConv1dFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, activation):
        silu = _silu_flag(activation)
        ctx.silu, ctx.w_shape, ctx.w_dtype = silu, weight.shape, weight.dtype
        ctx.has_bias = bias is not None
        ctx.save_for_backward(x, weight, bias)
        return causal_conv1d_fwd_function(x, weight, bias, None, None, None, silu)

    @staticmethod
    def backward(ctx, dout):
        x, weight, bias = ctx.saved_tensors
        dx, dw, db, _ = causal_conv1d_bwd_function(x, weight, bias, dout, None, None, None, None, False, ctx.silu)
        dw = dw.reshape(ctx.w_shape).to(ctx.w_dtype)
        db = db.to(bias.dtype) if ctx.has_bias else None
        return dx, dw, db, None


def causal_conv1d_fn(x, weight, bias=None, seq_idx=None, initial_states=None, return_final_states=False,
                     final_states_out=None, activation=None):
    """x (b, d, l); weight (d, w); bias (d,) or None; activation None / "silu" / "swish".
    Returns (b, d, l) in x's dtype."""
    if seq_idx is not None or initial_states is not None or return_final_states or final_states_out is not None:
        raise NotImplementedError("seq_idx / initial_states / final states are not supported")
    return CausalConv1dFn.apply(x, weight, bias, activation)


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None, cache_seqlens=None,
                         conv_state_indices=None):
    """One decode step (or a few): x (b, d) or (b, d, l_new); conv_state
    (b, d, s) with s >= w - 1, shifted in place.  Returns out like x."""
    if cache_seqlens is not None or conv_state_indices is not None:
        raise NotImplementedError("cache_seqlens / conv_state_indices are not supported")
    squeeze = x.dim() == 2
    xs = x.unsqueeze(-1) if squeeze else x
    _lib.require_gpu(conv_state)
    if conv_state.dtype != x.dtype:
        raise RuntimeError("conv_state must have the dtype of x")
    a, keep = _args(xs, weight, bias, _silu_flag(activation))
    out = torch.empty_like(xs)
    a.out = _lib.view_full(out)
    a.state_len = conv_state.shape[-1]
    a.conv_state = _lib.view_full(conv_state)
    with _lib.on_device(x):
        _lib.check(_lib.lib().lrnnx_causal_conv1d_update(a, _lib.stream_of(x)), "causal_conv1d_update")
    return out.squeeze(-1) if squeeze else out
