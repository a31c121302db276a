"""Fused residual-add LayerNorm / RMSNorm with the API of the reference's Triton
module (reference lrnnx/ops/triton/layer_norm.py): ``_layer_norm_fwd``,
``_layer_norm_bwd``, ``LayerNormFn``, ``layer_norm_fn``, ``rms_norm_fn`` and the
``RMSNorm`` module, with the compute in the gfx950 kernels of liblrnnx_scan.so
(``lrnnx_layer_norm_fwd`` / ``lrnnx_layer_norm_bwd``).

lrnnx calls it from its blocks (lrnnx/layers/block.py:77-87, :112-122) and its
language model (lrnnx/architectures/language_model.py:378-388, :417-427,
:440-450, :499-509) as ``layer_norm_fn(x, w, b, residual=..., prenorm=...,
residual_in_fp32=..., eps=..., is_rms_norm=...)``.  Semantics follow the Triton
kernels (layer_norm.py:202-322, :490-649): x + residual summed in fp32, stored
as residual_out in the residual dtype, normalised unrounded; the backward
recomputes xhat from residual_out.

Not supported (each raises NotImplementedError; lrnnx never passes them):
dropout_p > 0, rowscale, the parallel second norm (x1 / weight1 / bias1) and
``recompute_output``.  ``LayerNormLinearFn`` / ``layer_norm_linear_fn``
(layer_norm.py:1097-1260; no caller in lrnnx) are the norm followed by a
linear layer, computed as that composition and differentiated by autograd (the
reference recomputes y in its backward instead of keeping it).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib

_F32_TYPES = (torch.float32, torch.float16, torch.bfloat16)


def _unsupported(x1=None, weight1=None, bias1=None, dropout_p=0.0, rowscale=None):
    if x1 is not None or weight1 is not None or bias1 is not None:
        raise NotImplementedError("layer_norm: the parallel norm (x1 / weight1 / bias1) is not supported")
    if dropout_p > 0.0:
        raise NotImplementedError("layer_norm: dropout_p > 0 is not supported")
    if rowscale is not None:
        raise NotImplementedError("layer_norm: rowscale is not supported")


def _check_dtype(t, what):
    if t is not None and t.dtype not in _F32_TYPES:
        raise RuntimeError(f"layer_norm: {what} must be float32, float16 or bfloat16 (got {t.dtype})")


def _weights(weight, bias):
    """weight / bias share one dtype code in the kernel: upcast both to fp32 when
    they differ (the kernel reads them as fp32 values either way)."""
    if bias is not None and bias.dtype != weight.dtype:
        return weight.float().contiguous(), bias.float().contiguous()
    return weight.contiguous(), (bias.contiguous() if bias is not None else None)


def _base_args(M, N, xdt, rdt, weight, bias, eps, is_rms_norm):
    a = _lib.LayerNormArgs()
    a.rows, a.cols = M, N
    a.xtype, a.rtype, a.wtype = _lib.dtype_code(xdt), _lib.dtype_code(rdt), _lib.dtype_code(weight.dtype)
    a.is_rms_norm = int(bool(is_rms_norm))
    a.eps = float(eps)
    a.weight = _lib.view(weight)
    a.bias = _lib.view(bias)
    return a


def _layer_norm_fwd(x, weight, bias, eps, residual=None, x1=None, weight1=None, bias1=None, dropout_p=0.0,
                    rowscale=None, out_dtype=None, residual_dtype=None, is_rms_norm=False,
                    return_dropout_mask=False):
    """Reference ``_layer_norm_fwd`` (layer_norm.py:323-470).  x (M, N).
    Returns (y, y1, mean, rstd, residual_out or x, seeds, dropout_mask,
    dropout_mask1) with y1, seeds and the masks None."""
    _unsupported(x1, weight1, bias1, dropout_p, rowscale)
    _lib.require_gpu(x, weight, bias, residual)
    if residual is not None:
        residual_dtype = residual.dtype
    M, N = x.shape
    assert x.stride(-1) == 1
    if residual is not None:
        assert residual.stride(-1) == 1
        assert residual.shape == (M, N)
    assert weight.shape == (N,)
    assert weight.stride(-1) == 1
    if bias is not None:
        assert bias.stride(-1) == 1
        assert bias.shape == (N,)
    for t, n in ((x, "x"), (residual, "residual"), (weight, "weight"), (bias, "bias")):
        _check_dtype(t, n)
    if residual_dtype is not None and residual_dtype not in _F32_TYPES:
        raise RuntimeError(f"layer_norm: residual_dtype must be a floating type (got {residual_dtype})")
    if N * x.element_size() > 65536:
        raise RuntimeError("This layer norm doesn't support feature dim >= 64KB.")
    w, b = _weights(weight, bias)
    y = torch.empty_like(x, dtype=x.dtype, memory_format=torch.contiguous_format)
    if residual is not None or (residual_dtype is not None and residual_dtype != x.dtype):
        residual_out = torch.empty(M, N, device=x.device,
                                   dtype=residual_dtype if residual_dtype is not None else x.dtype)
    else:
        residual_out = None
    rdt = residual_out.dtype if residual_out is not None else x.dtype
    mean = torch.empty((M,), dtype=torch.float32, device=x.device) if not is_rms_norm else None
    rstd = torch.empty((M,), dtype=torch.float32, device=x.device)
    if M > 0:
        a = _base_args(M, N, x.dtype, rdt, w, b, eps, is_rms_norm)
        a.x = _lib.view(x)
        a.residual = _lib.view(residual)
        a.y = _lib.view(y)
        a.residual_out = _lib.view(residual_out)
        a.mean = mean.data_ptr() if mean is not None else None
        a.rstd = rstd.data_ptr()
        with _lib.on_device(x):
            _lib.check(_lib.lib().lrnnx_layer_norm_fwd(a, _lib.stream_of(x)), "layer_norm_fwd")
    if out_dtype is not None and out_dtype != y.dtype:
        y = y.to(out_dtype)
    return (y, None, mean, rstd, residual_out if residual_out is not None else x, None, None, None)


def _layer_norm_bwd(dy, x, weight, bias, eps, mean, rstd, dresidual=None, dy1=None, weight1=None, bias1=None,
                    seeds=None, dropout_p=0.0, rowscale=None, has_residual=False, has_x1=False, is_rms_norm=False,
                    x_dtype=None, recompute_output=False):
    """Reference ``_layer_norm_bwd`` (layer_norm.py:650-805).  x is the saved
    pre-norm input (residual_out, or x when there was none).  Returns
    (dx, dw, db, dresidual_in, dx1, dw1, db1) with dx1 / dw1 / db1 None."""
    _unsupported(None, weight1, bias1, dropout_p, rowscale)
    if dy1 is not None or has_x1 or seeds is not None:
        raise NotImplementedError("layer_norm: the parallel norm / dropout backward is not supported")
    if recompute_output:
        raise NotImplementedError("layer_norm: recompute_output is not supported")
    _lib.require_gpu(dy, x, weight, bias, dresidual)
    M, N = x.shape
    assert x.stride(-1) == 1
    assert dy.stride(-1) == 1
    assert dy.shape == (M, N)
    if dresidual is not None:
        assert dresidual.stride(-1) == 1
        assert dresidual.shape == (M, N)
    assert weight.shape == (N,)
    assert weight.stride(-1) == 1
    if bias is not None:
        assert bias.stride(-1) == 1
        assert bias.shape == (N,)
    xdt = x.dtype if x_dtype is None else x_dtype
    if N * x.element_size() > 65536:
        raise RuntimeError("This layer norm doesn't support feature dim >= 64KB.")
    if dy.dtype != xdt:
        dy = dy.to(xdt)
    if dresidual is not None and dresidual.dtype != x.dtype:
        dresidual = dresidual.to(x.dtype)
    w, b = _weights(weight, bias)
    dx = torch.empty(M, N, dtype=xdt, device=x.device)
    dresidual_in = torch.empty_like(x) if has_residual and dx.dtype != x.dtype else None
    dw = torch.empty(N, dtype=w.dtype, device=x.device)
    db = torch.empty(N, dtype=w.dtype, device=x.device) if bias is not None else None
    if M > 0:
        a = _base_args(M, N, xdt, x.dtype, w, b, eps, is_rms_norm)
        a.mean = mean.data_ptr() if (mean is not None and not is_rms_norm) else None
        a.rstd = rstd.data_ptr()
        a.x_saved = _lib.view(x)
        a.dy = _lib.view(dy)
        a.dresidual = _lib.view(dresidual)
        a.dx = _lib.view(dx)
        a.dresidual_in = _lib.view(dresidual_in)
        a.dweight = _lib.view(dw)
        a.dbias = _lib.view(db)
        L = _lib.lib()
        ws_bytes = L.lrnnx_layer_norm_workspace_size(a)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws_bytes
        with _lib.on_device(x):
            _lib.check(L.lrnnx_layer_norm_bwd(a, _lib.stream_of(x)), "layer_norm_bwd")
    else:
        dw.zero_()
        if db is not None:
            db.zero_()
    dw = dw.to(weight.dtype)
    db = db.to(bias.dtype) if bias is not None else None
    if has_residual and dx.dtype == x.dtype:
        dresidual_in = dx
    return dx, dw, db, dresidual_in, None, None, None


class LayerNormFn(torch.autograd.Function):
    """Reference ``LayerNormFn`` (layer_norm.py:808-990)."""

    @staticmethod
    def forward(ctx, x, weight, bias, residual=None, x1=None, weight1=None, bias1=None, eps=1e-6, dropout_p=0.0,
                rowscale=None, prenorm=False, residual_in_fp32=False, is_rms_norm=False, return_dropout_mask=False):
        _unsupported(x1, weight1, bias1, dropout_p, rowscale)
        x_shape_og = x.shape
        x = x.reshape(-1, x.shape[-1])
        if x.stride(-1) != 1:
            x = x.contiguous()
        if residual is not None:
            assert residual.shape == x_shape_og
            residual = residual.reshape(-1, residual.shape[-1])
            if residual.stride(-1) != 1:
                residual = residual.contiguous()
        weight = weight.contiguous()
        if bias is not None:
            bias = bias.contiguous()
        residual_dtype = residual.dtype if residual is not None else (torch.float32 if residual_in_fp32 else None)
        y, _, mean, rstd, residual_out, _, _, _ = _layer_norm_fwd(
            x, weight, bias, eps, residual, residual_dtype=residual_dtype, is_rms_norm=is_rms_norm)
        ctx.save_for_backward(residual_out, weight, bias, mean, rstd)
        ctx.x_shape_og = x_shape_og
        ctx.eps = eps
        ctx.is_rms_norm = is_rms_norm
        ctx.has_residual = residual is not None
        ctx.prenorm = prenorm
        ctx.x_dtype = x.dtype
        y = y.reshape(x_shape_og)
        residual_out = residual_out.reshape(x_shape_og)
        if not return_dropout_mask:
            return y if not prenorm else (y, residual_out)
        return (y, None, None) if not prenorm else (y, residual_out, None, None)

    @staticmethod
    def backward(ctx, dy, *args):
        x, weight, bias, mean, rstd = ctx.saved_tensors
        dy = dy.reshape(-1, dy.shape[-1])
        if dy.stride(-1) != 1:
            dy = dy.contiguous()
        assert dy.shape == x.shape
        if ctx.prenorm and args and args[0] is not None:
            dresidual = args[0].reshape(-1, args[0].shape[-1])
            if dresidual.stride(-1) != 1:
                dresidual = dresidual.contiguous()
            assert dresidual.shape == x.shape
        else:
            dresidual = None
        dx, dw, db, dresidual_in, _, _, _ = _layer_norm_bwd(
            dy, x, weight, bias, ctx.eps, mean, rstd, dresidual, has_residual=ctx.has_residual,
            is_rms_norm=ctx.is_rms_norm, x_dtype=ctx.x_dtype)
        return (dx.reshape(ctx.x_shape_og), dw, db,
                dresidual_in.reshape(ctx.x_shape_og) if ctx.has_residual else None,
                None, None, None, None, None, None, None, None, None, None)


def layer_norm_fn(x, weight, bias, residual=None, x1=None, weight1=None, bias1=None, eps=1e-6, dropout_p=0.0,
                  rowscale=None, prenorm=False, residual_in_fp32=False, is_rms_norm=False,
                  return_dropout_mask=False):
    """Reference ``layer_norm_fn`` (layer_norm.py:993-1023)."""
    return LayerNormFn.apply(x, weight, bias, residual, x1, weight1, bias1, eps, dropout_p, rowscale, prenorm,
                             residual_in_fp32, is_rms_norm, return_dropout_mask)


def rms_norm_fn(x, weight, bias, residual=None, x1=None, weight1=None, bias1=None, eps=1e-6, dropout_p=0.0,
                rowscale=None, prenorm=False, residual_in_fp32=False, return_dropout_mask=False):
    """Reference ``rms_norm_fn`` (layer_norm.py:1026-1055)."""
    return LayerNormFn.apply(x, weight, bias, residual, x1, weight1, bias1, eps, dropout_p, rowscale, prenorm,
                             residual_in_fp32, True, return_dropout_mask)


class RMSNorm(torch.nn.Module):
    """Reference ``RMSNorm`` (layer_norm.py:1058-1093): weight initialised to
    ones, no bias; forward(x, residual=None, prenorm=False,
    residual_in_fp32=False)."""

    def __init__(self, hidden_size, eps=1e-5, dropout_p=0.0, device=None, dtype=None):
        factory_kwargs = {"device": device, "dtype": dtype}
        super().__init__()
        self.eps = eps
        self.drop = torch.nn.Dropout(dropout_p) if dropout_p > 0.0 else None
        self.weight = torch.nn.Parameter(torch.empty(hidden_size, **factory_kwargs))
        self.register_parameter("bias", None)
        self.reset_parameters()

    def reset_parameters(self):
        torch.nn.init.ones_(self.weight)

    def forward(self, x, residual=None, prenorm=False, residual_in_fp32=False):
        return rms_norm_fn(x, self.weight, self.bias, residual=residual, eps=self.eps,
                           dropout_p=self.drop.p if self.drop is not None and self.training else 0.0,
                           prenorm=prenorm, residual_in_fp32=residual_in_fp32)


def _layer_norm_linear(x, norm_weight, norm_bias, linear_weight, linear_bias, residual=None, eps=1e-6,
                       prenorm=False, residual_in_fp32=False, is_rms_norm=False):
    y, residual_out = LayerNormFn.apply(x, norm_weight, norm_bias, residual, None, None, None, eps, 0.0, None, True,
                                        residual_in_fp32, is_rms_norm, False)
    # the linear layer runs in the autocast dtype when autocast is on (layer_norm.py:1135-1150)
    dtype = torch.get_autocast_gpu_dtype() if torch.is_autocast_enabled() else y.dtype
    out = F.linear(y.to(dtype), linear_weight.to(dtype), linear_bias.to(dtype) if linear_bias is not None else None)
    return out if not prenorm else (out, residual_out)


class LayerNormLinearFn:
    """Reference ``LayerNormLinearFn`` (layer_norm.py:1097-1217): ``apply`` with the
    same arguments returns linear(norm(x + residual)) (and residual_out when
    prenorm)."""

    apply = staticmethod(_layer_norm_linear)


def layer_norm_linear_fn(x, norm_weight, norm_bias, linear_weight, linear_bias, residual=None, eps=1e-6,
                         prenorm=False, residual_in_fp32=False, is_rms_norm=False):
    """Reference ``layer_norm_linear_fn`` (layer_norm.py:1220-1245)."""
    return _layer_norm_linear(x, norm_weight, norm_bias, linear_weight, linear_bias, residual, eps, prenorm,
                              residual_in_fp32, is_rms_norm)
