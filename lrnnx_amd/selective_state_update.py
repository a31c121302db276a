"""One-token state update for decoding, with the reference's API.

Mirrors ``selective_state_update`` (reference
lrnnx/ops/triton/selective_state_update.py:300-476): same arguments, the same
optional heads / groups / batch-index forms, in-place update of ``state``.
The Triton kernel is replaced by a gfx950 HIP kernel; no allocation besides
``out``, no host synchronisation, so it can be captured in a HIP graph.
"""

from __future__ import annotations

import torch

from . import _lib

_DISC = {"zoh": 0, "bilinear": 1, "dirac": 2, "mamba": 3, "s7": 4, "rglru": 5}


def _with_head(t, at):
    """(shape, strides) of t with a size-1 head dimension inserted at `at`
    (stride 0), without making a new tensor view."""
    sh, st = tuple(t.shape), t.stride()
    return sh[:at] + (1,) + sh[at:], st[:at] + (0,) + st[at:]


def _geom(t, full_dims, at):
    """(shape, strides) of t in its headed form: as is when it has `full_dims`
    dimensions, else with the head inserted at `at`."""
    if t.dim() == full_dims:
        return tuple(t.shape), t.stride()
    return _with_head(t, at)


def _fields(t, strides, n):
    """The (pointer, strides...) run of one tensor in lrnnx_state_update_args."""
    if t is None:
        return (None,) + (0,) * n
    return (t.data_ptr(),) + tuple(strides)


def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None, dt_softplus=False, deltaA=None,
                           state_batch_indices=None, discretization="mamba"):
    """state: (batch, dim, dstate) or (batch, nheads, dim, dstate), updated in place.
    Returns out: (batch, dim) or (batch, nheads, dim).

    The head-less forms are one head with stride 0.  Shapes and strides are
    checked and passed as tuples, so a call makes no tensor views (host time
    per call matters to eager decoding)."""
    has_heads = state.dim() > 3
    _lib.require_gpu(state, x, dt, A, B, C, D, z, dt_bias, deltaA)
    if A.dtype != torch.float32:
        A = A.float()
    if D is not None and D.dtype != torch.float32:
        D = D.float()
    if dt_bias is not None and dt_bias.dtype != torch.float32:
        dt_bias = dt_bias.float()
    if dt.dtype != x.dtype:
        dt = dt.to(x.dtype)
    if z is not None and z.dtype != x.dtype:
        z = z.to(x.dtype)
    if deltaA is not None and deltaA.dtype != x.dtype:
        deltaA = deltaA.to(x.dtype)
    if C.dtype != B.dtype:
        C = C.to(B.dtype)
    st_sh, st_st = _geom(state, 4, 1)
    x_sh, x_st = _geom(x, 3, 1)
    dt_sh, dt_st = _geom(dt, 3, 1)
    A_sh, A_st = _geom(A, 3, 0)
    B_sh, B_st = _geom(B, 3, 1)
    C_sh, C_st = _geom(C, 3, 1)
    _, nheads, dim, dstate = st_sh
    batch = x_sh[0]
    assert x_sh == (batch, nheads, dim)
    assert dt_sh == x_sh
    assert A_sh == (nheads, dim, dstate)
    ngroups = B_sh[1]
    assert nheads % ngroups == 0, "nheads must be divisible by ngroups"
    assert B_sh == (batch, ngroups, dstate)
    assert C_sh == B_sh
    D_st = z_st = dtb_st = dA_st = ()
    if D is not None:
        D_sh, D_st = _geom(D, 2, 0)
        assert D_sh == (nheads, dim)
    if z is not None:
        z_sh, z_st = _geom(z, 3, 1)
        assert z_sh == x_sh
    if dt_bias is not None:
        dtb_sh, dtb_st = _geom(dt_bias, 2, 0)
        assert dtb_sh == (nheads, dim)
    if deltaA is not None:
        dA_sh, dA_st = _geom(deltaA, 3, 1)
        assert dA_sh == x_sh
    sbi = None
    if state_batch_indices is not None:
        assert tuple(state_batch_indices.shape) == (batch,)
        sbi = state_batch_indices.to(torch.int32)
    out = torch.empty(x_sh, dtype=x.dtype, device=x.device)
    a = _lib.StateUpdateArgs(
        batch, nheads, dim, dstate, ngroups,
        _lib.dtype_code(state.dtype), _lib.dtype_code(x.dtype), _lib.dtype_code(B.dtype),
        _DISC.get(discretization.lower(), 3), int(bool(dt_softplus)),
        *_fields(state, st_st, 4), *_fields(x, x_st, 3), *_fields(dt, dt_st, 3), *_fields(A, A_st, 3),
        *_fields(B, B_st, 3), *_fields(C, C_st, 3), *_fields(D, D_st, 2), *_fields(z, z_st, 3),
        *_fields(dt_bias, dtb_st, 2), *_fields(deltaA, dA_st, 3),
        sbi.data_ptr() if sbi is not None else None,
        *_fields(out, out.stride(), 3))
    with _lib.on_device(x):
        _lib.check(_lib.lib().lrnnx_selective_state_update(a, _lib.stream_of(x)), "selective_state_update")
    return out if has_heads else out.squeeze(1)
