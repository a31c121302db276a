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


# stride fields of each pointer in lrnnx_state_update_args (include/lrnnx_scan.h)
_STRIDE_FIELDS = {
    "state": ("state_s0", "state_s1", "state_s2", "state_s3"),
    "x": ("x_s0", "x_s1", "x_s2"), "dt": ("dt_s0", "dt_s1", "dt_s2"), "A": ("A_s0", "A_s1", "A_s2"),
    "B": ("B_s0", "B_s1", "B_s2"), "C": ("C_s0", "C_s1", "C_s2"), "D": ("D_s0", "D_s1"),
    "z": ("z_s0", "z_s1", "z_s2"), "dt_bias": ("dtb_s0", "dtb_s1"), "deltaA": ("dA_s0", "dA_s1", "dA_s2"),
    "out": ("out_s0", "out_s1", "out_s2"),
}


def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None, dt_softplus=False, deltaA=None,
                           state_batch_indices=None, discretization="mamba"):
    """state: (batch, dim, dstate) or (batch, nheads, dim, dstate), updated in place.
    Returns out: (batch, dim) or (batch, nheads, dim)."""
    has_heads = state.dim() > 3
    if state.dim() == 3:
        state = state.unsqueeze(1)
    if x.dim() == 2:
        x = x.unsqueeze(1)
    if dt.dim() == 2:
        dt = dt.unsqueeze(1)
    if A.dim() == 2:
        A = A.unsqueeze(0)
    if B.dim() == 2:
        B = B.unsqueeze(1)
    if C.dim() == 2:
        C = C.unsqueeze(1)
    if D is not None and D.dim() == 1:
        D = D.unsqueeze(0)
    if z is not None and z.dim() == 2:
        z = z.unsqueeze(1)
    if dt_bias is not None and dt_bias.dim() == 1:
        dt_bias = dt_bias.unsqueeze(0)
    if deltaA is not None and deltaA.dim() == 2:
        deltaA = deltaA.unsqueeze(1)
    _, nheads, dim, dstate = state.shape
    batch = x.shape[0]
    assert x.shape == (batch, nheads, dim)
    assert dt.shape == x.shape
    assert A.shape == (nheads, dim, dstate)
    ngroups = B.shape[1]
    assert nheads % ngroups == 0, "nheads must be divisible by ngroups"
    assert B.shape == (batch, ngroups, dstate)
    assert C.shape == B.shape
    if D is not None:
        assert D.shape == (nheads, dim)
    if z is not None:
        assert z.shape == x.shape
    if dt_bias is not None:
        assert dt_bias.shape == (nheads, dim)
    if deltaA is not None:
        assert deltaA.shape == (batch, nheads, dim)
    if state_batch_indices is not None:
        assert state_batch_indices.shape == (batch,)
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
    sbi = None
    if state_batch_indices is not None:
        sbi = state_batch_indices.to(torch.int32)
    out = torch.empty_like(x)
    a = _lib.StateUpdateArgs()
    a.batch, a.nheads, a.dim, a.dstate, a.ngroups = batch, nheads, dim, dstate, ngroups
    a.state_type, a.x_type, a.bc_type = (_lib.dtype_code(t.dtype) for t in (state, x, B))
    a.method = _DISC.get(discretization.lower(), 3)
    a.dt_softplus = int(bool(dt_softplus))

    for name, t in (("state", state), ("x", x), ("dt", dt), ("A", A), ("B", B), ("C", C), ("D", D), ("z", z),
                    ("dt_bias", dt_bias), ("deltaA", deltaA), ("out", out)):
        if t is None:
            continue
        setattr(a, name, t.data_ptr())
        for f, st in zip(_STRIDE_FIELDS[name], t.stride()):
            setattr(a, f, st)
    if sbi is not None:
        a.state_batch_indices = sbi.data_ptr()
    with _lib.on_device(x):
        _lib.check(_lib.lib().lrnnx_selective_state_update(a, _lib.stream_of(x)), "selective_state_update")
    return out if has_heads else out.squeeze(1)
