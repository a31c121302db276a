"""One-token S5 decode update with the reference's API.

Mirrors ``simplified_state_update`` (reference
lrnnx/ops/triton/simplified_state_update.py:254-401): same arguments, the same
shape checks (AssertionError), ``dt`` / ``deltaA`` given per (batch, P) or per
state (P,), in-place update of the complex ``state``.  The Triton kernel is
replaced by a gfx950 HIP kernel reached through the C ABI
(``lrnnx_simplified_state_update``); besides ``out`` nothing is allocated and
nothing synchronises with the host, so the call can be captured in a HIP graph
(the reference instead copies the state's real and imaginary parts to
temporaries and back).
"""

from __future__ import annotations

import torch

from . import _lib

_DISC = {"zoh": 0, "bilinear": 1, "dirac": 2}


def simplified_state_update(state, x, dt, A, B, C, D=None, deltaA=None, discretization="bilinear",
                            conj_sym=True):
    """state (batch, P) complex64, updated in place; x (batch, H) float32;
    dt, deltaA (batch, P) or (P,) float32; A (P,), B (P, H), C (H, P) complex64;
    D (H, H) float32 or None.  Returns out (batch, H) float32."""
    assert state.is_complex(), "state must be complex64"
    assert A.is_complex(), "A must be complex64"
    assert B.is_complex(), "B must be complex64"
    assert C.is_complex(), "C must be complex64"
    assert not x.is_complex(), "x must be real (float32)"
    batch, P = state.shape
    H = x.shape[1]
    assert x.shape == (batch, H)
    assert A.shape == (P,)
    assert B.shape == (P, H)
    assert C.shape == (H, P)
    if D is not None:
        assert D.shape == (H, H)
    if dt.dim() == 1:
        assert dt.shape == (P,)
    else:
        assert dt.shape == (batch, P)
    if deltaA is not None:
        if deltaA.dim() == 1:
            assert deltaA.shape == (P,)
        else:
            assert deltaA.shape == (batch, P)
    method = _DISC.get(discretization.lower())
    if method is None:
        raise ValueError(f"discretization must be one of {list(_DISC)}, got '{discretization}'")
    _lib.require_gpu(state, x, dt, A, B, C, D, deltaA)
    if state.dtype != torch.complex64 or A.dtype != torch.complex64 or B.dtype != torch.complex64 \
            or C.dtype != torch.complex64:
        raise RuntimeError("state, A, B, C must be complex64")
    x = x.float()
    dt = dt.float()
    D = D.float() if D is not None else None
    deltaA = deltaA.float() if deltaA is not None else None
    out = torch.empty(batch, H, device=x.device, dtype=torch.float32)
    a = _lib.SimplifiedStateUpdateArgs()
    a.batch, a.H, a.P = batch, H, P
    a.method, a.conj_sym = method, int(bool(conj_sym))

    def put(name, t, prefix=None):
        prefix = prefix or name
        if t is None:
            return
        setattr(a, name, t.data_ptr())
        if t.dim() == 1:   # (P,) vectors shared by the batch; A
            if name == "A":
                a.A_s0 = t.stride(0)
            else:
                setattr(a, f"{prefix}_s0", 0)
                setattr(a, f"{prefix}_s1", t.stride(0))
        else:
            setattr(a, f"{prefix}_s0", t.stride(0))
            setattr(a, f"{prefix}_s1", t.stride(1))

    put("state", state)
    put("x", x)
    put("dt", dt)
    put("A", A)
    put("B", B)
    put("C", C)
    put("D", D)
    put("deltaA", deltaA, "dA")
    put("out", out)
    with _lib.on_device(x):
        _lib.check(_lib.lib().lrnnx_simplified_state_update(a, _lib.stream_of(x)), "simplified_state_update")
    return out
