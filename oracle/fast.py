"""ctypes wrapper of the float64 C restatement of the selective scan
(``oracle/selective_scan_ref.c``, "mamba" method, forward + backward).
TEST INFRASTRUCTURE ONLY: the GPU parity tests use it as the checker at
shapes where ``scan_ref.selective_scan_ref`` plus autograd is too slow (its
backward grows with L^2); the product never imports it.

Pinned in ``tests/test_oracle.py`` against fp64 autograd of
``scan_ref.selective_scan_ref`` (itself pinned by brute force, closed forms
and gradcheck) for every option the function takes.

Build: ``make -C oracle`` (``__graft_entry__.build()`` runs it), which writes
``oracle/liboracle_ss.so``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_ss.so")
_lib = None


def build():
    """Compile the C restatement with gcc (``make -C oracle``)."""
    r = subprocess.run(["make", "-C", _HERE, "-s"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}{r.stderr}")
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        I = ctypes.c_int
        L.lrnnx_oracle_ss_mamba.restype = I
        L.lrnnx_oracle_ss_mamba.argtypes = [I64, I64, I64, I64, I64] + [P] * 7 + [I, I, P, P, I, I] + [P] * 11
        L.lrnnx_oracle_ss_threads.restype = I
        _lib = L
    return _lib


def _f32(t):
    return None if t is None else t.detach().to("cpu", torch.float32).contiguous()


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def selective_scan_mamba(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False, dout=None,
                         threads=0, want_out_pre=False):
    """float64 forward (+ backward when ``dout`` is given) of the selective scan
    with the "mamba" discretisation, real weights, no deltaA.

    Shapes as ``selective_scan_fn``: u, delta, z, dout (b, d, l); A (d, n);
    B / C (d, n) constant or (b, n, l) / (b, g, n, l) variable; D, delta_bias
    (d,).  Inputs are taken as float32 values (bf16 / fp16 inputs convert
    exactly).  Returns a dict of float64 CPU tensors: out (z-gated when z is
    given), last_state (b, d, n) (the state h_L, B included also for a
    constant B, as the reference wrapper returns it), optionally out_pre
    (before the gate), and with ``dout`` du, ddelta, dA, dB, dC (shapes of
    B / C), dD, ddelta_bias, dz."""
    Bt, Dm, L = u.shape
    N = A.shape[1]
    varB, varC = B.dim() >= 3, C.dim() >= 3
    squeeze_B, squeeze_C = B.dim() == 3, C.dim() == 3
    Bv = B.unsqueeze(1) if squeeze_B else B
    Cv = C.unsqueeze(1) if squeeze_C else C
    G = Bv.shape[1] if varB else (Cv.shape[1] if varC else 1)
    uu, dd, zz, do = _f32(u), _f32(delta), _f32(z), _f32(dout)
    AA, BB, CC, DD, bb = _f32(A), _f32(Bv), _f32(Cv), _f32(D), _f32(delta_bias)
    f64 = dict(dtype=torch.float64)
    res = {"out": torch.empty(Bt, Dm, L, **f64), "last_state": torch.empty(Bt, Dm, N, **f64)}
    out_pre = torch.empty(Bt, Dm, L, **f64) if want_out_pre else None
    g = {}
    if dout is not None:
        g = {"du": torch.empty(Bt, Dm, L, **f64), "ddelta": torch.empty(Bt, Dm, L, **f64),
             "dA": torch.empty(Dm, N, **f64), "dB": torch.empty(BB.shape, **f64),
             "dC": torch.empty(CC.shape, **f64),
             "dD": torch.empty(Dm, **f64) if D is not None else None,
             "ddelta_bias": torch.empty(Dm, **f64) if delta_bias is not None else None,
             "dz": torch.empty(Bt, Dm, L, **f64) if z is not None else None}
    rc = lib().lrnnx_oracle_ss_mamba(
        Bt, Dm, L, N, G, _ptr(uu), _ptr(dd), _ptr(zz), _ptr(do), _ptr(AA), _ptr(BB), _ptr(CC), int(varB), int(varC),
        _ptr(DD), _ptr(bb), int(bool(delta_softplus)), int(threads), _ptr(res["out"]), _ptr(out_pre),
        _ptr(res["last_state"]), _ptr(g.get("du")), _ptr(g.get("ddelta")), _ptr(g.get("dA")), _ptr(g.get("dB")),
        _ptr(g.get("dC")), _ptr(g.get("dD")), _ptr(g.get("ddelta_bias")), _ptr(g.get("dz")))
    if rc != 0:
        raise MemoryError("oracle: allocation failed")
    if out_pre is not None:
        res["out_pre"] = out_pre
    if g:
        if squeeze_B:
            g["dB"] = g["dB"].squeeze(1)
        if squeeze_C:
            g["dC"] = g["dC"].squeeze(1)
        res.update(g)
    return res
