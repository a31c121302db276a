"""Scalar float64 brute force for tiny shapes.  TEST INFRASTRUCTURE ONLY.

Deliberately a *different* algorithm from ``scan_ref``: the state is formed as
the explicit sum  h_t = sum_{s<=t} (prod_{r=s+1..t} A_bar_r) * Bbar_s u_s
(O(L^2) per channel/state) with Python ``math``/``cmath`` scalars, so an
index, sign or term error in the vectorised recurrence does not repeat here.
Discretisation formulas follow lrnnx/ops/selective_scan.py:249-323 and
csrc/selective_scan/selective_scan.cuh:287-302.
"""

from __future__ import annotations

import cmath
import math


def softplus(x):
    return x if x > 20.0 else math.log1p(math.exp(x))


def _disc(method, d, dA, a, is_c):
    """Return (A_bar, B_bar) for scalar delta d, A-timestep dA, eigenvalue a."""
    ex = cmath.exp if is_c else math.exp
    if method in ("mamba", "zoh", "dirac"):
        Ab = ex(dA * a)
        if method == "mamba":
            Bb = d
        elif method == "zoh":
            Bb = (ex(d * a) - 1.0) / a
        else:
            Bb = 1.0
    elif method == "bilinear":
        Ab = (1.0 + 0.5 * dA * a) / (1.0 - 0.5 * dA * a)
        Bb = d / (1.0 - 0.5 * d * a)
    elif method == "s7":
        Ab = 1.0 - 1.0 / (d * d + 0.5)
        Bb = 1.0
    elif method == "rglru":
        Ab = math.exp(d * math.log(a))
        Bb = math.sqrt(1.0 - Ab * Ab)
    else:
        raise ValueError(method)
    return Ab, Bb


def selective_scan(u, delta, A, B, C, D=None, z=None, delta_bias=None, deltaA=None,
                   softplus_on=False, method="mamba"):
    """Nested lists / scalars in, nested lists out.

    u, delta, z, deltaA: [b][d][l]; A: [d][n] (float or complex);
    B, C: either [d][n] (constant) or [b][g][n][l] (variable; complex values
    given directly as Python complex).  Returns out[b][d][l] (before casting)
    and last[b][d][n].
    """
    nb, nd, L = len(u), len(u[0]), len(u[0][0])
    N = len(A[0])
    is_c = isinstance(A[0][0], complex)
    varB = isinstance(B[0][0], list)
    varC = isinstance(C[0][0], list)
    out = [[[0.0] * L for _ in range(nd)] for _ in range(nb)]
    last = [[[0.0] * N for _ in range(nd)] for _ in range(nb)]
    for b in range(nb):
        for d in range(nd):
            dl = []
            for t in range(L):
                v = delta[b][d][t] + (delta_bias[d] if delta_bias is not None else 0.0)
                dl.append(softplus(v) if softplus_on else v)
            for n in range(N):
                a = A[d][n]
                Ab, term = [], []
                for t in range(L):
                    dA = deltaA[b][d][t] if deltaA is not None else dl[t]
                    ab, bb = _disc(method, dl[t], dA, a, is_c)
                    if varB:
                        g = d // (nd // len(B[b]))
                        bin_ = 1.0 if method == "rglru" else B[b][g][n][t]
                    else:
                        bin_ = 1.0 if method == "rglru" else B[d][n]
                    Ab.append(ab)
                    term.append(bb * bin_ * u[b][d][t])
                for t in range(L):
                    h = 0.0
                    for s in range(t + 1):
                        p = term[s]
                        for r in range(s + 1, t + 1):
                            p = p * Ab[r]
                        h = h + p
                    if varC:
                        g = d // (nd // len(C[b]))
                        c = C[b][g][n][t]
                    else:
                        c = C[d][n]
                    if method == "rglru" and not varB:
                        c = c * B[d][n]
                    contrib = c * h
                    out[b][d][t] += 2.0 * contrib.real if is_c else contrib
                    if t == L - 1:
                        # returned last state = kernel state times a constant B
                        # (selective_scan.py:87-92); for rglru B is not in h
                        last[b][d][n] = h * B[d][n] if (method == "rglru" and not varB) else h
            for t in range(L):
                if D is not None:
                    out[b][d][t] += D[d] * u[b][d][t]
                if z is not None:
                    zz = z[b][d][t]
                    out[b][d][t] *= zz / (1.0 + math.exp(-zz))
    return out, last


def simplified_scan_states(u, delta, A, deltaA=None, method="bilinear"):
    """u: [b][p][l] complex, delta/deltaA: [b][p][l], A: [p] complex.
    Returns states h[b][p][l] (identity B/C)."""
    nb, npp, L = len(u), len(u[0]), len(u[0][0])
    out = [[[0j] * L for _ in range(npp)] for _ in range(nb)]
    for b in range(nb):
        for p in range(npp):
            Ab, term = [], []
            for t in range(L):
                d = delta[b][p][t]
                dA = deltaA[b][p][t] if deltaA is not None else d
                ab, bb = _disc(method, d, dA, A[p], True)
                Ab.append(ab)
                term.append(bb * u[b][p][t])
            for t in range(L):
                h = 0j
                for s in range(t + 1):
                    q = term[s]
                    for r in range(s + 1, t + 1):
                        q *= Ab[r]
                    h += q
                out[b][p][t] = h
    return out
