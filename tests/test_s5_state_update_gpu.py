"""GPU parity of the S5 decode update (simplified_state_update, HIP kernel
through the C ABI) against the float64 oracle (restatement of
simplified_state_update_ref, lrnnx/ops/triton/simplified_state_update.py:404-469).

Tolerance: rtol 1e-4, atol 1e-5 * max|ref| (complex64 state, fp32 arithmetic).
"""

import math

import pytest
import torch

from lrnnx_amd import s5_inner_fn, simplified_state_update
from oracle import scan_ref as R
from tests.parity import close

pytestmark = pytest.mark.gpu


def _case(b, H, P, seed, dt_per_state=False, deltaA=None, D=True):
    g = torch.Generator().manual_seed(seed)
    cplx = lambda *s: torch.complex(torch.randn(*s, generator=g), torch.randn(*s, generator=g))
    state = cplx(b, P)
    x = torch.randn(b, H, generator=g)
    dt = 0.05 + 0.2 * torch.rand(*((P,) if dt_per_state else (b, P)), generator=g)
    A = torch.complex(-0.2 - torch.rand(P, generator=g), torch.randn(P, generator=g))
    Bm, Cm = cplx(P, H) / math.sqrt(H), cplx(H, P) / math.sqrt(P)
    Dm = torch.randn(H, H, generator=g) / math.sqrt(H) if D else None
    dA = None
    if deltaA == "batch":
        dA = 0.05 + 0.2 * torch.rand(b, P, generator=g)
    elif deltaA == "state":
        dA = 0.05 + 0.2 * torch.rand(P, generator=g)
    return state, x, dt, A, Bm, Cm, Dm, dA


def _check(dev, case, method, conj_sym):
    state, x, dt, A, Bm, Cm, Dm, dA = case
    c128 = lambda t: None if t is None else (t.to(torch.complex128) if t.is_complex() else t.double())
    st_ref = c128(state).clone()
    out_ref = R.simplified_state_update_ref(st_ref, c128(x), c128(dt), c128(A), c128(Bm), c128(Cm), c128(Dm),
                                            c128(dA), method, conj_sym, compute_dtype=torch.float64)
    st = state.to(dev)
    out = simplified_state_update(st, x.to(dev), dt.to(dev), A.to(dev), Bm.to(dev), Cm.to(dev),
                                  None if Dm is None else Dm.to(dev), None if dA is None else dA.to(dev),
                                  method, conj_sym)
    torch.cuda.synchronize()
    close("out", out, out_ref, 1e-4, 1e-5)
    close("state", st, st_ref, 1e-4, 1e-5)


@pytest.mark.parametrize("method", ["bilinear", "zoh", "dirac"])
@pytest.mark.parametrize("conj_sym", [True, False])
@pytest.mark.parametrize("D", [True, False])
def test_s5_state_update_methods(dev, method, conj_sym, D):
    _check(dev, _case(4, 24, 16, seed=1, D=D), method, conj_sym)


@pytest.mark.parametrize("deltaA", ["batch", "state"])
@pytest.mark.parametrize("dt_per_state", [False, True])
def test_s5_state_update_dt_forms(dev, deltaA, dt_per_state):
    _check(dev, _case(3, 40, 33, seed=2, dt_per_state=dt_per_state, deltaA=deltaA), "zoh", True)


@pytest.mark.parametrize("H,P", [(300, 200), (1, 1), (129, 7), (64, 512)])
def test_s5_state_update_shapes(dev, H, P):
    # H > 128 is the case the reference's Triton launch splits into several
    # programs per batch row; every state element must be updated once
    _check(dev, _case(5, H, P, seed=H + P), "bilinear", True)


def test_s5_state_update_strided_state(dev):
    state, x, dt, A, Bm, Cm, Dm, dA = _case(4, 16, 12, seed=3)
    big = torch.zeros(4, 24, dtype=torch.complex64, device=dev)
    big[:, ::2] = state.to(dev)
    view = big[:, ::2]
    st_ref = state.to(torch.complex128).clone()
    out_ref = R.simplified_state_update_ref(st_ref, x.double(), dt.double(), A.to(torch.complex128),
                                            Bm.to(torch.complex128), Cm.to(torch.complex128), Dm.double(), None,
                                            "dirac", True, compute_dtype=torch.float64)
    out = simplified_state_update(view, x.to(dev), dt.to(dev), A.to(dev), Bm.to(dev), Cm.to(dev), Dm.to(dev), None,
                                  "dirac", True)
    torch.cuda.synchronize()
    close("out", out, out_ref, 1e-4, 1e-5)
    close("state", view, st_ref, 1e-4, 1e-5)
    assert big[:, 1::2].abs().max().item() == 0.0   # the other columns are untouched


@pytest.mark.parametrize("method", ["bilinear", "zoh"])
def test_s5_decode_loop_matches_scan(dev, method):
    # L decode steps from the zero state == s5_inner_fn over the sequence (both
    # HIP paths; the decode's dense D taken diagonal as s5_inner's D (H,))
    g = torch.Generator().manual_seed(4)
    b, H, P, L = 2, 8, 16, 40
    A = torch.complex(-0.5 - torch.rand(P, generator=g), torch.randn(P, generator=g))
    Bm = torch.complex(torch.randn(P, H, generator=g), torch.randn(P, H, generator=g)) / math.sqrt(H)
    Cm = torch.complex(torch.randn(H, P, generator=g), torch.randn(H, P, generator=g)) / math.sqrt(P)
    u = torch.randn(b, H, L, generator=g)
    delta = 0.05 + 0.2 * torch.rand(b, P, L, generator=g)
    Dv = torch.randn(H, generator=g)
    y_scan = s5_inner_fn(torch.complex(u, torch.zeros_like(u)).to(dev), delta.to(dev), A.to(dev), Bm.to(dev),
                         Cm.to(dev), Dv.to(dev), discretization=method, conj_sym=True)
    st = torch.zeros(b, P, dtype=torch.complex64, device=dev)
    Dm = torch.diag(Dv).to(dev)
    outs = [simplified_state_update(st, u[..., t].contiguous().to(dev), delta[..., t].contiguous().to(dev),
                                    A.to(dev), Bm.to(dev), Cm.to(dev), Dm, None, method, True) for t in range(L)]
    torch.cuda.synchronize()
    close("decode vs scan", torch.stack(outs, -1), y_scan.detach().cpu().double(), 1e-4, 1e-5)
