"""GPU parity of the simplified complex scan (S5 / LRU) against the float64
CPU oracle (restatements of simplified_scan_ref / s5_inner_ref,
lrnnx/ops/simplified_scan.py:233-340, :586-640).

Tolerance: rtol 1e-4, atol 1e-5 * max|ref| for outputs and du; reductions
(dA, dB, dC, dD) and ddelta rtol 1e-4, atol 1e-4 * max|ref| (complex64
state, fp32 arithmetic).
"""

import math

import pytest
import torch

from lrnnx_amd import s5_inner_fn, simplified_scan_cuda, simplified_scan_fn
from oracle import scan_ref as R
from tests.parity import close

pytestmark = pytest.mark.gpu


def _inputs(B, H, P, L, seed, dt_scale=0.1):
    g = torch.Generator().manual_seed(seed)
    A = torch.complex(-0.5 - torch.rand(P, generator=g), math.pi * torch.randn(P, generator=g))
    Bm = torch.complex(torch.randn(P, H, generator=g), torch.randn(P, H, generator=g)) / math.sqrt(2 * H)
    Cm = torch.complex(torch.randn(H, P, generator=g), torch.randn(H, P, generator=g)) / math.sqrt(2 * P)
    u = torch.complex(torch.randn(B, H, L, generator=g), torch.randn(B, H, L, generator=g))
    delta = dt_scale * (0.5 + torch.rand(B, P, L, generator=g))
    deltaA = dt_scale * (0.5 + torch.rand(B, P, L, generator=g))
    D = torch.randn(H, generator=g)
    dout = torch.complex(torch.randn(B, H, L, generator=g), torch.randn(B, H, L, generator=g))
    return A, Bm, Cm, u, delta, deltaA, D, dout


@pytest.mark.parametrize("method", ["bilinear", "zoh", "dirac"])
@pytest.mark.parametrize("L", [1, 31, 100, 2100])
@pytest.mark.parametrize("use_deltaA", [False, True])
def test_simplified_scan_fn(dev, method, L, use_deltaA):
    A, Bm, Cm, u, delta, deltaA, D, dout = _inputs(2, 8, 16, L, seed=L)
    dA_in = deltaA if use_deltaA else None
    leaves = [t.double() if not t.is_complex() else t.to(torch.complex128) for t in (u, delta, A, Bm, Cm)]
    for t in leaves:
        t.requires_grad_(True)
    dA_ref_leaf = dA_in.double().requires_grad_(True) if dA_in is not None else None
    y_ref, last_ref = R.simplified_scan_ref(*leaves, deltaA=dA_ref_leaf, return_last_state=True,
                                            discretization=method, compute_dtype=torch.float64)
    y_ref.backward(dout.to(torch.complex128))
    dl = [t.to(dev).requires_grad_(True) for t in (u, delta, A, Bm, Cm)]
    dA_dev = dA_in.to(dev).requires_grad_(True) if dA_in is not None else None
    y, last = simplified_scan_fn(*dl, deltaA=dA_dev, return_last_state=True, discretization=method)
    y.backward(dout.to(dev))
    torch.cuda.synchronize()
    close("y", y, y_ref.detach(), 1e-4, 1e-5)
    close("last_state", last, last_ref.detach(), 1e-4, 1e-5)
    for name, got, ref in zip(("du", "ddelta", "dA", "dB", "dC"), dl, leaves):
        red = name != "du"
        close(name, got.grad, ref.grad, 1e-4, 1e-4 if red else 1e-5)
    if dA_dev is not None:
        close("ddeltaA", dA_dev.grad, dA_ref_leaf.grad, 1e-4, 1e-4)


@pytest.mark.parametrize("method", ["bilinear", "zoh", "dirac"])
@pytest.mark.parametrize("conj_sym", [True, False])
def test_s5_inner_fn(dev, method, conj_sym):
    A, Bm, Cm, u, delta, deltaA, D, dout = _inputs(2, 8, 16, 200, seed=7)
    dout = dout.real.contiguous()
    leaves = [t.double() if not t.is_complex() else t.to(torch.complex128) for t in (u, delta, A, Bm, Cm, D)]
    for t in leaves:
        t.requires_grad_(True)
    y_ref = R.s5_inner_ref(*leaves, discretization=method, conj_sym=conj_sym, compute_dtype=torch.float64)
    y_ref.backward(dout.double())
    dl = [t.to(dev).requires_grad_(True) for t in (u, delta, A, Bm, Cm, D)]
    y = s5_inner_fn(*dl, discretization=method, conj_sym=conj_sym)
    y.backward(dout.to(dev))
    torch.cuda.synchronize()
    close("y", y, y_ref.detach(), 1e-4, 1e-5)
    for name, got, ref in zip(("du", "ddelta", "dA", "dB", "dC", "dD"), dl, leaves):
        close(name, got.grad, ref.grad, 1e-4, 1e-4 if name != "du" else 1e-5)


def test_lru_config1_shape_slice(dev):
    # config 1 at the boundary: dirac, delta = 1 broadcast along L (stride 0),
    # A = log(Lambda), identity B/C; states h_t = Lambda h_{t-1} + Bu_t.
    d = R.make_lru_inputs(2, 1024, 16, seed=1)
    lam, Bu = d["Lambda"], d["Bu"]
    A = torch.log(lam).to(torch.complex64).unsqueeze(-1)
    ones = torch.ones(16, 1, dtype=torch.complex64)
    delta = torch.ones(1, 1, 1).expand(2, 16, 1024)
    out, x = simplified_scan_cuda.fwd(Bu.to(dev), delta.to(dev), A.to(dev), ones.to(dev), ones.to(dev), None, "dirac")
    h = torch.zeros(2, 16, dtype=torch.complex128)
    ref = []
    lam64 = lam.to(torch.complex128)
    for t in range(1024):
        h = lam64 * h + Bu[:, :, t].to(torch.complex128)
        ref.append(h)
    ref = torch.stack(ref, -1)
    torch.cuda.synchronize()
    close("states", out, ref, 1e-4, 1e-5)


# ---- one state per channel with delta constant along L: the fast LRU path
# (one wave per sequence, cross-lane scan) of the simplified-scan kernels

def _bcast_inputs(B, H, P, L, seed):
    A, Bm, Cm, u, _, _, D, dout = _inputs(B, H, P, L, seed)
    g = torch.Generator().manual_seed(seed + 50)
    delta = 0.1 * (0.5 + torch.rand(B, P, 1, generator=g))
    deltaA = 0.1 * (0.5 + torch.rand(B, P, 1, generator=g))
    return A, Bm, Cm, u, delta, deltaA, D, dout


@pytest.mark.parametrize("method", ["bilinear", "zoh", "dirac"])
@pytest.mark.parametrize("L", [1, 37, 512, 1000, 4113])
@pytest.mark.parametrize("use_deltaA", [False, True])
def test_simplified_scan_fn_broadcast_delta(dev, method, L, use_deltaA):
    A, Bm, Cm, u, delta, deltaA, D, dout = _bcast_inputs(2, 8, 16, L, seed=L + 3)
    dA_in = deltaA if use_deltaA else None
    leaves = [t.double() if not t.is_complex() else t.to(torch.complex128) for t in (u, delta, A, Bm, Cm)]
    for t in leaves:
        t.requires_grad_(True)
    dA_ref_leaf = dA_in.double().requires_grad_(True) if dA_in is not None else None
    y_ref, last_ref = R.simplified_scan_ref(leaves[0], leaves[1].expand(-1, -1, L), *leaves[2:],
                                            deltaA=dA_ref_leaf.expand(-1, -1, L) if dA_ref_leaf is not None else None,
                                            return_last_state=True, discretization=method,
                                            compute_dtype=torch.float64)
    y_ref.backward(dout.to(torch.complex128))
    dl = [t.to(dev).requires_grad_(True) for t in (u, delta, A, Bm, Cm)]
    dA_dev = dA_in.to(dev).requires_grad_(True) if dA_in is not None else None
    y, last = simplified_scan_fn(dl[0], dl[1].expand(-1, -1, L), *dl[2:],
                                 deltaA=dA_dev.expand(-1, -1, L) if dA_dev is not None else None,
                                 return_last_state=True, discretization=method)
    y.backward(dout.to(dev))
    torch.cuda.synchronize()
    close("y", y, y_ref.detach(), 1e-4, 1e-5)
    close("last_state", last, last_ref.detach(), 1e-4, 1e-5)
    for name, got, ref in zip(("du", "ddelta", "dA", "dB", "dC"), dl, leaves):
        close(name, got.grad, ref.grad, 1e-4, 1e-4 if name != "du" else 1e-5)
    if dA_dev is not None:
        close("ddeltaA", dA_dev.grad, dA_ref_leaf.grad, 1e-4, 1e-4)


@pytest.mark.parametrize("method", ["bilinear", "dirac"])
def test_s5_inner_fn_broadcast_delta(dev, method):
    A, Bm, Cm, u, delta, deltaA, D, dout = _bcast_inputs(2, 8, 16, 700, seed=11)
    dout = dout.real.contiguous()
    leaves = [t.double() if not t.is_complex() else t.to(torch.complex128) for t in (u, delta, A, Bm, Cm, D)]
    for t in leaves:
        t.requires_grad_(True)
    y_ref = R.s5_inner_ref(leaves[0], leaves[1].expand(-1, -1, 700), *leaves[2:], discretization=method,
                           conj_sym=True, compute_dtype=torch.float64)
    y_ref.backward(dout.double())
    dl = [t.to(dev).requires_grad_(True) for t in (u, delta, A, Bm, Cm, D)]
    y = s5_inner_fn(dl[0], dl[1].expand(-1, -1, 700), *dl[2:], discretization=method, conj_sym=True)
    y.backward(dout.to(dev))
    torch.cuda.synchronize()
    close("y", y, y_ref.detach(), 1e-4, 1e-5)
    for name, got, ref in zip(("du", "ddelta", "dA", "dB", "dC", "dD"), dl, leaves):
        close(name, got.grad, ref.grad, 1e-4, 1e-4 if name != "du" else 1e-5)


@pytest.mark.parametrize("method", ["zoh", "dirac"])
def test_simplified_kernel_x_carries_broadcast(dev, method):
    # the reference boundary's outputs, incl. the chunk carries x = (prod A_bar, h)
    # at every 2048-step chunk end and at L - 1
    d = R.make_lru_inputs(2, 4500, 8, seed=2)
    A = torch.log(d["Lambda"]).to(torch.complex64).unsqueeze(-1)
    g = torch.Generator().manual_seed(3)
    Bw = torch.complex(torch.randn(8, 1, generator=g), torch.randn(8, 1, generator=g))
    Cw = torch.complex(torch.randn(8, 1, generator=g), torch.randn(8, 1, generator=g))
    delta = (0.5 + torch.rand(2, 8, 1, generator=g)).expand(2, 8, 4500)
    out, x = simplified_scan_cuda.fwd(d["Bu"].to(dev), delta.to(dev), A.to(dev), Bw.to(dev), Cw.to(dev), None, method)
    ref_out, ref_x = R.simplified_scan_kernel_ref(d["Bu"], delta, A, Bw, Cw, None, method,
                                                  compute_dtype=torch.float64)
    torch.cuda.synchronize()
    close("out", out, ref_out, 1e-4, 1e-5)
    close("x", x, ref_x, 1e-4, 1e-5)


@pytest.mark.parametrize("method", ["bilinear", "zoh"])
def test_simplified_fast_matches_generic(dev, method, monkeypatch):
    A, Bm, Cm, u, delta, deltaA, D, dout = _bcast_inputs(2, 8, 16, 1500, seed=21)
    res = []
    for generic in ("0", "1"):
        monkeypatch.setenv("LRNNX_SCAN_GENERIC", generic)
        dl = [t.to(dev).requires_grad_(True) for t in (u, delta, A, Bm, Cm)]
        y, last = simplified_scan_fn(dl[0], dl[1].expand(-1, -1, 1500), *dl[2:], return_last_state=True,
                                     discretization=method)
        y.backward(dout.to(dev))
        torch.cuda.synchronize()
        res.append([y.detach(), last.detach()] + [t.grad for t in dl])
    for n, a, b in zip(("y", "last", "du", "ddelta", "dA", "dB", "dC"), res[0], res[1]):
        close(n, a, b.cpu().to(torch.complex128 if b.is_complex() else torch.float64), 1e-5, 1e-5)


@pytest.mark.parametrize("method", ["bilinear", "zoh", "dirac"])
@pytest.mark.parametrize("use_deltaA", [False, True])
def test_simplified_kernel_time_varying_delta(dev, method, use_deltaA):
    """The binding's fwd / bwd (reference boundary, chunk carries x, no
    checkpoints handed to the backward) with delta varying along L."""
    d = R.make_lru_inputs(2, 4500, 8, seed=4)
    A = torch.log(d["Lambda"]).to(torch.complex64).unsqueeze(-1)
    g = torch.Generator().manual_seed(5)
    Bw = torch.complex(torch.randn(8, 1, generator=g), torch.randn(8, 1, generator=g))
    Cw = torch.complex(torch.randn(8, 1, generator=g), torch.randn(8, 1, generator=g))
    delta = 0.2 + torch.rand(2, 8, 4500, generator=g)
    deltaA = (0.2 + torch.rand(2, 8, 4500, generator=g)) if use_deltaA else None
    dout = torch.complex(torch.randn(2, 8, 4500, generator=g), torch.randn(2, 8, 4500, generator=g))
    leaves = [d["Bu"].to(torch.complex128), delta.double(), A.to(torch.complex128), Bw.to(torch.complex128),
              Cw.to(torch.complex128)]
    for t in leaves:
        t.requires_grad_(True)
    dA_leaf = deltaA.double().requires_grad_(True) if use_deltaA else None
    ref_out, ref_x = R.simplified_scan_kernel_ref(*leaves, dA_leaf, method, compute_dtype=torch.float64)
    ref_out.backward(dout.to(torch.complex128))
    dv = lambda t: t.to(dev) if t is not None else None
    out, x = simplified_scan_cuda.fwd(dv(d["Bu"]), dv(delta), dv(A), dv(Bw), dv(Cw), dv(deltaA), method)
    grads = simplified_scan_cuda.bwd(dv(d["Bu"]), dv(delta), dv(A), dv(Bw), dv(Cw), dv(deltaA), dv(dout), x, method)
    torch.cuda.synchronize()
    close("out", out, ref_out.detach(), 1e-4, 1e-5)
    close("x", x, ref_x.detach(), 1e-4, 1e-5)
    for name, got, ref in zip(("du", "ddelta", "dA", "dB", "dC"), grads, leaves):
        close(name, got, ref.grad, 1e-4, 1e-5 if name == "du" else 1e-4)
    if use_deltaA:
        close("ddeltaA", grads[5], dA_leaf.grad, 1e-4, 1e-4)


@pytest.mark.parametrize("method", ["bilinear", "zoh", "dirac"])
@pytest.mark.parametrize("use_deltaA", [False, True])
def test_simplified_fast_matches_generic_time_varying(dev, method, use_deltaA, monkeypatch):
    A, Bm, Cm, u, delta, deltaA, D, dout = _inputs(2, 8, 16, 1300, seed=22)
    res = []
    for generic in ("0", "1"):
        monkeypatch.setenv("LRNNX_SCAN_GENERIC", generic)
        dl = [t.to(dev).requires_grad_(True) for t in (u, delta, A, Bm, Cm)]
        dA_dev = deltaA.to(dev).requires_grad_(True) if use_deltaA else None
        y, last = simplified_scan_fn(*dl, deltaA=dA_dev, return_last_state=True, discretization=method)
        y.backward(dout.to(dev))
        torch.cuda.synchronize()
        res.append([y.detach(), last.detach()] + [t.grad for t in dl] + ([dA_dev.grad] if use_deltaA else []))
    names = ("y", "last", "du", "ddelta", "dA", "dB", "dC", "ddeltaA")
    for n, a, b in zip(names, res[0], res[1]):
        close(n, a, b.cpu().to(torch.complex128 if b.is_complex() else torch.float64), 1e-4, 1e-5)
