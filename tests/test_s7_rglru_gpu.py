"""GPU parity of the S7 and RG-LRU wrappers (the scan through the C ABI with the
"s7" / "rglru" discretisations) and of their fused blocks, against fp64
autograd of the oracle's restatements (s7_scan_ref, rglru_scan_ref,
s7_inner_ref, rglru_inner_ref).

Tolerances (fp32): rtol 1e-4, atol 1e-5 x max|ref| for outputs; gradients that
sum over batch and length (dA of the RG-LRU, base_params, the projection
weights) atol 1e-4 x max|ref|.
"""

import pytest
import torch

from lrnnx_amd import rglru_inner_fn, rglru_scan_fn, s7_inner_fn, s7_scan_fn
from oracle import scan_ref as R
from tests.parity import close

pytestmark = pytest.mark.gpu
D64 = torch.float64


def _leaves(ts):
    return [t.double().requires_grad_(True) if t is not None else None for t in ts]


def _dev(ts, dev):
    return [t.to(dev).requires_grad_(True) if t is not None else None for t in ts]


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("L", [7, 300])
def test_s7_scan_fn(dev, bias, L):
    g = torch.Generator().manual_seed(51 + L)
    b, dim, n = 2, 6, 8
    u = torch.randn(b, dim, L, generator=g)
    A = torch.randn(b, n, L, generator=g)
    B = torch.randn(b, n, dim, L, generator=g) * 0.4
    C = torch.randn(b, dim, n, L, generator=g) * 0.4
    bs = torch.randn(b, n, L, generator=g) * 0.1 if bias else None
    dout = torch.randn(b, dim, L, generator=g)
    ref_l = _leaves([u, A, B, C, bs])
    y_r, last_r = R.s7_scan_ref(*ref_l, return_last_state=True, compute_dtype=D64)
    y_r.backward(dout.double())
    dv = _dev([u, A, B, C, bs], dev)
    y, last = s7_scan_fn(*dv, return_last_state=True)
    y.backward(dout.to(dev))
    torch.cuda.synchronize()
    close("out", y, y_r.detach(), 1e-4, 1e-5)
    close("last_state", last, last_r.detach(), 1e-4, 1e-5)
    for name, got, ref in zip(("du", "dA", "dB", "dC", "dbias"), dv, ref_l):
        if got is None:
            continue
        close(name, got.grad, ref.grad, 1e-4, 1e-5)


@pytest.mark.parametrize("L", [5, 2100])
def test_rglru_scan_fn(dev, L):
    g = torch.Generator().manual_seed(61 + L)
    b, dim, n = 2, 8, 2
    u = torch.randn(b, dim, L, generator=g)
    delta = 8.0 * torch.sigmoid(torch.randn(b, dim, L, generator=g))
    A = torch.rand(dim, n, generator=g) * 0.5 + 0.45
    dout = torch.randn(b, dim, L, generator=g)
    ref_l = _leaves([u, delta, A])
    y_r, last_r = R.rglru_scan_ref(*ref_l, return_last_state=True, compute_dtype=D64)
    y_r.backward(dout.double())
    dv = _dev([u, delta, A], dev)
    y, last = rglru_scan_fn(*dv, return_last_state=True)
    y.backward(dout.to(dev))
    torch.cuda.synchronize()
    close("out", y, y_r.detach(), 1e-4, 1e-5)
    close("last_state", last, last_r.detach(), 1e-4, 1e-5)
    close("du", dv[0].grad, ref_l[0].grad, 1e-4, 1e-5)
    close("ddelta", dv[1].grad, ref_l[1].grad, 1e-4, 1e-5)
    close("dA", dv[2].grad, ref_l[2].grad, 1e-4, 1e-4)


def test_s7_inner_fn(dev):
    g = torch.Generator().manual_seed(71)
    b, L, dm, n = 2, 50, 8, 4
    hs = torch.randn(b, L, dm, generator=g)
    Wi = torch.randn(dm, dm, generator=g) * 0.3
    Wx = torch.randn(n + 2 * dm * n + dm + n, dm, generator=g) * 0.2
    Wg = torch.randn(dm, dm, generator=g) * 0.3
    base = torch.randn(n, generator=g)
    dout = torch.randn(b, L, dm, generator=g)
    ref_l = _leaves([hs, Wi, Wx, Wg, base])
    out_r = R.s7_inner_ref(ref_l[0], ref_l[1], ref_l[2], ref_l[3], n, ref_l[4], compute_dtype=D64)
    out_r.backward(dout.double())
    dv = _dev([hs, Wi, Wx, Wg, base], dev)
    out = s7_inner_fn(dv[0], dv[1], dv[2], dv[3], n, dv[4])
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    close("out", out, out_r.detach(), 1e-4, 1e-5)
    for name, got, ref in zip(("dhidden", "din_proj", "dx_proj", "dgate_proj", "dbase"), dv, ref_l):
        close(name, got.grad, ref.grad, 1e-4, 1e-4)


@pytest.mark.parametrize("a_1d", [False, True])
def test_rglru_inner_fn(dev, a_1d):
    g = torch.Generator().manual_seed(81)
    b, d, L, w, n, dm = 2, 16, 70, 4, (1 if a_1d else 2), 12
    x = torch.randn(b, d, L, generator=g)
    cw = torch.randn(d, 1, w, generator=g) * 0.5
    cb = torch.randn(d, generator=g) * 0.1
    a = torch.rand(d, generator=g) * 0.5 + 0.45 if a_1d else torch.rand(d, n, generator=g) * 0.5 + 0.45
    Wr, Wi = torch.randn(d, d, generator=g) * 0.3, torch.randn(d, d, generator=g) * 0.3
    br, bi = torch.randn(d, generator=g) * 0.1, torch.randn(d, generator=g) * 0.1
    Wo, bo = torch.randn(dm, d, generator=g) * 0.3, torch.randn(dm, generator=g) * 0.1
    gate = torch.randn(b, L, d, generator=g)
    dout = torch.randn(b, L, dm, generator=g)
    ts = [x, cw, cb, a, Wr, br, Wi, bi, Wo, bo, gate]
    ref_l = _leaves(ts)
    out_r = R.rglru_inner_ref(*ref_l, 8.0, compute_dtype=D64)
    out_r.backward(dout.double())
    dv = _dev(ts, dev)
    out = rglru_inner_fn(*dv, 8.0)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    close("out", out, out_r.detach(), 1e-4, 1e-5)
    names = ("dx", "dconv_w", "dconv_b", "da", "dWr", "dbr", "dWi", "dbi", "dWo", "dbo", "dgate")
    for name, got, ref in zip(names, dv, ref_l):
        close(name, got.grad, ref.grad, 1e-4, 1e-4)
