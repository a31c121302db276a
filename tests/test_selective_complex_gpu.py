"""GPU parity of the complex-weight selective scan (A and constant B/C
complex64; variable B/C real (.., 2L) interleaved) against the fp64 oracle.

Reference semantics: lrnnx/ops/selective_scan.py:200-360 with complex A
(zoh / bilinear / dirac / mamba), kernels selective_scan.cuh:229-286 and
selective_scan_backward.cuh with complex weight_t.  Complex gradients follow
PyTorch's convention (the oracle's autograd).  Tolerance: fp32, rtol 1e-4,
atol 1e-5 x max|ref| (1e-4 for batch-reduced gradients)."""

import pytest
import torch

from lrnnx_amd import selective_scan_fn
from oracle import scan_ref as R
from parity import close, oracle_selective, to_dev

pytestmark = pytest.mark.gpu


def _run(dev, B, D, L, N, method="mamba", varB=True, varC=True, has_z=True, has_D=True, has_bias=True,
         softplus=True, groups=None, seed=0, with_deltaA=False):
    inp = R.make_selective_inputs(B, D, L, N, seed=seed, groups=groups, varB=varB, varC=varC, has_z=has_z,
                                  has_D=has_D, has_bias=has_bias, complex_A=True)
    if not softplus:
        inp["delta"] = inp["delta"].abs() * 0.2 + 1e-3
        if inp.get("delta_bias") is not None:
            inp["delta_bias"] = inp["delta_bias"].abs() * 0.01
    g = torch.Generator().manual_seed(seed + 100)
    dout = torch.randn(B, D, L, generator=g)
    deltaA = 0.5 * torch.rand(B, D, L, generator=g) if with_deltaA else None
    ref_out, ref_last, ref_g = oracle_selective(inp, method, softplus, deltaA, True, dout)
    d = to_dev(inp, dev)
    leaves = {k: d[k].clone().requires_grad_(True) for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
              if d.get(k) is not None}
    dA_dev = deltaA.to(dev).requires_grad_(True) if deltaA is not None else None
    out, last = selective_scan_fn(leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"],
                                  leaves.get("D"), leaves.get("z"), leaves.get("delta_bias"), dA_dev, softplus,
                                  True, method)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    close("out", out, ref_out, 1e-4, 1e-5)
    close("last_state", last, ref_last, 1e-4, 1e-5)
    for k, v in leaves.items():
        red = k in ("A", "D", "delta_bias") or (k == "B" and not varB) or (k == "C" and not varC)
        close(f"d{k}", v.grad, ref_g[k], 1e-4, 1e-4 if red else 1e-5)
    if dA_dev is not None:
        close("ddeltaA", dA_dev.grad, ref_g["deltaA"], 1e-4, 1e-5)


@pytest.mark.parametrize("method", ["mamba", "zoh", "bilinear", "dirac"])
@pytest.mark.parametrize("varB,varC", [(True, True), (False, False), (True, False), (False, True)])
def test_complex_methods(dev, method, varB, varC):
    _run(dev, 2, 64, 40, 4, method=method, varB=varB, varC=varC)


@pytest.mark.parametrize("method", ["mamba", "zoh", "bilinear", "dirac"])
def test_complex_methods_two_states_per_wave(dev, method):
    # 9 <= N <= 16 runs two states per wave (here 6 waves, the last one full)
    _run(dev, 2, 64, 40, 12, method=method)


@pytest.mark.parametrize("N", [1, 3, 8, 16, 30, 40, 100])
def test_complex_dstate(dev, N):
    _run(dev, 1, 70, 33, N)


@pytest.mark.parametrize("L", [1, 17, 100, 2100])
def test_complex_lengths(dev, L):
    _run(dev, 1, 64, L, 4)


def test_complex_groups_deltaA_options(dev):
    _run(dev, 2, 128, 48, 4, groups=2)
    _run(dev, 2, 64, 48, 4, with_deltaA=True)
    _run(dev, 1, 64, 48, 4, has_z=False, has_D=False, has_bias=False, softplus=False)


@pytest.mark.parametrize("method", ["mamba", "zoh", "bilinear"])
def test_complex_x_carries_vs_oracle(dev, method):
    """Both halves of the complex chunk carries of ``selective_scan_cuda.fwd``
    over three 2048-step chunks: the product of A_bar since the sequence start
    (the reference's running prefix, selective_scan.cuh:316-333) and the
    state, against oracle.selective_scan_fwd_ref."""
    from lrnnx_amd import selective_scan_cuda as ssc

    inp = R.make_selective_inputs(1, 64, 4200, 4, seed=81, complex_A=True)
    inp["delta"] = inp["delta"] * 0.1   # keep the products above underflow for a while
    ro, rx, roz = R.selective_scan_fwd_ref(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"],
                                           inp["delta_bias"], None, True, method, compute_dtype=torch.float64)
    d = to_dev(inp, dev)
    B, C = d["B"].unsqueeze(1).contiguous(), d["C"].unsqueeze(1).contiguous()
    out, x = ssc.fwd(d["u"], d["delta"], d["A"], B, C, d["D"], d["z"], d["delta_bias"], None, True, method)[:2]
    torch.cuda.synchronize()
    assert x.shape == rx.shape and x.is_complex()
    # products over up to 4200 steps carry up to ~4200 * 2^-24 relative rounding (see the real-weight test)
    close(f"x products ({method})", x[..., 0::2], rx[..., 0::2], 2e-3, 1e-6)
    close(f"x states ({method})", x[..., 1::2], rx[..., 1::2], 1e-4, 1e-5)
