"""GPU parity of the depthwise causal conv1d (HIP kernels through the C ABI)
against the float64 oracle (restatement of the Mamba layer's fallbacks,
lrnnx/models/ltv/mamba.py:271, :398-410).

Tolerances: fp32 rtol 1e-4, atol 1e-5 * max|ref| (dweight / dbias, which sum
over batch x length: atol 1e-4 * max|ref|); bf16 / fp16 I/O rtol 2e-2,
atol 1e-2 * max|ref| (the inputs are the rounded values on both sides).
"""

import pytest
import torch

from lrnnx_amd import causal_conv1d_fn, causal_conv1d_update
from oracle import scan_ref as R
from tests.parity import close

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-4, 1e-5, 1e-4), torch.bfloat16: (2e-2, 1e-2, 1e-2), torch.float16: (1e-2, 5e-3, 5e-3)}


def _inputs(b, d, L, w, dtype, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(b, d, L, generator=g).to(dtype)
    wt = (torch.randn(d, w, generator=g) * 0.5).to(dtype)
    bs = (torch.randn(d, generator=g) * 0.1).to(dtype) if bias else None
    dout = torch.randn(b, d, L, generator=g).to(dtype)
    return x, wt, bs, dout


def _check(dev, b, d, L, w, dtype=torch.float32, act="silu", bias=True, seed=0, strided=False):
    x, wt, bs, dout = _inputs(b, d, L, w, dtype, seed, bias)
    leaves = [x.double().requires_grad_(True), wt.double().requires_grad_(True)]
    if bias:
        leaves.append(bs.double().requires_grad_(True))
    ref = R.causal_conv1d_ref(leaves[0], leaves[1], leaves[2] if bias else None, act, compute_dtype=torch.float64)
    ref.backward(dout.double())
    if strided:   # x as the first half of an (b, 2d, L) tensor, as Mamba's xz.chunk gives it
        big = torch.zeros(b, 2 * d, L, dtype=dtype, device=dev)
        big[:, :d] = x.to(dev)
        xd = big[:, :d].detach().requires_grad_(True)
    else:
        xd = x.to(dev).requires_grad_(True)
    wd = wt.to(dev).requires_grad_(True)
    bd = bs.to(dev).requires_grad_(True) if bias else None
    out = causal_conv1d_fn(xd, wd, bd, activation=act)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    rt, at, atr = TOL[dtype]
    close("out", out, ref.detach(), rt, at)
    close("dx", xd.grad, leaves[0].grad, rt, at)
    close("dweight", wd.grad, leaves[1].grad, rt, atr)
    if bias:
        close("dbias", bd.grad, leaves[2].grad, rt, atr)


@pytest.mark.parametrize("w", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("act", [None, "silu"])
def test_causal_conv1d_widths(dev, w, act):
    _check(dev, 2, 64, 600, w, act=act, seed=w)


@pytest.mark.parametrize("L", [1, 3, 8, 100, 512, 513, 1000, 4100])
def test_causal_conv1d_lengths(dev, L):
    _check(dev, 2, 16, L, 4, seed=L)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_causal_conv1d_low_precision(dev, dtype):
    _check(dev, 2, 32, 2048, 4, dtype=dtype, seed=5)


def test_causal_conv1d_no_bias_strided(dev):
    _check(dev, 3, 24, 777, 4, bias=False, seed=6, strided=True)


@pytest.mark.parametrize("state_len", [4, 7])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_causal_conv1d_update_steps(dev, state_len, dtype):
    # decode steps from a zero state continue the full convolution
    x, wt, bs, _ = _inputs(3, 40, 20, 4, dtype, seed=9)
    full = R.causal_conv1d_ref(x.double(), wt.double(), bs.double(), "silu", compute_dtype=torch.float64)
    st = torch.zeros(3, 40, state_len, dtype=dtype, device=dev)
    outs = [causal_conv1d_update(x[..., t].to(dev), st, wt.to(dev), bs.to(dev), "silu") for t in range(12)]
    more = causal_conv1d_update(x[..., 12:].to(dev), st, wt.to(dev), bs.to(dev), "silu")   # 8 steps in one call
    torch.cuda.synchronize()
    rt, at, _ = TOL[dtype]
    close("update", torch.cat([torch.stack(outs, -1), more], -1), full, rt, at)
    st_ref = torch.zeros(3, 40, state_len, dtype=torch.float64)
    st_ref[..., -min(state_len, 20):] = x[..., 20 - min(state_len, 20):].double()
    close("conv_state", st, st_ref, 0.0, 1e-7)
