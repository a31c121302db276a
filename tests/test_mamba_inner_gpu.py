"""GPU parity of the fused Mamba inner block (mamba_inner_fn: causal conv +
projections + selective scan, this package's HIP kernels and torch GEMMs)
against the float64 oracle restatement of mamba_inner_ref
(lrnnx/ops/selective_scan.py:789-846), output and every gradient.

The B / C / dt RMSNorm options are checked too, gradients of the norm
weights included (the oracle applies them where MambaInnerFn's forward does,
selective_scan.py:501-518).

Tolerance: fp32 rtol 1e-3, atol 1e-4 * max|ref| (a chain of four GEMMs, a
conv and a scan in fp32); bf16 rtol 5e-2, atol 3e-2 * max|ref|.
"""

import pytest
import torch

from lrnnx_amd import mamba_inner_fn
from oracle import scan_ref as R
from tests.parity import close

pytestmark = pytest.mark.gpu

NAMES = ("xz", "conv1d_weight", "conv1d_bias", "x_proj_weight", "delta_proj_weight", "out_proj_weight",
         "out_proj_bias", "A", "D", "delta_bias", "b_rms_weight", "c_rms_weight", "dt_rms_weight")


def _params(b, dm, d, n, r, L, w, seed, out_bias, rms=False):
    g = torch.Generator().manual_seed(seed)
    p = dict(
        xz=torch.randn(b, 2 * d, L, generator=g),
        conv1d_weight=torch.randn(d, 1, w, generator=g) * 0.4,
        conv1d_bias=torch.randn(d, generator=g) * 0.1,
        x_proj_weight=torch.randn(r + 2 * n, d, generator=g) / d ** 0.5,
        delta_proj_weight=torch.randn(d, r, generator=g) / r ** 0.5,
        out_proj_weight=torch.randn(dm, d, generator=g) / d ** 0.5,
        out_proj_bias=torch.randn(dm, generator=g) if out_bias else None,
        A=-torch.exp(torch.rand(d, n, generator=g) * 2.0),
        D=torch.randn(d, generator=g),
        delta_bias=torch.log(torch.expm1(0.001 + 0.1 * torch.rand(d, generator=g))),
        b_rms_weight=(torch.rand(n, generator=g) + 0.5) if rms else None,
        c_rms_weight=(torch.rand(n, generator=g) + 0.5) if rms else None,
        dt_rms_weight=(0.05 * torch.rand(d, generator=g) + 0.02) if rms else None,
    )
    dout = torch.randn(b, L, dm, generator=g)
    return p, dout


def _run(dev, dtype, out_bias, L=128, seed=0, rms=False, checkpoint_lvl=1):
    p, dout = _params(2, 32, 64, 16, 4, L, 4, seed, out_bias, rms)
    ref_leaves = {k: (v.double().requires_grad_(True) if v is not None else None) for k, v in p.items()}
    a = ref_leaves
    ref = R.mamba_inner_ref(a["xz"], a["conv1d_weight"], a["conv1d_bias"], a["x_proj_weight"],
                            a["delta_proj_weight"], a["out_proj_weight"], a["out_proj_bias"], a["A"], None, None,
                            a["D"], a["delta_bias"], b_rms_weight=a["b_rms_weight"],
                            c_rms_weight=a["c_rms_weight"], dt_rms_weight=a["dt_rms_weight"], b_c_dt_rms_eps=1e-5,
                            compute_dtype=torch.float64)
    ref.backward(dout.double())
    big = dict(xz=dtype, conv1d_weight=dtype, conv1d_bias=dtype, x_proj_weight=dtype, delta_proj_weight=dtype,
               out_proj_weight=dtype, out_proj_bias=dtype, A=torch.float32, D=torch.float32,
               delta_bias=torch.float32, b_rms_weight=torch.float32, c_rms_weight=torch.float32,
               dt_rms_weight=torch.float32)
    leaves = {k: (v.to(big[k]).to(dev).requires_grad_(True) if v is not None else None) for k, v in p.items()}
    t = leaves
    out = mamba_inner_fn(t["xz"], t["conv1d_weight"], t["conv1d_bias"], t["x_proj_weight"], t["delta_proj_weight"],
                         t["out_proj_weight"], t["out_proj_bias"], t["A"], None, None, t["D"], t["delta_bias"],
                         delta_softplus=True, checkpoint_lvl=checkpoint_lvl, b_rms_weight=t["b_rms_weight"],
                         c_rms_weight=t["c_rms_weight"], dt_rms_weight=t["dt_rms_weight"], b_c_dt_rms_eps=1e-5)
    out.backward(dout.to(dtype).to(dev))
    torch.cuda.synchronize()
    rt, at = (1e-3, 1e-4) if dtype == torch.float32 else (5e-2, 3e-2)
    close("out", out, ref.detach(), rt, at)
    for k in NAMES:
        if ref_leaves[k] is None:
            continue
        close(f"d{k}", leaves[k].grad, ref_leaves[k].grad, rt, at)


@pytest.mark.parametrize("out_bias", [False, True])
def test_mamba_inner_fp32(dev, out_bias):
    _run(dev, torch.float32, out_bias)


def test_mamba_inner_fp32_long(dev):
    # crosses the fast path's 2048-step chunk carries and the conv's 512-step chunks
    _run(dev, torch.float32, False, L=2080, seed=1)


def test_mamba_inner_bf16(dev):
    _run(dev, torch.bfloat16, False, L=256, seed=2)


@pytest.mark.parametrize("checkpoint_lvl", [0, 1])
def test_mamba_inner_rms_norms(dev, checkpoint_lvl):
    # B / C / dt RMSNorms with their full backward (norm weights included)
    _run(dev, torch.float32, True, L=160, seed=3, rms=True, checkpoint_lvl=checkpoint_lvl)


def test_mamba_inner_rms_norms_bf16(dev):
    _run(dev, torch.bfloat16, False, L=256, seed=4, rms=True)
