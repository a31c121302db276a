"""GPU parity of the fused residual-add LayerNorm / RMSNorm (HIP kernels through
the C ABI) against the oracle's restatement of the reference's Triton kernels
(lrnnx/ops/triton/layer_norm.py:202-322, :490-649), run on the CPU in the same
fp32 arithmetic on the same rounded inputs.

Tolerances: y / dx in fp32 rtol 1e-4, atol 1e-5 * max|ref|; in bf16 rtol 2e-2,
fp16 rtol 1e-2 (one rounding of the output on each side), atol 1e-2 * max|ref|;
mean / rstd rtol 1e-5; dweight / dbias (sums over rows) rtol 1e-4, atol
1e-4 * max|ref|; residual_out bit-exact (one fp32 add, one rounding).

Shapes cover both kernel families (fast: cols % 4 == 0 and <= 4096 with 1, 2 or
4 waves per row; generic: other widths, misaligned rows), rows beyond one pass
of the grid (10000 x 256 forward, 1501 x 2048 and 2100 x 4096 backward, so
that a workgroup's row groups end on different iterations), 1-row inputs and
an empty input.
"""

import pytest
import torch
import torch.nn.functional as F

from lrnnx_amd import RMSNorm, layer_norm_fn, rms_norm_fn
from lrnnx_amd.layer_norm import _layer_norm_bwd, _layer_norm_fwd
from oracle import scan_ref as R
from tests.parity import close

pytestmark = pytest.mark.gpu

YTOL = {torch.float32: (1e-4, 1e-5), torch.bfloat16: (2e-2, 1e-2), torch.float16: (1e-2, 1e-2)}
SHAPES = [(1, 64), (7, 256), (33, 1000), (300, 2048), (129, 4096), (5, 37), (40, 5000), (10000, 256),
          (1501, 2048), (2100, 4096), (3, 1002)]


def _inputs(M, N, dtype, res_mode, bias, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, N, generator=g) * 2 + 0.3).to(dtype)
    res = None
    if res_mode == "same":
        res = torch.randn(M, N, generator=g).to(dtype)
    elif res_mode == "fp32":
        res = torch.randn(M, N, generator=g)
    w = (1 + 0.5 * torch.randn(N, generator=g))
    b = 0.1 * torch.randn(N, generator=g) if bias else None
    dy = torch.randn(M, N, generator=g).to(dtype)
    dres = torch.randn(M, N, generator=g).to(res.dtype if res is not None else dtype)
    return x, res, w, b, dy, dres


def _run(dev, M, N, dtype, res_mode, bias, rms, seed, prenorm=True, eps=1e-5, residual_in_fp32=False):
    x, res, w, b, dy, dres = _inputs(M, N, dtype, res_mode, bias, seed)
    rdt = torch.float32 if (res is None and residual_in_fp32) else None
    # oracle (CPU, fp32 arithmetic, same rounding points as the kernels)
    y_r, mean_r, rstd_r, xs_r = R.layer_norm_fwd_ref(x, w, b, res, eps=eps, residual_dtype=rdt, is_rms_norm=rms)
    has_res = res is not None
    dres_r = dres.to(xs_r.dtype) if prenorm else None
    dx_r, dw_r, db_r, dri_r = R.layer_norm_bwd_ref(dy, xs_r, w, b, mean_r, rstd_r, dresidual=dres_r,
                                                   has_residual=has_res, is_rms_norm=rms, x_dtype=dtype)
    # HIP path
    xd, wd = x.to(dev), w.to(dev)
    bd = b.to(dev) if b is not None else None
    rd = res.to(dev) if res is not None else None
    y, _, mean, rstd, xs, _, _, _ = _layer_norm_fwd(xd, wd, bd, eps, rd, residual_dtype=rdt, is_rms_norm=rms)
    dx, dw, db, dri, _, _, _ = _layer_norm_bwd(dy.to(dev), xs, wd, bd, eps, mean, rstd,
                                               dres_r.to(dev) if prenorm else None, has_residual=has_res,
                                               is_rms_norm=rms, x_dtype=dtype)
    torch.cuda.synchronize()
    rt, at = YTOL[dtype]
    tag = f"M={M} N={N} {dtype} res={res_mode} bias={bias} rms={rms}"
    assert y.dtype == dtype and dx.dtype == dtype, tag
    close(f"y {tag}", y, y_r.float(), rt, at)
    assert xs.dtype == xs_r.dtype, tag
    assert torch.equal(xs.cpu(), xs_r), f"residual_out {tag}"
    close(f"rstd {tag}", rstd, rstd_r, 1e-5, 0.0)
    if rms:
        assert mean is None
    else:
        close(f"mean {tag}", mean, mean_r, 1e-5, 1e-6)
    close(f"dx {tag}", dx, dx_r.float(), rt, at)
    close(f"dw {tag}", dw, dw_r, 1e-4, 1e-4)
    if bias:
        close(f"db {tag}", db, db_r, 1e-4, 1e-4)
    if has_res:
        assert dri.dtype == xs_r.dtype, tag
        close(f"dresidual_in {tag}", dri, dri_r.float(), rt if dri.dtype != torch.float32 else 1e-4,
              at if dri.dtype != torch.float32 else 1e-5)


@pytest.mark.parametrize("rms", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", SHAPES)
def test_layer_norm_parity(dev, shape, dtype, rms):
    i = SHAPES.index(shape)
    res_mode = ("none", "same", "fp32")[i % 3]
    if dtype == torch.float32 and res_mode == "fp32":
        res_mode = "same"
    _run(dev, *shape, dtype, res_mode, bias=(i % 2 == 0), rms=rms, seed=100 + i)


@pytest.mark.parametrize("rms", [False, True])
@pytest.mark.parametrize("res_mode", ["none", "same", "fp32"])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("prenorm", [False, True])
def test_layer_norm_options(dev, rms, res_mode, bias, prenorm):
    _run(dev, 65, 768, torch.bfloat16, res_mode, bias, rms, seed=7, prenorm=prenorm)


def test_residual_in_fp32_without_residual(dev):
    # the first block of a model: no residual yet, residual_out created in fp32 (layer_norm.py:857-861)
    _run(dev, 17, 512, torch.bfloat16, "none", True, True, seed=9, residual_in_fp32=True)


@pytest.mark.parametrize("N", [1024, 2048])
def test_strided_and_misaligned_rows(dev, N):
    """Rows with a stride > cols (aligned: fast path) and rows starting one
    element off a 4-element boundary (generic path) give the contiguous result."""
    M = 9
    x, res, w, b, dy, _ = _inputs(M, N, torch.bfloat16, "same", True, 3)
    wd, bd = w.to(dev), b.to(dev)
    y0, _, m0, r0, xs0, _, _, _ = _layer_norm_fwd(x.to(dev), wd, bd, 1e-5, res.to(dev))
    dx0, dw0, db0, _, _, _, _ = _layer_norm_bwd(dy.to(dev), xs0, wd, bd, 1e-5, m0, r0, has_residual=True)
    for off in (0, 1):
        big = torch.zeros(M, 2 * N + 8, dtype=torch.bfloat16, device=dev)
        bigr = torch.zeros_like(big)
        bigdy = torch.zeros_like(big)
        big[:, off:off + N] = x.to(dev)
        bigr[:, off:off + N] = res.to(dev)
        bigdy[:, off:off + N] = dy.to(dev)
        xv, rv, dyv = big[:, off:off + N], bigr[:, off:off + N], bigdy[:, off:off + N]
        y, _, m, r, xs, _, _, _ = _layer_norm_fwd(xv, wd, bd, 1e-5, rv)
        dx, dw, db, _, _, _, _ = _layer_norm_bwd(dyv, xs, wd, bd, 1e-5, m, r, has_residual=True)
        torch.cuda.synchronize()
        close(f"y off={off}", y, y0.float().cpu(), 2e-2, 1e-2)
        assert torch.equal(xs.cpu(), xs0.cpu())
        close(f"rstd off={off}", r, r0.cpu(), 1e-5, 0.0)
        close(f"dx off={off}", dx, dx0.float().cpu(), 2e-2, 1e-2)
        close(f"dw off={off}", dw, dw0.cpu(), 1e-4, 1e-4)
        close(f"db off={off}", db, db0.cpu(), 1e-4, 1e-4)


@pytest.mark.parametrize("rms", [False, True])
def test_layer_norm_fn_autograd_matches_oracle(dev, rms):
    """The block's call (block.py:77-87): 3-D bf16 input, fp32 residual stream,
    prenorm; gradients reach x, residual, weight and bias through LayerNormFn."""
    g = torch.Generator().manual_seed(21)
    B, L, D = 2, 33, 384
    x = torch.randn(B, L, D, generator=g).to(torch.bfloat16)
    res = torch.randn(B, L, D, generator=g)
    w = 1 + 0.2 * torch.randn(D, generator=g)
    b = 0.1 * torch.randn(D, generator=g)
    dy = torch.randn(B, L, D, generator=g).to(torch.bfloat16)
    dres = torch.randn(B, L, D, generator=g)
    xd, rd = x.to(dev).requires_grad_(), res.to(dev).requires_grad_()
    wd, bd = w.to(dev).requires_grad_(), b.to(dev).requires_grad_()
    y, ro = layer_norm_fn(xd, wd, bd, residual=rd, prenorm=True, residual_in_fp32=True, eps=1e-5, is_rms_norm=rms)
    torch.autograd.backward([y, ro], [dy.to(dev), dres.to(dev)])
    torch.cuda.synchronize()
    y_r, mean_r, rstd_r, xs_r = R.layer_norm_fwd_ref(x.reshape(-1, D), w, b, res.reshape(-1, D), eps=1e-5,
                                                     is_rms_norm=rms)
    dx_r, dw_r, db_r, dri_r = R.layer_norm_bwd_ref(dy.reshape(-1, D), xs_r, w, b, mean_r, rstd_r,
                                                   dresidual=dres.reshape(-1, D), has_residual=True,
                                                   is_rms_norm=rms, x_dtype=torch.bfloat16)
    assert y.shape == (B, L, D) and ro.shape == (B, L, D) and ro.dtype == torch.float32
    close("y", y.reshape(-1, D), y_r.float(), 2e-2, 1e-2)
    assert torch.equal(ro.detach().reshape(-1, D).cpu(), xs_r)
    close("dx", xd.grad.reshape(-1, D), dx_r.float(), 2e-2, 1e-2)
    close("dresidual", rd.grad.reshape(-1, D), dri_r, 1e-4, 1e-5)
    close("dweight", wd.grad, dw_r, 1e-4, 1e-4)
    close("dbias", bd.grad, db_r, 1e-4, 1e-4)


def test_rmsnorm_module_and_final_norm(dev):
    """RMSNorm(d) as the model's norm_f (language_model.py:440-450: no
    prenorm) equals rms_norm_fn with the module's eps and ones weight."""
    torch.manual_seed(0)
    m = RMSNorm(256).to(dev)
    x = torch.randn(4, 10, 256, device=dev, dtype=torch.bfloat16)
    r = torch.randn(4, 10, 256, device=dev)
    y = m(x, residual=r)
    y2 = rms_norm_fn(x, torch.ones(256, device=dev), None, residual=r, eps=1e-5)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    y_r, _, _, _ = R.layer_norm_fwd_ref(x.reshape(-1, 256).cpu(), torch.ones(256), None, r.reshape(-1, 256).cpu(),
                                        eps=1e-5, is_rms_norm=True)
    close("y", y.reshape(-1, 256), y_r.float(), 2e-2, 1e-2)


def test_empty_rows(dev):
    x = torch.empty(0, 64, device=dev)
    w = torch.ones(64, device=dev)
    y, _, mean, rstd, xs, _, _, _ = _layer_norm_fwd(x, w, None, 1e-5)
    assert y.shape == (0, 64) and rstd.shape == (0,)
    dx, dw, db, _, _, _, _ = _layer_norm_bwd(torch.empty(0, 64, device=dev), xs, w, None, 1e-5, mean, rstd)
    torch.cuda.synchronize()
    assert dx.shape == (0, 64) and torch.equal(dw.cpu(), torch.zeros(64))


@pytest.mark.parametrize("prenorm", [False, True])
def test_layer_norm_linear_fn(dev, prenorm):
    """linear(norm(x + residual)) against the library routines in fp64."""
    from lrnnx_amd import layer_norm_linear_fn

    g = torch.Generator().manual_seed(27)
    x = torch.randn(2, 9, 128, generator=g)
    res = torch.randn(2, 9, 128, generator=g)
    w, b = 1 + 0.1 * torch.randn(128, generator=g), 0.1 * torch.randn(128, generator=g)
    lw, lb = torch.randn(64, 128, generator=g) / 11, torch.randn(64, generator=g)
    dy = torch.randn(2, 9, 64, generator=g)
    ref_l = [t.double().requires_grad_() for t in (x, res, w, b, lw, lb)]
    s = ref_l[0] + ref_l[1]
    ref = F.linear(F.layer_norm(s, (128,), ref_l[2], ref_l[3], 1e-5), ref_l[4], ref_l[5])
    ref.backward(dy.double())
    dv = [t.to(dev).requires_grad_() for t in (x, res, w, b, lw, lb)]
    out = layer_norm_linear_fn(dv[0], dv[2], dv[3], dv[4], dv[5], residual=dv[1], eps=1e-5, prenorm=prenorm)
    if prenorm:
        out, ro = out
        assert torch.allclose(ro.detach().cpu(), (x + res))
    out.backward(dy.to(dev))
    torch.cuda.synchronize()
    close("out", out, ref.detach(), 1e-4, 1e-5)
    for name, got, r in zip(("dx", "dres", "dw", "db", "dlw", "dlb"), dv, ref_l):
        close(name, got.grad, r.grad, 1e-4, 1e-4)
