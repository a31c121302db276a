"""GPU parity of the one-step decode update against the CPU oracle
(restatement of selective_state_update_ref,
lrnnx/ops/triton/selective_state_update.py:479-599) and against one step of
the selective-scan oracle.  Tolerance: fp32 rtol 1e-4 / atol 1e-5 * max|ref|;
bf16 state rtol 2e-2 / atol 1e-2 * max|ref|."""

import pytest
import torch

from lrnnx_amd import selective_state_update
from oracle import scan_ref as R
from tests.parity import close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("method", ["mamba", "zoh", "bilinear", "dirac", "s7", "rglru"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("heads", [False, True])
@pytest.mark.parametrize("n", [16, 64])
def test_state_update(dev, method, dtype, heads, n):
    g = torch.Generator().manual_seed(3)
    b, h, d, grp = 3, (2 if heads else 1), 96, (2 if heads else 1)
    shp = (b, h, d) if heads else (b, d)
    state = torch.randn(*((b, h, d, n) if heads else (b, d, n)), generator=g).to(dtype)
    x = torch.randn(*shp, generator=g).to(dtype)
    dt = (0.5 * torch.randn(*shp, generator=g)).to(dtype)
    if method == "rglru":
        A = torch.rand(*((h, d, n) if heads else (d, n)), generator=g) * 0.5 + 0.45
    else:
        A = -torch.rand(*((h, d, n) if heads else (d, n)), generator=g) - 0.5
    Bm = torch.randn(*((b, grp, n) if heads else (b, n)), generator=g).to(dtype)
    Cm = torch.randn(*((b, grp, n) if heads else (b, n)), generator=g).to(dtype)
    D = torch.randn(*((h, d) if heads else (d,)), generator=g)
    z = torch.randn(*shp, generator=g).to(dtype)
    dt_bias = 0.1 * torch.randn(*((h, d) if heads else (d,)), generator=g)
    st_ref = state.clone().double()
    out_ref = R.selective_state_update_ref(st_ref, x.double(), dt.double(), A.double(), Bm.double(), Cm.double(),
                                           D.double(), z.double(), dt_bias.double(), True, None, method,
                                           compute_dtype=torch.float64)
    st_dev = state.to(dev)
    out = selective_state_update(st_dev, x.to(dev), dt.to(dev), A.to(dev), Bm.to(dev), Cm.to(dev), D.to(dev),
                                 z.to(dev), dt_bias.to(dev), True, None, None, method)
    torch.cuda.synchronize()
    rt, at = (1e-4, 1e-5) if dtype == torch.float32 else (2e-2, 1e-2)
    close("state", st_dev, st_ref, rt, at)
    close("out", out, out_ref, rt, at)


def test_state_update_batch_indices(dev):
    g = torch.Generator().manual_seed(4)
    b, d, n = 4, 64, 8
    state = torch.randn(6, d, n, generator=g)
    idx = torch.tensor([5, 0, 3, 1], dtype=torch.int32)
    x, dt = torch.randn(b, d, generator=g), torch.randn(b, d, generator=g)
    A = -torch.rand(d, n, generator=g) - 0.5
    Bm, Cm = torch.randn(b, n, generator=g), torch.randn(b, n, generator=g)
    st_ref = state.clone().double()
    sub = st_ref[idx.long()]
    out_ref = R.selective_state_update_ref(sub, x.double(), dt.double(), A.double(), Bm.double(), Cm.double(),
                                           dt_softplus=True, compute_dtype=torch.float64)
    st_ref[idx.long()] = sub
    st_dev = state.to(dev)
    out = selective_state_update(st_dev, x.to(dev), dt.to(dev), A.to(dev), Bm.to(dev), Cm.to(dev),
                                 dt_softplus=True, state_batch_indices=idx.to(dev))
    torch.cuda.synchronize()
    close("state", st_dev, st_ref, 1e-4, 1e-5)
    close("out", out, out_ref, 1e-4, 1e-5)


_LAYOUT_DSTATE = {"dstate32": 32, "dstate64": 64, "f32_state_dstate32": 32, "f32_state_dstate64": 64, "dstate24": 24}


@pytest.mark.parametrize("layout", ["rows16_batch_indices", "strided_state16", "dstate32", "dstate64",
                                    "f32_state_dstate32", "f32_state_dstate64", "dstate24", "f16_state"])
def test_state_update_layouts(dev, layout):
    """Both kernels of the update: the row-at-once path (d_state 16 / 32 / 64,
    unit-stride aligned rows: 2 to 16 lanes per row with bf16 / fp16 / fp32
    states; here also with state_batch_indices) and the entry-by-entry path (a
    state view with stride 2 along d_state; d_state 24)."""
    g = torch.Generator().manual_seed(5)
    b, d = 4, 200
    n = _LAYOUT_DSTATE.get(layout, 16)
    sdt = {"f16_state": torch.float16, "f32_state_dstate32": torch.float32,
           "f32_state_dstate64": torch.float32}.get(layout, torch.bfloat16)
    pool = 6 if layout == "rows16_batch_indices" else b
    if layout == "strided_state16":
        big = torch.randn(pool, d, 2 * n, generator=g).to(sdt)
        state_cpu = big[..., ::2]
    else:
        state_cpu = torch.randn(pool, d, n, generator=g).to(sdt)
    idx = torch.tensor([5, 0, 3, 1], dtype=torch.int32) if layout == "rows16_batch_indices" else None
    x = torch.randn(b, d, generator=g).to(torch.bfloat16)
    dt = (0.5 * torch.randn(b, d, generator=g)).to(torch.bfloat16)
    A = -torch.rand(d, n, generator=g) - 0.5
    Bm, Cm = torch.randn(b, n, generator=g).to(torch.bfloat16), torch.randn(b, n, generator=g).to(torch.bfloat16)
    D = torch.randn(d, generator=g)
    z = torch.randn(b, d, generator=g).to(torch.bfloat16)
    dt_bias = 0.1 * torch.randn(d, generator=g)
    st_ref = state_cpu.clone().double()
    sel = idx.long() if idx is not None else torch.arange(b)
    sub = st_ref[sel]
    out_ref = R.selective_state_update_ref(sub, x.double(), dt.double(), A.double(), Bm.double(), Cm.double(),
                                           D.double(), z.double(), dt_bias.double(), True, None, "mamba",
                                           compute_dtype=torch.float64)
    st_ref[sel] = sub
    if layout == "strided_state16":
        big_dev = big.to(dev)
        st_dev = big_dev[..., ::2]
    else:
        st_dev = state_cpu.to(dev)
    out = selective_state_update(st_dev, x.to(dev), dt.to(dev), A.to(dev), Bm.to(dev), Cm.to(dev), D.to(dev),
                                 z.to(dev), dt_bias.to(dev), True, None, idx.to(dev) if idx is not None else None)
    torch.cuda.synchronize()
    close(f"state {layout}", st_dev, st_ref, 2e-2, 1e-2)
    close(f"out {layout}", out, out_ref, 2e-2, 1e-2)
    if layout == "strided_state16":   # the entries between the view's are untouched
        assert torch.equal(big_dev[..., 1::2].cpu(), big[..., 1::2])
