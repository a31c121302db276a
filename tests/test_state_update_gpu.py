"""GPU parity of the one-step decode update against the CPU oracle
(restatement of selective_state_update_ref,
lrnnx/ops/triton/selective_state_update.py:479-599), and of a decode loop
against the selective scan over the same sequence.  Tolerance: fp32 rtol
1e-4 / atol 1e-5 * max|ref|; bf16 state rtol 2e-2 / atol 1e-2 * max|ref|."""

import pytest
import torch

from lrnnx_amd import selective_scan_fn, selective_state_update
from oracle import scan_ref as R
from tests.parity import close, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("method", ["mamba", "zoh", "bilinear", "dirac", "s7", "rglru"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("heads", [False, True])
@pytest.mark.parametrize("n", [16, 64, 128, 256])
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


_LAYOUT_DSTATE = {"dstate32": 32, "dstate64": 64, "f32_state_dstate32": 32, "f32_state_dstate64": 64, "dstate24": 24,
                  "dstate128": 128, "dstate256": 256, "f32_state_dstate128": 128, "f32_state_dstate256": 256}


@pytest.mark.parametrize("layout", ["rows16_batch_indices", "strided_state16", "dstate32", "dstate64",
                                    "f32_state_dstate32", "f32_state_dstate64", "dstate24", "f16_state",
                                    "dstate128", "dstate256", "f32_state_dstate128", "f32_state_dstate256"])
def test_state_update_layouts(dev, layout):
    """Both kernels of the update: the row-at-once path (d_state 16 / 32 / 64 /
    128 / 256, unit-stride aligned rows: 2 to 16 lanes per row, 16 to 64 bytes
    of state per lane, with bf16 / fp16 / fp32 states; here also with
    state_batch_indices) and the entry-by-entry path (a state view with stride
    2 along d_state; d_state 24)."""
    g = torch.Generator().manual_seed(5)
    b, d = 4, 200
    n = _LAYOUT_DSTATE.get(layout, 16)
    sdt = {"f16_state": torch.float16, "f32_state_dstate32": torch.float32, "f32_state_dstate64": torch.float32,
           "f32_state_dstate128": torch.float32, "f32_state_dstate256": torch.float32}.get(layout, torch.bfloat16)
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


@pytest.mark.parametrize("method", ["mamba", "zoh", "rglru"])
@pytest.mark.parametrize("n", [16, 24, 64, 128, 256])
@pytest.mark.parametrize("form", ["deltaA", "bare"])
def test_state_update_deltaA_and_bare(dev, method, n, form):
    """The operand forms the reference callers use besides the full one:
    deltaA given (the event-mode Mamba step, lrnnx/models/ltv/mamba.py:441-455)
    and the bare call without D, z, dt_bias and softplus (the RG-LRU step,
    lrnnx/models/ltv/rglru.py:315-325), on the row kernel (d_state 16, 64,
    128, 256) and the entry-by-entry kernel (d_state 24)."""
    g = torch.Generator().manual_seed(6 + n)
    b, d = 3, 160
    dtype = torch.bfloat16
    state = torch.randn(b, d, n, generator=g).to(dtype)
    x = torch.randn(b, d, generator=g).to(dtype)
    if form == "bare":  # no softplus: the step must already be positive
        dt = (0.3 * torch.rand(b, d, generator=g) + 1e-3).to(dtype)
    else:
        dt = (0.5 * torch.randn(b, d, generator=g)).to(dtype)
    A = (torch.rand(d, n, generator=g) * 0.5 + 0.45) if method == "rglru" else (-torch.rand(d, n, generator=g) - 0.5)
    Bm, Cm = torch.randn(b, n, generator=g).to(dtype), torch.randn(b, n, generator=g).to(dtype)
    if form == "deltaA":
        D = torch.randn(d, generator=g)
        z = torch.randn(b, d, generator=g).to(dtype)
        dt_bias = 0.1 * torch.randn(d, generator=g)
        dA_in = (0.4 * torch.rand(b, d, generator=g)).to(dtype)
        sp = True
    else:
        D = z = dt_bias = dA_in = None
        sp = False
    st_ref = state.clone().double()
    dbl = lambda t: None if t is None else t.double()
    out_ref = R.selective_state_update_ref(st_ref, x.double(), dt.double(), A.double(), Bm.double(), Cm.double(),
                                           dbl(D), dbl(z), dbl(dt_bias), sp, dbl(dA_in), method,
                                           compute_dtype=torch.float64)
    dv = lambda t: None if t is None else t.to(dev)
    st_dev = state.to(dev)
    out = selective_state_update(st_dev, x.to(dev), dt.to(dev), A.to(dev), Bm.to(dev), Cm.to(dev), dv(D), dv(z),
                                 dv(dt_bias), sp, dv(dA_in), None, method)
    torch.cuda.synchronize()
    close(f"state {form}", st_dev, st_ref, 2e-2, 1e-2)
    close(f"out {form}", out, out_ref, 2e-2, 1e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_loop_equals_scan(dev, dtype):
    """L steps of selective_state_update from a zero state reproduce
    selective_scan_fn over the same sequence, step by step and in the final
    state: the reference's parallel == recurrent bar
    (tests/models/test_ltv/test_mamba.py:51-87).  With a bf16 state (rounded
    every step) the loop is compared with the oracle's loop, which rounds the
    same way."""
    g = torch.Generator().manual_seed(17)
    Bt, D, L, N = 3, 128, 40, 16
    inp = R.make_selective_inputs(Bt, D, L, N, seed=17, itype=torch.float32)
    inp["A"] = -torch.rand(D, N, generator=g) - 0.5
    d = to_dev(inp, dev)
    out_scan, last_scan = selective_scan_fn(d["u"], d["delta"], d["A"], d["B"], d["C"], d["D"], d["z"],
                                            d["delta_bias"], None, True, True, "mamba")
    state = torch.zeros(Bt, D, N, device=dev, dtype=dtype)
    st_ref = torch.zeros(Bt, D, N, dtype=dtype)
    outs, outs_ref = [], []
    for t in range(L):
        outs.append(selective_state_update(state, d["u"][:, :, t], d["delta"][:, :, t], d["A"], d["B"][:, :, t],
                                           d["C"][:, :, t], d["D"], d["z"][:, :, t], d["delta_bias"], True))
        if dtype != torch.float32:
            outs_ref.append(R.selective_state_update_ref(
                st_ref, inp["u"][:, :, t].double(), inp["delta"][:, :, t].double(), inp["A"].double(),
                inp["B"][:, :, t].double(), inp["C"][:, :, t].double(), inp["D"].double(),
                inp["z"][:, :, t].double(), inp["delta_bias"].double(), True, None, "mamba",
                compute_dtype=torch.float64))
    torch.cuda.synchronize()
    loop = torch.stack(outs, dim=2)
    if dtype == torch.float32:
        close("decode loop out vs scan", loop, out_scan.cpu().double(), 1e-4, 1e-5)
        close("decode loop state vs scan last_state", state, last_scan.cpu().double(), 1e-4, 1e-5)
    else:
        close("decode loop out vs oracle loop", loop, torch.stack(outs_ref, dim=2), 2e-2, 1e-2)
        close("decode loop state vs oracle loop", state, st_ref.double(), 2e-2, 1e-2)
        # and the bf16-state loop stays near the fp32-state scan
        close("bf16 decode loop vs scan", loop, out_scan.cpu().double(), 5e-2, 3e-2)
