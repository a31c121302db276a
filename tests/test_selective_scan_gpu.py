"""GPU parity of the selective scan (HIP kernels through the C ABI) against the
float64 CPU oracle (oracle/scan_ref.py, a restatement of the reference's
selective_scan_ref, lrnnx/ops/selective_scan.py:200-360).

Tolerances (elementwise |got-ref| <= atol + rtol |ref|, atol relative to the
tensor's max magnitude):
  fp32 I/O  : outputs rtol 1e-4, atol 1e-5 * max|ref|; gradients the same,
              except reductions over batch*length (dA, dD, ddelta_bias,
              constant dB/dC) rtol 1e-4, atol 1e-4 * max|ref|.
  bf16 I/O  : rtol 2e-2, atol 1e-2 * max|ref| (fp32 state; inputs are the
              bf16-rounded values given to both sides).
"""

import pytest
import torch

from lrnnx_amd import selective_scan_fn
from oracle import scan_ref as R
from tests.parity import close, oracle_selective, to_dev

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-4, 1e-5, 1e-4), torch.bfloat16: (2e-2, 1e-2, 1e-2), torch.float16: (1e-2, 5e-3, 5e-3)}


def _run(dev, B, D, L, N, itype=torch.float32, method="mamba", varB=True, varC=True, has_z=True, has_D=True,
         has_bias=True, softplus=True, groups=None, seed=0, with_deltaA=False, A_override=None):
    inp = R.make_selective_inputs(B, D, L, N, seed=seed, itype=itype, groups=groups, varB=varB, varC=varC,
                                  has_z=has_z, has_D=has_D, has_bias=has_bias)
    if A_override is not None:
        inp["A"] = A_override
    if not softplus:
        # without softplus the time step delta + delta_bias must already be positive
        # (as the callers guarantee)
        inp["delta"] = (inp["delta"].float().abs() * 0.2 + 1e-3).to(itype)
        if inp.get("delta_bias") is not None:
            inp["delta_bias"] = inp["delta_bias"].abs() * 0.01
    g = torch.Generator().manual_seed(seed + 100)
    dout = torch.randn(B, D, L, generator=g).to(itype)
    deltaA = (0.5 * torch.rand(B, D, L, generator=g)).to(itype) if with_deltaA else None
    ref_out, ref_last, ref_g = oracle_selective(inp, method, softplus, deltaA, True, dout)
    d = to_dev(inp, dev)
    leaves = {}
    for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias"):
        if d.get(k) is not None:
            leaves[k] = d[k].clone().requires_grad_(True)
    dA_dev = deltaA.to(dev).requires_grad_(True) if deltaA is not None else None
    out, last = selective_scan_fn(leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"],
                                  leaves.get("D"), leaves.get("z"), leaves.get("delta_bias"), dA_dev, softplus,
                                  True, method)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    rt, at, atr = TOL[itype]
    close("out", out, ref_out, rt, at)
    close("last_state", last, ref_last, rt, at)
    for k, v in leaves.items():
        red = k in ("A", "D", "delta_bias") or (k == "B" and not varB) or (k == "C" and not varC)
        close(f"d{k}", v.grad, ref_g[k], rt, atr if red else at)
    if dA_dev is not None:
        close("ddeltaA", dA_dev.grad, ref_g["deltaA"], rt, at)


@pytest.mark.parametrize("L", [1, 7, 32, 100, 256, 511])
def test_mamba_fp32_lengths(dev, L):
    _run(dev, 2, 64, L, 16)


@pytest.mark.parametrize("varB,varC", [(True, True), (True, False), (False, True), (False, False)])
def test_mamba_fp32_var_const(dev, varB, varC):
    _run(dev, 2, 70, 96, 16, varB=varB, varC=varC)


@pytest.mark.parametrize("N", [1, 3, 8, 16, 20, 32, 33, 64, 100, 128, 256])
def test_mamba_fp32_dstate(dev, N):
    # N > 64 runs the 32-states-per-wave instantiation (the reference accepts
    # N <= 256; its LM tests use d_state 128)
    _run(dev, 1, 64, 80, N)


@pytest.mark.parametrize("N", [128, 256])
def test_mamba_bf16_large_dstate(dev, N):
    _run(dev, 2, 64, 96, N, itype=torch.bfloat16, seed=N)


@pytest.mark.parametrize("flags", [dict(has_z=False), dict(has_D=False), dict(has_bias=False), dict(softplus=False)])
def test_mamba_fp32_options(dev, flags):
    _run(dev, 2, 64, 64, 16, **flags)


def test_mamba_fp32_groups(dev):
    _run(dev, 2, 128, 64, 16, groups=2)


def test_mamba_fp32_deltaA(dev):
    _run(dev, 2, 64, 64, 16, with_deltaA=True)


@pytest.mark.parametrize("method", ["zoh", "bilinear", "dirac"])
@pytest.mark.parametrize("varB,varC", [(True, True), (False, False)])
def test_other_methods_fp32(dev, method, varB, varC):
    _run(dev, 2, 64, 72, 8, method=method, varB=varB, varC=varC)


@pytest.mark.parametrize("method", ["zoh", "bilinear", "dirac"])
def test_other_methods_deltaA(dev, method):
    _run(dev, 2, 64, 48, 8, method=method, with_deltaA=True)


def test_s7_fp32(dev):
    _run(dev, 2, 64, 64, 1, method="s7", varB=False, varC=False, has_z=False, has_D=False, has_bias=False,
         softplus=False)


def test_rglru_fp32(dev):
    A = torch.rand(64, 1) * 0.5 + 0.45
    _run(dev, 2, 64, 64, 1, method="rglru", varB=False, varC=False, has_z=False, has_D=False, has_bias=False,
         softplus=False, A_override=A)


@pytest.mark.parametrize("L,has_D", [(7, False), (513, True), (2100, False), (4100, True)])
def test_rglru_fast_path_lengths(dev, L, has_D):
    # one state per channel takes the lanes-along-L kernels: lengths inside one
    # lane, across the 512-step chunk, and across the 2048-step carries (last_state)
    A = torch.rand(64, 1, generator=torch.Generator().manual_seed(L)) * 0.5 + 0.45
    _run(dev, 2, 64, L, 1, method="rglru", varB=False, varC=False, has_z=False, has_D=has_D, has_bias=False,
         softplus=False, A_override=A, seed=L)


@pytest.mark.parametrize("L", [513, 2100])
def test_s7_fast_path_lengths(dev, L):
    _run(dev, 2, 64, L, 1, method="s7", varB=False, varC=False, has_z=False, has_D=True, has_bias=False,
         softplus=False, seed=L + 1)


def _rglru_leaves(dev, L, seed):
    inp = R.make_selective_inputs(2, 48, L, 1, seed=seed, varB=False, varC=False, has_z=False, has_D=True,
                                  has_bias=False)
    inp["A"] = torch.rand(48, 1, generator=torch.Generator().manual_seed(seed)) * 0.5 + 0.45
    inp["delta"] = inp["delta"].float().abs() * 0.2 + 1e-3
    d = to_dev(inp, dev)
    return {k: d[k].clone().requires_grad_(True) for k in ("u", "delta", "A", "B", "C", "D")}


@pytest.mark.parametrize("method", ["rglru", "s7"])
@pytest.mark.parametrize("fwd_generic,bwd_generic", [("0", "1"), ("1", "0"), ("1", "1")])
def test_rglru_fast_path_matches_generic(dev, monkeypatch, method, fwd_generic, bwd_generic):
    """The one-state rglru / s7 fast kernels write and read the general path's
    checkpoint layout: a forward on one path followed by a backward on the
    other gives the results of the fast path on both."""
    L = 1100
    dout = torch.randn(2, 48, L, generator=torch.Generator().manual_seed(3)).to(dev)
    res = []
    for fg, bg in (("0", "0"), (fwd_generic, bwd_generic)):
        lv = _rglru_leaves(dev, L, 11)
        monkeypatch.setenv("LRNNX_SCAN_GENERIC", fg)
        out, last = selective_scan_fn(lv["u"], lv["delta"], lv["A"], lv["B"], lv["C"], lv["D"], None, None, None,
                                      False, True, method)
        monkeypatch.setenv("LRNNX_SCAN_GENERIC", bg)
        out.backward(dout)
        torch.cuda.synchronize()
        res.append([out.detach(), last.detach()] + [lv[k].grad for k in lv])
    names = ["out", "last_state"] + ["d" + k for k in ("u", "delta", "A", "B", "C", "D")]
    for n, a, b in zip(names, res[0], res[1]):
        # same fp32 math; the scan across lanes and the sums run in another order
        close(n, a, b.cpu().double(), 1e-4, 1e-4 if n in ("dA", "dB", "dC", "dD") else 1e-5)


@pytest.mark.parametrize("itype", [torch.bfloat16, torch.float16])
def test_mamba_low_precision(dev, itype):
    _run(dev, 2, 64, 128, 16, itype=itype)


def test_mamba_bf16_cfg2_slice(dev):
    # config-2 distributions on a channel slice (the full shape is timed by bench.py)
    _run(dev, 2, 64, 2048, 16, itype=torch.bfloat16, seed=2)


def test_mamba_fp32_long_chunks(dev):
    # crosses the 2048-step chunk of the reference x carries
    _run(dev, 1, 64, 4100, 16, seed=5)


@pytest.mark.parametrize("itype", [torch.float32, torch.bfloat16])
def test_mamba_fast_path_long_chunks(dev, itype):
    # L a multiple of the fast path's tile: the fast kernels run, and the
    # 2048-step chunk carries (last_state) cross two chunk ends
    _run(dev, 1, 64, 4160, 16, itype=itype, seed=6)


@pytest.mark.parametrize("N", [12, 16])
def test_mamba_fast_path_dstate(dev, N):
    _run(dev, 2, 64, 96, N, itype=torch.bfloat16, seed=7)


@pytest.mark.parametrize("itype", [torch.float32, torch.bfloat16])
def test_fast_path_matches_generic(dev, itype, monkeypatch):
    """The fast kernels and the generic kernels (LRNNX_SCAN_GENERIC=1) agree on
    the same inputs (both fp32 state; only the order of the final sums differs)."""
    inp = R.make_selective_inputs(2, 128, 512, 16, seed=8, itype=itype, groups=2)
    g = torch.Generator().manual_seed(9)
    dout = torch.randn(2, 128, 512, generator=g).to(itype).to(dev)
    d = to_dev(inp, dev)
    res = []
    for generic in ("0", "1"):
        monkeypatch.setenv("LRNNX_SCAN_GENERIC", generic)
        leaves = {k: d[k].clone().requires_grad_(True) for k in ("u", "delta", "A", "B", "C", "D", "z",
                                                                 "delta_bias")}
        out, last = selective_scan_fn(leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"],
                                      leaves["D"], leaves["z"], leaves["delta_bias"], None, True, True, "mamba")
        out.backward(dout)
        torch.cuda.synchronize()
        res.append([out.detach().float(), last.detach()] + [leaves[k].grad.float() for k in leaves])
    names = ["out", "last_state"] + ["d" + k for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")]
    rt = 1e-5 if itype == torch.float32 else 1e-2
    for n, a, b in zip(names, res[0], res[1]):
        close(n, a, b.cpu().double(), rt, rt)


def test_binding_bwd_recompute_out_z(dev):
    """selective_scan_cuda.bwd with recompute_out_z=True appends out_z, equal to
    the forward's (selective_scan_cpu.cpp:627-631 return order)."""
    from lrnnx_amd import selective_scan_cuda as ssc

    inp = R.make_selective_inputs(2, 64, 96, 16, seed=12)
    d = to_dev(inp, dev)
    g = torch.Generator().manual_seed(13)
    dout = torch.randn(2, 64, 96, generator=g).to(dev)
    d["B"], d["C"] = d["B"].unsqueeze(1).contiguous(), d["C"].unsqueeze(1).contiguous()  # (b, g, n, l)
    fwd = ssc.fwd(d["u"], d["delta"], d["A"], d["B"], d["C"], d["D"], d["z"], d["delta_bias"], None, True, "mamba")
    out, x, out_z = fwd
    res = ssc.bwd(d["u"], d["delta"], d["A"], d["B"], d["C"], d["D"], d["z"], d["delta_bias"], None, dout, x, out,
                  None, True, True, "mamba")
    assert len(res) == 9  # du, ddelta, dA, dB, dC, dD, ddelta_bias, dz, out_z
    close("out_z", res[-1], out_z.cpu().double(), 1e-6, 1e-6)
    ref = ssc.bwd(d["u"], d["delta"], d["A"], d["B"], d["C"], d["D"], d["z"], d["delta_bias"], None, dout, x, out,
                  None, True, False, "mamba")
    assert len(ref) == 8
    for n, a_, b_ in zip(("du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz"), res[:8], ref):
        close(n, a_, b_.cpu().double(), 1e-6, 1e-6)


@pytest.mark.parametrize("itype", [torch.float32, torch.bfloat16])
def test_fast_forward_split_matches_unsplit(dev, itype):
    """A small grid (B=1, D=64: one workgroup) splits L into segments when the
    forward gets a workspace; without one it runs unsplit.  Both give the same
    out, x carries (chunk products and states) and checkpoints, up to the
    rounding of the carry chain."""
    from lrnnx_amd import _lib
    from lrnnx_amd import selective_scan_cuda as ssc

    L = 4160  # 2048-step chunk ends inside the run, a ragged last chunk
    inp = R.make_selective_inputs(1, 64, L, 16, seed=21, itype=itype)
    d = to_dev(inp, dev)
    d["B"], d["C"] = d["B"].unsqueeze(1).contiguous(), d["C"].unsqueeze(1).contiguous()
    res = []
    for split in (True, False):
        a = ssc.build_args(d["u"], d["delta"], d["A"], d["B"], d["C"], d["D"], d["z"], d["delta_bias"], None, True,
                           "mamba")
        if split:
            assert _lib.lib().lrnnx_selective_scan_workspace_size(a, 0) > 0
            out, x, out_z, ckpt = ssc.run_fwd(a, d["u"], d["delta"], d["A"], d["z"], want_ckpt=True)
        else:
            out = torch.empty_like(d["u"])
            out_z = torch.empty_like(d["z"])
            x = torch.empty((1, 64, 3, 32), dtype=torch.float32, device=dev)
            ckpt = torch.empty(_lib.lib().lrnnx_selective_scan_ckpt_size(a) // 4, dtype=torch.float32, device=dev)
            a.out, a.out_z = _lib.view(out, 2), _lib.view(out_z, 2)
            a.x, a.ckpt = x.data_ptr(), ckpt.data_ptr()
            a.workspace, a.workspace_bytes = None, 0
            _lib.check(_lib.lib().lrnnx_selective_scan_fwd(a, _lib.stream_of(d["u"])), "fwd")
        torch.cuda.synchronize()
        res.append((out.float(), out_z.float(), x, ckpt))
    tol = 1e-5 if itype == torch.float32 else 2e-2
    for name, s_, u_ in zip(("out", "out_z", "x", "ckpt"), res[0], res[1]):
        close(name, s_, u_.cpu().double(), tol if name in ("out", "out_z") else 1e-5, tol if name in ("out", "out_z") else 1e-5)


# "dirac" (input term B u) on the fast kernels: fp32 input, d_state <= 16,
# L a multiple of 16.  Small grids split L (the default) or run unsplit in
# 64- or 32-channel workgroups (LRNNX_SCAN_NO_SPLIT, LRNNX_SCAN_CHANNELS).
@pytest.mark.parametrize("schedule", ["split", "unsplit64", "unsplit32"])
@pytest.mark.parametrize("opts", [dict(), dict(has_z=False, softplus=False, N=13), dict(groups=2, has_bias=False)],
                         ids=["z_softplus", "noz_nosoftplus_n13", "groups2"])
def test_dirac_fast_path_vs_oracle(dev, monkeypatch, schedule, opts):
    if schedule != "split":
        monkeypatch.setenv("LRNNX_SCAN_NO_SPLIT", "1")
        monkeypatch.setenv("LRNNX_SCAN_CHANNELS", schedule[-2:])
    opts = dict(opts)
    N = opts.pop("N", 16)
    print(f"dirac fast path, schedule {schedule}, N={N}, {opts}", flush=True)
    _run(dev, 2, 128, 512, N, method="dirac", seed=51, **opts)


@pytest.mark.parametrize("no_split", ["0", "1"])
def test_dirac_fast_path_long_chunks(dev, monkeypatch, no_split):
    # the 2048-step chunk carries (last_state) across two chunk ends and a
    # ragged last chunk, split into segments and unsplit
    monkeypatch.setenv("LRNNX_SCAN_NO_SPLIT", no_split)
    _run(dev, 1, 64, 4160, 16, method="dirac", seed=52)


def test_dirac_fast_path_matches_generic(dev, monkeypatch):
    """The fast kernels and the generic kernels (LRNNX_SCAN_GENERIC=1) agree on
    "dirac" (both fp32 state; only the order of the final sums differs)."""
    inp = R.make_selective_inputs(2, 128, 512, 16, seed=53, groups=2)
    dout = torch.randn(2, 128, 512, generator=torch.Generator().manual_seed(54)).to(dev)
    d = to_dev(inp, dev)
    res = []
    for generic in ("0", "1"):
        monkeypatch.setenv("LRNNX_SCAN_GENERIC", generic)
        leaves = {k: d[k].clone().requires_grad_(True) for k in ("u", "delta", "A", "B", "C", "D", "z",
                                                                 "delta_bias")}
        out, last = selective_scan_fn(leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"],
                                      leaves["D"], leaves["z"], leaves["delta_bias"], None, True, True, "dirac")
        out.backward(dout)
        torch.cuda.synchronize()
        res.append([out.detach(), last.detach()] + [leaves[k].grad for k in leaves])
    names = ["out", "last_state"] + ["d" + k for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")]
    for n, a, b in zip(names, res[0], res[1]):
        close(n, a, b.cpu().double(), 1e-5, 1e-5)


@pytest.mark.parametrize("save", ["checkpoints", "x"])
@pytest.mark.parametrize("no_split", ["0", "1"])
def test_dirac_binding_fwd_then_bwd(dev, monkeypatch, save, no_split):
    """selective_scan_cuda.fwd -> bwd(x, out) for "dirac": with the forward's
    checkpoints, or rebuilding them on the fast path's states-only forward
    (split on this small grid, or one 2048-step chunk per grid slice from the
    x carries when unsplit)."""
    from lrnnx_amd import selective_scan_cuda as ssc

    monkeypatch.setenv("LRNNX_SCAN_NO_SPLIT", no_split)
    prev = ssc.save_mode()
    ssc.set_save_mode(save)
    try:
        Bt, D, L = 1, 64, 4160
        inp = R.make_selective_inputs(Bt, D, L, 16, seed=55)
        dout = torch.randn(Bt, D, L, generator=torch.Generator().manual_seed(56))
        ro, rl, rg = oracle_selective(inp, "dirac", True, None, True, dout)
        d = to_dev(inp, dev)
        u, dl, A, B, C, Dv, z, db = (d[k] for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias"))
        B, C = B.unsqueeze(1).contiguous(), C.unsqueeze(1).contiguous()  # (b, g, n, l), as the autograd wrapper
        out, x, out_z = ssc.fwd(u, dl, A, B, C, Dv, z, db, None, True, "dirac")[:3]
        g = ssc.bwd(u, dl, A, B, C, Dv, z, db, None, dout.to(dev), x, out, None, True, False, "dirac")
        torch.cuda.synchronize()
    finally:
        ssc.set_save_mode(prev)
    close("out", out_z, ro, 1e-4, 1e-5)
    close("last_state", x[:, :, -1, 1::2], rl, 1e-4, 1e-5)
    for i, k in enumerate(("u", "delta", "A", "B", "C", "D", "delta_bias")):
        close(f"d{k}", g[i], rg[k], 1e-4, 1e-4 if k in ("A", "D", "delta_bias") else 1e-5)
    close("dz", g[7], rg["z"], 1e-4, 1e-5)


# d_state > 64 (real weights): blocks of at most 64 states along the grid's z
# dimension, on the 8-states-per-wave kernels; their sums over states (y, and
# the du / ddelta / ddeltaA terms) are fp32 partials combined in block order.
@pytest.mark.parametrize("method,N,extra", [
    ("mamba", 100, {}),                                  # blocks of 56 + 44 states
    ("mamba", 128, dict(groups=2)),
    ("mamba", 128, dict(varB=False, varC=False)),
    ("mamba", 96, dict(with_deltaA=True)),
    ("mamba", 200, dict(has_z=False, softplus=False)),   # four blocks of 56, 56, 56, 32
    ("zoh", 80, {}),
    ("zoh", 96, dict(with_deltaA=True)),
    ("bilinear", 72, {}),
    ("dirac", 128, dict(varB=True, varC=False)),
], ids=lambda v: str(v) if not isinstance(v, dict) else "-".join(f"{k}={x}" for k, x in v.items()) or "default")
def test_state_blocks_vs_oracle(dev, method, N, extra):
    print(f"state blocks: {method} N={N} {extra}", flush=True)
    _run(dev, 2, 64, 200, N, method=method, seed=61 + N, **extra)


def test_state_blocks_one_state_methods(dev):
    """s7 and rglru with 80 states (constant B / C), on the state blocks."""
    _run(dev, 2, 64, 96, 80, method="s7", varB=False, varC=False, has_z=False, has_D=True, has_bias=False,
         softplus=False, seed=63)
    A = torch.rand(64, 80, generator=torch.Generator().manual_seed(64)) * 0.5 + 0.45
    _run(dev, 2, 64, 96, 80, method="rglru", varB=False, varC=False, has_z=False, has_D=False, has_bias=False,
         softplus=False, A_override=A, seed=64)


def test_state_blocks_long_chunks_bf16(dev):
    # the 2048-step chunk carries of every block (last_state) across a chunk end
    _run(dev, 1, 64, 2100, 128, itype=torch.bfloat16, seed=65)


def test_state_blocks_without_workspace(dev):
    """d_state > 64 without a forward workspace: every state in one workgroup
    (the fallback), with the checkpoint interval of the blocks.  out, out_z, x
    and the checkpoints match the state-block forward; the allocation-free
    forward takes the same path; the backward (state blocks) from the
    fallback's checkpoints matches the fp64 oracle."""
    from lrnnx_amd import _lib
    from lrnnx_amd import selective_scan_cuda as ssc

    Bt, D, L, N = 2, 64, 160, 128
    inp = R.make_selective_inputs(Bt, D, L, N, seed=66)
    dout = torch.randn(Bt, D, L, generator=torch.Generator().manual_seed(67))
    ro, rl, rg = oracle_selective(inp, "mamba", True, None, True, dout)
    d = to_dev(inp, dev)
    d["B"], d["C"] = d["B"].unsqueeze(1).contiguous(), d["C"].unsqueeze(1).contiguous()

    def args():
        return ssc.build_args(d["u"], d["delta"], d["A"], d["B"], d["C"], d["D"], d["z"], d["delta_bias"], None,
                              True, "mamba")

    a = args()
    assert _lib.lib().lrnnx_selective_scan_workspace_size(a, 0) == 2 * Bt * D * L * 4   # two blocks of 64
    res = {"blocks": ssc.run_fwd(a, d["u"], d["delta"], d["A"], d["z"], want_ckpt=True)}
    for entry in ("lrnnx_selective_scan_fwd", "lrnnx_selective_scan_fwd_noalloc"):
        a = args()
        out, out_z = torch.empty_like(d["u"]), torch.empty_like(d["z"])
        x = torch.empty((Bt, D, 1, 2 * N), dtype=torch.float32, device=dev)
        ckpt = torch.empty(_lib.lib().lrnnx_selective_scan_ckpt_size(a) // 4, dtype=torch.float32, device=dev)
        a.out, a.out_z = _lib.view(out, 2), _lib.view(out_z, 2)
        a.x, a.ckpt = x.data_ptr(), ckpt.data_ptr()
        a.workspace, a.workspace_bytes = None, 0
        _lib.check(getattr(_lib.lib(), entry)(a, _lib.stream_of(d["u"])), entry)
        torch.cuda.synchronize()
        res[entry] = (out, x, out_z, ckpt)
    ref = res["blocks"]
    for entry in ("lrnnx_selective_scan_fwd", "lrnnx_selective_scan_fwd_noalloc"):
        for name, g_, r_ in zip(("out", "x", "out_z", "ckpt"), res[entry], ref):
            close(f"{name} ({entry})", g_, r_.cpu().double(), 1e-5, 1e-5)
    out, x, out_z, ckpt = res["lrnnx_selective_scan_fwd"]
    close("out_z vs oracle", out_z, ro, 1e-4, 1e-5)
    g = ssc.run_bwd(args(), d["u"], d["delta"], d["A"], d["B"], d["C"], d["D"], d["z"], d["delta_bias"], None,
                    dout.to(dev), out, ckpt)
    torch.cuda.synchronize()
    for i, k in enumerate(("u", "delta", "A", "B", "C", "D", "delta_bias")):
        gk = g[i].squeeze(1) if k in ("B", "C") else g[i]
        close(f"d{k}", gk, rg[k], 1e-4, 1e-4 if k in ("A", "D", "delta_bias") else 1e-5)
    close("dz", g[7], rg["z"], 1e-4, 1e-5)


@pytest.mark.parametrize("itype", [torch.float32, torch.bfloat16])
def test_state_blocks_ragged_shapes(dev, itype):
    """State blocks on ragged shapes: D = 200 in two groups (50-channel
    workgroups: partial channel blocks, synchronous tile fetches) and L = 203
    (a partial last tile; the partial sums' rows are not 16-byte multiples)."""
    _run(dev, 2, 200, 203, 100, itype=itype, groups=2, seed=68)


# deltaA (Mamba's event mode, lrnnx/models/ltv/mamba.py:303-330: delta without
# softplus or bias, deltaA the step of A_bar) on the fast kernels, both
# directions, with and without softplus.
@pytest.mark.parametrize("itype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("schedule", ["split", "unsplit64", "unsplit32"])
def test_deltaA_fast_path_vs_oracle(dev, monkeypatch, itype, schedule):
    if schedule != "split":
        monkeypatch.setenv("LRNNX_SCAN_NO_SPLIT", "1")
        monkeypatch.setenv("LRNNX_SCAN_CHANNELS", schedule[-2:])
    print(f"deltaA fast path, {schedule}, {itype}", flush=True)
    _run(dev, 2, 128, 512, 16, itype=itype, has_bias=False, softplus=False, with_deltaA=True, seed=71)


def test_deltaA_fast_forward_softplus_long(dev):
    # with softplus and bias too; two chunk ends and a ragged last chunk (x carries over deltaA)
    _run(dev, 1, 64, 4160, 13, itype=torch.bfloat16, with_deltaA=True, seed=72)


@pytest.mark.parametrize("save", ["checkpoints", "x"])
def test_deltaA_binding_fwd_then_bwd(dev, monkeypatch, save):
    """selective_scan_cuda.fwd -> bwd(x, out) with deltaA: the backward gets
    the forward's checkpoints, or rebuilds them on the fast states-only
    forward from the x carries (unsplit grid: one 2048-step chunk per slice)."""
    from lrnnx_amd import selective_scan_cuda as ssc

    monkeypatch.setenv("LRNNX_SCAN_NO_SPLIT", "1")
    prev = ssc.save_mode()
    ssc.set_save_mode(save)
    try:
        Bt, D, L = 1, 64, 4160
        inp = R.make_selective_inputs(Bt, D, L, 16, seed=73, has_bias=False)
        inp["delta"] = inp["delta"].abs() * 0.2 + 1e-3
        g = torch.Generator().manual_seed(74)
        dA = 0.5 * torch.rand(Bt, D, L, generator=g)
        dout = torch.randn(Bt, D, L, generator=g)
        ro, rl, rg = oracle_selective(inp, "mamba", False, dA, True, dout)
        d = to_dev(inp, dev)
        u, dl, A, B, C, Dv, z = (d[k] for k in ("u", "delta", "A", "B", "C", "D", "z"))
        B, C = B.unsqueeze(1).contiguous(), C.unsqueeze(1).contiguous()
        dA_dev = dA.to(dev)
        out, x, out_z = ssc.fwd(u, dl, A, B, C, Dv, z, None, dA_dev, False, "mamba")[:3]
        res = ssc.bwd(u, dl, A, B, C, Dv, z, None, dA_dev, dout.to(dev), x, out, None, False, False, "mamba")
        torch.cuda.synchronize()
    finally:
        ssc.set_save_mode(prev)
    close("out", out_z, ro, 1e-4, 1e-5)
    close("last_state", x[:, :, -1, 1::2], rl, 1e-4, 1e-5)
    # du, ddelta, dA, dB, dC, dD, ddelta_bias (None), ddeltaA, dz
    for i, k in ((0, "u"), (1, "delta"), (2, "A"), (3, "B"), (4, "C"), (5, "D")):
        gk = res[i].squeeze(1) if k in ("B", "C") else res[i]
        close(f"d{k}", gk, rg[k], 1e-4, 1e-4 if k in ("A", "D") else 1e-5)
    close("ddeltaA", res[7], rg["deltaA"], 1e-4, 1e-5)
    close("dz", res[8], rg["z"], 1e-4, 1e-5)


@pytest.mark.parametrize("itype", [torch.float32, torch.bfloat16])
def test_deltaA_fast_forward_matches_generic(dev, monkeypatch, itype):
    """The deltaA forward on the fast and on the general kernels: out, x
    carries and checkpoints agree (fp32 state; sums in another order)."""
    from lrnnx_amd import _lib
    from lrnnx_amd import selective_scan_cuda as ssc

    inp = R.make_selective_inputs(2, 128, 512, 16, seed=75, itype=itype, has_bias=False)
    inp["delta"] = (inp["delta"].float().abs() * 0.2 + 1e-3).to(itype)
    dA = (0.5 * torch.rand(2, 128, 512, generator=torch.Generator().manual_seed(76))).to(itype)
    d = to_dev(inp, dev)
    d["B"], d["C"] = d["B"].unsqueeze(1).contiguous(), d["C"].unsqueeze(1).contiguous()
    res = []
    for generic in ("0", "1"):
        monkeypatch.setenv("LRNNX_SCAN_GENERIC", generic)
        a = ssc.build_args(d["u"], d["delta"], d["A"], d["B"], d["C"], d["D"], d["z"], None, dA.to(dev), False,
                           "mamba")
        res.append(ssc.run_fwd(a, d["u"], d["delta"], d["A"], d["z"], want_ckpt=True))
        torch.cuda.synchronize()
    tol = 1e-5 if itype == torch.float32 else 1e-2
    for name, f_, g_ in zip(("out", "x", "out_z", "ckpt"), res[0], res[1]):
        t = tol if name in ("out", "out_z") else 1e-5
        close(f"{name} fast vs general", f_.float(), g_.float().cpu().double(), t, t)


@pytest.mark.parametrize("itype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_z", [True, False])
@pytest.mark.parametrize("softplus", [False, True])
def test_deltaA_fast_path_matches_generic(dev, monkeypatch, itype, with_z, softplus):
    """deltaA fwd + bwd on the fast and on the general kernels, without
    softplus (event mode) and with it: every output and gradient, ddeltaA
    included (fp32 state; sums in another order)."""
    inp = R.make_selective_inputs(2, 128, 512, 16, seed=77, itype=itype, has_bias=False, has_z=with_z)
    if not softplus:
        inp["delta"] = (inp["delta"].float().abs() * 0.2 + 1e-3).to(itype)
    g = torch.Generator().manual_seed(78)
    dA = (0.5 * torch.rand(2, 128, 512, generator=g)).to(itype)
    dout = torch.randn(2, 128, 512, generator=g).to(itype).to(dev)
    d = to_dev(inp, dev)
    res = []
    for generic in ("0", "1"):
        monkeypatch.setenv("LRNNX_SCAN_GENERIC", generic)
        lv = {k: d[k].clone().requires_grad_(True) for k in ("u", "delta", "A", "B", "C", "D")}
        z = d["z"].clone().requires_grad_(True) if with_z else None
        dA_dev = dA.to(dev).requires_grad_(True)
        out, last = selective_scan_fn(lv["u"], lv["delta"], lv["A"], lv["B"], lv["C"], lv["D"], z, None, dA_dev,
                                      softplus, True, "mamba")
        out.backward(dout)
        torch.cuda.synchronize()
        res.append([out.detach().float(), last.detach()] + [lv[k].grad.float() for k in lv] +
                   [dA_dev.grad.float()] + ([z.grad.float()] if with_z else []))
    names = ["out", "last_state", "du", "ddelta", "dA", "dB", "dC", "dD", "ddeltaA"] + (["dz"] if with_z else [])
    rt = 1e-5 if itype == torch.float32 else 1e-2
    for n, a_, b_ in zip(names, res[0], res[1]):
        close(f"{n} fast vs general", a_, b_.cpu().double(), rt, rt)


@pytest.mark.parametrize("path", ["fast_split", "fast_unsplit64", "fast_unsplit32", "general", "state_blocks"])
@pytest.mark.parametrize("itype", [torch.float32, torch.bfloat16])
def test_x_carries_vs_oracle(dev, monkeypatch, path, itype):
    """Both halves of every chunk carry of ``selective_scan_cuda.fwd``'s x over
    three 2048-step chunks: the product of A_bar since the sequence start (the
    reference's running prefix, selective_scan.cuh:316-333) and the state,
    against oracle.selective_scan_fwd_ref."""
    from lrnnx_amd import selective_scan_cuda as ssc

    N = 80 if path == "state_blocks" else 16
    if path.startswith("fast_unsplit"):
        monkeypatch.setenv("LRNNX_SCAN_NO_SPLIT", "1")
        monkeypatch.setenv("LRNNX_SCAN_CHANNELS", path[-2:])
    if path == "general":
        monkeypatch.setenv("LRNNX_SCAN_GENERIC", "1")
    Bt, D, L = 1, 64, 4160
    inp = R.make_selective_inputs(Bt, D, L, N, seed=79, itype=itype)
    inp["delta"] = (inp["delta"].float() * 0.1).to(itype)   # keep the products above underflow for a while
    ro, rx, roz = R.selective_scan_fwd_ref(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"],
                                           inp["delta_bias"], None, True, compute_dtype=torch.float64)
    d = to_dev(inp, dev)
    B, C = d["B"].unsqueeze(1).contiguous(), d["C"].unsqueeze(1).contiguous()
    out, x = ssc.fwd(d["u"], d["delta"], d["A"], B, C, d["D"], d["z"], d["delta_bias"], None, True, "mamba")[:2]
    torch.cuda.synchronize()
    assert x.shape == rx.shape
    # a product over up to 4160 steps (an exp of an fp32 sum of as many delta') carries up to
    # ~4160 * 2^-24 relative rounding, as the reference's own fp32 running product does
    close(f"x products ({path})", x[..., 0::2], rx[..., 0::2], 2e-3, 1e-6)
    close(f"x states ({path})", x[..., 1::2], rx[..., 1::2], 1e-4, 1e-5)


# zoh and bilinear (fp32) on the fast kernels: the forward in either channel
# form (bilinear never splits L: its A_bar is not exp-form; zoh does on small
# grids), the backward in 32-channel workgroups, unsplit.
@pytest.mark.parametrize("method", ["zoh", "bilinear"])
@pytest.mark.parametrize("schedule", ["default", "unsplit64", "unsplit32"])
def test_zoh_bilinear_fast_path_vs_oracle(dev, monkeypatch, method, schedule):
    if schedule != "default":
        monkeypatch.setenv("LRNNX_SCAN_NO_SPLIT", "1")
        monkeypatch.setenv("LRNNX_SCAN_CHANNELS", schedule[-2:])
    print(f"{method} fast path, {schedule}", flush=True)
    _run(dev, 2, 128, 512, 16, method=method, seed=83)
    _run(dev, 2, 128, 512, 11, method=method, has_z=False, softplus=False, seed=84)


@pytest.mark.parametrize("method", ["zoh", "bilinear"])
@pytest.mark.parametrize("no_split", ["0", "1"])
def test_zoh_bilinear_x_carries_vs_oracle(dev, monkeypatch, method, no_split):
    """out, out_z and both halves of x over three chunks (bilinear's products
    from a running product of A_bar, zoh's from exp(A sum delta'))."""
    from lrnnx_amd import selective_scan_cuda as ssc

    monkeypatch.setenv("LRNNX_SCAN_NO_SPLIT", no_split)
    Bt, D, L = 1, 64, 4160
    inp = R.make_selective_inputs(Bt, D, L, 16, seed=85)
    inp["delta"] = inp["delta"] * 0.1
    ro, rx, roz = R.selective_scan_fwd_ref(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"],
                                           inp["delta_bias"], None, True, method, compute_dtype=torch.float64)
    d = to_dev(inp, dev)
    B, C = d["B"].unsqueeze(1).contiguous(), d["C"].unsqueeze(1).contiguous()
    out, x, out_z = ssc.fwd(d["u"], d["delta"], d["A"], B, C, d["D"], d["z"], d["delta_bias"], None, True, method)[:3]
    torch.cuda.synchronize()
    close(f"out ({method})", out, ro, 1e-4, 1e-5)
    close(f"out_z ({method})", out_z, roz, 1e-4, 1e-5)
    close(f"x products ({method})", x[..., 0::2], rx[..., 0::2], 2e-3, 1e-6)
    close(f"x states ({method})", x[..., 1::2], rx[..., 1::2], 1e-4, 1e-5)


@pytest.mark.parametrize("method", ["zoh", "bilinear"])
def test_zoh_bilinear_fast_forward_matches_generic(dev, monkeypatch, method):
    from lrnnx_amd import selective_scan_cuda as ssc

    inp = R.make_selective_inputs(2, 128, 512, 16, seed=86, groups=2)   # B / C (b, g, n, l)
    d = to_dev(inp, dev)
    res = []
    for generic in ("0", "1"):
        monkeypatch.setenv("LRNNX_SCAN_GENERIC", generic)
        a = ssc.build_args(d["u"], d["delta"], d["A"], d["B"], d["C"], d["D"], d["z"], d["delta_bias"], None, True,
                           method)
        res.append(ssc.run_fwd(a, d["u"], d["delta"], d["A"], d["z"], want_ckpt=True))
        torch.cuda.synchronize()
    for name, f_, g_ in zip(("out", "x", "out_z", "ckpt"), res[0], res[1]):
        close(f"{name} fast vs general ({method})", f_, g_.cpu().double(), 1e-5, 1e-5)


@pytest.mark.parametrize("method", ["zoh", "bilinear"])
@pytest.mark.parametrize("with_z", [True, False])
def test_zoh_bilinear_fast_path_matches_generic(dev, monkeypatch, method, with_z):
    """fwd + bwd of zoh / bilinear on the fast and on the general kernels:
    every output and gradient (fp32 state; sums in another order)."""
    inp = R.make_selective_inputs(2, 128, 512, 16, seed=87, groups=2, has_z=with_z)
    dout = torch.randn(2, 128, 512, generator=torch.Generator().manual_seed(88)).to(dev)
    d = to_dev(inp, dev)
    keys = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias") if with_z else ("u", "delta", "A", "B", "C", "D",
                                                                                  "delta_bias")
    res = []
    for generic in ("0", "1"):
        monkeypatch.setenv("LRNNX_SCAN_GENERIC", generic)
        lv = {k: d[k].clone().requires_grad_(True) for k in keys}
        out, last = selective_scan_fn(lv["u"], lv["delta"], lv["A"], lv["B"], lv["C"], lv["D"], lv.get("z"),
                                      lv["delta_bias"], None, True, True, method)
        out.backward(dout)
        torch.cuda.synchronize()
        res.append([out.detach(), last.detach()] + [lv[k].grad for k in keys])
    names = ["out", "last_state"] + ["d" + k for k in keys]
    for n, a_, b_ in zip(names, res[0], res[1]):
        close(f"{n} fast vs general ({method})", a_, b_.cpu().double(), 1e-5, 1e-5)


@pytest.mark.parametrize("method", ["zoh", "bilinear"])
@pytest.mark.parametrize("no_split", ["0", "1"])
def test_zoh_bilinear_binding_bwd_from_x(dev, monkeypatch, method, no_split):
    """selective_scan_cuda.fwd -> bwd(x, out) in save mode "x": the backward
    rebuilds the checkpoints on the fast states-only forward (zoh: split on
    this small grid or, unsplit, one 2048-step chunk per grid slice from the x
    carries; bilinear never splits) and runs the fast backward."""
    from lrnnx_amd import selective_scan_cuda as ssc

    monkeypatch.setenv("LRNNX_SCAN_NO_SPLIT", no_split)
    prev = ssc.save_mode()
    ssc.set_save_mode("x")
    try:
        Bt, D, L = 1, 64, 4160
        inp = R.make_selective_inputs(Bt, D, L, 16, seed=89)
        dout = torch.randn(Bt, D, L, generator=torch.Generator().manual_seed(90))
        ro, rl, rg = oracle_selective(inp, method, True, None, True, dout)
        d = to_dev(inp, dev)
        u, dl, A, B, C, Dv, z, db = (d[k] for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias"))
        B, C = B.unsqueeze(1).contiguous(), C.unsqueeze(1).contiguous()
        out, x, out_z = ssc.fwd(u, dl, A, B, C, Dv, z, db, None, True, method)[:3]
        g = ssc.bwd(u, dl, A, B, C, Dv, z, db, None, dout.to(dev), x, out, None, True, False, method)
        torch.cuda.synchronize()
    finally:
        ssc.set_save_mode(prev)
    close("out", out_z, ro, 1e-4, 1e-5)
    for i, k in enumerate(("u", "delta", "A", "B", "C", "D", "delta_bias")):
        gk = g[i].squeeze(1) if k in ("B", "C") else g[i]
        close(f"d{k}", gk, rg[k], 1e-4, 1e-4 if k in ("A", "D", "delta_bias") else 1e-5)
    close("dz", g[7], rg["z"], 1e-4, 1e-5)


# d_state 17..32: 8 states per wave in at most 4 waves, with LDS (and, for the
# 16-bit forward, 16-step tiles) sized for 4 waves
@pytest.mark.parametrize("case", [
    ("mamba_bf16", dict(itype=torch.bfloat16)),
    ("mamba_const_bc", dict(varB=False, varC=False)),
    ("mamba_deltaA", dict(with_deltaA=True)),
    ("zoh", dict(method="zoh")),
    ("bilinear_groups", dict(method="bilinear", groups=2)),
], ids=lambda c: c[0])
@pytest.mark.parametrize("N", [24, 32])
def test_dstate_17_to_32_four_waves(dev, case, N):
    _run(dev, 2, 128, 300, N, seed=90 + N, **case[1])
