"""GPU parity at the grids the bench times, against the float64 C oracle
(oracle/selective_scan_ref.c, pinned in tests/test_oracle.py against fp64
autograd of the restated selective_scan_ref, lrnnx/ops/selective_scan.py:
200-360).

* Config 3 (B=8, D=4096, L=4096, N=16, G=1, bf16; 512 workgroups) and
  config 2 (B=8, D=1536, L=2048; 192 workgroups) in full: every output and
  gradient of ``selective_scan_fn`` on every element.
* Grids just above the 128-workgroup split limit (unsplit fast kernels at
  moderate L): bf16 B=3 D=2816 L=1024 and fp32 B=2 D=4160 L=512.
* d_state 24 / 64 (bf16) and 32 / 48 (fp32) on the general kernels at 512
  workgroups (B=8 D=4096 L=256).
* The small-grid split of L against the unsplit schedule
  (LRNNX_SCAN_NO_SPLIT=1) at B=1 D=64 L=4160, both against the oracle.
* 64 and 32 channels per workgroup (LRNNX_SCAN_CHANNELS) on one unsplit grid, both forms
  with d_state 1, 3, 8, 9 and 13 (waves whose states are all or part padding), and the
  32-channel form with padded states, groups and several chunk ends.
* The binding's own call sequence ``selective_scan_cuda.fwd`` -> ``bwd(x)``
  in both save modes: "checkpoints" (fwd attaches them to x) and "x" (the
  backward rebuilds them: split on small grids, one 2048-step chunk per grid
  slice from the x carries on long sequences, one pass otherwise); the
  autograd path in the "x" mode at config 2.

Tolerance, elementwise |got - ref| <= atol + rtol |ref|:
  fp32 I/O: north_star's bound as stated, rtol 1e-4 and an absolute atol of
  1e-5, on every output and every gradient; for the gradients summed over
  batch and length (dA, dD, ddelta_bias) atol is max(1e-5, 1e-6 max|ref|):
  a sum of B L fp32 terms that cancels to a small value carries rounding in
  proportion to the sum of the terms' magnitudes, not to its own value (the
  report still counts every element outside the plain bound);
  bf16 I/O (fp32 state): rtol 2e-2, atol 1e-2 max|ref| of the tensor (the
  outputs are rounded to bf16, a relative step of 2^-8).
Each comparison also prints (and with $LRNNX_PARITY_REPORT set, records) the
max abs / rel error and the count of elements outside the fp32 bound.
"""

import pytest
import torch

import bench
from lrnnx_amd import selective_scan_cuda as ssc
from lrnnx_amd import selective_scan_fn
from oracle import fast as OF
from oracle import scan_ref as R
from tests.parity import close, close_dev, oracle_selective, to_dev

pytestmark = pytest.mark.gpu

_REDUCED = ("dA", "dD", "ddelta_bias", "dB", "dC")


@pytest.fixture(params=["checkpoints", "x"])
def save_mode(request):
    prev = ssc.save_mode()
    ssc.set_save_mode(request.param)
    yield request.param
    ssc.set_save_mode(prev)


def _tol(itype):
    """(rtol, atol relative to max|ref|, absolute atol)"""
    return (1e-4, 0.0, 1e-5) if itype == torch.float32 else (2e-2, 1e-2, 0.0)


def _gpu_inputs(dev, Bt, D, L, N, seed, itype):
    inp = bench.make_cfg3(dev, torch, None, Bt, D, L, N, seed=seed, io=itype)
    return inp


def _oracle(inp):
    return OF.selective_scan_mamba(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"],
                                   inp["delta_bias"], True, inp["dout"])


def _run_fn(inp):
    """selective_scan_fn fwd + bwd (the autograd drop-in path)."""
    lv = {k: (inp[k].clone().requires_grad_(True) if inp[k] is not None else None)
          for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")}
    out, last = selective_scan_fn(lv["u"], lv["delta"], lv["A"], lv["B"], lv["C"], lv["D"], lv["z"],
                                  lv["delta_bias"], None, True, True, "mamba")
    out.backward(inp["dout"])
    torch.cuda.synchronize()
    res = {"out": out.detach(), "last_state": last.detach()}
    for k, gk in (("u", "du"), ("delta", "ddelta"), ("A", "dA"), ("B", "dB"), ("C", "dC"), ("D", "dD"),
                  ("z", "dz"), ("delta_bias", "ddelta_bias")):
        res[gk] = lv[k].grad if lv[k] is not None else None
    return res


_SUMMED = ("dA", "dD", "ddelta_bias")


def _tol_of(name, itype):
    """_tol, with the fp32 absolute term of the batch- and length-summed
    gradients relative to the tensor's magnitude."""
    rt, at, aa = _tol(itype)
    if itype == torch.float32 and name.split(" ")[0] in _SUMMED:
        at = 1e-6
    return rt, at, aa


def _compare(got, ref, itype):
    for name in ("out", "last_state", "du", "ddelta", "dz", "dA", "dB", "dC", "dD", "ddelta_bias"):
        close_dev(name, got[name], ref[name], *_tol_of(name, itype))


@pytest.mark.parametrize("case", [
    # (name, B, D, L, seed, itype): configs 2 and 3 of the benchmark, then grids just above 128 workgroups
    ("cfg3", 8, 4096, 4096, 3, torch.bfloat16),
    ("cfg2", 8, 1536, 2048, 2, torch.bfloat16),
    ("grid132", 3, 2816, 1024, 7, torch.bfloat16),
    ("grid130_f32", 2, 4160, 512, 8, torch.float32),
], ids=lambda c: c[0])
def test_full_grid_vs_oracle(dev, case):
    _full_grid(dev, case)


@pytest.mark.parametrize("N,itype", [(24, torch.bfloat16), (32, torch.float32), (48, torch.float32), (64, torch.bfloat16)],
                         ids=["n24_bf16", "n32_f32", "n48_f32", "n64_bf16"])
def test_general_dstate_large_grid_vs_oracle(dev, N, itype):
    """d_state 17..64 on the general kernels on a 512-workgroup grid, every
    element: 17..32 in 4-wave workgroups (two per CU), 33..64 in 8-wave ones
    (fp32: 32-step forward and 16-step backward tiles)."""
    _full_grid(dev, (f"general_n{N}", 8, 4096, 256, 11, itype), N=N)


def test_cfg2_autograd_save_x_vs_oracle(dev):
    """SelectiveScanFn keeping only x (the reference's saved state): the
    backward rebuilds the checkpoints."""
    prev = ssc.save_mode()
    ssc.set_save_mode("x")
    try:
        _full_grid(dev, ("cfg2_save_x", 8, 1536, 2048, 2, torch.bfloat16))
    finally:
        ssc.set_save_mode(prev)


def _full_grid(dev, case, N=16):
    name, Bt, D, L, seed, itype = case
    print(f"[{name}] B={Bt} D={D} L={L} N={N} {itype} seed={seed}: GPU fwd+bwd", flush=True)
    inp = _gpu_inputs(dev, Bt, D, L, N, seed, itype)
    got = _run_fn(inp)
    print(f"[{name}] oracle (C, fp64, {OF.lib().lrnnx_oracle_ss_threads()} threads)", flush=True)
    ref = _oracle(inp)
    _compare(got, ref, itype)


@pytest.mark.parametrize("itype", [torch.float32, torch.bfloat16])
def test_small_grid_split_and_unsplit_vs_oracle(dev, monkeypatch, itype):
    """B=1, D=64 is one workgroup: by default both directions split L into
    segments; LRNNX_SCAN_NO_SPLIT=1 runs the unsplit kernels.  Both schedules
    match the oracle, and each other."""
    inp = _gpu_inputs(dev, 1, 64, 4160, 16, 21, itype)
    ref = _oracle(inp)
    res = {}
    for mode in ("split", "unsplit"):
        monkeypatch.setenv("LRNNX_SCAN_NO_SPLIT", "1" if mode == "unsplit" else "0")
        print(f"[{mode}] {itype}", flush=True)
        res[mode] = _run_fn(inp)
        _compare(res[mode], ref, itype)
    for name in res["split"]:
        close_dev(f"{name} split/unsplit", res["split"][name], res["unsplit"][name].double(), *_tol_of(name, itype))


def _binding_fwd_bwd(inp, method="mamba", softplus=True):
    """selective_scan_cuda.fwd then bwd with the forward's x and out, as the
    reference's SelectiveScanFn calls them (selective_scan.py:70-82, :116-135)."""
    u, dl, A, B, C, D, z, db = (inp.get(k) for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias"))
    r = ssc.fwd(u, dl, A, B, C, D, z, db, None, softplus, method)
    out, x = r[0], r[1]
    g = ssc.bwd(u, dl, A, B, C, D, z, db, None, inp["dout"], x, out, None, softplus, False, method)
    torch.cuda.synchronize()
    res = {"out": r[2] if z is not None else out, "last_state": x[:, :, -1, 1::2],
           "du": g[0], "ddelta": g[1], "dA": g[2], "dB": g[3], "dC": g[4], "dD": g[5], "ddelta_bias": g[6]}
    if z is not None:
        res["dz"] = g[7]
    return res


@pytest.mark.parametrize("case", [
    ("small_f32", 2, 64, 512, torch.float32),
    ("small_bf16", 2, 64, 512, torch.bfloat16),
    ("small_long_bf16", 1, 64, 4160, torch.bfloat16),
    ("grid132_bf16", 3, 2816, 1024, torch.bfloat16),
    ("grid132_long_bf16", 3, 2816, 4160, torch.bfloat16),
    ("grid130_f32", 2, 4160, 256, torch.float32),
], ids=lambda c: c[0])
def test_binding_fwd_then_bwd_x_vs_oracle(dev, case, save_mode):
    """The boundary's own sequence, the path the reference's SelectiveScanFn,
    S7ScanFn and RGLRUScanFn take after the import swap: bwd gets x and out."""
    name, Bt, D, L, itype = case
    inp = _gpu_inputs(dev, Bt, D, L, 16, 31, itype)
    print(f"[{name}] fwd -> bwd(x), save mode {save_mode}", flush=True)
    got = _binding_fwd_bwd(inp)
    ref = _oracle(inp)
    _compare(got, ref, itype)


@pytest.mark.parametrize("method", ["rglru", "s7"])
def test_binding_fwd_then_bwd_x_one_state_methods(dev, method, save_mode):
    """The S7 / RG-LRU wrappers' binding calls (N = 1, constant B / C, fp32)
    through fwd -> bwd(x), against fp64 autograd of the restated oracle."""
    g = torch.Generator().manual_seed(41)
    Bt, D, L = 2, 96, 700
    inp = R.make_selective_inputs(Bt, D, L, 1, seed=41, varB=False, varC=False, has_z=False, has_D=True,
                                  has_bias=False)
    inp["delta"] = inp["delta"].abs() * 0.2 + 1e-3
    if method == "rglru":
        inp["A"] = torch.rand(D, 1, generator=g) * 0.5 + 0.45
    dout = torch.randn(Bt, D, L, generator=g)
    ro, rl, rg = oracle_selective(inp, method, False, None, True, dout)
    d = to_dev(inp, dev)
    d["dout"] = dout.to(dev)
    got = _binding_fwd_bwd(d, method, softplus=False)
    close("out", got["out"], ro, 1e-4, 1e-5)
    for k, gk in (("u", "du"), ("delta", "ddelta"), ("A", "dA"), ("B", "dB"), ("C", "dC"), ("D", "dD")):
        close(gk, got[gk], rg[k], 1e-4, 1e-4 if gk in _REDUCED else 1e-5)


@pytest.mark.parametrize("itype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_z", [True, False])
def test_channels_per_workgroup_64_and_32_vs_oracle(dev, monkeypatch, itype, with_z):
    """The fast forward with 64 channels per workgroup (lane = channel, 4
    states per lane) and with 32 (two lane halves of 2 states; the default
    for grids of at most 256 64-channel workgroups), forced by
    LRNNX_SCAN_CHANNELS on the same unsplit grid, against the oracle and each
    other (fwd + bwd through selective_scan_fn)."""
    inp = _gpu_inputs(dev, 2, 128, 4160, 16, 23, itype)
    if not with_z:
        inp["z"] = None
    ref = OF.selective_scan_mamba(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"],
                                  inp["delta_bias"], True, inp["dout"])
    monkeypatch.setenv("LRNNX_SCAN_NO_SPLIT", "1")
    rt, at, aa = _tol(itype)
    res = {}
    for chans in ("64", "32"):
        monkeypatch.setenv("LRNNX_SCAN_CHANNELS", chans)
        print(f"[channels {chans}] {itype} z={with_z}", flush=True)
        res[chans] = _run_fn(inp)
        names = ["out", "last_state", "du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias"] + (["dz"] if with_z else [])
        for name in names:
            close_dev(f"{name} channels={chans}", res[chans][name], ref[name], *_tol_of(name, itype))
    for name in res["64"]:
        if res["64"][name] is not None:
            close_dev(f"{name} 32 vs 64 channels", res["32"][name], res["64"][name].double(), *_tol_of(name, itype))


@pytest.mark.parametrize("itype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N", [1, 3, 8, 9, 13])
@pytest.mark.parametrize("chans", ["64", "32"])
def test_partially_padded_wave_states_vs_oracle(dev, monkeypatch, itype, N, chans):
    """d_state 9 and 13: one wave's four states are part real, part padding;
    1, 3 and 8: whole waves hold padding only; in both channel forms
    (LRNNX_SCAN_CHANNELS).  The backward's dB / dC
    reduce-scatter gives each lane its states in a lane-dependent register
    order, so real and padded states share registers across lanes, and a
    lane writes its partial only where the state it ends with is real."""
    monkeypatch.setenv("LRNNX_SCAN_NO_SPLIT", "1")
    monkeypatch.setenv("LRNNX_SCAN_CHANNELS", chans)
    inp = _gpu_inputs(dev, 2, 128, 512, N, 41 + N, itype)
    ref = _oracle(inp)
    print(f"[padded states] N={N} channels={chans} {itype}", flush=True)
    got = _run_fn(inp)
    for name in ("out", "last_state", "du", "ddelta", "dz", "dA", "dB", "dC", "dD", "ddelta_bias"):
        close_dev(f"{name} N={N} channels={chans}", got[name], ref[name], *_tol_of(name, itype))


@pytest.mark.parametrize("itype", [torch.float32, torch.bfloat16])
def test_channels_32_d_state_and_chunks_vs_oracle(dev, monkeypatch, itype):
    """32-channel workgroups with fewer than 16 states (padded states in both
    lane halves), a group count of 2 and a length past two 2048-step chunk
    ends (x carries of every chunk), against the oracle."""
    monkeypatch.setenv("LRNNX_SCAN_NO_SPLIT", "1")
    monkeypatch.setenv("LRNNX_SCAN_CHANNELS", "32")
    inp = R.make_selective_inputs(2, 128, 4160, 12, seed=33, itype=itype, groups=2)
    dout = torch.randn(2, 128, 4160, generator=torch.Generator().manual_seed(34)).to(itype)
    ref = OF.selective_scan_mamba(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"],
                                  inp["delta_bias"], True, dout)
    d = {k: v.to(dev) for k, v in inp.items()}
    d["dout"] = dout.to(dev)
    rt, at, aa = _tol(itype)
    got = _run_fn(d)
    for name in ("out", "last_state", "du", "ddelta", "dz", "dA", "dB", "dC", "dD", "ddelta_bias"):
        close_dev(f"{name} 32ch N=12 G=2", got[name], ref[name], *_tol_of(name, itype))
    # the x carries of both chunk ends, through the binding
    u, dl, A, B, C, D, z, db = (d.get(k) for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias"))
    x = ssc.fwd(u, dl, A, B, C, D, z, db, None, True, "mamba")[1]
    ro = OF.selective_scan_mamba(inp["u"][..., :4096], inp["delta"][..., :4096], inp["A"], inp["B"][..., :4096],
                                 inp["C"][..., :4096], inp["D"], inp["z"][..., :4096], inp["delta_bias"], True)
    close_dev("x carry h at 4096, 32ch", x[:, :, 1, 1::2], ro["last_state"], rt, at, aa)


def test_bf16_length_16_mod_32_vs_oracle(dev):
    """bf16 with L = 16 (mod 32): the fast forward needs L % 32 == 0 and the
    general forward runs; the fast backward takes its one-tile raw fetches
    (the two-tile form needs an even tile count)."""
    inp = _gpu_inputs(dev, 2, 128, 1040, 16, 29, torch.bfloat16)
    ref = _oracle(inp)
    _compare(_run_fn(inp), ref, torch.bfloat16)
