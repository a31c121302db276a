"""Golden fixtures (tests/golden/*.pt, written by tests/golden/make_golden.py
from the pinned float64 oracle): the oracle must keep reproducing them (CPU),
and the HIP kernels must match them (GPU, fp32 kernels vs float64 values:
rtol 1e-4, atol 1e-5 * max|ref|; gradients that sum over batch x length
atol 1e-4 * max|ref|)."""

import glob
import os

import pytest
import torch

from oracle import scan_ref as R
from tests.parity import close

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SEL = sorted(glob.glob(os.path.join(HERE, "selective_*.pt")))
SIMP = sorted(glob.glob(os.path.join(HERE, "simplified_*.pt")))
SU = sorted(glob.glob(os.path.join(HERE, "state_update_*.pt")))
S5U = sorted(glob.glob(os.path.join(HERE, "s5_state_update_*.pt")))


def _load(p):
    return torch.load(p, weights_only=True)


def _sel_oracle(rec):
    i = {k: v.clone().requires_grad_(True) for k, v in rec["inputs"].items()}
    out, last = R.selective_scan_ref(i["u"], i["delta"], i["A"], i["B"], i["C"], i["D"], i["z"], i["delta_bias"],
                                     i.get("deltaA"), True, True, rec["meta"]["method"], compute_dtype=torch.float64)
    out.backward(rec["dout"])
    return out, last, i


@pytest.mark.parametrize("path", SEL, ids=[os.path.basename(p) for p in SEL])
def test_oracle_reproduces_selective_fixture(path):
    rec = _load(path)
    out, last, i = _sel_oracle(rec)
    assert torch.equal(out.detach(), rec["out"])
    assert torch.equal(last.detach(), rec["last_state"])
    for k, v in i.items():
        g = v.grad if v.grad is not None else torch.zeros_like(v)
        assert torch.equal(g, rec["grads"][k]), k


@pytest.mark.parametrize("path", SIMP, ids=[os.path.basename(p) for p in SIMP])
def test_oracle_reproduces_simplified_fixture(path):
    rec = _load(path)
    i = {k: v.clone().requires_grad_(True) for k, v in rec["inputs"].items()}
    y, last = R.simplified_scan_ref(i["u"], i["delta"], i["A"], i["B"], i["C"], deltaA=i.get("deltaA"),
                                    return_last_state=True, discretization=rec["meta"]["method"],
                                    compute_dtype=torch.float64)
    y.backward(rec["dout"])
    assert torch.equal(y.detach(), rec["out"]) and torch.equal(last.detach(), rec["last_state"])


@pytest.mark.parametrize("path", SU, ids=[os.path.basename(p) for p in SU])
def test_oracle_reproduces_state_update_fixture(path):
    rec = _load(path)
    i = rec["inputs"]
    st = i["state"].clone()
    out = R.selective_state_update_ref(st, i["x"], i["dt"], i["A"], i["B"], i["C"], i["D"], i["z"], i["dt_bias"],
                                       True, None, rec["meta"]["method"], compute_dtype=torch.float64)
    assert torch.equal(out, rec["out"]) and torch.equal(st, rec["state_after"])


@pytest.mark.parametrize("path", S5U, ids=[os.path.basename(p) for p in S5U])
def test_oracle_reproduces_s5_state_update_fixture(path):
    rec = _load(path)
    i = rec["inputs"]
    st = i["state"].clone()
    out = R.simplified_state_update_ref(st, i["x"], i["dt"], i["A"], i["B"], i["C"], i.get("D"), i.get("deltaA"),
                                        rec["meta"]["method"], rec["meta"]["conj_sym"], compute_dtype=torch.float64)
    assert torch.equal(out, rec["out"]) and torch.equal(st, rec["state_after"])


# ---------------------------------------------------------------- GPU side
def _f32(t, dev):
    t = t.to(torch.complex64) if t.is_complex() else t.float()
    return t.to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize("path", SEL, ids=[os.path.basename(p) for p in SEL])
def test_kernel_matches_selective_fixture(dev, path):
    from lrnnx_amd import selective_scan_fn

    rec = _load(path)
    i = {k: _f32(v, dev).requires_grad_(True) for k, v in rec["inputs"].items()}
    out, last = selective_scan_fn(i["u"], i["delta"], i["A"], i["B"], i["C"], i["D"], i["z"], i["delta_bias"],
                                  i.get("deltaA"), True, True, rec["meta"]["method"])
    out.backward(_f32(rec["dout"], dev))
    torch.cuda.synchronize()
    close("out", out, rec["out"], 1e-4, 1e-5)
    close("last_state", last, rec["last_state"], 1e-4, 1e-5)
    varB, varC = rec["inputs"]["B"].dim() >= 3, rec["inputs"]["C"].dim() >= 3
    for k, v in i.items():
        red = k in ("A", "D", "delta_bias") or (k == "B" and not varB) or (k == "C" and not varC)
        close(f"d{k}", v.grad, rec["grads"][k], 1e-4, 1e-4 if red else 1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("path", SIMP, ids=[os.path.basename(p) for p in SIMP])
def test_kernel_matches_simplified_fixture(dev, path):
    from lrnnx_amd import simplified_scan_fn

    rec = _load(path)
    i = {k: _f32(v, dev).requires_grad_(True) for k, v in rec["inputs"].items()}
    y, last = simplified_scan_fn(i["u"], i["delta"], i["A"], i["B"], i["C"], deltaA=i.get("deltaA"),
                                 return_last_state=True, discretization=rec["meta"]["method"])
    y.backward(_f32(rec["dout"], dev))
    torch.cuda.synchronize()
    close("y", y, rec["out"], 1e-4, 1e-5)
    close("last_state", last, rec["last_state"], 1e-4, 1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("path", SU, ids=[os.path.basename(p) for p in SU])
def test_kernel_matches_state_update_fixture(dev, path):
    from lrnnx_amd import selective_state_update

    rec = _load(path)
    i = {k: _f32(v, dev) for k, v in rec["inputs"].items()}
    st = i["state"].clone()
    out = selective_state_update(st, i["x"], i["dt"], i["A"], i["B"], i["C"], i["D"], i["z"], i["dt_bias"], True,
                                 None, None, rec["meta"]["method"])
    torch.cuda.synchronize()
    close("out", out, rec["out"], 1e-4, 1e-5)
    close("state", st, rec["state_after"], 1e-4, 1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("path", S5U, ids=[os.path.basename(p) for p in S5U])
def test_kernel_matches_s5_state_update_fixture(dev, path):
    from lrnnx_amd import simplified_state_update

    rec = _load(path)
    i = {k: _f32(v, dev) for k, v in rec["inputs"].items()}
    st = i["state"].clone()
    out = simplified_state_update(st, i["x"], i["dt"], i["A"], i["B"], i["C"], i.get("D"), i.get("deltaA"),
                                  rec["meta"]["method"], rec["meta"]["conj_sym"])
    torch.cuda.synchronize()
    close("out", out, rec["out"], 1e-4, 1e-5)
    close("state", st, rec["state_after"], 1e-4, 1e-5)
