"""Helpers shared by the GPU parity tests: oracle runs (CPU, float64) and
tolerance checks.  The oracle is the checker only."""

from __future__ import annotations

import json
import os

import torch

from oracle import scan_ref as R

# north_star's fp32 bound, checked (and reported) for every comparison:
# |got - ref| <= NS_ATOL + NS_RTOL |ref| elementwise, with an absolute atol
NS_RTOL, NS_ATOL = 1e-4, 1e-5


def _report(rec):
    """Append one comparison record to $LRNNX_PARITY_REPORT (JSON lines)."""
    path = os.environ.get("LRNNX_PARITY_REPORT")
    if path:
        with open(path, "a") as fh:
            fh.write(json.dumps(rec) + "\n")


def error_stats(got, ref):
    """max |err|, max |ref|, the largest relative error over elements with
    |ref| >= 1e-2 max|ref|, and the count of elements outside north_star's
    fp32 bound (absolute atol 1e-5, rtol 1e-4)."""
    err = (got - ref).abs()
    aref = ref.abs()
    scale = aref.max().item() if ref.numel() else 0.0
    big = aref >= 1e-2 * scale
    rel = (err[big] / aref[big]).max().item() if big.any() else 0.0
    ns_bad = int((err > NS_ATOL + NS_RTOL * aref).sum())
    return {"max_abs": err.max().item() if err.numel() else 0.0, "max_ref": scale, "max_rel": rel,
            "ns_fp32_out_of_bound": ns_bad, "numel": ref.numel()}


def to_dev(d, dev):
    return {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}


def close(name, got, ref, rtol, atol_rel, atol_abs=0.0):
    """|got - ref| <= atol + rtol |ref| elementwise, atol = max(atol_abs, atol_rel * max|ref|)."""
    if ref is None:  # the oracle does not depend on this input: the gradient must be zero
        g = got.detach().cpu()
        if g.abs().max().item() != 0.0:
            raise AssertionError(f"{name}: expected an all-zero gradient, max |got| = {g.abs().max().item()}")
        return 0.0
    got = got.detach().cpu().to(ref.dtype)
    ref = ref.detach().cpu()
    scale = ref.abs().max().item() if ref.numel() else 0.0
    atol = max(atol_abs, atol_rel * scale)
    err = (got - ref).abs()
    bad = err > atol + rtol * ref.abs()
    if os.environ.get("LRNNX_PARITY_REPORT"):
        rec = error_stats(got, ref)
        rec.update(name=name, test=os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0], rtol=rtol, atol=atol)
        _report(rec)
    if bad.any():
        i = bad.flatten().nonzero()[0].item()
        raise AssertionError(
            f"{name}: {int(bad.sum())}/{bad.numel()} elements out of tolerance "
            f"(rtol={rtol}, atol={atol:.3g}); max abs err {err.max().item():.3g}, "
            f"first bad flat index {i}: got {got.flatten()[i].item()} ref {ref.flatten()[i].item()}")
    return err.max().item()


def oracle_selective(inp, method="mamba", softplus=True, deltaA=None, grads=True, dout=None):
    """fp64 oracle forward (+ autograd gradients) on the CPU copies of `inp`."""
    leaves = {}
    for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias"):
        v = inp.get(k)
        if v is None:
            continue
        t = v.detach().cpu()
        t = t.to(torch.complex128) if t.is_complex() else t.double()
        leaves[k] = t.requires_grad_(grads)
    dA_ = None
    if deltaA is not None:
        dA_ = deltaA.detach().cpu().double().requires_grad_(grads)
    out, last = R.selective_scan_ref(
        leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"], leaves.get("D"), leaves.get("z"),
        leaves.get("delta_bias"), dA_, softplus, True, method, compute_dtype=torch.float64)
    g = {}
    if grads:
        out.backward(dout.detach().cpu().double())
        g = {k: v.grad for k, v in leaves.items()}
        if dA_ is not None:
            g["deltaA"] = dA_.grad
    return out.detach(), last.detach(), g


def close_dev(name, got, ref, rtol, atol_rel, atol_abs=0.0):
    """``close`` for full-size tensors: the float64 reference is moved to the
    device of ``got`` and compared there (the same bound: |got - ref| <=
    atol + rtol |ref| with atol = max(atol_abs, atol_rel max|ref|)).  Returns
    error_stats."""
    ref = ref.to(got.device, torch.float64)
    got = got.detach().to(torch.float64)
    st = error_stats(got, ref)
    atol = max(atol_abs, atol_rel * st["max_ref"])
    err = (got - ref).abs()
    bad = err > atol + rtol * ref.abs()
    n_bad = int(bad.sum())
    st.update(name=name, test=os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0], rtol=rtol, atol=atol)
    _report(st)
    print(f"  {name:12s} max|err| {st['max_abs']:.3e}  max|ref| {st['max_ref']:.3e}  max rel (|ref| >= 1% max) "
          f"{st['max_rel']:.3e}  outside fp32 north-star bound {st['ns_fp32_out_of_bound']}/{st['numel']}",
          flush=True)
    if n_bad:
        i = bad.flatten().nonzero()[0].item()
        raise AssertionError(
            f"{name}: {n_bad}/{bad.numel()} elements out of tolerance (rtol={rtol}, atol={atol:.3g}); "
            f"max abs err {st['max_abs']:.3g}, first bad flat index {i}: got {got.flatten()[i].item()} "
            f"ref {ref.flatten()[i].item()}")
    return st
