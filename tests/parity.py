"""Helpers shared by the GPU parity tests: oracle runs (CPU, float64) and
tolerance checks.  The oracle is the checker only."""

from __future__ import annotations

import torch

from oracle import scan_ref as R


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
