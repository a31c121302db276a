"""Write the golden fixtures of tests/golden/ from the float64 oracle.

The reference ships no golden vectors for the scan path (its tests compare the
CUDA op with *_ref at run time), so these fixtures are produced by the
restated oracle after tests/test_oracle.py has pinned it (brute force, closed
forms, lfilter, invariants, gradcheck).  They freeze inputs and expected
outputs / gradients independently of the torch RNG stream.

    python tests/golden/make_golden.py
"""

import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import scan_ref as R  # noqa: E402

D64 = torch.float64


def selective_case(name, method, cplx=False, varB=True, varC=True, b=2, d=8, L=37, n=4, seed=0, deltaA=False):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(b, d, L, generator=g, dtype=D64)
    delta = 0.5 * torch.randn(b, d, L, generator=g, dtype=D64)
    z = torch.randn(b, d, L, generator=g, dtype=D64)
    Dv = torch.randn(d, generator=g, dtype=D64)
    bias = -2.0 + 0.3 * torch.randn(d, generator=g, dtype=D64)
    A = (torch.rand(d, n, generator=g, dtype=D64) * 0.5 + 0.4) if method == "rglru" else \
        -(torch.arange(1, n + 1, dtype=D64).repeat(d, 1) * (0.5 + torch.rand(d, 1, generator=g, dtype=D64)))
    if cplx:
        A = torch.complex(A, torch.randn(d, n, generator=g, dtype=D64))
    Lb = 2 * L if cplx else L
    B = torch.randn(b, 1, n, Lb, generator=g, dtype=D64) if varB else torch.randn(d, n, dtype=A.dtype, generator=g)
    C = torch.randn(b, 1, n, Lb, generator=g, dtype=D64) if varC else torch.randn(d, n, dtype=A.dtype, generator=g)
    dA = torch.rand(b, d, L, generator=g, dtype=D64) if deltaA else None
    dout = torch.randn(b, d, L, generator=g, dtype=D64)
    leaves = dict(u=u, delta=delta, A=A, B=B, C=C, D=Dv, z=z, delta_bias=bias)
    if dA is not None:
        leaves["deltaA"] = dA
    lv = {k: v.clone().requires_grad_(True) for k, v in leaves.items()}
    out, last = R.selective_scan_ref(lv["u"], lv["delta"], lv["A"], lv["B"], lv["C"], lv["D"], lv["z"],
                                     lv["delta_bias"], lv.get("deltaA"), True, True, method, compute_dtype=D64)
    out.backward(dout)
    rec = {"inputs": leaves, "dout": dout, "out": out.detach(), "last_state": last.detach(),
           "grads": {k: (v.grad if v.grad is not None else torch.zeros_like(v)) for k, v in lv.items()},
           "meta": {"method": method, "delta_softplus": True}}
    torch.save(rec, os.path.join(HERE, name + ".pt"))


def simplified_case(name, method, b=2, H=3, P=4, L=41, seed=1, deltaA=False):
    g = torch.Generator().manual_seed(seed)
    u = torch.complex(torch.randn(b, H, L, generator=g, dtype=D64), torch.randn(b, H, L, generator=g, dtype=D64))
    delta = 0.1 + 0.2 * torch.rand(b, P, L, generator=g, dtype=D64)
    A = torch.complex(-0.5 - torch.rand(P, generator=g, dtype=D64), torch.randn(P, generator=g, dtype=D64))
    Bm = torch.complex(torch.randn(P, H, generator=g, dtype=D64), torch.randn(P, H, generator=g, dtype=D64))
    Cm = torch.complex(torch.randn(H, P, generator=g, dtype=D64), torch.randn(H, P, generator=g, dtype=D64))
    dA = 0.1 + 0.2 * torch.rand(b, P, L, generator=g, dtype=D64) if deltaA else None
    dout = torch.complex(torch.randn(b, H, L, generator=g, dtype=D64), torch.randn(b, H, L, generator=g, dtype=D64))
    leaves = dict(u=u, delta=delta, A=A, B=Bm, C=Cm)
    if dA is not None:
        leaves["deltaA"] = dA
    lv = {k: v.clone().requires_grad_(True) for k, v in leaves.items()}
    y, last = R.simplified_scan_ref(lv["u"], lv["delta"], lv["A"], lv["B"], lv["C"], deltaA=lv.get("deltaA"),
                                    return_last_state=True, discretization=method, compute_dtype=D64)
    y.backward(dout)
    rec = {"inputs": leaves, "dout": dout, "out": y.detach(), "last_state": last.detach(),
           "grads": {k: (v.grad if v.grad is not None else torch.zeros_like(v)) for k, v in lv.items()},
           "meta": {"method": method}}
    torch.save(rec, os.path.join(HERE, name + ".pt"))


def state_update_case(name, method, seed=2):
    g = torch.Generator().manual_seed(seed)
    b, d, n = 3, 16, 8
    state = torch.randn(b, d, n, generator=g, dtype=D64)
    x, dt = torch.randn(b, d, generator=g, dtype=D64), 0.5 * torch.randn(b, d, generator=g, dtype=D64)
    A = (torch.rand(d, n, generator=g, dtype=D64) * 0.5 + 0.4) if method == "rglru" else \
        -torch.rand(d, n, generator=g, dtype=D64) - 0.5
    Bm, Cm = torch.randn(b, n, generator=g, dtype=D64), torch.randn(b, n, generator=g, dtype=D64)
    Dv, z = torch.randn(d, generator=g, dtype=D64), torch.randn(b, d, generator=g, dtype=D64)
    bias = 0.1 * torch.randn(d, generator=g, dtype=D64)
    st = state.clone()
    out = R.selective_state_update_ref(st, x, dt, A, Bm, Cm, Dv, z, bias, True, None, method, compute_dtype=D64)
    rec = {"inputs": dict(state=state, x=x, dt=dt, A=A, B=Bm, C=Cm, D=Dv, z=z, dt_bias=bias), "out": out,
           "state_after": st, "meta": {"method": method, "dt_softplus": True}}
    torch.save(rec, os.path.join(HERE, name + ".pt"))


def simplified_state_update_case(name, method, seed, deltaA=False, D=True, dt_per_state=False):
    g = torch.Generator().manual_seed(seed)
    b, H, P = 3, 20, 12
    cplx = lambda *shape: torch.complex(torch.randn(*shape, generator=g, dtype=D64),
                                        torch.randn(*shape, generator=g, dtype=D64))
    state = cplx(b, P)
    x = torch.randn(b, H, generator=g, dtype=D64)
    dt = 0.05 + 0.2 * torch.rand(*((P,) if dt_per_state else (b, P)), generator=g, dtype=D64)
    A = torch.complex(-0.2 - torch.rand(P, generator=g, dtype=D64), torch.randn(P, generator=g, dtype=D64))
    Bm, Cm = cplx(P, H) / H ** 0.5, cplx(H, P) / P ** 0.5
    Dm = torch.randn(H, H, generator=g, dtype=D64) / H ** 0.5 if D else None
    dA = 0.05 + 0.2 * torch.rand(b, P, generator=g, dtype=D64) if deltaA else None
    st = state.clone()
    out = R.simplified_state_update_ref(st, x, dt, A, Bm, Cm, Dm, dA, method, True, compute_dtype=D64)
    inputs = dict(state=state, x=x, dt=dt, A=A, B=Bm, C=Cm)
    if Dm is not None:
        inputs["D"] = Dm
    if dA is not None:
        inputs["deltaA"] = dA
    rec = {"inputs": inputs, "out": out, "state_after": st, "meta": {"method": method, "conj_sym": True}}
    torch.save(rec, os.path.join(HERE, name + ".pt"))


def main():
    selective_case("selective_mamba_var", "mamba")
    selective_case("selective_mamba_const_deltaA", "mamba", varB=False, varC=False, deltaA=True, seed=3)
    selective_case("selective_zoh_mixed", "zoh", varB=True, varC=False, seed=4)
    selective_case("selective_bilinear_mixed", "bilinear", varB=False, varC=True, seed=5)
    selective_case("selective_dirac_var", "dirac", seed=6)
    selective_case("selective_mamba_complex_const", "mamba", cplx=True, varB=False, varC=False, seed=7)
    selective_case("selective_mamba_complex_var", "mamba", cplx=True, seed=8)
    selective_case("selective_s7", "s7", varB=False, varC=False, n=1, seed=9)
    selective_case("selective_rglru", "rglru", varB=False, varC=False, n=2, seed=10)
    for m in ("bilinear", "zoh", "dirac"):
        simplified_case(f"simplified_{m}", m, seed=11)
    simplified_case("simplified_zoh_deltaA", "zoh", seed=12, deltaA=True)
    for m in ("mamba", "zoh", "bilinear", "dirac", "s7", "rglru"):
        state_update_case(f"state_update_{m}", m)
    simplified_state_update_case("s5_state_update_bilinear", "bilinear", seed=15)
    simplified_state_update_case("s5_state_update_zoh_deltaA", "zoh", seed=16, deltaA=True, dt_per_state=True)
    simplified_state_update_case("s5_state_update_dirac_noD", "dirac", seed=17, D=False)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
