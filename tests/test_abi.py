"""CPU tests of the drop-in boundary: the C ABI library loads, exports every
symbol include/lrnnx_scan.h declares, its structs have the layout the
Python binding assumes, argument checks fail with the reference's messages
(host code only, no GPU call), and the Python API refuses CPU tensors
(there is no CPU fallback)."""

import ctypes
import os
import re
import subprocess
import tempfile

import pytest
import torch

from lrnnx_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lrnnx_scan.h")


def _declared_functions():
    src = open(HEADER).read()
    decl = re.compile(r"^\s*(?:const\s+)?(?:int|int64_t|char|void)\s*\*?\s*(lrnnx_[a-z0-9_]+)\s*\(", re.M)
    return sorted(set(decl.findall(src)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = _declared_functions()
    assert len(names) >= 11
    for n in names:
        assert hasattr(L, n), f"{n} declared in lrnnx_scan.h but not exported"
    assert set(_lib.EXPORTS) <= set(names)
    assert L.lrnnx_abi_version() == _lib.ABI_VERSION


def test_struct_layout_matches_c():
    prog = r'''
#include <stdio.h>
#include <stddef.h>
#include "lrnnx_scan.h"
int main(void) {
  printf("%zu %zu %zu %zu\n", sizeof(lrnnx_view), sizeof(lrnnx_selective_scan_args),
         sizeof(lrnnx_simplified_scan_args), sizeof(lrnnx_state_update_args));
  printf("%zu %zu %zu %zu %zu\n", offsetof(lrnnx_selective_scan_args, u), offsetof(lrnnx_selective_scan_args, x),
         offsetof(lrnnx_selective_scan_args, dout), offsetof(lrnnx_selective_scan_args, workspace),
         offsetof(lrnnx_selective_scan_args, dz));
  printf("%zu %zu %zu\n", offsetof(lrnnx_simplified_scan_args, x), offsetof(lrnnx_simplified_scan_args, dout),
         offsetof(lrnnx_simplified_scan_args, workspace_bytes));
  printf("%zu %zu %zu\n", offsetof(lrnnx_state_update_args, state), offsetof(lrnnx_state_update_args, deltaA),
         offsetof(lrnnx_state_update_args, out_s2));
  printf("%zu %zu %zu %zu\n", sizeof(lrnnx_causal_conv1d_args), offsetof(lrnnx_causal_conv1d_args, x),
         offsetof(lrnnx_causal_conv1d_args, conv_state), offsetof(lrnnx_causal_conv1d_args, workspace_bytes));
  printf("%zu %zu %zu %zu %zu\n", sizeof(lrnnx_simplified_state_update_args),
         offsetof(lrnnx_simplified_state_update_args, state), offsetof(lrnnx_simplified_state_update_args, A_s0),
         offsetof(lrnnx_simplified_state_update_args, deltaA), offsetof(lrnnx_simplified_state_update_args, out_s1));
  printf("%zu %zu %zu %zu %zu %zu\n", sizeof(lrnnx_layer_norm_args), offsetof(lrnnx_layer_norm_args, eps),
         offsetof(lrnnx_layer_norm_args, x), offsetof(lrnnx_layer_norm_args, mean),
         offsetof(lrnnx_layer_norm_args, x_saved), offsetof(lrnnx_layer_norm_args, workspace_bytes));
  return 0;
}
'''
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "t.c")
        open(c, "w").write(prog)
        exe = os.path.join(d, "t")
        subprocess.check_call(["gcc", "-std=c99", "-I", os.path.dirname(HEADER), c, "-o", exe])
        got = subprocess.check_output([exe]).decode().split("\n")
    S, M, U = _lib.SelectiveScanArgs, _lib.SimplifiedScanArgs, _lib.StateUpdateArgs
    assert got[0].split() == [str(ctypes.sizeof(t)) for t in (_lib.View, S, M, U)]
    assert got[1].split() == [str(getattr(S, f).offset) for f in ("u", "x", "dout", "workspace", "dz")]
    assert got[2].split() == [str(getattr(M, f).offset) for f in ("x", "dout", "workspace_bytes")]
    assert got[3].split() == [str(getattr(U, f).offset) for f in ("state", "deltaA", "out_s2")]
    K = _lib.CausalConv1dArgs
    assert got[4].split() == [str(ctypes.sizeof(K))] + [str(getattr(K, f).offset)
                                                        for f in ("x", "conv_state", "workspace_bytes")]
    Z = _lib.SimplifiedStateUpdateArgs
    assert got[5].split() == [str(ctypes.sizeof(Z))] + [str(getattr(Z, f).offset)
                                                        for f in ("state", "A_s0", "deltaA", "out_s1")]
    N = _lib.LayerNormArgs
    assert got[6].split() == [str(ctypes.sizeof(N))] + [str(getattr(N, f).offset)
                                                        for f in ("eps", "x", "mean", "x_saved", "workspace_bytes")]


def _err():
    return _lib.lib().lrnnx_last_error().decode()


def test_argument_checks_mirror_reference_messages():
    L = _lib.lib()
    a = _lib.SelectiveScanArgs()
    a.batch, a.dim, a.seqlen, a.dstate, a.n_groups = 1, 4, 8, 4, 1
    a.itype, a.wtype, a.method = _lib.F32, _lib.F32, 99
    assert L.lrnnx_selective_scan_fwd(a, None) != 0
    assert "Discretization method not supported" in _err()
    a.method = _lib.METHODS["mamba"]
    a.dstate = 300
    assert L.lrnnx_selective_scan_fwd(a, None) != 0
    assert "state dimension <= 256" in _err()
    a.dstate = 4
    a.method, a.wtype = _lib.METHODS["s7"], _lib.C64
    assert L.lrnnx_selective_scan_fwd(a, None) != 0
    assert "S7 discretization only supports real" in _err()
    a.method, a.wtype, a.itype = _lib.METHODS["zoh"], _lib.F32, _lib.BF16
    assert L.lrnnx_selective_scan_fwd(a, None) != 0
    assert "float32 input only" in _err()
    a.itype = _lib.F32
    assert L.lrnnx_selective_scan_fwd(a, None) != 0   # null tensors
    assert "required" in _err()
    assert L.lrnnx_selective_scan_fwd(None, None) != 0
    m = _lib.SimplifiedScanArgs()
    m.batch, m.dim, m.seqlen, m.dstate, m.method = 1, 2, 3, 1, _lib.METHODS["mamba"]
    assert L.lrnnx_simplified_scan_fwd(m, None) != 0
    assert "Discretization method not supported" in _err()
    u = _lib.StateUpdateArgs()
    u.batch, u.nheads, u.dim, u.dstate, u.ngroups, u.method = 1, 3, 4, 4, 2, 3
    assert L.lrnnx_selective_state_update(u, None) != 0
    assert "divisible" in _err()
    z = _lib.SimplifiedStateUpdateArgs()
    z.batch, z.H, z.P, z.method = 1, 4, 4, _lib.METHODS["mamba"]
    assert L.lrnnx_simplified_state_update(z, None) != 0
    assert "discretization must be one of" in _err()
    z.method = _lib.METHODS["zoh"]
    assert L.lrnnx_simplified_state_update(z, None) != 0   # null tensors
    assert "required" in _err()
    c = _lib.CausalConv1dArgs()
    c.batch, c.dim, c.seqlen, c.width, c.itype = 1, 4, 8, 9, _lib.F32
    assert L.lrnnx_causal_conv1d_fwd(c, None) != 0
    assert "width must be between 1 and 8" in _err()
    c.width = 4
    assert L.lrnnx_causal_conv1d_fwd(c, None) != 0   # null tensors
    assert "required" in _err()
    assert L.lrnnx_causal_conv1d_workspace_size(c) == 1 * 4 * 5 * 4
    n = _lib.LayerNormArgs()
    n.rows, n.cols, n.xtype, n.rtype, n.wtype = 4, 40000, _lib.F16, _lib.F16, _lib.F32
    assert L.lrnnx_layer_norm_fwd(n, None) != 0
    assert "feature dim >= 64KB" in _err()   # layer_norm.py:405-411
    n.cols = 64
    assert L.lrnnx_layer_norm_fwd(n, None) != 0   # null tensors
    assert "required" in _err()
    n.xtype = 7
    assert L.lrnnx_layer_norm_fwd(n, None) != 0
    assert "unsupported dtype" in _err()
    n.xtype = _lib.F16
    # fast path (cols % 4 == 0, <= 4096): one partial per workgroup (1 row each here)
    assert L.lrnnx_layer_norm_workspace_size(n) == (1 + 16) * 2 * 64 * 4
    n.cols = 5000   # generic path: min(rows, 64) row blocks
    assert L.lrnnx_layer_norm_workspace_size(n) == (4 + 16) * 2 * 5000 * 4


def test_python_api_refuses_cpu_tensors():
    from lrnnx_amd import selective_scan_cuda, selective_scan_fn

    u = torch.randn(1, 4, 8)
    A = -torch.ones(4, 2)
    B = torch.randn(1, 2, 8)
    with pytest.raises(RuntimeError, match="GPU only"):
        selective_scan_fn(u, u.clone(), A, B, B.clone())
    with pytest.raises(RuntimeError, match="GPU only"):
        selective_scan_cuda.fwd(u, u.clone(), A, B[:, None], B[:, None].clone(), None, None, None, None, False,
                                "mamba")


def test_simplified_state_update_refuses_cpu_tensors():
    from lrnnx_amd import simplified_state_update

    st = torch.zeros(2, 3, dtype=torch.complex64)
    A = torch.zeros(3, dtype=torch.complex64)
    B = torch.zeros(3, 4, dtype=torch.complex64)
    with pytest.raises(RuntimeError, match="GPU only"):
        simplified_state_update(st, torch.zeros(2, 4), torch.ones(3), A, B, B.T.contiguous())
    with pytest.raises(AssertionError):   # the reference's shape assertions
        simplified_state_update(st, torch.zeros(2, 5), torch.ones(3), A, B, B.T.contiguous())


def test_layer_norm_refuses_cpu_tensors():
    from lrnnx_amd import RMSNorm, layer_norm_fn

    x = torch.randn(2, 3, 8)
    w = torch.ones(8)
    with pytest.raises(RuntimeError, match="GPU only"):
        layer_norm_fn(x, w, None, residual=x.clone(), prenorm=True)
    with pytest.raises(RuntimeError, match="GPU only"):
        RMSNorm(8)(x)
    with pytest.raises(NotImplementedError, match="dropout"):
        layer_norm_fn(x, w, None, dropout_p=0.1)


def test_workspace_queries_are_host_only():
    L = _lib.lib()
    a = _lib.SelectiveScanArgs()
    a.batch, a.dim, a.seqlen, a.dstate, a.n_groups = 8, 4096, 4096, 16, 1
    a.itype, a.wtype, a.method, a.var_B, a.var_C = _lib.BF16, _lib.F32, 3, 1, 1
    ck = L.lrnnx_selective_scan_ckpt_size(a)
    assert ck == 8 * (4096 // 16) * 16 * 4096 * 4
    assert L.lrnnx_selective_scan_workspace_size(a, 0) == 0   # 512 workgroups: no split of L
    assert L.lrnnx_selective_scan_workspace_size(a, 1) > 0
    # one workgroup (B=1, D=64): L = 2048 in 16 segments of 128 steps; h_end and h_init
    # (seg, b, n, d) plus two (seg, b, d) sums of delta', fp32
    a.batch, a.dim, a.seqlen = 1, 64, 2048
    assert L.lrnnx_selective_scan_workspace_size(a, 0) == (2 * 16 * 16 * 64 + 2 * 16 * 64) * 4
    a.method = 0  # zoh at bf16: the general kernels (the reference takes zoh at fp32 only), unsplit
    assert L.lrnnx_selective_scan_workspace_size(a, 0) == 0
    a.itype = _lib.F32  # zoh at fp32: the fast forward, split like mamba (exp-form A_bar)
    assert L.lrnnx_selective_scan_workspace_size(a, 0) == (2 * 16 * 16 * 64 + 2 * 16 * 64) * 4
    a.method = 1  # bilinear: the fast forward, never split (its A_bar is not exp-form)
    assert L.lrnnx_selective_scan_workspace_size(a, 0) == 0


def test_state_block_sizes_are_host_only():
    """d_state > 64: blocks of at most 64 states with 8-step checkpoints; the
    forward's optional workspace holds one fp32 partial y per block, the
    backward's the blocks' du / ddelta term sums (two for mamba, three for zoh)."""
    L = _lib.lib()
    a = _lib.SelectiveScanArgs()
    a.batch, a.dim, a.seqlen, a.n_groups = 2, 64, 160, 1
    a.itype, a.wtype, a.method, a.var_B, a.var_C = _lib.F32, _lib.F32, 3, 1, 1
    for n, nsb in ((64, 1), (65, 2), (128, 2), (200, 4), (256, 4)):
        a.dstate = n
        assert L.lrnnx_selective_scan_ckpt_size(a) == 2 * (160 // 8) * n * 64 * 4, n
        fws = L.lrnnx_selective_scan_workspace_size(a, 0)
        assert fws == (nsb * 2 * 64 * 160 * 4 if nsb > 1 else 0), (n, fws)
    a.dstate = 128
    bws_mamba = L.lrnnx_selective_scan_workspace_size(a, 1)
    a.method = 0
    bws_zoh = L.lrnnx_selective_scan_workspace_size(a, 1)
    assert bws_mamba >= 2 * 2 * 2 * 64 * 160 * 4          # blocks x terms x B x D x L fp32
    assert bws_zoh - bws_mamba == 2 * 2 * 64 * 160 * 4     # zoh's third term
    a.dstate = 16   # d_state <= 16: 16-step checkpoints (the fast kernels' interval)
    assert L.lrnnx_selective_scan_ckpt_size(a) == 2 * (160 // 16) * 16 * 64 * 4
