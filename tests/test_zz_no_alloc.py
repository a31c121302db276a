"""GPU test of lrnnx_selective_scan_fwd_noalloc, the forward entry point that
allocates nothing: called through the C ABI, it must give bit for bit the
results of lrnnx_selective_scan_fwd with a caller-allocated workspace (same
kernels), on two calls in a row, the second with a smaller input (the
scratch keeps the first call's contents), both taking the small-grid split
of L that uses the scratch."""

import pytest
import torch

import bench
from lrnnx_amd import _lib
from lrnnx_amd import selective_scan_cuda as ssc

pytestmark = pytest.mark.gpu


def _fwd(dev, inp, noalloc):
    a = ssc.build_args(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"], inp["delta_bias"],
                       None, True, "mamba")
    Bt, D, L = inp["u"].shape
    N = inp["A"].shape[1]
    out = torch.empty_like(inp["u"])
    out_z = torch.empty_like(inp["z"])
    x = torch.empty((Bt, D, (L + 2047) // 2048, 2 * N), dtype=torch.float32, device=dev)
    ckpt = torch.empty(_lib.lib().lrnnx_selective_scan_ckpt_size(a) // 4, dtype=torch.float32, device=dev)
    a.out, a.out_z = _lib.view(out, 2), _lib.view(out_z, 2)
    a.x, a.ckpt = x.data_ptr(), ckpt.data_ptr()
    need = _lib.lib().lrnnx_selective_scan_workspace_size(a, 0)
    assert 0 < need <= 4456448, need   # the call takes the split, within the scratch's bound
    stream = torch.cuda.current_stream(dev).cuda_stream
    if noalloc:
        a.workspace, a.workspace_bytes = None, 0
        before = torch.cuda.memory_allocated(dev)
        _lib.check(_lib.lib().lrnnx_selective_scan_fwd_noalloc(a, stream), "fwd_noalloc")
        assert torch.cuda.memory_allocated(dev) == before
    else:
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = ws.data_ptr(), need
        _lib.check(_lib.lib().lrnnx_selective_scan_fwd(a, stream), "fwd")
    torch.cuda.synchronize()
    return {"out": out, "out_z": out_z, "x": x, "ckpt": ckpt}


@pytest.mark.parametrize("itype", [torch.bfloat16, torch.float32])
def test_fwd_noalloc_matches_workspace_entry_point(dev, itype):
    # two calls in a row, the second smaller: B=1 D=256 L=4096 (4 workgroups,
    # 32 segments), then B=1 D=64 L=1024 (1 workgroup, 8 segments)
    for i, (Bt, D, L) in enumerate(((1, 256, 4096), (1, 64, 1024))):
        print(f"[noalloc] call {i}: B={Bt} D={D} L={L} {itype}", flush=True)
        inp = bench.make_cfg3(dev, torch, None, Bt, D, L, 16, seed=50 + i, io=itype)
        ref = _fwd(dev, inp, noalloc=False)
        got = _fwd(dev, inp, noalloc=True)
        for k in ref:
            assert torch.equal(got[k], ref[k]), f"call {i}: {k} differs from lrnnx_selective_scan_fwd"


def test_fwd_noalloc_unsplit_call_and_errors(dev):
    """A grid that does not split runs without touching the scratch, and the
    argument checks are those of lrnnx_selective_scan_fwd."""
    inp = bench.make_cfg3(dev, torch, None, 4, 2560, 256, 16, seed=60, io=torch.bfloat16)
    a = ssc.build_args(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"], inp["delta_bias"],
                       None, True, "mamba")
    assert _lib.lib().lrnnx_selective_scan_workspace_size(a, 0) == 0
    out, out_z = torch.empty_like(inp["u"]), torch.empty_like(inp["z"])
    a.out, a.out_z = _lib.view(out, 2), _lib.view(out_z, 2)
    stream = torch.cuda.current_stream(dev).cuda_stream
    _lib.check(_lib.lib().lrnnx_selective_scan_fwd_noalloc(a, stream), "fwd_noalloc")
    ref = ssc.fwd(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"], inp["delta_bias"],
                  None, True, "mamba")
    torch.cuda.synchronize()
    assert torch.equal(out_z, ref[2])
    a.out_z = _lib.view(None, 2)
    assert _lib.lib().lrnnx_selective_scan_fwd_noalloc(a, stream) != 0
    assert b"out_z is required" in _lib.lib().lrnnx_last_error()
