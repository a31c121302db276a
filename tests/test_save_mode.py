"""Host logic of the selective scan's save modes (CPU; no kernel runs).

What a wrapper keeps for the backward: "checkpoints" (default; the forward's
fp32 states, attached to the returned x) or "x" (the reference's chunk
carries only, selective_scan.py:93-100).  The GPU tests run both modes
against the oracle (tests/test_grid_gpu.py); these check the selection, the
validation and that a CPU call fails before anything is launched.
"""

import os
import subprocess
import sys

import pytest
import torch

from lrnnx_amd import selective_scan_cuda as ssc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture
def restore_mode():
    prev = ssc.save_mode()
    yield
    ssc.set_save_mode(prev)


def test_default_mode_keeps_checkpoints(restore_mode):
    env = {k: v for k, v in os.environ.items() if k != "LRNNX_SCAN_SAVE"}
    out = subprocess.run([sys.executable, "-c",
                          "from lrnnx_amd import selective_scan_cuda as s; print(s.save_mode(), s.keeps_checkpoints())"],
                         cwd=ROOT, env=env, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.split() == ["checkpoints", "True"]


def test_env_selects_x_mode():
    env = dict(os.environ, LRNNX_SCAN_SAVE="x")
    out = subprocess.run([sys.executable, "-c",
                          "from lrnnx_amd import selective_scan_cuda as s; print(s.save_mode(), s.keeps_checkpoints())"],
                         cwd=ROOT, env=env, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.split() == ["x", "False"]


def test_env_rejects_unknown_mode():
    env = dict(os.environ, LRNNX_SCAN_SAVE="everything")
    out = subprocess.run([sys.executable, "-c", "from lrnnx_amd import selective_scan_cuda"],
                         cwd=ROOT, env=env, capture_output=True, text=True, timeout=120)
    assert out.returncode != 0
    assert "LRNNX_SCAN_SAVE must be one of" in out.stderr


def test_set_save_mode_validates(restore_mode):
    with pytest.raises(ValueError, match="save mode must be one of"):
        ssc.set_save_mode("ckpt")
    ssc.set_save_mode("x")
    assert ssc.save_mode() == "x" and not ssc.keeps_checkpoints()
    ssc.set_save_mode("checkpoints")
    assert ssc.save_mode() == "checkpoints" and ssc.keeps_checkpoints()


def test_for_backward_selection(restore_mode):
    x = torch.zeros(2, 64, 1, 32)          # (B, D, n_chunks, 2N) carries
    ck = torch.zeros(2 * 1 * 16 * 64)      # flat fp32 checkpoints
    ssc.set_save_mode("checkpoints")
    assert ssc.for_backward(x, ck) is ck
    assert ssc.for_backward(x, None) is x   # a forward that wrote none (no backward was needed)
    ssc.set_save_mode("x")
    assert ssc.for_backward(x, ck) is x
    assert ssc.for_backward(x, None) is x


@pytest.mark.parametrize("mode", ["checkpoints", "x"])
def test_backward_refuses_cpu_tensors_in_both_modes(restore_mode, mode):
    """No CPU fallback whichever tensor was saved: the binding raises before
    any launch."""
    ssc.set_save_mode(mode)
    Bt, D, L, N = 1, 64, 32, 16
    u = torch.randn(Bt, D, L)
    delta = torch.rand(Bt, D, L)
    A = -torch.rand(D, N)
    B = torch.randn(Bt, 1, N, L)
    C = torch.randn(Bt, 1, N, L)
    x = torch.zeros(Bt, D, 1, 2 * N)
    with pytest.raises(RuntimeError, match="GPU only"):
        ssc.bwd(u, delta, A, B, C, None, None, None, None, torch.randn(Bt, D, L), x, None, None, False, False,
                "mamba")
