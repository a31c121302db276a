"""ctypes binding of liblrnnx_scan.so (the C ABI declared in include/lrnnx_scan.h).

The library is loaded lazily on first use.  There is no CPU fallback: if the
library is missing, or a tensor is not on a ROCm device, the call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

_LIB_PATH = Path(os.environ.get("LRNNX_LIB", Path(__file__).resolve().parent / "liblrnnx_scan.so"))
_lock = threading.Lock()
_lib = None

F32, F16, BF16, C64 = 0, 1, 2, 3
METHODS = {"zoh": 0, "bilinear": 1, "dirac": 2, "mamba": 3, "s7": 4, "rglru": 5}
_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.complex64: C64}

c_i64 = ctypes.c_int64
c_i32 = ctypes.c_int32
c_vp = ctypes.c_void_p


class View(ctypes.Structure):
    _fields_ = [("ptr", c_vp), ("s0", c_i64), ("s1", c_i64), ("s2", c_i64)]


class SelectiveScanArgs(ctypes.Structure):
    _fields_ = (
        [(n, c_i64) for n in ("batch", "dim", "seqlen", "dstate", "n_groups")]
        + [(n, c_i32) for n in ("itype", "wtype", "method", "var_B", "var_C", "delta_softplus")]
        + [(n, View) for n in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias", "deltaA", "out", "out_z")]
        + [("x", c_vp), ("ckpt", c_vp)]
        + [(n, View) for n in ("dout", "out_saved", "du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias",
                               "ddeltaA", "dz")]
        + [("workspace", c_vp), ("workspace_bytes", c_i64)]
    )


class SimplifiedScanArgs(ctypes.Structure):
    _fields_ = (
        [(n, c_i64) for n in ("batch", "dim", "seqlen", "dstate")]
        + [("method", c_i32), ("need_ddelta", c_i32)]
        + [(n, View) for n in ("u", "delta", "A", "B", "C", "deltaA", "out")]
        + [("x", c_vp), ("ckpt", c_vp), ("dout", View)]
        + [(n, View) for n in ("du", "ddelta", "dA", "dB", "dC", "ddeltaA")]
        + [("workspace", c_vp), ("workspace_bytes", c_i64)]
    )


def _ptr_fields(name, n):
    return [(name, c_vp)] + [(f"{name}_s{i}", c_i64) for i in range(n)]


class StateUpdateArgs(ctypes.Structure):
    _fields_ = (
        [(n, c_i64) for n in ("batch", "nheads", "dim", "dstate", "ngroups")]
        + [(n, c_i32) for n in ("state_type", "x_type", "bc_type", "method", "dt_softplus")]
        + _ptr_fields("state", 4) + _ptr_fields("x", 3) + _ptr_fields("dt", 3) + _ptr_fields("A", 3)
        + _ptr_fields("B", 3) + _ptr_fields("C", 3) + _ptr_fields("D", 2) + _ptr_fields("z", 3)
        + [("dt_bias", c_vp), ("dtb_s0", c_i64), ("dtb_s1", c_i64)]
        + [("deltaA", c_vp), ("dA_s0", c_i64), ("dA_s1", c_i64), ("dA_s2", c_i64)]
        + [("state_batch_indices", c_vp)]
        + _ptr_fields("out", 3)
    )


class SimplifiedStateUpdateArgs(ctypes.Structure):
    _fields_ = (
        [(n, c_i64) for n in ("batch", "H", "P")]
        + [(n, c_i32) for n in ("method", "conj_sym")]
        + _ptr_fields("state", 2) + _ptr_fields("x", 2) + _ptr_fields("dt", 2) + _ptr_fields("A", 1)
        + _ptr_fields("B", 2) + _ptr_fields("C", 2) + _ptr_fields("D", 2)
        + [("deltaA", c_vp), ("dA_s0", c_i64), ("dA_s1", c_i64)]
        + _ptr_fields("out", 2)
    )


class CausalConv1dArgs(ctypes.Structure):
    _fields_ = (
        [(n, c_i64) for n in ("batch", "dim", "seqlen", "width", "state_len")]
        + [(n, c_i32) for n in ("itype", "silu")]
        + [(n, View) for n in ("x", "weight", "bias", "out", "dout", "dx", "dweight", "dbias", "conv_state")]
        + [("workspace", c_vp), ("workspace_bytes", c_i64)]
    )


class LayerNormArgs(ctypes.Structure):
    _fields_ = (
        [("rows", c_i64), ("cols", c_i64)]
        + [(n, c_i32) for n in ("xtype", "rtype", "wtype", "is_rms_norm")]
        + [("eps", ctypes.c_float), ("reserved", c_i32)]
        + [(n, View) for n in ("x", "residual", "weight", "bias", "y", "residual_out")]
        + [("mean", c_vp), ("rstd", c_vp)]
        + [(n, View) for n in ("x_saved", "dy", "dresidual", "dx", "dresidual_in", "dweight", "dbias")]
        + [("workspace", c_vp), ("workspace_bytes", c_i64)]
    )


EXPORTS = (
    "lrnnx_selective_scan_ckpt_size",
    "lrnnx_selective_scan_workspace_size",
    "lrnnx_selective_scan_fwd",
    "lrnnx_selective_scan_fwd_noalloc",
    "lrnnx_selective_scan_bwd",
    "lrnnx_simplified_scan_ckpt_size",
    "lrnnx_simplified_scan_workspace_size",
    "lrnnx_simplified_scan_fwd",
    "lrnnx_simplified_scan_bwd",
    "lrnnx_selective_state_update",
    "lrnnx_simplified_state_update",
    "lrnnx_causal_conv1d_fwd",
    "lrnnx_causal_conv1d_bwd",
    "lrnnx_causal_conv1d_update",
    "lrnnx_causal_conv1d_workspace_size",
    "lrnnx_layer_norm_fwd",
    "lrnnx_layer_norm_bwd",
    "lrnnx_layer_norm_workspace_size",
    "lrnnx_last_error",
    "lrnnx_abi_version",
)

ABI_VERSION = 4


def lib():
    """Load (once) and return the ctypes library; raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not _LIB_PATH.exists():
            raise RuntimeError(
                f"lrnnx_amd: native library {_LIB_PATH} not found; build it with "
                "`python -m lrnnx_amd.build` (there is no CPU fallback)")
        L = ctypes.CDLL(str(_LIB_PATH))
        P = ctypes.POINTER
        L.lrnnx_selective_scan_ckpt_size.argtypes = [P(SelectiveScanArgs)]
        L.lrnnx_selective_scan_ckpt_size.restype = c_i64
        L.lrnnx_selective_scan_workspace_size.argtypes = [P(SelectiveScanArgs), ctypes.c_int]
        L.lrnnx_selective_scan_workspace_size.restype = c_i64
        L.lrnnx_selective_scan_fwd.argtypes = [P(SelectiveScanArgs), c_vp]
        L.lrnnx_selective_scan_fwd_noalloc.argtypes = [P(SelectiveScanArgs), c_vp]
        L.lrnnx_selective_scan_bwd.argtypes = [P(SelectiveScanArgs), c_vp]
        L.lrnnx_simplified_scan_ckpt_size.argtypes = [P(SimplifiedScanArgs)]
        L.lrnnx_simplified_scan_ckpt_size.restype = c_i64
        L.lrnnx_simplified_scan_workspace_size.argtypes = [P(SimplifiedScanArgs), ctypes.c_int]
        L.lrnnx_simplified_scan_workspace_size.restype = c_i64
        L.lrnnx_simplified_scan_fwd.argtypes = [P(SimplifiedScanArgs), c_vp]
        L.lrnnx_simplified_scan_bwd.argtypes = [P(SimplifiedScanArgs), c_vp]
        L.lrnnx_selective_state_update.argtypes = [P(StateUpdateArgs), c_vp]
        L.lrnnx_simplified_state_update.argtypes = [P(SimplifiedStateUpdateArgs), c_vp]
        for fn in ("lrnnx_causal_conv1d_fwd", "lrnnx_causal_conv1d_bwd", "lrnnx_causal_conv1d_update"):
            getattr(L, fn).argtypes = [P(CausalConv1dArgs), c_vp]
            getattr(L, fn).restype = ctypes.c_int
        L.lrnnx_causal_conv1d_workspace_size.argtypes = [P(CausalConv1dArgs)]
        L.lrnnx_causal_conv1d_workspace_size.restype = c_i64
        for fn in ("lrnnx_layer_norm_fwd", "lrnnx_layer_norm_bwd"):
            getattr(L, fn).argtypes = [P(LayerNormArgs), c_vp]
            getattr(L, fn).restype = ctypes.c_int
        L.lrnnx_layer_norm_workspace_size.argtypes = [P(LayerNormArgs)]
        L.lrnnx_layer_norm_workspace_size.restype = c_i64
        L.lrnnx_last_error.restype = ctypes.c_char_p
        for fn in ("lrnnx_selective_scan_fwd", "lrnnx_selective_scan_fwd_noalloc", "lrnnx_selective_scan_bwd",
                   "lrnnx_simplified_scan_fwd",
                   "lrnnx_simplified_scan_bwd", "lrnnx_selective_state_update",
                   "lrnnx_simplified_state_update", "lrnnx_abi_version"):
            getattr(L, fn).restype = ctypes.c_int
        if L.lrnnx_abi_version() != ABI_VERSION:
            raise RuntimeError(f"lrnnx_amd: ABI version mismatch ({L.lrnnx_abi_version()} != {ABI_VERSION})")
        _lib = L
        return _lib


def check(rc: int, what: str):
    if rc != 0:
        msg = lib().lrnnx_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg}")


def dtype_code(t: torch.dtype) -> int:
    try:
        return _DT[t]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {t}") from None


def require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("lrnnx_amd ops run on the GPU only (tensor on %s); there is no CPU path" % t.device)


def view(t, ndim_lead: int | None = None) -> View:
    """View of a tensor: pointer + element strides of the leading dims.
    Strides of complex tensors count complex elements (as torch does)."""
    if t is None:
        return View()
    st = t.stride()
    lead = st[:-1] if ndim_lead is None else st[:ndim_lead]
    return View(t.data_ptr(), *lead[:3])


def view_full(t) -> View:
    """All strides (up to 3) of a tensor, including the last one."""
    if t is None:
        return View()
    return View(t.data_ptr(), *t.stride()[:3])


class _NoGuard:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NO_GUARD = _NoGuard()


def on_device(t):
    """Device guard for a launch on t's device: a no-op when that device is
    already current (the common case), torch.cuda.device otherwise."""
    idx = t.device.index
    if idx is None or idx == torch.cuda.current_device():
        return _NO_GUARD
    return torch.cuda.device(idx)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t) -> int:
    """The current stream of t's device (a hipStream_t as an integer)."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream
