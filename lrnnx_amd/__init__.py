"""lrnnx_amd: the lrnnx scan hot path on AMD Instinct MI355X (gfx950).

Public API (same names, arguments and return conventions as the reference's
``lrnnx.ops``):

* ``selective_scan_fn`` / ``SelectiveScanFn``   (lrnnx/ops/selective_scan.py)
* ``simplified_scan_fn`` / ``SimplifiedScanFn``, ``s5_inner_fn`` / ``S5InnerFn``
  (lrnnx/ops/simplified_scan.py)
* ``selective_state_update``  (lrnnx/ops/triton/selective_state_update.py)
* ``simplified_state_update``  (lrnnx/ops/triton/simplified_state_update.py)
* ``causal_conv1d_fn``, ``causal_conv1d_update`` and the ``causal_conv1d_fwd_function`` /
  ``causal_conv1d_bwd_function`` pair: the causal-conv1d package's API that lrnnx calls
* ``mamba_inner_fn`` / ``MambaInnerFn``  (lrnnx/ops/selective_scan.py:389-786)
* ``layer_norm_fn``, ``rms_norm_fn``, ``LayerNormFn``, ``RMSNorm``,
  ``layer_norm_linear_fn``: the fused residual-add LayerNorm / RMSNorm
  (lrnnx/ops/triton/layer_norm.py)
* ``s7_scan_fn`` / ``S7ScanFn``, ``s7_inner_fn``  (lrnnx/ops/s7_scan.py)
* ``rglru_scan_fn`` / ``RGLRUScanFn``, ``rglru_inner_fn``  (lrnnx/ops/rglru_scan.py)
* ``selective_scan_cuda``, ``simplified_scan_cuda``: drop-in replacements of
  the reference's pybind11 extension modules (``fwd`` / ``bwd``).

All compute runs in hand-written HIP kernels in ``liblrnnx_scan.so`` (C ABI:
include/lrnnx_scan.h).  There is no CPU fallback.
"""

from . import selective_scan_cuda, simplified_scan_cuda  # noqa: F401
from .causal_conv1d import (causal_conv1d_bwd_function, causal_conv1d_fn, causal_conv1d_fwd_function,  # noqa: F401
                            causal_conv1d_update)
from .layer_norm import (LayerNormFn, LayerNormLinearFn, RMSNorm, layer_norm_fn, layer_norm_linear_fn,  # noqa: F401
                         rms_norm_fn)
from .mamba_inner import MambaInnerFn, mamba_inner_fn  # noqa: F401
from .rglru_scan import RGLRUScanFn, rglru_inner_fn, rglru_scan_fn  # noqa: F401
from .s7_scan import S7ScanFn, s7_inner_fn, s7_scan_fn  # noqa: F401
from .selective_scan import SelectiveScanFn, selective_scan_fn  # noqa: F401
from .selective_state_update import selective_state_update  # noqa: F401
from .simplified_state_update import simplified_state_update  # noqa: F401
from .simplified_scan import S5InnerFn, SimplifiedScanFn, s5_inner_fn, simplified_scan_fn  # noqa: F401
