"""CPU oracle for the lrnnx scan hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (``lrnnx_amd``)
imports this package; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker (or the
timed CPU baseline), never as the thing that computes a product result.

Contents
--------
``scan_ref``  PyTorch restatements of the reference's pure-PyTorch scans
              (``lrnnx/ops/selective_scan.py:200-360``,
              ``lrnnx/ops/simplified_scan.py:233-340,586-640``,
              ``lrnnx/ops/triton/selective_state_update.py:479-599``,
              ``lrnnx/ops/s7_scan.py:179-233``, ``lrnnx/ops/rglru_scan.py:148-203``)
              plus the kernel-boundary semantics of ``selective_scan_cuda.fwd``
              and ``simplified_scan_cuda.fwd`` (chunk carries ``x``).  Every
              function takes a compute dtype so that tests can run it in
              float64; gradients come from autograd through it.
``brute``     Scalar triple loops in float64 (pure Python, tiny shapes only)
              used to pin ``scan_ref`` independently of its vectorised form.

Pinning (what checks each function; see ``tests/test_oracle.py``)
---------------------------------------------------------------------
* selective scan, every discretisation, real and complex: brute-force scalar
  loop, closed forms (geometric series, cumsum for A=0, L=1, IIR filter via
  ``scipy.signal.lfilter``), invariants (z-gating, D skip, G=1 4-D == 3-D
  B/C, deltaA == delta for mamba, chunk-split continuation) and fp64
  ``torch.autograd.gradcheck``.
* simplified scan / s5_inner: brute-force loop, complex IIR closed form
  (``lfilter``), gradcheck.
* selective_state_update: equality with one step of the selective scan
  oracle (same discretisation) and brute force.
* The reference holds no golden vectors for this path (its tests compare the
  CUDA op with ``*_ref`` at run time), so the committed fixtures under
  ``tests/golden/`` are written from this oracle in float64 after the checks
  above pass.
"""
