"""CPU oracle for the Hyena long-convolution hot path -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (``nvsubquadratic_amd``) imports this package.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
use it, and only as the checker / the timed CPU baseline.

Contents:

* :mod:`oracle.fftconv_ref` -- restatement of the reference torch.fft path
  (``nvsubquadratic/ops/fftconv.py``) on the CPU: a float32 torch version (the
  reference algorithm, autograd-capable) and a float64 numpy version.
* :mod:`oracle.direct` -- ctypes binding of ``direct_conv.c``: brute-force
  float64 direct convolutions that pin the FFT restatement independently of any
  FFT.
* :mod:`oracle.direct_ref` -- torch restatements of the depthwise causal conv
  (``CausalConv1D``) and of the B2B block's specification.
* :mod:`oracle.circular_ref` -- circular and mixed-boundary restatements
  (``ops/circular_fftconv.py``, ``ops/mixed_fftconv.py``) and their float64
  brute forces.
* :mod:`oracle.gated_ref` -- the Hyena gate compositions around the long conv.
* :mod:`oracle.siren_ref` -- the SIREN implicit filter generator
  (``modules/kernels_nd.py``, ``SIRENKernelND`` without FiLM) in float32 or
  float64 torch.
* :mod:`oracle.norm_ref` -- the Hyena gate + RMSNorm over channels + layout
  sequence at the norm sites (torch on the CPU, autograd backward).

The seeded synthetic inputs of the benchmark configs are product-side
(``nvsubquadratic_amd.workloads``): they are data, not a checker.

Parity status of every function is listed in the module docstrings; a function
with no independent check says "parity unpinned".
"""
