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
* :mod:`oracle.inputs` -- seeded synthetic inputs for the BASELINE configs.

Parity status of every function is listed in the module docstrings; a function
with no independent check says "parity unpinned".
"""
