"""nvsubquadratic_amd: MI355X-native (gfx950) Hyena long-convolution hot path.

``fft_backend="hip"`` counterpart of the reference's ``nvsubquadratic.ops``
FFT-conv / causal-conv ops.  Importing the package never touches the GPU; the
native library ``libnsq_hip.so`` is loaded on first use.
"""

__version__ = "0.1.0"
