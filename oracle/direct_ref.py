"""CPU restatements for the direct-conv rows -- TEST INFRASTRUCTURE ONLY.

* :func:`causal_conv1d_torch` restates ``CausalConv1D.forward``
  (nvsubquadratic/modules/causal_conv1d.py:113-139: left pad K-1, depthwise
  F.conv1d) plus the activation of ``causal_conv1d_custom.causal_conv1d``
  (nvsubquadratic/ops/causal_conv1d_custom.py:81-98), exactly the reference
  test helper tests/ops/test_causal_conv1d_custom.py:65-72.  Float32 CPU torch,
  autograd-capable.
* :func:`b2b_causal_conv1d_torch` is this build's specification of the B2B
  block (projection conv -> z = k*v -> mixer conv + skip*z -> q*h), which the
  reference leaves to an external package (causal_conv1d_custom.py:101-121);
  fp32 throughout, output cast to x.dtype.

Pinning (tests/test_oracle_direct.py): both are compared with the brute-force
float64 C loops of oracle/direct_conv.c and with the golden fixtures
tests/golden/direct1d.npz, plus closed forms (delta weights reduce B2B to
q * k * v * (1 + skip)).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def causal_conv1d_torch(x, weight, bias=None, activation="identity"):
    K = weight.shape[-1]
    y = F.conv1d(F.pad(x, (K - 1, 0)), weight.unsqueeze(1), bias, groups=weight.shape[0])
    return F.silu(y) if activation == "silu" else y


def b2b_causal_conv1d_torch(x, weight_proj, weight_mixer, skip_bias):
    C = x.shape[1] // 3
    p = causal_conv1d_torch(x.float(), weight_proj.float())
    q, k, v = p[:, :C], p[:, C:2 * C], p[:, 2 * C:]
    z = k * v
    h = causal_conv1d_torch(z, weight_mixer.float())
    if skip_bias is not None:
        h = h + skip_bias.float().view(1, C, 1) * z
    return (q * h).to(x.dtype)
