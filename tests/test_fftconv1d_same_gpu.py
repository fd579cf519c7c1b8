"""GPU parity of the zero-padded non-causal 1D FFT conv (``fftconv1d_bhl``, reference
``nvsubquadratic/ops/fftconv.py:603-660``; ``mixed_fftconv1d`` with ``periodic=(False,)``).

The oracle is the CPU restatement in ``oracle/circular_ref.py`` (brute-force sum, and the
torch.fft recipe in float64 for autograd), itself pinned against numpy's full convolution
in ``tests/test_oracle_circular.py``.  Tolerances: 1e-4 rel-L2 for fp32, 2e-2 for bf16 I/O.
"""

import numpy as np
import pytest
import torch

from nvsubquadratic_amd import _lib, dispatch
from nvsubquadratic_amd import fftconv_hip as Z
from nvsubquadratic_amd import mixed_fftconv_hip as M
from oracle.circular_ref import mixed_conv_direct_np, mixed_fftconv_torch

pytestmark = pytest.mark.gpu


def rel_l2(ref, out) -> float:
    r = torch.as_tensor(np.asarray(ref) if not torch.is_tensor(ref) else ref.detach().cpu()).double()
    o = out.detach().cpu().double()
    return float((o - r).norm() / r.norm().clamp_min(1e-30))


# (B, H, L, K): odd / even K, K = 2L, K = 1, L = 1, lengths that are not powers of two, and the largest
# L + ceil(K/2) the fused kernels take (16384; longer ones run the 4-step plan, tested below)
CASES = [(2, 16, 64, 7), (2, 8, 64, 8), (1, 8, 100, 200), (3, 4, 333, 1), (2, 3, 1, 2), (2, 4, 1000, 129),
         (1, 4, 4096, 4096), (1, 2, 12288, 8192), (2, 16, 2048, 33), (4, 32, 8192, 16)]


@pytest.mark.parametrize("B,H,L,K", CASES)
def test_same_1d_forward_vs_brute_force(B, H, L, K):
    rng = np.random.default_rng(B * 1000 + L + K)
    x = rng.standard_normal((B, H, L)).astype(np.float32)
    k = rng.standard_normal((1, H, K)).astype(np.float32)
    s = rng.standard_normal(H).astype(np.float32)
    print(f"same1d fwd B={B} H={H} L={L} K={K}", flush=True)
    y = Z.fftconv1d_bhl(torch.tensor(x).cuda(), torch.tensor(k).cuda(), torch.tensor(s).cuda())
    if L * K <= 1 << 20:
        ref = mixed_conv_direct_np(x.astype(np.float64), k.astype(np.float64), (False,), s.astype(np.float64))
    else:
        ref = mixed_fftconv_torch(torch.tensor(x), torch.tensor(k), (False,), torch.tensor(s),
                                  compute_dtype=torch.float64)
    assert y.shape == (B, H, L) and y.dtype == torch.float32
    assert rel_l2(ref, y) < 1e-4


def _fwd_bwd(B, H, L, K, kb=1, dtype=torch.float32, tol=1e-4):
    torch.manual_seed(L + K)
    x = torch.randn(B, H, L).to(dtype).requires_grad_(True)
    k = torch.randn(kb, H, K, requires_grad=True)
    s = torch.randn(H).to(dtype).requires_grad_(True)
    y_ref = mixed_fftconv_torch(x, k, (False,), s, compute_dtype=torch.float64)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg, kg, sg = (t.detach().cuda().requires_grad_(True) for t in (x, k, s))
    print(f"same1d fwd+bwd B={B} H={H} L={L} K={K} kb={kb} {dtype}", flush=True)
    y = Z.fftconv1d_bhl(xg, kg, sg)
    y.backward(g.cuda())
    assert y.dtype == dtype
    assert rel_l2(y_ref, y) < tol
    assert rel_l2(x.grad, xg.grad) < tol
    assert rel_l2(k.grad, kg.grad) < tol
    assert rel_l2(s.grad, sg.grad) < tol


@pytest.mark.parametrize("B,H,L,K", [(2, 8, 64, 7), (2, 8, 64, 8), (1, 4, 100, 200), (3, 4, 333, 1),
                                     (2, 3, 1, 2), (2, 4, 1000, 129), (1, 4, 8192, 8191)])
def test_same_1d_fwd_bwd(B, H, L, K):
    _fwd_bwd(B, H, L, K)


@pytest.mark.parametrize("B,H,L,K", [(3, 4, 256, 31), (2, 8, 100, 64)])
def test_same_1d_per_sample_kernel(B, H, L, K):
    _fwd_bwd(B, H, L, K, kb=B)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_same_1d_half_io(dtype):
    _fwd_bwd(2, 16, 512, 65, dtype=dtype, tol=2e-2)


def test_same_1d_routing_chunking_and_layouts_bitwise():
    torch.manual_seed(3)
    x = torch.randn(2, 20, 300, device="cuda")
    k = torch.randn(1, 20, 41, device="cuda")
    s = torch.randn(20, device="cuda")
    y = Z.fftconv1d_bhl(x, k, s)
    assert torch.equal(M.mixed_fftconv1d_fp32_bhl(x, k, (False,), s), y)
    assert torch.equal(Z.fftconv1d_bhl_chunked(x, k, s, chunk_size=8), y)
    yw = Z.fftconv1d_bhl_w_reshape(x.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous(), s)
    assert torch.equal(yw.transpose(1, 2), y)
    assert torch.equal(Z.fftconv1d_blh_chunked(x.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous(), s,
                                               chunk_size=7).transpose(1, 2), y)
    fn, fn_bhl = dispatch.hip_fftconv_fns(1, False, "zero")
    assert torch.equal(fn_bhl(x, k, s), y)


def test_same_1d_limits():
    x = torch.randn(1, 2, 2**24 - 100, device="cuda")
    with pytest.raises(NotImplementedError, match="FFT length"):
        Z.fftconv1d_bhl(x, torch.randn(1, 2, 400, device="cuda"))  # L + ceil(K/2) > 2^24
    with pytest.raises(AssertionError, match="2 \\* seq_len"):
        Z.fftconv1d_bhl(torch.randn(1, 2, 8, device="cuda"), torch.randn(1, 2, 17, device="cuda"))
    # the C-ABI's own checks: K > 2L and a mask naming axis 1
    lib = _lib.get_lib()
    xs = torch.randn(1, 2, 8, device="cuda")
    k = torch.randn(2, 17, device="cuda")
    y = torch.empty_like(xs)
    with pytest.raises(ValueError, match="2\\*L"):
        Z.mixed_fftconv1d_fwd_raw(xs, k, None, y, 1, 0)
    with pytest.raises(ValueError, match="periodic mask"):
        _lib.check(lib.nsq_mixed_fftconv1d_fwd(xs.data_ptr(), k.data_ptr(), None, y.data_ptr(), 0, 1, 2, 8, 3, 1, 2,
                                               None, 0, _lib.stream_ptr(xs.device)))


# --- beyond the fused kernels: the 4-step plan with a rolled operand -------------
LONG = [(1, 4, 20000, 3001, False), (2, 2, 40000, 80000, False), (1, 3, 32768, 31, True), (2, 2, 65536, 65536, True),
        (1, 2, 131072, 1000, True), (1, 2, 100000, 17, False)]


@pytest.mark.parametrize("B,H,L,K,periodic", LONG)
def test_long_shifted_1d_fwd_bwd(B, H, L, K, periodic):
    """Zero-padded "same" and circular 1D at FFT lengths 2^15..2^18 (4-step plan): forward and all gradients
    against the float64 torch.fft restatement."""
    from oracle.circular_ref import mixed_fftconv_torch

    torch.manual_seed(L + K)
    x = torch.randn(B, H, L, requires_grad=True)
    k = (torch.randn(1, H, K) * torch.exp(-torch.arange(K) / (K / 4))).requires_grad_(True)
    s = torch.randn(H, requires_grad=True)
    y_ref = mixed_fftconv_torch(x, k, (periodic,), s, compute_dtype=torch.float64)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg, kg, sg = (t.detach().cuda().requires_grad_(True) for t in (x, k, s))
    print(f"long shifted 1d B={B} H={H} L={L} K={K} periodic={periodic}", flush=True)
    y = M.mixed_fftconv1d_fp32_bhl(xg, kg, (periodic,), sg)
    y.backward(g.cuda())
    for ref, out in ((y_ref, y), (x.grad, xg.grad), (k.grad, kg.grad), (s.grad, sg.grad)):
        assert rel_l2(ref, out) < 1e-4


def test_long_shifted_1d_bf16_per_sample():
    from oracle.circular_ref import mixed_fftconv_torch

    torch.manual_seed(9)
    B, H, L, K = 2, 3, 50000, 777
    x = torch.randn(B, H, L).to(torch.bfloat16).requires_grad_(True)
    k = (torch.randn(B, H, K) / K ** 0.5).requires_grad_(True)
    y_ref = mixed_fftconv_torch(x, k, (False,), None, compute_dtype=torch.float64)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg, kg = (t.detach().cuda().requires_grad_(True) for t in (x, k))
    print("long shifted 1d bf16 per-sample", flush=True)
    y = Z.fftconv1d_bhl(xg, kg)
    y.backward(g.cuda())
    for ref, out in ((y_ref, y), (x.grad, xg.grad), (k.grad, kg.grad)):
        assert rel_l2(ref, out) < 2e-2
