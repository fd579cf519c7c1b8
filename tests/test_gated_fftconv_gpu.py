"""GPU parity of the Hyena-gated causal FFT conv against the CPU oracle composition.

Covers the fused plan (FFT length <= 16384: the gated forward kernel below 2^22 elements, gate kernels around the
plain fused kernel above, including the K > L+1 fold), the multi-kernel plan (elementwise gate kernels around the
4-step conv), every gate pair the reference configs use (SiLU / Sigmoid, Identity), per-sample filters and bf16
I/O.  Tolerances: rel-L2 <= 1e-4 fp32, <= 2e-2 bf16.  The reference computes gradients with autograd through the
composition; the oracle does the same on the CPU.  The two forward routes of the fused plan give the same bits.
"""

import pytest
import torch

from nvsubquadratic_amd.gated_fftconv_hip import hyena_gated_causal_fftconv1d_bhl
from oracle.fftconv_ref import rel_l2
from oracle.gated_ref import gated_causal_fftconv1d_torch


pytestmark = pytest.mark.gpu


def _check(B, H, L, K, g1, g2, kb=1, dtype=torch.float32, tol=1e-4, shortcut=True):
    torch.manual_seed(B * 131 + L + K)
    q, k, v = (torch.randn(B, H, L).to(dtype).requires_grad_(True) for _ in range(3))
    w = (torch.randn(kb, H, K) / K ** 0.5).requires_grad_(True)
    s = torch.randn(H).to(dtype).requires_grad_(True) if shortcut else None
    y_ref = gated_causal_fftconv1d_torch(q, k, v, w, s, g1, g2)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    qg, kg, vg, wg = (t.detach().cuda().requires_grad_(True) for t in (q, k, v, w))
    sg = s.detach().cuda().requires_grad_(True) if shortcut else None
    y = hyena_gated_causal_fftconv1d_bhl(qg, kg, vg, wg, sg, g1, g2)
    y.backward(g.cuda())
    assert y.dtype == dtype
    assert rel_l2(y_ref, y) < tol
    for ref_t, hip_t in ((q, qg), (k, kg), (v, vg), (w, wg)) + (((s, sg),) if shortcut else ()):
        assert rel_l2(ref_t.grad, hip_t.grad) < tol


@pytest.mark.parametrize("g1,g2", [("silu", "sigmoid"), ("identity", "identity"), ("silu", "silu"),
                                   ("sigmoid", "identity")])
@pytest.mark.parametrize("B,H,L,K", [(2, 16, 1024, 1024), (3, 8, 300, 17), (2, 4, 100, 180), (1, 4, 8192, 8192)])
def test_fused_plan(B, H, L, K, g1, g2):
    _check(B, H, L, K, g1, g2)


@pytest.mark.parametrize("g1,g2", [("silu", "sigmoid"), ("identity", "identity")])
@pytest.mark.parametrize("B,H,L,K", [(2, 3, 16384, 16384), (1, 2, 65536, 4000), (2, 2, 20001, 9000),
                                     (2, 2, 20000, 36000)])
def test_multi_kernel_plan(B, H, L, K, g1, g2):
    _check(B, H, L, K, g1, g2)


@pytest.mark.parametrize("L", [2048, 32768])
def test_per_sample_filters_and_no_shortcut(L):
    _check(3, 4, L, 257, "silu", "sigmoid", kb=3)
    _check(2, 4, L, 64, "silu", "sigmoid", shortcut=False)


@pytest.mark.parametrize("L", [4096, 65536])
def test_bf16_io(L):
    _check(2, 8, L, L, "silu", "sigmoid", dtype=torch.bfloat16, tol=2e-2)


def test_modules_as_gates_and_default_second_gate():
    torch.manual_seed(3)
    q, k, v = (torch.randn(2, 4, 512, device="cuda") for _ in range(3))
    w = torch.randn(1, 4, 512, device="cuda") / 512 ** 0.5
    a = hyena_gated_causal_fftconv1d_bhl(q, k, v, w, None, torch.nn.SiLU())
    b = hyena_gated_causal_fftconv1d_bhl(q, k, v, w, None, "silu", "silu")
    assert torch.equal(a, b)
    with pytest.raises(NotImplementedError):
        hyena_gated_causal_fftconv1d_bhl(q, k, v, w, None, torch.nn.GELU())


def test_multi_kernel_plan_odd_numel_bf16_and_split_views():
    """4-step plan (elementwise gate kernels around the conv) with B*H*L odd: every workspace sub-buffer
    must start 16-byte aligned.  q / k / v are x.split(H, dim=1) views at B = 1 (k and v start at odd
    element offsets); a no-grad forward keeps y1 in the workspace."""
    B, H, L, K = 1, 3, 20001, 9001
    torch.manual_seed(13)
    x = torch.randn(B, 3 * H, L).to(torch.bfloat16)
    w = torch.randn(1, H, K) / K ** 0.5
    s = torch.randn(H).to(torch.bfloat16)
    xg = x.cuda().requires_grad_(True)
    q, kk, v = xg.split(H, dim=1)
    assert kk.data_ptr() % 16 != 0
    wg, sg = w.cuda().requires_grad_(True), s.cuda().requires_grad_(True)
    y = hyena_gated_causal_fftconv1d_bhl(q, kk, v, wg, sg, "silu", "sigmoid")
    g = torch.randn(y.shape).to(torch.bfloat16)
    y.backward(g.cuda())
    xr = x.clone().requires_grad_(True)
    qr, kr, vr = xr.split(H, dim=1)
    wr, sr = w.clone().requires_grad_(True), s.clone().requires_grad_(True)
    y_ref = gated_causal_fftconv1d_torch(qr, kr, vr, wr, sr, "silu", "sigmoid")
    y_ref.backward(g)
    assert rel_l2(y_ref, y) < 2e-2
    for a, b in ((xr, xg), (wr, wg), (sr, sg)):
        assert rel_l2(a.grad, b.grad) < 2e-2
    with torch.no_grad():
        y0 = hyena_gated_causal_fftconv1d_bhl(q, kk, v, wg, sg, "silu", "sigmoid")
    assert torch.equal(y0, y)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_plan_forward_routes_agree(dtype):
    """B*H*L = 2^22 runs the gate kernels around the plain fused kernel, each half (2^21) the gated kernel: the
    same bits, outputs and gradients; and the large call against the oracle."""
    B, H, L, K = 4, 128, 8192, 8192
    print(f"gated routes B={B} H={H} L={L} {dtype}", flush=True)
    gen = torch.Generator().manual_seed(11)
    q, k, v = (torch.randn(B, H, L, generator=gen).to(dtype) for _ in range(3))
    w = torch.randn(H, K, generator=gen) / K ** 0.5
    s = torch.randn(H, generator=gen).to(dtype)
    g = torch.randn(B, H, L, generator=gen).to(dtype)

    def run(sl):
        ts = [t[sl].cuda().requires_grad_(True) for t in (q, k, v)]
        wg, sg = w.cuda().requires_grad_(True), s.cuda().requires_grad_(True)
        y = hyena_gated_causal_fftconv1d_bhl(*ts, wg, sg, "silu", "sigmoid")
        y.backward(g[sl].cuda())
        return y.detach(), [t.grad for t in ts], wg.grad, sg.grad

    y, gq, gw, gs = run(slice(0, B))
    halves = [run(slice(0, B // 2)), run(slice(B // 2, B))]
    assert torch.equal(y, torch.cat([h[0] for h in halves]))
    for i in range(3):
        assert torch.equal(gq[i], torch.cat([h[1][i] for h in halves]))
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert rel_l2(halves[0][2] + halves[1][2], gw) < 1e-5 and rel_l2(halves[0][3] + halves[1][3], gs) < tol
    y_ref = gated_causal_fftconv1d_torch(q, k, v, w, s, "silu", "sigmoid")
    assert rel_l2(y_ref, y) < tol
