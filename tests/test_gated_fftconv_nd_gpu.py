"""GPU parity of the Hyena-gated 2D/3D FFT conv (``hyena_gated_fftconv{2,3}d_bhl``) against the CPU
composition of the reference (``hyena_nd.py:546-570`` around CKConvND's N-d conv), restated in
``oracle/gated_ref.py``: forward and the gradients of q, k, v, the filter and the shortcut.
Tolerances: 1e-4 rel-L2 for fp32, 2e-2 for bf16 I/O."""

import pytest
import torch

from nvsubquadratic_amd import gated_fftconv_hip as G
from nvsubquadratic_amd import fftconv_hip as Z
from oracle.gated_ref import gated_fftconv_nd_torch

pytestmark = pytest.mark.gpu


def rel_l2(ref, out) -> float:
    r = ref.detach().cpu().double()
    o = out.detach().cpu().double()
    return float((o - r).norm() / r.norm().clamp_min(1e-30))


def _check(S, K, periodic, gate, gate_2, dtype=torch.float32, kb=1, B=2, H=6, tol=1e-4, shortcut=True):
    torch.manual_seed(sum(S) + sum(K))
    q, kg, v = (torch.randn(B, H, *S).to(dtype).requires_grad_(True) for _ in range(3))
    k = torch.randn(kb, H, *K, requires_grad=True)
    s = torch.randn(H).to(dtype).requires_grad_(True) if shortcut else None
    per = (False,) * len(S) if periodic is None else periodic
    y_ref = gated_fftconv_nd_torch(q, kg, v, k, per, s, gate, gate_2, compute_dtype=torch.float64)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    leaves = [q, kg, v, k] + ([s] if shortcut else [])
    dev = [t.detach().cuda().requires_grad_(True) for t in leaves]
    print(f"gated nd S={S} K={K} periodic={periodic} {gate}/{gate_2} {dtype} kb={kb}", flush=True)
    y = G.hyena_gated_fftconv_nd_bhl(dev[0], dev[1], dev[2], dev[3], dev[4] if shortcut else None, gate, gate_2,
                                     periodic)
    y.backward(g.cuda())
    assert y.dtype == dtype and y.shape == q.shape
    assert rel_l2(y_ref, y) < tol
    for a, b in zip(leaves, dev):
        assert rel_l2(a.grad, b.grad) < tol


@pytest.mark.parametrize("gate,gate_2", [("silu", None), ("sigmoid", "identity"), ("identity", "silu")])
def test_gated_2d(gate, gate_2):
    _check((16, 24), (5, 7), None, gate, gate_2)


@pytest.mark.parametrize("periodic", [(True, False), (True, True)])
def test_gated_2d_periodic_axes(periodic):
    _check((32, 16), (5, 9), periodic, "silu", None)


@pytest.mark.parametrize("S,K,periodic", [((24, 20), (5, 7), (True, False)), ((24, 20), (5, 6), (True, True)),
                                          ((12, 10, 8), (3, 4, 5), (True, True, False))])
def test_gated_periodic_non_power_of_two(S, K, periodic):
    """Periodic lengths that are not powers of two: torch gates around the conv on the periodic extension."""
    _check(S, K, periodic, "silu", "sigmoid")
    _check(S, K, periodic, "identity", None, dtype=torch.bfloat16, tol=2e-2)


def test_gated_3d():
    _check((8, 16, 12), (3, 5, 4), None, "silu", "sigmoid", H=4)


def test_gated_3d_mixed_per_sample_filter():
    _check((16, 8, 16), (5, 3, 4), (True, False, True), "sigmoid", None, kb=2, H=4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gated_2d_half_io(dtype):
    _check((32, 32), (9, 9), None, "silu", None, dtype=dtype, tol=2e-2)


def test_gated_2d_no_shortcut_identity_gates_equal_plain_conv():
    torch.manual_seed(4)
    x = torch.randn(2, 8, 24, 20, device="cuda")
    k = torch.randn(1, 8, 7, 5, device="cuda")
    one = torch.ones_like(x)
    y = G.hyena_gated_fftconv2d_bhl(x, one, one, k, None, "identity", "identity")
    assert rel_l2(Z.fftconv2d_bhl(x, k), y) < 1e-6


def test_gated_nd_argument_errors():
    q = torch.randn(1, 2, 8, 8, device="cuda")
    with pytest.raises(ValueError, match="share one"):
        G.hyena_gated_fftconv_nd_bhl(q, q, q[..., :4], torch.randn(1, 2, 3, 3, device="cuda"))
    with pytest.raises(ValueError, match="periodic"):
        G.hyena_gated_fftconv2d_bhl(q, q, q, torch.randn(1, 2, 3, 3, device="cuda"), periodic=(True,))
    with pytest.raises(NotImplementedError):
        G.hyena_gated_fftconv2d_bhl(q, q, q, torch.randn(1, 2, 3, 3, device="cuda"), gate_nonlinear=torch.nn.GELU())


def test_gated_2d_odd_numel_bf16_and_split_views():
    """B*H*prod(S) odd: the workspace sub-buffers (z, y1, dy1, dz) follow one another and must each start
    16-byte aligned for the vectorized gate kernels.  The q / k / v come from x.split(H, dim=1) at B = 1,
    as Hyena takes them, so k and v start at odd element offsets; a no-grad forward keeps y1 in the
    workspace."""
    B, H, S, K = 1, 3, (15, 17), (5, 7)
    torch.manual_seed(12)
    x = torch.randn(B, 3 * H, *S).to(torch.bfloat16)
    w = torch.randn(1, H, *K)
    s = torch.randn(H).to(torch.bfloat16)
    xg = x.cuda().requires_grad_(True)
    q, kk, v = xg.split(H, dim=1)
    assert kk.data_ptr() % 16 != 0
    wg, sg = w.cuda().requires_grad_(True), s.cuda().requires_grad_(True)
    y = G.hyena_gated_fftconv2d_bhl(q, kk, v, wg, sg, "silu", "sigmoid")
    g = torch.randn(y.shape).to(torch.bfloat16)
    y.backward(g.cuda())
    xr = x.clone().requires_grad_(True)
    qr, kr, vr = xr.split(H, dim=1)
    wr, sr = w.clone().requires_grad_(True), s.clone().requires_grad_(True)
    y_ref = gated_fftconv_nd_torch(qr, kr, vr, wr, (False, False), sr, "silu", "sigmoid",
                                   compute_dtype=torch.float64)
    y_ref.backward(g)
    assert rel_l2(y_ref, y) < 2e-2
    for a, b in ((xr, xg), (wr, wg), (sr, sg)):
        assert rel_l2(a.grad, b.grad) < 2e-2
    with torch.no_grad():
        y0 = G.hyena_gated_fftconv2d_bhl(q, kk, v, wg, sg, "silu", "sigmoid")
    assert torch.equal(y0, y)
