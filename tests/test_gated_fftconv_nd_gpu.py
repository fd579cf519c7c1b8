"""GPU parity of the Hyena-gated 2D/3D FFT conv (``hyena_gated_fftconv{2,3}d_bhl``) against the CPU
composition of the reference (``hyena_nd.py:546-570`` around CKConvND's N-d conv), restated in
``oracle/gated_ref.py``: forward and the gradients of q, k, v, the filter and the shortcut.
Tolerances: 1e-4 rel-L2 for fp32, 2e-2 for bf16 I/O.  Plans with the gates fused into the conv's first and
last passes are also checked bitwise against the gate kernels composed around the plain conv
(``NSQ_ND_GATES_FUSED=0``)."""

import os

import pytest
import torch

from nvsubquadratic_amd import _lib
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


# Plans whose gates run inside the conv's passes: packed 2D rows with the vector epilogue (even crop offset
# along the last axis, its length a multiple of 8) and 3D plane passes (F1 * F2/2 >= 4096).
FUSED_CASES = [  # (S, K, periodic, gate, gate_2, dtype, kb, shortcut)
    ((32, 32), (9, 9), None, "silu", None, torch.float32, 1, True),
    ((32, 32), (9, 9), None, "sigmoid", "silu", torch.bfloat16, 1, True),
    ((32, 16), (5, 9), (True, False), "identity", "sigmoid", torch.float16, 1, False),
    ((24, 40), (7, 13), None, "silu", "identity", torch.bfloat16, 2, True),
    ((8, 8), (3, 3), (False, True), "silu", "silu", torch.float32, 1, True),  # tiled period 8 on the last axis
    ((8, 64, 64), (3, 9, 9), None, "silu", "sigmoid", torch.bfloat16, 1, True),
    ((8, 64, 64), (3, 9, 8), (False, True, False), "sigmoid", None, torch.float32, 2, True),
]


def _gated_run(S, K, periodic, gate, gate_2, dtype, kb, shortcut, fused):
    # The fused gates live in the power-of-two plan's passes (NSQ_ND_R3=0 keeps shapes that the mixed-radix
    # plan would take, which runs the gate kernels around its conv, on that plan).
    old = os.environ.get("NSQ_ND_GATES_FUSED")
    old_r3 = os.environ.get("NSQ_ND_R3")
    os.environ["NSQ_ND_GATES_FUSED"] = "1" if fused else "0"
    os.environ["NSQ_ND_R3"] = "0"
    try:
        torch.manual_seed(7)
        B, H = 2, 4
        leaves = [torch.randn(B, H, *S, device="cuda").to(dtype) for _ in range(3)]
        leaves.append(torch.randn(kb, H, *K, device="cuda"))
        if shortcut:
            leaves.append(torch.randn(H, device="cuda").to(dtype))
        leaves = [t.requires_grad_(True) for t in leaves]
        y = G.hyena_gated_fftconv_nd_bhl(leaves[0], leaves[1], leaves[2], leaves[3],
                                         leaves[4] if shortcut else None, gate, gate_2, periodic)
        g = torch.randn(y.shape, device="cuda", generator=torch.Generator("cuda").manual_seed(3)).to(dtype)
        y.backward(g)
        with torch.no_grad():  # a forward that keeps no y1
            y_ng = G.hyena_gated_fftconv_nd_bhl(*[t.detach() for t in leaves[:4]],
                                                leaves[4].detach() if shortcut else None, gate, gate_2, periodic)
        per = 0 if periodic is None else sum(1 << d for d, f in enumerate(periodic) if f)
        ws = G._gated_nd_ws(leaves[0], torch.empty(kb * H, *K), kb, per, _lib.NSQ_DIR_BWD)
        torch.cuda.synchronize()
        return [y, y_ng] + [t.grad for t in leaves], ws
    finally:
        if old is None:
            del os.environ["NSQ_ND_GATES_FUSED"]
        else:
            os.environ["NSQ_ND_GATES_FUSED"] = old
        if old_r3 is None:
            del os.environ["NSQ_ND_R3"]
        else:
            os.environ["NSQ_ND_R3"] = old_r3


@pytest.mark.parametrize("case", FUSED_CASES)
def test_gates_fused_into_passes_equal_gate_kernels(case):
    """The fused loaders and epilogues round as the gate kernels do, so every output is bitwise equal; the fused
    plan also needs only the conv's workspace (checks that the fused path is the one that ran)."""
    print(f"gated fused vs composed {case}", flush=True)
    fused, ws_f = _gated_run(*case, fused=True)
    comp, ws_c = _gated_run(*case, fused=False)
    assert ws_f < ws_c
    for a, b in zip(fused, comp):
        assert torch.equal(a, b)


def test_gated_3d_plane_fused_against_oracle():
    _check((8, 64, 64), (3, 9, 9), None, "silu", "sigmoid", H=3, B=2)
    _check((8, 64, 64), (3, 9, 9), None, "sigmoid", None, dtype=torch.bfloat16, H=3, B=2, tol=2e-2)
