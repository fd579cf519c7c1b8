"""GPU parity of the 2D / 3D FFT conv on the reference's own FFT sizes (3 * 2^m axes).

The reference pads each axis to F_d = S_d + ceil(K_d / 2) and lets torch.fft run
a mixed-radix plan (nvsubquadratic/ops/fftconv.py:699-702, 774-778); the HIP plan
in csrc/fftconv_nd_r3.h runs the lengths 48, 96 and 192 wherever their spectrum
is smaller than the power-of-two one.  The shapes below reach every plane
instance ((F2/2, F1) in {24, 48} x {48, 96}), every 2D row length (F2/2 in {24,
48, 96}), every axis-0 length, first passes with and without the two-thirds
zero fold (S <= 2F/3), odd and unaligned row lengths, per-sample filters, and
the batch-split adjoint (few channels).
Oracle: fftconv_nd_torch (the reference's torch.fft formula on the CPU) and the
float64 numpy restatement.  Tolerances: rel-L2 <= 1e-4 fp32, <= 2e-2 16-bit I/O.
"""

import pytest
import torch

from nvsubquadratic_amd import _lib
from nvsubquadratic_amd import fftconv_hip as F
from oracle.fftconv_ref import fftconv_nd_np, fftconv_nd_torch, rel_l2


pytestmark = pytest.mark.gpu

# (x shape, kernel shape, FFT lengths of the mixed-radix plan)
R3_SHAPES = [
    ((2, 3, 32, 32, 32), (32, 32, 32), (48, 48, 48)),     # plane (24, 48), two-thirds fold
    ((2, 2, 40, 40, 40), (16, 16, 16), (48, 48, 48)),     # no fold (S > 2F/3), K < S
    ((2, 3, 33, 45, 27), (29, 7, 41), (48, 96, 48)),      # plane (24, 96), odd, unaligned rows
    ((1, 3, 20, 30, 64), (9, 30, 64), (48, 48, 96)),      # plane (48, 48)
    ((1, 2, 50, 60, 70), (40, 50, 30), (96, 96, 96)),     # plane (48, 96), no fold in the plane
    ((1, 2, 128, 32, 32), (128, 32, 32), (192, 48, 48)),  # axis 0 of 192
]


def _nd_fft_lengths(xs, ks, kb=1):
    """FFT lengths the library plans, read back from its workspace size."""
    lib = _lib.get_lib()
    S, K = _lib.i64_array(xs[2:]), _lib.i64_array(ks)
    return lib.nsq_fftconv_nd_workspace_bytes(3, xs[0], xs[1], S, K, kb, _lib.NSQ_DIR_FWD)


def _grad_check(xs, ks, kb=1, dtype=torch.float32, tol=1e-4, seed=0):
    torch.manual_seed(seed)
    H = xs[1]
    x = torch.randn(*xs).to(dtype).requires_grad_(True)
    k = torch.randn(kb, H, *ks, requires_grad=True)
    s = torch.randn(H).to(dtype).requires_grad_(True)
    y_ref = fftconv_nd_torch(x, k, s)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg = x.detach().cuda().requires_grad_(True)
    kg = k.detach().cuda().requires_grad_(True)
    sg = s.detach().cuda().requires_grad_(True)
    y = F.fftconv3d_bhl(xg, kg, sg)
    y.backward(g.cuda())
    assert y.dtype == dtype
    assert rel_l2(y_ref, y) < tol
    assert rel_l2(x.grad, xg.grad) < tol
    assert rel_l2(k.grad, kg.grad) < tol
    assert rel_l2(s.grad, sg.grad) < tol
    return y


@pytest.mark.parametrize("xs,ks,fl", R3_SHAPES)
def test_r3_plan_is_taken(xs, ks, fl):
    """The workspace is sized for the mixed-radix spectrum (F0 F1 (F2/2 + 1) per block)."""
    B, H = xs[0], xs[1]
    assert _nd_fft_lengths(xs, ks) == (B * H + H) * fl[0] * fl[1] * (fl[2] // 2 + 1) * 8


@pytest.mark.parametrize("xs,ks,fl", R3_SHAPES)
def test_r3_fwd_bwd(xs, ks, fl):
    _grad_check(xs, ks)


@pytest.mark.parametrize("xs,ks,fl", [R3_SHAPES[0], R3_SHAPES[2], R3_SHAPES[5]])
def test_r3_film_per_sample_kernel(xs, ks, fl):
    _grad_check(xs, ks, kb=xs[0], seed=1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_r3_16bit_io(dtype):
    y = _grad_check((2, 2, 64, 64, 64), (64, 64, 64), dtype=dtype, tol=2e-2, seed=2)
    torch.manual_seed(2)
    x = torch.randn(2, 2, 64, 64, 64).to(dtype)
    k = torch.randn(1, 2, 64, 64, 64)
    s = torch.randn(2).to(dtype)
    y64 = fftconv_nd_np(x.float().numpy(), k.numpy(), s.float().numpy())
    assert rel_l2(y64, y) < 5e-3


@pytest.mark.parametrize("xs,ks,fl", [R3_SHAPES[0], R3_SHAPES[3], R3_SHAPES[4]])
def test_r3_matches_power_of_two_plan(xs, ks, fl, monkeypatch):
    """The mixed-radix and the power-of-two plans agree to fp32 rounding."""
    torch.manual_seed(3)
    x = torch.randn(*xs, device="cuda", requires_grad=True)
    k = torch.randn(xs[1], *ks, device="cuda", requires_grad=True)
    s = torch.randn(xs[1], device="cuda", requires_grad=True)
    g = torch.randn(*xs, device="cuda")
    outs = []
    for flag in ("1", "0"):
        monkeypatch.setenv("NSQ_ND_R3", flag)
        for t in (x, k, s):
            t.grad = None
        y = F.fftconv3d_bhl(x, k, s)
        y.backward(g)
        outs.append([y.detach().clone(), x.grad.clone(), k.grad.clone(), s.grad.clone()])
    monkeypatch.delenv("NSQ_ND_R3")
    for a, b in zip(*outs):
        assert rel_l2(b, a) < 1e-5


@pytest.mark.parametrize("xs,ks,kb", [((2, 3, 32, 32, 32), (32, 32, 32), 1), ((2, 2, 50, 60, 70), (40, 50, 30), 2)])
def test_r3_backward_reusing_forward_state_is_bitwise_equal(xs, ks, kb):
    torch.manual_seed(4)
    x = torch.randn(*xs, device="cuda")
    k = torch.randn(kb * xs[1], *ks, device="cuda")
    s = torch.randn(xs[1], device="cuda")
    g = torch.randn(*xs, device="cuda")
    lib = _lib.get_lib()
    S, K = _lib.i64_array(xs[2:]), _lib.i64_array(ks)
    need = lib.nsq_fftconv_nd_workspace_bytes(3, xs[0], xs[1], S, K, kb, _lib.NSQ_DIR_BWD)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    y = torch.empty_like(x)
    F.fftconv_nd_fwd_raw(x, k, s, y, kb, ws)
    outs = []
    for state, w in ((True, ws), (False, None)):
        gx, gk, gs = torch.empty_like(x), torch.empty_like(k), torch.empty(kb * xs[1], device="cuda")
        F.fftconv_nd_bwd_raw(g, x, k, s, gx, gk, gs, kb, w, fwd_state=state)
        outs.append((gx, gk, gs))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    y2 = torch.empty_like(x)
    F.fftconv_nd_fwd_raw(x, k, s, y2, kb)  # minimum workspace: product in place
    assert torch.equal(y, y2)


def test_r3_chunked_bitwise():
    torch.manual_seed(5)
    x = torch.randn(1, 40, 32, 32, 32, device="cuda")
    k = torch.randn(40, 32, 32, 32, device="cuda")
    assert torch.equal(F.fftconv3d_bhl(x, k), F.fftconv3d_bhl_chunked(x, k, chunk_size=16))


# 2D: (x shape, kernel shape, FFT lengths (F0, F2)); row kernels at F2/2 in {24, 48, 96}, axis 0 of 48 / 96 / 192.
R3_SHAPES_2D = [
    ((2, 3, 128, 128), (128, 128), (192, 192)),  # config 4's geometry
    ((2, 4, 64, 64), (64, 64), (96, 96)),
    ((3, 2, 32, 32), (32, 32), (48, 48)),
    ((2, 3, 90, 27), (7, 41), (96, 48)),        # odd, unaligned rows, no fold on axis 0
    ((1, 2, 120, 70), (100, 41), (192, 96)),    # no fold on the rows
]


def _grad_check_2d(xs, ks, kb=1, dtype=torch.float32, tol=1e-4, seed=0):
    torch.manual_seed(seed)
    H = xs[1]
    x = torch.randn(*xs).to(dtype).requires_grad_(True)
    k = torch.randn(kb, H, *ks, requires_grad=True)
    s = torch.randn(H).to(dtype).requires_grad_(True)
    y_ref = fftconv_nd_torch(x, k, s)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg, kg, sg = (t.detach().cuda().requires_grad_(True) for t in (x, k, s))
    y = F.fftconv2d_bhl(xg, kg, sg)
    y.backward(g.cuda())
    assert y.dtype == dtype
    assert rel_l2(y_ref, y) < tol
    assert rel_l2(x.grad, xg.grad) < tol
    assert rel_l2(k.grad, kg.grad) < tol
    assert rel_l2(s.grad, sg.grad) < tol
    return y


@pytest.mark.parametrize("xs,ks,fl", R3_SHAPES_2D)
def test_r3_2d_plan_is_taken(xs, ks, fl):
    lib = _lib.get_lib()
    S, K = _lib.i64_array(xs[2:]), _lib.i64_array(ks)
    got = lib.nsq_fftconv_nd_workspace_bytes(2, xs[0], xs[1], S, K, 1, _lib.NSQ_DIR_FWD)
    assert got == (xs[0] * xs[1] + xs[1]) * fl[0] * (fl[1] // 2 + 1) * 8


@pytest.mark.parametrize("xs,ks,fl", R3_SHAPES_2D)
def test_r3_2d_fwd_bwd(xs, ks, fl):
    _grad_check_2d(xs, ks)


@pytest.mark.parametrize("xs,ks,fl", [R3_SHAPES_2D[0], R3_SHAPES_2D[3]])
def test_r3_2d_film_per_sample_kernel(xs, ks, fl):
    _grad_check_2d(xs, ks, kb=xs[0], seed=1)


def test_r3_2d_bf16_config4_geometry():
    """Config 4's geometry (128^2, K = 128, FFT 192^2) in bf16 I/O against the float64 restatement."""
    y = _grad_check_2d((2, 4, 128, 128), (128, 128), dtype=torch.bfloat16, tol=2e-2, seed=2)
    torch.manual_seed(2)
    x = torch.randn(2, 4, 128, 128).to(torch.bfloat16)
    k = torch.randn(1, 4, 128, 128)
    s = torch.randn(4).to(torch.bfloat16)
    assert rel_l2(fftconv_nd_np(x.float().numpy(), k.numpy(), s.float().numpy()), y) < 5e-3


@pytest.mark.parametrize("xs,ks,fl", [R3_SHAPES_2D[0], R3_SHAPES_2D[4]])
def test_r3_2d_matches_power_of_two_plan(xs, ks, fl, monkeypatch):
    torch.manual_seed(3)
    x = torch.randn(*xs, device="cuda", requires_grad=True)
    k = torch.randn(xs[1], *ks, device="cuda", requires_grad=True)
    s = torch.randn(xs[1], device="cuda", requires_grad=True)
    g = torch.randn(*xs, device="cuda")
    outs = []
    for flag in ("1", "0"):
        monkeypatch.setenv("NSQ_ND_R3", flag)
        for t in (x, k, s):
            t.grad = None
        y = F.fftconv2d_bhl(x, k, s)
        y.backward(g)
        outs.append([y.detach().clone(), x.grad.clone(), k.grad.clone(), s.grad.clone()])
    monkeypatch.delenv("NSQ_ND_R3")
    for a, b in zip(*outs):
        assert rel_l2(b, a) < 1e-5


def test_r3_2d_backward_reusing_forward_state_is_bitwise_equal():
    torch.manual_seed(4)
    xs, ks, kb = (2, 3, 128, 128), (128, 128), 2
    x = torch.randn(*xs, device="cuda")
    k = torch.randn(kb * xs[1], *ks, device="cuda")
    s = torch.randn(xs[1], device="cuda")
    g = torch.randn(*xs, device="cuda")
    lib = _lib.get_lib()
    S, K = _lib.i64_array(xs[2:]), _lib.i64_array(ks)
    need = lib.nsq_fftconv_nd_workspace_bytes(2, xs[0], xs[1], S, K, kb, _lib.NSQ_DIR_BWD)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    y = torch.empty_like(x)
    F.fftconv_nd_fwd_raw(x, k, s, y, kb, ws)
    outs = []
    for state, w in ((True, ws), (False, None)):
        gx, gk, gs = torch.empty_like(x), torch.empty_like(k), torch.empty(kb * xs[1], device="cuda")
        F.fftconv_nd_bwd_raw(g, x, k, s, gx, gk, gs, kb, w, fwd_state=state)
        outs.append((gx, gk, gs))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    y2 = torch.empty_like(x)
    F.fftconv_nd_fwd_raw(x, k, s, y2, kb)
    assert torch.equal(y, y2)


# The one-kernel image forward on the 192 x 192 plane (fftconv2d_image192.h) runs a 2D forward that keeps no
# state (no gradient wanted) when F0 = F2 = 192, S0, S2 <= 128, S2 % 8 == 0 and K2 // 2 is even; forwards that keep
# a state run the three passes.  Both against the oracle, and against each other.
IMAGE192_SHAPES = [
    ((2, 8, 128, 128), (128, 128)),   # config 4's geometry: every row and column of the tile
    ((3, 5, 100, 104), (100, 168)),   # a partial row group, crop offsets 50 / 84
    ((2, 3, 128, 128), (127, 128)),   # odd K0 (o0 = 63)
    ((1, 2, 128, 120), (65, 129)),    # o2 = 64 from an odd K2, S2 = 120
]


@pytest.mark.parametrize("xs,ks", IMAGE192_SHAPES)
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2), (torch.float16, 2e-2)])
@pytest.mark.parametrize("shortcut", [True, False])
def test_image192_forward(xs, ks, dtype, tol, shortcut):
    print(f"image192 case {xs} {ks} {dtype} shortcut={shortcut}", flush=True)
    torch.manual_seed(6)
    H = xs[1]
    x = torch.randn(*xs).to(dtype)
    k = torch.randn(H, *ks)
    s = torch.randn(H).to(dtype) if shortcut else None
    y_ref = fftconv_nd_torch(x, k[None], s if s is not None else torch.zeros(H, dtype=dtype))
    xg, kg = x.cuda(), k.cuda()
    sg = s.cuda() if s is not None else None
    with torch.no_grad():
        y = F.fftconv2d_bhl(xg, kg, sg)
    assert y.dtype == dtype
    assert rel_l2(y_ref, y) < tol
    # the three passes (a forward that keeps its state for the backward) on the same inputs
    xr = xg.clone().requires_grad_(True)
    y3 = F.fftconv2d_bhl(xr, kg, sg)
    assert rel_l2(y3.detach(), y) < (1e-5 if dtype == torch.float32 else 1e-2)


def test_image192_config4_fp32_against_float64():
    torch.manual_seed(7)
    x = torch.randn(2, 8, 128, 128)
    k = torch.randn(8, 128, 128)
    s = torch.randn(8)
    with torch.no_grad():
        y = F.fftconv2d_bhl(x.cuda(), k.cuda(), s.cuda())
    assert rel_l2(fftconv_nd_np(x.numpy(), k[None].numpy(), s.numpy()), y) < 2e-6
