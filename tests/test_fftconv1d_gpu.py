"""GPU parity of the HIP causal 1D FFT conv against the CPU oracle.

Mirrors the reference's own test matrix (tests/ops/test_fftconv_custom_1d.py:
shapes :106-113, BLH :133-144, shortcut :146-156, chunked :159-180, backward
:183-200, dtypes :203-212, long kernels :215-228) and adds the BASELINE
configs: config 1 whole, config 3 on a channel sample at full length, and
size-independent properties (adjoint identity, delta filter) at full size.

Tolerances: rel-L2 <= 1e-4 for fp32, <= 2e-2 for bf16
I/O; the reference tests' own elementwise bounds are also applied where they
mirror a reference test.
"""

import os

import numpy as np
import pytest
import torch

from nvsubquadratic_amd import fftconv_hip as F
from nvsubquadratic_amd.workloads import causal1d_case
from oracle.fftconv_ref import causal_fftconv1d_np, causal_fftconv1d_torch, rel_l2


pytestmark = pytest.mark.gpu

RTOL_F32_L2 = 1e-4
RTOL_BF16_L2 = 2e-2
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "causal1d.npz")

SHARED_SHAPES = [
    (2, 64, 256, 7),
    (4, 128, 512, 7),
    (1, 256, 1024, 15),
    (2, 32, 128, 3),
    (1, 96, 2048, 65),
    (2, 64, 64, 64),  # K == L
]


def _ref(x, k, s=None):
    return causal_fftconv1d_torch(x.detach().cpu(), k.detach().cpu(), None if s is None else s.detach().cpu())


@pytest.mark.parametrize("B,H,L,K", SHARED_SHAPES)
def test_bhl_shared_kernel(B, H, L, K):
    torch.manual_seed(42)
    x = torch.randn(B, H, L)
    k = torch.randn(1, H, K)
    y = F.causal_fftconv1d_bhl(x.cuda(), k.cuda())
    y_ref = _ref(x, k)
    torch.testing.assert_close(y.cpu(), y_ref, atol=1e-3, rtol=1e-4)
    assert rel_l2(y_ref, y) < RTOL_F32_L2


@pytest.mark.parametrize("B,H,L,K", SHARED_SHAPES)
def test_blh_shared_kernel(B, H, L, K):
    torch.manual_seed(42)
    x = torch.randn(B, L, H)
    k = torch.randn(1, K, H)
    y = F.causal_fftconv1d_bhl_w_reshape(x.cuda(), k.cuda())
    xb = x.permute(0, 2, 1)
    kb = k.permute(0, 2, 1)
    y_ref = _ref(xb, kb).permute(0, 2, 1)
    torch.testing.assert_close(y.cpu(), y_ref, atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("B,H,L,K", SHARED_SHAPES[:3])
def test_shortcut_semantics(B, H, L, K):
    torch.manual_seed(42)
    x = torch.randn(B, H, L)
    k = torch.randn(1, H, K)
    s = torch.randn(H)
    y = F.causal_fftconv1d_bhl(x.cuda(), k.cuda(), s.cuda())
    torch.testing.assert_close(y.cpu(), _ref(x, k, s), atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("B,H,L,K", SHARED_SHAPES[:4])
@pytest.mark.parametrize("chunk_size", [16, 32, 128])
def test_chunked_matches_bitwise(B, H, L, K, chunk_size):
    torch.manual_seed(42)
    x = torch.randn(B, H, L, device="cuda")
    k = torch.randn(1, H, K, device="cuda")
    s = torch.randn(H, device="cuda")
    y = F.causal_fftconv1d_bhl(x, k, s)
    yc = F.causal_fftconv1d_bhl_chunked(x, k, s, chunk_size)
    assert torch.equal(y, yc)


def test_blh_chunked_matches():
    torch.manual_seed(42)
    x = torch.randn(2, 256, 64, device="cuda")
    k = torch.randn(1, 7, 64, device="cuda")
    y = F.causal_fftconv1d_bhl_w_reshape(x, k)
    yc = F.causal_fftconv1d_blh_chunked(x, k, chunk_size=32)
    assert torch.equal(y, yc)


@pytest.mark.parametrize("B,H,L,K", [(2, 64, 256, 7), (4, 32, 128, 5), (2, 16, 64, 64), (1, 8, 1024, 1024)])
def test_grad_matches_reference(B, H, L, K):
    torch.manual_seed(42)
    x = torch.randn(B, H, L, requires_grad=True)
    k = torch.randn(1, H, K, requires_grad=True)
    s = torch.randn(H, requires_grad=True)
    y_ref = causal_fftconv1d_torch(x, k, s)
    gy = torch.randn_like(y_ref)
    y_ref.backward(gy)
    xg = x.detach().cuda().requires_grad_(True)
    kg = k.detach().cuda().requires_grad_(True)
    sg = s.detach().cuda().requires_grad_(True)
    y = F.causal_fftconv1d_bhl(xg, kg, sg)
    y.backward(gy.cuda())
    torch.testing.assert_close(xg.grad.cpu(), x.grad, atol=1e-2, rtol=1e-3)
    torch.testing.assert_close(kg.grad.cpu(), k.grad, atol=1e-2, rtol=1e-3)
    torch.testing.assert_close(sg.grad.cpu(), s.grad, atol=1e-2, rtol=1e-3)
    assert rel_l2(x.grad, xg.grad) < RTOL_F32_L2
    assert rel_l2(k.grad, kg.grad) < RTOL_F32_L2
    assert rel_l2(s.grad, sg.grad) < RTOL_F32_L2


@pytest.mark.parametrize("in_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dtype_preserved(in_dtype):
    torch.manual_seed(0)
    x = torch.randn(2, 32, 128, device="cuda", dtype=in_dtype)
    k = torch.randn(1, 32, 5, device="cuda", dtype=in_dtype)
    y = F.causal_fftconv1d_bhl(x, k)
    assert y.dtype == in_dtype
    assert torch.isfinite(y).all()
    y_ref = _ref(x, k)
    assert rel_l2(y_ref, y) < (RTOL_F32_L2 if in_dtype == torch.float32 else RTOL_BF16_L2)


@pytest.mark.parametrize("K", [128, 512, 2048])
def test_long_kernel_matches_reference(K):
    torch.manual_seed(42)
    B, H, L = 1, 32, max(K, 256)
    x = torch.randn(B, H, L)
    k = torch.randn(1, H, K)
    y = F.causal_fftconv1d_bhl(x.cuda(), k.cuda())
    torch.testing.assert_close(y.cpu(), _ref(x, k), atol=1e-3, rtol=1e-4)


def test_golden_fixtures_forward_and_backward():
    d = np.load(GOLDEN)
    for i in range(int(d["n_causal"])):
        x = torch.tensor(d[f"c{i}_x"], dtype=torch.float32, device="cuda", requires_grad=True)
        k = torch.tensor(d[f"c{i}_k"], dtype=torch.float32, device="cuda", requires_grad=True)
        s = torch.tensor(d[f"c{i}_s"], dtype=torch.float32, device="cuda", requires_grad=True)
        y = F.causal_fftconv1d_bhl(x, k[None], s)
        assert rel_l2(d[f"c{i}_y"], y) < 1e-5, f"case {i} y"
        y.backward(torch.tensor(d[f"c{i}_g"], dtype=torch.float32, device="cuda"))
        assert rel_l2(d[f"c{i}_gx"], x.grad) < 1e-5, f"case {i} gx"
        assert rel_l2(d[f"c{i}_gk"], k.grad) < 1e-5, f"case {i} gk"
        assert rel_l2(d[f"c{i}_gs"], s.grad) < 1e-5, f"case {i} gs"


@pytest.mark.parametrize("B,H,L,K", [(1, 4, 100, 150), (2, 3, 1000, 2000), (1, 2, 4096, 8192), (2, 2, 33, 60)])
def test_kernel_longer_than_l_plus_one_wraps_like_reference(B, H, L, K):
    torch.manual_seed(3)
    x = torch.randn(B, H, L, requires_grad=True)
    k = torch.randn(1, H, K, requires_grad=True)
    y_ref = causal_fftconv1d_torch(x, k)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg = x.detach().cuda().requires_grad_(True)
    kg = k.detach().cuda().requires_grad_(True)
    y = F.causal_fftconv1d_bhl(xg, kg)
    y.backward(g.cuda())
    assert rel_l2(y_ref, y) < RTOL_F32_L2
    assert rel_l2(x.grad, xg.grad) < RTOL_F32_L2
    assert rel_l2(k.grad, kg.grad) < RTOL_F32_L2


@pytest.mark.parametrize("L,K", [(3, 3), (1, 1), (1, 2), (5, 1), (257, 3), (8191, 8191)])
def test_ragged_and_tiny_lengths(L, K):
    torch.manual_seed(5)
    x = torch.randn(3, 5, L)
    k = torch.randn(5, K)
    s = torch.randn(5)
    y = F.causal_fftconv1d_bhl(x.cuda(), k.cuda(), s.cuda())
    assert rel_l2(_ref(x, k, s), y) < RTOL_F32_L2


# ---------------------------------------------------------------------------
# 4-step plan (FFT length >= 2^15) and the BASELINE configs
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("B", [1, 2])
@pytest.mark.parametrize("L,K", [(16384, 16384), (20000, 9000), (65536, 65536), (131072, 1000)])
def test_four_step_fp32_fwd_bwd(L, K, B):
    torch.manual_seed(7)
    H = 3
    x = torch.randn(B, H, L, requires_grad=True)
    k = torch.randn(1, H, K, requires_grad=True)
    s = torch.randn(H, requires_grad=True)
    y_ref = causal_fftconv1d_torch(x, k, s)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg = x.detach().cuda().requires_grad_(True)
    kg = k.detach().cuda().requires_grad_(True)
    sg = s.detach().cuda().requires_grad_(True)
    y = F.causal_fftconv1d_bhl(xg, kg, sg)
    y.backward(g.cuda())
    assert rel_l2(y_ref, y) < RTOL_F32_L2
    assert rel_l2(x.grad, xg.grad) < RTOL_F32_L2
    assert rel_l2(k.grad, kg.grad) < RTOL_F32_L2
    assert rel_l2(s.grad, sg.grad) < RTOL_F32_L2


@pytest.mark.parametrize("B,H,L,K,kb", [(1, 3, 32768, 65536, 1), (2, 2, 20000, 30000, 1), (1, 2, 12000, 24000, 1),
                                        (2, 2, 20000, 40000, 2), (1, 2, 40000, 40002, 1)])
def test_four_step_kernel_longer_than_l_plus_one(B, H, L, K, kb):
    """K > L+1 beyond the fused plan (FFT length >= 2^15): the reference's length-2L FFT wraps
    (fftconv.py:576-580); the 4-step plan adds the wrap through a copy of x (forward) or g (backward)
    at the wrap offset.  L = 2^15, K = 2L is the longest kernel the reference accepts at that length;
    kb = B runs per-sample filters; K = L + 2 is the first length that wraps."""
    torch.manual_seed(L + K)
    x = torch.randn(B, H, L, requires_grad=True)
    k = (torch.randn(kb, H, K) / K ** 0.5).requires_grad_(True)
    s = torch.randn(H, requires_grad=True)
    y_ref = causal_fftconv1d_torch(x, k, s)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg, kg, sg = (t.detach().cuda().requires_grad_(True) for t in (x, k, s))
    y = F.causal_fftconv1d_bhl(xg, kg, sg)
    y.backward(g.cuda())
    assert rel_l2(y_ref, y) < RTOL_F32_L2
    assert rel_l2(x.grad, xg.grad) < RTOL_F32_L2
    assert rel_l2(k.grad, kg.grad) < RTOL_F32_L2
    assert rel_l2(s.grad, sg.grad) < RTOL_F32_L2
    # no-grad forward (the conv runs in place of x's block, no kept state) gives the same y
    with torch.no_grad():
        assert torch.equal(F.causal_fftconv1d_bhl(xg, kg, sg), y)


def test_four_step_fold_bf16_against_float64():
    torch.manual_seed(12)
    B, H, L, K = 1, 4, 32768, 65536
    x = torch.randn(B, H, L).to(torch.bfloat16)
    k = torch.randn(H, K) / K ** 0.5
    y = F.causal_fftconv1d_bhl(x.cuda(), k.cuda())
    y64 = causal_fftconv1d_np(x.float().numpy(), k.numpy())
    assert rel_l2(y64, y) < 5e-3


def test_config1_fp32_fwd_bwd():
    """B=2, D=128, L=4096, fp32, decaying filter a~U(1,10)."""
    c = causal1d_case(2, 128, 4096, torch.float32, (1.0, 10.0))
    x = c.x.clone().requires_grad_(True)
    k = c.k[None].clone().requires_grad_(True)
    s = c.s.clone().requires_grad_(True)
    y_ref = causal_fftconv1d_torch(x, k, s)
    y_ref.backward(c.g)
    xg = c.x.cuda().requires_grad_(True)
    kg = c.k[None].cuda().requires_grad_(True)
    sg = c.s.cuda().requires_grad_(True)
    y = F.causal_fftconv1d_bhl(xg, kg, sg)
    y.backward(c.g.cuda())
    assert rel_l2(y_ref, y) < RTOL_F32_L2
    assert rel_l2(x.grad, xg.grad) < RTOL_F32_L2
    assert rel_l2(k.grad, kg.grad) < RTOL_F32_L2
    assert rel_l2(s.grad, sg.grad) < RTOL_F32_L2


@pytest.mark.parametrize("L", [2048, 4096, 8192])
@pytest.mark.parametrize("dtype,film", [(torch.float32, False), (torch.bfloat16, False), (torch.float32, True)])
def test_fused_pair_and_single_kernels_agree(L, dtype, film):
    """The fused forward runs up to 1536 / 1536 / 256 rows (B*H) of FFT lengths 4096 / 8192 / 16384 on the
    two-transform (filter | row) workgroup and larger grids on the one-transform kernel: 8 channels past that bound
    take the latter, the bound's worth of them the former.  At FFT length 16384 both run radix-16 passes and agree
    bit for bit; up to 8192 the pair kernel runs radix-8 passes (8 points per thread, twice the threads), so the two
    agree to fp32 rounding (rel-L2 <= 1e-6 on fp32 outputs; <= 1e-3 on bf16 outputs, where a rounding difference can
    move an output by one bf16 step) and the pair kernel repeats bit for bit.  Both meet the oracle."""
    torch.manual_seed(31)
    B = 2 if film else 1
    rows = {2048: 1536, 4096: 1536, 8192: 256}[L]
    H, Hp = rows // B + 8, rows // B
    x = torch.randn(B, H, L).to(dtype)
    k = torch.randn(B if film else 1, H, L) * torch.exp(-torch.linspace(0, 8, L))
    s = torch.randn(H).to(dtype)
    xd, kd, sd = x.cuda(), k.cuda(), s.cuda()
    y_single = F.causal_fftconv1d_bhl(xd, kd, sd)
    y_pair = F.causal_fftconv1d_bhl(xd[:, :Hp].contiguous(), kd[:, :Hp].contiguous(), sd[:Hp].contiguous())
    if L == 8192:
        assert torch.equal(y_pair, y_single[:, :Hp])
    else:
        assert rel_l2(y_single[:, :Hp], y_pair) < (1e-6 if dtype == torch.float32 else 1e-3)
        y_again = F.causal_fftconv1d_bhl(xd[:, :Hp].contiguous(), kd[:, :Hp].contiguous(), sd[:Hp].contiguous())
        assert torch.equal(y_pair, y_again)
    tol = RTOL_F32_L2 if dtype == torch.float32 else RTOL_BF16_L2
    y64 = np.concatenate([causal_fftconv1d_np(x[b:b + 1].float().numpy(), k[b if film else 0].numpy(),
                                              s.float().numpy()) for b in range(B)])
    assert rel_l2(y64, y_single) < tol
    assert rel_l2(y64[:, :Hp], y_pair) < tol


def test_config3_channel_sample_bf16_fwd_bwd():
    """BASELINE config 3 at full length L=262144 on a 4-channel sample (bf16 I/O)."""
    L = 262144
    c = causal1d_case(1, 4096, L, torch.bfloat16, (1.0, 50.0), channels=slice(1000, 1004))
    x = c.x.clone().requires_grad_(True)
    k = c.k[None].clone().requires_grad_(True)
    s = c.s.clone().requires_grad_(True)
    y_ref = causal_fftconv1d_torch(x, k, s)
    y_ref.backward(c.g)
    xg = c.x.cuda().requires_grad_(True)
    kg = c.k[None].cuda().requires_grad_(True)
    sg = c.s.cuda().requires_grad_(True)
    y = F.causal_fftconv1d_bhl(xg, kg, sg)
    y.backward(c.g.cuda())
    assert y.dtype == torch.bfloat16
    assert rel_l2(y_ref, y) < RTOL_BF16_L2
    assert rel_l2(x.grad, xg.grad) < RTOL_BF16_L2
    assert rel_l2(k.grad, kg.grad) < RTOL_BF16_L2
    assert rel_l2(s.grad, sg.grad) < RTOL_BF16_L2
    # the fp32 spectrum path itself is far tighter than the bf16 budget
    y64 = causal_fftconv1d_np(c.x.float().numpy(), c.k.numpy(), c.s.float().numpy())
    assert rel_l2(y64, y) < 5e-3


def test_config3_full_size_properties():
    """Full config-3 shape (B=1, D=4096, L=262144): size-independent checks.

    * adjoint identity <conv(x), g> == <x, conv^T(g)> and <conv(x), g> == <k, gk>
      (float32 I/O so no output rounding enters);
    * a delta filter reproduces the input exactly (up to fp32 FFT error);
    * the bf16 forward agrees with the CPU oracle on 3 sampled channels.
    """
    H, L = 4096, 262144
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    x = torch.randn(1, H, L, device="cuda", generator=gen)
    a = torch.rand(H, 1, device="cuda", generator=gen) * 49 + 1
    k = torch.randn(H, L, device="cuda", generator=gen)
    k *= torch.exp(-a * torch.arange(L, device="cuda").float().view(1, L) / L)
    g = torch.randn(1, H, L, device="cuda", generator=gen)
    y = F.causal_fftconv1d_bhl(x, k)
    gx = torch.empty_like(x)
    gk = torch.empty_like(k)
    F.causal_fftconv1d_bwd_raw(g, x, k, None, gx, gk, None)
    lhs = torch.dot(y.flatten().double(), g.flatten().double()).item()
    rhs1 = torch.dot(x.flatten().double(), gx.flatten().double()).item()
    rhs2 = torch.dot(k.flatten().double(), gk.flatten().double()).item()
    scale = y.double().norm().item() * g.double().norm().item()
    assert abs(lhs - rhs1) / scale < 1e-5
    assert abs(lhs - rhs2) / scale < 1e-5
    # sampled channels vs oracle
    for h in (0, 1777, 4095):
        y_ref = causal_fftconv1d_np(x[:, h:h + 1].cpu().numpy(), k[h:h + 1].cpu().numpy())
        assert rel_l2(y_ref, y[:, h:h + 1]) < RTOL_F32_L2
    del gx, gk
    # delta filter
    kd = torch.zeros_like(k)
    kd[:, 0] = 1.0
    yd = F.causal_fftconv1d_bhl(x, kd)
    assert rel_l2(x, yd) < 1e-5


@pytest.mark.parametrize("B", [1, 2])
@pytest.mark.parametrize("L", [16384, 65536])
def test_backward_reusing_forward_state_is_bitwise_equal(L, B):
    """The forward keeps its transformed x, k in a backward-sized workspace; reuse == recompute."""
    from nvsubquadratic_amd import _lib

    torch.manual_seed(8)
    H = 3
    x = torch.randn(B, H, L, device="cuda").to(torch.bfloat16)
    k = torch.randn(H, L, device="cuda")
    s = torch.randn(H, device="cuda").to(torch.bfloat16)
    g = torch.randn(B, H, L, device="cuda").to(torch.bfloat16)
    need = _lib.get_lib().nsq_fftconv1d_causal_workspace_bytes(B, H, L, L, _lib.NSQ_DIR_BWD)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    y = torch.empty_like(x)
    F.causal_fftconv1d_fwd_raw(x, k, s, y, ws)
    outs = []
    for state, w in ((True, ws), (False, None)):
        gx, gk, gs = torch.empty_like(x), torch.empty_like(k), torch.empty(H, device="cuda")
        F.causal_fftconv1d_bwd_raw(g, x, k, s, gx, gk, gs, w, fwd_state=state)
        outs.append((gx, gk, gs))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    y2 = torch.empty_like(x)
    F.causal_fftconv1d_fwd_raw(x, k, s, y2)  # minimum workspace, in-place plan
    assert torch.equal(y, y2)


@pytest.mark.parametrize("L", [16384, 65536])
def test_single_row_backward_matches_batched(L):
    """B == 1 runs its own backward row kernel: per-row gx and gk agree with the batched call.

    The two kernels may contract products into FMAs differently, so agreement is to
    rounding (bf16 gx: a last-bit flip here and there), not bitwise.
    """
    torch.manual_seed(10)
    B, H = 2, 3
    x = torch.randn(B, H, L, device="cuda").to(torch.bfloat16)
    k = torch.randn(H, L, device="cuda")
    s = torch.randn(H, device="cuda").to(torch.bfloat16)
    g = torch.randn(B, H, L, device="cuda").to(torch.bfloat16)
    gx, gk, gs = torch.empty_like(x), torch.empty_like(k), torch.empty(H, device="cuda")
    F.causal_fftconv1d_bwd_raw(g, x, k, s, gx, gk, gs)
    gk_sum = torch.zeros_like(k)
    gs_sum = torch.zeros(H, device="cuda")
    for b in range(B):
        gx1, gk1, gs1 = torch.empty_like(x[b:b + 1]), torch.empty_like(k), torch.empty(H, device="cuda")
        F.causal_fftconv1d_bwd_raw(g[b:b + 1].contiguous(), x[b:b + 1].contiguous(), k, s, gx1, gk1, gs1)
        assert rel_l2(gx[b], gx1[0]) < 2e-3
        gk_sum += gk1
        gs_sum += gs1
    torch.testing.assert_close(gk_sum, gk, rtol=1e-5, atol=1e-5 * gk.abs().max().item())
    torch.testing.assert_close(gs_sum, gs, rtol=1e-5, atol=1e-5 * gs.abs().max().item())


def test_retain_graph_second_backward_matches_first():
    torch.manual_seed(9)
    x = torch.randn(1, 2, 20000, device="cuda", requires_grad=True)
    k = torch.randn(1, 2, 20000, device="cuda", requires_grad=True)
    g = torch.randn(1, 2, 20000, device="cuda")
    y = F.causal_fftconv1d_bhl(x, k)
    y.backward(g, retain_graph=True)
    gx1, gk1 = x.grad.clone(), k.grad.clone()
    x.grad = None
    k.grad = None
    y.backward(g)
    assert torch.equal(gx1, x.grad) and torch.equal(gk1, k.grad)


# --- per-sample (FiLM) filters [B, H, K] ------------------------------------------
@pytest.mark.parametrize("B,H,L,K", [(3, 16, 256, 7), (2, 8, 1000, 2000), (2, 5, 4096, 4096), (4, 3, 64, 64),
                                     (2, 3, 16384, 16384), (3, 2, 65536, 1000), (2, 2, 20000, 9000)])
def test_per_sample_filters_fwd_bwd(B, H, L, K):
    """Fused plan (incl. the K > L+1 fold) and 4-step plan, against the oracle's [B, H, K] path
    (fftconv.py:546-600 broadcasts the kernel batch); gk is per image, gs summed over images."""
    torch.manual_seed(11)
    x = torch.randn(B, H, L, requires_grad=True)
    k = torch.randn(B, H, K, requires_grad=True)
    s = torch.randn(H, requires_grad=True)
    y_ref = causal_fftconv1d_torch(x, k, s)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg, kg, sg = (t.detach().cuda().requires_grad_(True) for t in (x, k, s))
    y = F.causal_fftconv1d_bhl(xg, kg, sg)
    y.backward(g.cuda())
    assert kg.grad.shape == (B, H, K)
    assert rel_l2(y_ref, y) < RTOL_F32_L2
    assert rel_l2(x.grad, xg.grad) < RTOL_F32_L2
    assert rel_l2(k.grad, kg.grad) < RTOL_F32_L2
    assert rel_l2(s.grad, sg.grad) < RTOL_F32_L2


@pytest.mark.parametrize("L,K", [(512, 31), (32768, 32768)])
def test_per_sample_filters_equal_per_image_shared_calls_bitwise(L, K):
    torch.manual_seed(12)
    B, H = 3, 4
    x = torch.randn(B, H, L, device="cuda").to(torch.bfloat16)
    k = torch.randn(B, H, K, device="cuda")
    s = torch.randn(H, device="cuda").to(torch.bfloat16)
    y = F.causal_fftconv1d_bhl(x, k, s)
    for b in range(B):
        assert torch.equal(y[b:b + 1], F.causal_fftconv1d_bhl(x[b:b + 1].contiguous(), k[b:b + 1].contiguous(), s))
    yc = F.causal_fftconv1d_bhl_chunked(x, k, s, chunk_size=3)
    assert torch.equal(yc, y)
    y_blh = F.causal_fftconv1d_bhl_w_reshape(x.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous(), s)
    assert torch.equal(y_blh, y.transpose(1, 2))


def test_per_sample_filters_bf16_config3_shape_sample():
    """Config 3's length with per-sample filters on a channel sample (bf16 I/O)."""
    torch.manual_seed(13)
    B, H, L = 2, 2, 262144
    x = torch.randn(B, H, L).to(torch.bfloat16)
    k = torch.randn(B, H, L) * torch.exp(-torch.linspace(0, 20, L))
    y_ref = causal_fftconv1d_torch(x, k)
    y = F.causal_fftconv1d_bhl(x.cuda(), k.cuda())
    assert y.dtype == torch.bfloat16
    assert rel_l2(y_ref, y) < RTOL_BF16_L2


@pytest.mark.parametrize("L", [8192, 65536])
def test_state_budget_zero_recomputes_bitwise(monkeypatch, L):
    """A forward state above NSQ_STATE_MAX_BYTES is not kept; the backward then recomputes the transforms
    and gives the same gradients bit for bit (fused plan: no state either way; 4-step plan: two column passes)."""
    torch.manual_seed(21)
    x = torch.randn(2, 3, L, device="cuda", requires_grad=True)
    k = torch.randn(1, 3, L, device="cuda", requires_grad=True)
    s = torch.randn(3, device="cuda", requires_grad=True)
    g = torch.randn(2, 3, L, device="cuda")
    grads = []
    for budget in (None, "0"):
        if budget is None:
            monkeypatch.delenv("NSQ_STATE_MAX_BYTES", raising=False)
        else:
            monkeypatch.setenv("NSQ_STATE_MAX_BYTES", budget)
        for t in (x, k, s):
            t.grad = None
        F.causal_fftconv1d_bhl(x, k, s).backward(g)
        grads.append([t.grad.clone() for t in (x, k, s)])
    for a, b in zip(*grads):
        assert torch.equal(a, b)
