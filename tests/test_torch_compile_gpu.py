"""torch.compile through the HIP ops.

The reference runs Hyena under torch.compile (experiments/run.py:193-197) and checks that compiled
outputs and gradients match eager (tests/modules/test_torch_compile.py:153-163: rtol/atol 1e-4 for
outputs, 5e-4 for gradients).  Here every HIP op is a torch.library custom op (nsq_hip::*) with a fake
implementation and a registered backward op, so a Hyena-style block built from them compiles with
fullgraph=True.  Each block is checked against its eager run (same kernels: bitwise, or within the
reference test's tolerances where the compiled graph reorders the torch elementwise ops around them) and
against the CPU oracle (rel-L2 <= 1e-4, fp32).  torch.library.opcheck exercises each op's schema, fake
implementation and autograd registration.
"""

import pytest
import torch

from nvsubquadratic_amd import causal_conv1d_hip as CC
from nvsubquadratic_amd import fftconv_hip as F
from nvsubquadratic_amd import gated_fftconv_hip as G
from nvsubquadratic_amd import mixed_fftconv_hip as M
from nvsubquadratic_amd import siren_hip as S
from nvsubquadratic_amd.modules import HipCausalConv1d
from oracle.circular_ref import mixed_fftconv_torch
from oracle.direct_ref import b2b_causal_conv1d_torch, causal_conv1d_torch
from oracle.fftconv_ref import causal_fftconv1d_torch, rel_l2


pytestmark = pytest.mark.gpu


class Hyena1D(torch.nn.Module):
    """Hyena's data path (hyena_nd.py:503-570) in 1D: short conv, gates, causal long conv with shortcut."""

    def __init__(self, H, L, fused_gates=False):
        super().__init__()
        self.short = HipCausalConv1d(3 * H, 3 * H, 3, groups=3 * H, bias=True)
        self.kernel = torch.nn.Parameter(torch.randn(1, H, L) * torch.exp(-4 * torch.arange(L) / L) / 8)
        self.shortcut = torch.nn.Parameter(torch.randn(H))
        self.H, self.fused = H, fused_gates

    def forward(self, u):
        q, k, v = self.short(u).split(self.H, dim=1)
        if self.fused:
            return G.hyena_gated_causal_fftconv1d_bhl(q, k, v, self.kernel, self.shortcut, "silu", "sigmoid")
        y = F.causal_fftconv1d_bhl(q * torch.nn.functional.silu(k), self.kernel, self.shortcut)
        return y * torch.sigmoid(v)


class HyenaND(torch.nn.Module):
    """2D / 3D data path with the non-causal N-d conv (zero-padded or periodic per axis)."""

    def __init__(self, H, S, periodic=None):
        super().__init__()
        nd = len(S)
        self.kernel = torch.nn.Parameter(torch.randn(1, H, *S) / S[0])
        self.shortcut = torch.nn.Parameter(torch.randn(H))
        self.nd, self.periodic = nd, periodic

    def forward(self, q, k, v):
        z = q * torch.sigmoid(k)
        if self.periodic is not None:
            fn = M.mixed_fftconv2d_fp32_bhl if self.nd == 2 else M.mixed_fftconv3d_fp32_bhl
            y = fn(z, self.kernel, self.periodic, self.shortcut)
        else:
            y = (F.fftconv2d_bhl if self.nd == 2 else F.fftconv3d_bhl)(z, self.kernel, self.shortcut)
        return y * torch.nn.functional.silu(v)


def _compare(model, inputs, ref_fn=None, tol_bitwise=True):
    torch.manual_seed(0)
    leaves = [t.clone().requires_grad_(True) for t in inputs]
    y_e = model(*leaves)
    g = torch.randn_like(y_e)
    y_e.backward(g)
    grads_e = [t.grad.clone() for t in leaves] + [p.grad.clone() for p in model.parameters()]
    model.zero_grad()
    leaves_c = [t.clone().requires_grad_(True) for t in inputs]
    torch._dynamo.reset()
    compiled = torch.compile(model, backend="aot_eager", fullgraph=True)
    y_c = compiled(*leaves_c)
    y_c.backward(g)
    grads_c = [t.grad for t in leaves_c] + [p.grad for p in model.parameters()]
    torch.testing.assert_close(y_c, y_e, rtol=1e-4, atol=1e-4)
    for a, b in zip(grads_c, grads_e):
        torch.testing.assert_close(a, b, rtol=5e-4, atol=5e-4)
    if ref_fn is not None:
        y_ref = ref_fn(*[t.detach().cpu() for t in inputs])
        assert rel_l2(y_ref, y_c) < 1e-4
    return y_c


@pytest.mark.parametrize("fused", [False, True])
def test_compile_hyena_1d_causal(fused):
    torch.manual_seed(1)
    H, L = 8, 2048
    m = Hyena1D(H, L, fused).cuda()
    u = torch.randn(2, 3 * H, L, device="cuda")

    def ref(u):
        p = causal_conv1d_torch(u, m.short.weight.detach().cpu()[:, 0], m.short.bias.detach().cpu())
        q, k, v = p.split(H, dim=1)
        y = causal_fftconv1d_torch(q * torch.nn.functional.silu(k), m.kernel.detach().cpu(),
                                   m.shortcut.detach().cpu())
        return y * torch.sigmoid(v)

    _compare(m, [u], ref)


@pytest.mark.parametrize("S,periodic", [((24, 20), None), ((16, 32), (True, True)), ((16, 32), (True, False)),
                                        ((8, 12, 10), None)])
def test_compile_hyena_nd(S, periodic):
    torch.manual_seed(2)
    H = 6
    m = HyenaND(H, S, periodic).cuda()
    q, k, v = (torch.randn(2, H, *S, device="cuda") for _ in range(3))
    per = (False,) * len(S) if periodic is None else periodic

    def ref(q, k, v):
        z = q * torch.sigmoid(k)
        y = mixed_fftconv_torch(z, m.kernel.detach().cpu(), per, m.shortcut.detach().cpu())
        return y * torch.nn.functional.silu(v)

    _compare(m, [q, k, v], ref)


def test_compile_b2b_and_long_causal():
    """The B2B block and the 4-step causal plan (FFT length 2^16) under compile."""
    torch.manual_seed(3)
    C, L = 8, 1024
    wp = torch.nn.Parameter(torch.randn(3 * C, 3, device="cuda") / 3 ** 0.5)
    wm = torch.nn.Parameter(torch.randn(C, 128, device="cuda") / 128 ** 0.5)
    sk = torch.nn.Parameter(torch.randn(C, device="cuda"))

    class B2B(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.wp, self.wm, self.sk = wp, wm, sk

        def forward(self, x):
            return CC.b2b_causal_conv1d(x, self.wp, self.wm, self.sk)

    x = torch.randn(2, 3 * C, L, device="cuda")
    _compare(B2B(), [x], lambda x: b2b_causal_conv1d_torch(x, wp.detach().cpu(), wm.detach().cpu(),
                                                           sk.detach().cpu()))

    class Long(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.k = torch.nn.Parameter(torch.randn(1, 3, 40000, device="cuda") / 200)

        def forward(self, x):
            return F.causal_fftconv1d_bhl(x, self.k)

    long_model = Long()
    xl = torch.randn(1, 3, 40000, device="cuda")
    _compare(long_model, [xl], lambda x: causal_fftconv1d_torch(x, long_model.k.detach().cpu()))


def _opchecks():
    d = dict(device="cuda")
    x1, k1, s1 = torch.randn(2, 4, 256, **d), torch.randn(4, 100, **d), torch.randn(4, **d)
    x2, k2 = torch.randn(2, 4, 12, 10, **d), torch.randn(4, 5, 3, **d)
    xc, wc, bc = torch.randn(2, 6, 300, **d), torch.randn(6, 4, **d), torch.randn(6, **d)
    xb = torch.randn(2, 12, 300, **d)
    q, kg, v = (torch.randn(2, 4, 256, **d) for _ in range(3))
    qn, kgn, vn = (torch.randn(2, 4, 12, 10, **d) for _ in range(3))
    gs = torch.linspace(0, 1, 8200, **d).reshape(-1, 1)  # SIREN grid [G, 1]
    w0, b0 = torch.randn(16, 1, **d), torch.randn(16, **d)
    wh, bh = torch.randn(2 * 16 * 16, **d) / 4, torch.randn(2 * 16, **d)
    act = torch.cat([torch.randn(16, 8200, **d), torch.ones(1, 8200, **d)])  # [a^T; 1]
    return [
        (F.causal_fftconv1d_op, (x1, k1, s1, 1, False)),
        (F.fftconv_nd_op, (x2, k2, s1, 1, 0, False)),
        (F.fftconv_nd_op, (torch.randn(2, 4, 16, 10, **d), k2, None, 1, 1, False)),
        (F.shifted_fftconv1d_op, (x1, k1, s1, 1, 1)),
        (CC.causal_conv1d_op, (xc, wc, bc, 1)),
        (CC.b2b_causal_conv1d_op, (xb, torch.randn(12, 3, **d), torch.randn(4, 16, **d), torch.randn(4, **d))),
        (G.gated_causal_fftconv1d_op, (q, kg, v, k1, s1, 2, 1, 1, True)),
        (G.gated_fftconv_nd_op, (qn, kgn, vn, k2, s1, 2, 1, 1, 0, True)),
        (S.siren_mlp_op, (gs, w0, b0, wh, bh, 2, 16)),
        (S.siren_readout_causal_fftconv1d_op, (torch.randn(1, 4, 8200, **d), act, torch.randn(4, 16, **d),
                                               torch.randn(4, **d), s1, True)),
    ]


@pytest.mark.parametrize("i", range(10))
def test_opcheck(i):
    op, args = _opchecks()[i]
    args = tuple(a.requires_grad_(True) if isinstance(a, torch.Tensor) and a.is_floating_point() else a
                 for a in args)
    torch.library.opcheck(op, args, test_utils=("test_schema", "test_autograd_registration", "test_faketensor"))
