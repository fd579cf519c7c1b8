"""GPU parity of the causal 1D FFT conv's team plan (one cooperative kernel per direction, the
column/row exchange kept in the XCD's L2; selected with NSQ_1D_PLAN=team) against the default
multi-kernel plan (bitwise: both run the same transforms in the same order) and the oracle.

The team plan covers B = 1, a shared filter and FFT length 2^19 (config 3's band).  Its
workspace starts with a control block whose int32 status word (byte 68) is 0 after a call
whose team barriers all completed, 1 if any wait timed out.
"""

import pytest
import torch

from nvsubquadratic_amd import _lib
from nvsubquadratic_amd import fftconv_hip as F
from nvsubquadratic_amd.workloads import causal1d_case_fast
from oracle.fftconv_ref import causal_fftconv1d_np, causal_fftconv1d_torch, rel_l2


pytestmark = pytest.mark.gpu

STATUS_BYTE = 68


def _run(x, k, s, g):
    lib = _lib.get_lib()
    B, H, L = x.shape
    K = k.shape[-1]
    need = lib.nsq_fftconv1d_causal_workspace_bytes(B, H, L, K, _lib.NSQ_DIR_BWD)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    y = torch.empty_like(x)
    F.causal_fftconv1d_fwd_raw(x, k, s, y, ws)
    torch.cuda.synchronize()
    st_fwd = int(ws[STATUS_BYTE:STATUS_BYTE + 4].view(torch.int32).item())
    gx, gk, gs = torch.empty_like(x), torch.empty_like(k), torch.empty(H, device="cuda")
    F.causal_fftconv1d_bwd_raw(g, x, k, s, gx, gk, gs, ws, fwd_state=True)
    torch.cuda.synchronize()
    st_bwd = int(ws[STATUS_BYTE:STATUS_BYTE + 4].view(torch.int32).item())
    return (y, gx, gk, gs), need, (st_fwd, st_bwd)


@pytest.mark.parametrize("H,L,K,dtype", [(16, 262144, 262144, torch.float32), (12, 262144, 262144, torch.bfloat16),
                                         (3, 300000, 50000, torch.float32), (5, 140000, 140000, torch.float16)])
def test_team_plan_equals_multi_kernel_plan_and_oracle(monkeypatch, H, L, K, dtype):
    c = causal1d_case_fast(1, H, L, dtype, (1.0, 50.0), device="cuda", seed=3)
    k = c.k[:, :K].contiguous()
    print(f"team plan H={H} L={L} K={K} {dtype}", flush=True)
    monkeypatch.setenv("NSQ_1D_PLAN", "team")
    team, need_team, status = _run(c.x, k, c.s, c.g)
    assert status == (0, 0)
    monkeypatch.setenv("NSQ_1D_PLAN", "multi")
    multi, need_multi, _ = _run(c.x, k, c.s, c.g)
    assert need_team < need_multi or H < 64  # its workspace does not grow with D
    for a, b in zip(team, multi):
        assert torch.equal(a, b)
    tol = 1e-4 if dtype == torch.float32 else 5e-3
    for h in (0, H - 1):
        y64 = causal_fftconv1d_np(c.x[:, h:h + 1].float().cpu().numpy(), k[h:h + 1].cpu().numpy(),
                                  c.s[h:h + 1].float().cpu().numpy())
        assert rel_l2(y64, team[0][:, h:h + 1]) < tol


def test_team_plan_through_autograd(monkeypatch):
    monkeypatch.setenv("NSQ_1D_PLAN", "team")
    H, L = 6, 262144
    c = causal1d_case_fast(1, H, L, torch.float32, (1.0, 50.0), device="cpu", seed=9)
    x, k, s = (t.clone().requires_grad_(True) for t in (c.x, c.k[None], c.s))
    y_ref = causal_fftconv1d_torch(x, k, s)
    y_ref.backward(c.g)
    xg, kg, sg = (t.detach().cuda().requires_grad_(True) for t in (x, k, s))
    y = F.causal_fftconv1d_bhl(xg, kg, sg)
    y.backward(c.g.cuda())
    assert rel_l2(y_ref, y) < 1e-4
    for a, b in ((x, xg), (k, kg), (s, sg)):
        assert rel_l2(a.grad, b.grad) < 1e-4
